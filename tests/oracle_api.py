"""ctypes binding of the CPU oracle (oracle/lama_oracle.c).

Test infrastructure: the oracle is the checker, never the thing measured or
shipped.  The weight table handed to `OracleNet` is parsed here with Python's
own json module, independently of the product's safetensors reader.
"""
import ctypes
import json
import os
import struct

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.environ.get("LAMA_ORACLE_SO") or os.path.join(ROOT, "oracle", "_build", "liblama_oracle.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle not built: {ORACLE_SO} (run `make -C oracle`)")
        L = ctypes.CDLL(ORACLE_SO)
        fp = ctypes.POINTER(ctypes.c_float)
        L.or_reflect_index.restype = ctypes.c_size_t
        L.or_reflect_index.argtypes = [ctypes.c_long, ctypes.c_size_t]
        L.or_conv2d.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp, ctypes.c_int,
                                ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp]
        L.or_conv1x1.argtypes = [fp, ctypes.c_int, ctypes.c_long, fp, fp, ctypes.c_int, fp]
        L.or_conv_transpose.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp, ctypes.c_int, fp]
        L.or_rfft2_ortho.argtypes = [fp, ctypes.c_int, ctypes.c_int, fp]
        L.or_irfft2_ortho.argtypes = [fp, ctypes.c_int, ctypes.c_int, fp]
        L.or_bn_fold.argtypes = [fp, fp, fp, fp, ctypes.c_int, fp, fp]
        L.or_reflect_pad.argtypes = [fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp]
        L.or_net_load.restype = ctypes.c_void_p
        L.or_net_load.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        L.or_net_free.argtypes = [ctypes.c_void_p]
        L.or_net_forward.argtypes = [ctypes.c_void_p, fp, ctypes.c_int, ctypes.c_int, fp,
                                     ctypes.POINTER(fp)]
        L.or_step_numel.restype = ctypes.c_long
        L.or_step_numel.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        u8p = ctypes.POINTER(ctypes.c_uint8)
        L.or_build_input.argtypes = [u8p, u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp]
        L.or_composite.argtypes = [u8p, u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, u8p]
        L.or_num_threads.restype = ctypes.c_int
        L.or_net_spectral.argtypes = [ctypes.c_void_p, ctypes.c_int, fp, ctypes.c_int, ctypes.c_int, fp,
                                      ctypes.POINTER(fp)]
        _lib = L
    return _lib


def _f(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u8(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def reflect_index(i, n):
    return lib().or_reflect_index(i, n)


def conv2d(x, w, bias=None, pad=0, stride=1, reflect=True):
    x, w = f32(x), f32(w)
    cin, h, wd = x.shape
    cout, _, kh, kw = w.shape
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (wd + 2 * pad - kw) // stride + 1
    out = np.empty((cout, oh, ow), np.float32)
    b = f32(bias) if bias is not None else None
    lib().or_conv2d(_f(x), cin, h, wd, _f(w), _f(b) if b is not None else None, cout, kh, kw, pad, stride,
                    1 if reflect else 0, _f(out))
    return out


def conv1x1(x, w, bias=None):
    x, w = f32(x), f32(w)
    cin = x.shape[0]
    cout = w.shape[0]
    out = np.empty((cout,) + x.shape[1:], np.float32)
    b = f32(bias) if bias is not None else None
    lib().or_conv1x1(_f(x), cin, int(np.prod(x.shape[1:])), _f(w.reshape(cout, cin)),
                     _f(b) if b is not None else None, cout, _f(out))
    return out


def conv_transpose(x, w, bias):
    x, w, bias = f32(x), f32(w), f32(bias)
    cin, h, wd = x.shape
    cout = w.shape[1]
    out = np.empty((cout, 2 * h, 2 * wd), np.float32)
    lib().or_conv_transpose(_f(x), cin, h, wd, _f(w), _f(bias), cout, _f(out))
    return out


def rfft2_ortho(x):
    x = f32(x)
    h, w = x.shape
    out = np.empty((2, h, w // 2 + 1), np.float32)
    lib().or_rfft2_ortho(_f(x), h, w, _f(out))
    return out


def irfft2_ortho(spec, w):
    spec = f32(spec)
    h = spec.shape[1]
    out = np.empty((h, w), np.float32)
    lib().or_irfft2_ortho(_f(spec), h, w, _f(out))
    return out


def bn_fold(w, b, mean, var):
    w, b, mean, var = map(f32, (w, b, mean, var))
    n = w.shape[0]
    s = np.empty(n, np.float32)
    t = np.empty(n, np.float32)
    lib().or_bn_fold(_f(w), _f(b), _f(mean), _f(var), n, _f(s), _f(t))
    return s, t


def reflect_pad(x, pad):
    x = f32(x)
    c, h, w = x.shape
    out = np.empty((c, h + 2 * pad, w + 2 * pad), np.float32)
    lib().or_reflect_pad(_f(x), c, h, w, pad, _f(out))
    return out


def build_input(rgb, mask, pad_h, pad_w):
    rgb = np.ascontiguousarray(rgb, np.uint8)
    mask = np.ascontiguousarray(mask, np.uint8)
    h, w = mask.shape
    out = np.empty((4, h + pad_h, w + pad_w), np.float32)
    lib().or_build_input(_u8(rgb), _u8(mask), h, w, pad_h, pad_w, _f(out))
    return out


def composite(rgb, mask, net, pad_h, pad_w):
    rgb = np.ascontiguousarray(rgb, np.uint8)
    mask = np.ascontiguousarray(mask, np.uint8)
    net = f32(net)
    h, w = mask.shape
    out = np.empty((h, w, 3), np.uint8)
    lib().or_composite(_u8(rgb), _u8(mask), h, w, pad_h, pad_w, _f(net), _u8(out))
    return out


def step_numel(step, h, w):
    return lib().or_step_numel(step, h, w)


N_STEPS = 29


def read_safetensors(path):
    """Parse a safetensors file with the json module: {name: np.ndarray}, in order."""
    with open(path, "rb") as fh:
        raw = fh.read()
    (hl,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + hl])
    base = 8 + hl
    out = {}
    items = [(k, v) for k, v in header.items() if k != "__metadata__"]
    items.sort(key=lambda kv: kv[1]["data_offsets"][0])
    for k, v in items:
        assert v["dtype"] == "F32", k
        a, b = v["data_offsets"]
        out[k] = np.frombuffer(raw, dtype="<f4", count=(b - a) // 4, offset=base + a).reshape(v["shape"])
    return out


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.POINTER(ctypes.c_float)),
                ("ndim", ctypes.c_int), ("shape", ctypes.c_long * 4)]


class OracleNet:
    """The reference's CPU engine (cpu::Net) over a {name: array} weight dict."""

    def __init__(self, weights):
        self._keep = {k: f32(v) for k, v in weights.items()}
        arr = (_Tensor * len(self._keep))()
        self._names = []
        for i, (k, v) in enumerate(self._keep.items()):
            nm = k.encode()
            self._names.append(nm)
            arr[i].name = nm
            arr[i].data = _f(v)
            arr[i].ndim = v.ndim
            for d in range(4):
                arr[i].shape[d] = v.shape[d] if d < v.ndim else 1
        self._arr = arr
        err = ctypes.create_string_buffer(512)
        self._net = lib().or_net_load(ctypes.cast(arr, ctypes.c_void_p), len(self._keep), err, 512)
        if not self._net:
            raise RuntimeError(err.value.decode())

    def forward(self, x, steps=False):
        """x: [4][h][w] -> [3][h][w]; with steps=True also the 29 step dumps."""
        x = f32(x)
        _, h, w = x.shape
        out = np.empty((3, h, w), np.float32)
        bufs = None
        dumps = []
        if steps:
            bufs = (ctypes.POINTER(ctypes.c_float) * N_STEPS)()
            for i in range(N_STEPS):
                d = np.empty(step_numel(i, h, w), np.float32)
                dumps.append(d)
                bufs[i] = _f(d)
        lib().or_net_forward(self._net, _f(x), h, w, _f(out), bufs)
        return (out, dumps) if steps else out

    def spectral(self, k, x, stages=False):
        """FFC k's SpectralTransform alone (Spectral::forward, cpu.rs:239-265)
        over x [384][h][w]; with stages=True also (f, spectrum, FU conv output,
        f + FU(f)), the LAMA_DUMP_SPECTRAL stages."""
        x = f32(x)
        _, h, w = x.shape
        out = np.empty((384, h, w), np.float32)
        st = None
        arr = None
        if stages:
            wh = w // 2 + 1
            st = [np.empty((192, h, w), np.float32), np.empty((384, h, wh), np.float32),
                  np.empty((384, h, wh), np.float32), np.empty((192, h, w), np.float32)]
            arr = (ctypes.POINTER(ctypes.c_float) * 4)(*[_f(a) for a in st])
        if lib().or_net_spectral(self._net, k, _f(x), h, w, _f(out), arr):
            raise ValueError(f"no SpectralTransform {k}")
        return (out, st) if stages else out

    def __del__(self):
        if getattr(self, "_net", None):
            lib().or_net_free(self._net)
            self._net = None


def calibrated_weights(src_path, dst_path, image_hw=64, seed_image=1, seed_mask=2):
    """Writes a copy of `src_path` whose BN running statistics are re-fitted,
    by one oracle forward on a seeded image, to the statistics of each BN's own
    input ("calibrated-BN" fixture: activations stay O(1), so the final 8-bit
    output is not saturated).  Payload offsets are unchanged."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "lama-inpaint-rs_amd"))
    import host_api as H
    W = read_safetensors(src_path)
    net = OracleNet(W)
    img = H.synth_image(image_hw, image_hw, seed_image)
    m, _ = H.synth_mask_rect(image_hw, image_hw, max(1, image_hw // 4), max(1, image_hw // 6), seed_mask)
    x = H.build_input(img, m)
    out = np.empty((3, image_hw, image_hw), np.float32)
    L = lib()
    L.or_net_calibrate.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_float)]
    L.or_net_bn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_int,
                            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    L.or_net_calibrate(net._net, _f(x), image_hw, image_hw, _f(out))
    with open(src_path, "rb") as fh:
        raw = bytearray(fh.read())
    (hl,) = struct.unpack("<Q", raw[:8])
    header = json.loads(bytes(raw[8:8 + hl]))
    base = 8 + hl
    i = 0
    pref = ctypes.create_string_buffer(256)
    while True:
        n = L.or_net_bn(net._net, i, pref, 256, None, None)
        if n == 0:
            break
        mean = np.empty(n, np.float32)
        var = np.empty(n, np.float32)
        L.or_net_bn(net._net, i, pref, 256, _f(mean), _f(var))
        p = pref.value.decode()
        for key, arr in ((p + ".running_mean", mean), (p + ".running_var", var)):
            a, b = header[key]["data_offsets"]
            raw[base + a:base + b] = arr.astype("<f4").tobytes()
        i += 1
    with open(dst_path, "wb") as fh:
        fh.write(raw)
    return i
