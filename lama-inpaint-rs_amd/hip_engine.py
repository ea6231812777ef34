"""ctypes binding of liblama_hip.so (include/lama_hip.h), mirroring the
reference's engine interface: `run(store, model, input, h, w)` is
`cuda::run` (lama-rs/src/cuda.rs:1542-1548) and raises where it returns Err.

There is no fallback: if the library is not built or no gfx950 device can be
opened, every call raises.
"""
import ctypes
import os

import numpy as np

from . import host_api

HERE = os.path.dirname(os.path.abspath(__file__))
HIP_SO = os.path.join(HERE, "lib", "liblama_hip.so")

FAMILIES = ["conv7x7", "conv3x3s2", "conv3x3", "conv1x1", "convt", "rfft2", "irfft2", "tail", "finalize",
            "conv1x1res", "conv3x3g2l", "build_input"]
N_STEPS = 29

_lib = None


class LaunchTime(ctypes.Structure):
    _fields_ = [("family", ctypes.c_int32), ("stream", ctypes.c_int32), ("start_us", ctypes.c_double),
                ("end_us", ctypes.c_double)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(HIP_SO):
            raise RuntimeError(f"{HIP_SO} is not built: the HIP backend is unavailable (run __graft_entry__.build())")
        host_api.lib()  # liblama_hip.so links liblama_host.so
        L = ctypes.CDLL(HIP_SO)
        vp, cp, sz = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t
        fp = ctypes.POINTER(ctypes.c_float)
        L.lama_hip_open.argtypes = [ctypes.POINTER(vp), cp, sz]
        L.lama_hip_close.argtypes = [vp]
        L.lama_hip_load_weights.argtypes = [vp, vp, sz, ctypes.POINTER(host_api.TensorInfo), sz, cp, sz]
        L.lama_hip_forward.argtypes = [vp, fp, ctypes.c_int, ctypes.c_int, fp, cp, sz]
        L.lama_hip_forward_device.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, cp, sz]
        L.lama_hip_forward_steps.argtypes = [vp, fp, ctypes.c_int, ctypes.c_int, fp, ctypes.POINTER(fp), cp, sz]
        L.lama_hip_vram.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64), cp, sz, cp, sz]
        L.lama_hip_profile.argtypes = [vp, ctypes.c_uint32]
        L.lama_hip_profile_reset.argtypes = [vp]
        L.lama_hip_profile_read.argtypes = [vp, ctypes.c_int, cp, sz, ctypes.POINTER(ctypes.c_uint64),
                                            ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_double)]
        L.lama_hip_print_stats.argtypes = [vp]
        L.lama_hip_timeline.argtypes = [vp, ctypes.c_int]
        L.lama_hip_timeline_read.argtypes = [vp, ctypes.POINTER(LaunchTime), ctypes.c_int]
        L.lama_hip_profile_read_clock.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64),
                                                  ctypes.POINTER(ctypes.c_double)]
        L.lama_hip_launch_count.argtypes = [vp, ctypes.c_int, ctypes.c_int]
        L.lama_hip_plan_signature.argtypes = []
        L.lama_hip_plan_signature.restype = cp
        L.lama_hip_kernel_name.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                           ctypes.c_size_t]
        L.lama_hip_plan_bytes.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64),
                                          ctypes.POINTER(ctypes.c_uint64), cp, sz]
        L.lama_hip_malloc.argtypes = [vp, sz, ctypes.POINTER(vp), cp, sz]
        L.lama_hip_free.argtypes = [vp, vp]
        L.lama_hip_memcpy.argtypes = [vp, vp, vp, sz, ctypes.c_int, cp, sz]
        L.lama_hip_synchronize.argtypes = [vp, cp, sz]
        L.lama_hip_op_conv2d.argtypes = [vp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, fp, fp, ctypes.c_int, fp, cp, sz]
        L.lama_hip_op_conv_transpose.argtypes = [vp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp,
                                                 ctypes.c_int, fp, fp, ctypes.c_int, fp, cp, sz]
        L.lama_hip_op_rfft2.argtypes = [vp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, cp, sz]
        L.lama_hip_op_irfft2.argtypes = [vp, fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, cp, sz]
        L.lama_hip_op_tail.argtypes = [vp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp, fp, cp, sz]
        L.lama_hip_forward_device_noalloc.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, cp, sz]
        u8p = ctypes.POINTER(ctypes.c_uint8)
        L.lama_hip_inpaint.argtypes = [vp, u8p, u8p, ctypes.c_int, ctypes.c_int, u8p, fp, cp, sz]
        L.lama_hip_inpaint_device.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, cp, sz]
        L.lama_hip_spectral.argtypes = [vp, ctypes.c_int, fp, ctypes.c_int, ctypes.c_int, fp, ctypes.POINTER(fp),
                                        cp, sz]
        L.lama_hip_spectral_device.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, vp, vp, cp, sz]
        _lib = L
    return _lib


def _f(a):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _c(a):
    return None if a is None else np.ascontiguousarray(a, np.float32)


class HipError(RuntimeError):
    pass


class Engine:
    """One device context (lama_hip_open) with resident weights."""

    def __init__(self):
        self._err = ctypes.create_string_buffer(4096)
        h = ctypes.c_void_p()
        if lib().lama_hip_open(ctypes.byref(h), self._err, 4096):
            raise HipError(self._msg())
        self.ctx = h

    def _msg(self):
        return self._err.value.decode(errors="replace")

    def _check(self, rc):
        if rc:
            raise HipError(self._msg())

    def close(self):
        if getattr(self, "ctx", None):
            lib().lama_hip_close(self.ctx)
            self.ctx = None

    def __del__(self):
        self.close()

    def load_weights(self, store):
        """store: host_api.Store (the mapped container and its index)."""
        ptr, n = store.bytes_ptr()
        self._store = store  # the container must outlive the call
        self._check(lib().lama_hip_load_weights(self.ctx, ptr, n, store.table(), len(store), self._err, 4096))

    def forward(self, x):
        x = _c(x)
        _, h, w = x.shape
        out = np.empty((3, h, w), np.float32)
        self._check(lib().lama_hip_forward(self.ctx, _f(x), h, w, _f(out), self._err, 4096))
        return out

    def forward_steps(self, x, steps):
        """Forward that also returns {step: activation} for the requested
        plan steps (the reference's LAMA_DUMP_STEP layout)."""
        x = _c(x)
        _, h, w = x.shape
        out = np.empty((3, h, w), np.float32)
        arr = (ctypes.POINTER(ctypes.c_float) * N_STEPS)()
        dumps = {}
        for s in steps:
            d = np.empty(step_numel(s, h, w), np.float32)
            dumps[s] = d
            arr[s] = _f(d)
        self._check(lib().lama_hip_forward_steps(self.ctx, _f(x), h, w, _f(out), arr, self._err, 4096))
        return out, dumps

    def forward_device(self, d_in, h, w, d_out, stream=None):
        self._check(lib().lama_hip_forward_device(self.ctx, d_in, h, w, d_out, stream, self._err, 4096))

    def forward_device_noalloc(self, d_in, h, w, d_out, stream=None):
        """lama_hip_forward_device on the device's scratch array: no allocation."""
        self._check(lib().lama_hip_forward_device_noalloc(self.ctx, d_in, h, w, d_out, stream, self._err, 4096))

    def inpaint(self, rgb, mask, net_out=False):
        """The whole-image flow on the device (lama_hip_inpaint): u8 HWC image
        and [h][w] mask -> the u8 HWC composite; with net_out=True also the
        [3][H][W] sigmoid plane of the padded shape."""
        rgb = np.ascontiguousarray(rgb, np.uint8)
        mask = np.ascontiguousarray(mask, np.uint8)
        h, w = mask.shape
        assert rgb.shape == (h, w, 3)
        out = np.empty((h, w, 3), np.uint8)
        net = np.empty((3, h + (-h) % 8, w + (-w) % 8), np.float32) if net_out else None
        u8 = ctypes.POINTER(ctypes.c_uint8)
        self._check(lib().lama_hip_inpaint(self.ctx, rgb.ctypes.data_as(u8), mask.ctypes.data_as(u8), h, w,
                                           out.ctypes.data_as(u8), _f(net), self._err, 4096))
        return (out, net) if net_out else out

    def inpaint_device(self, d_rgb, d_mask, h, w, d_out, stream=None):
        self._check(lib().lama_hip_inpaint_device(self.ctx, d_rgb, d_mask, h, w, d_out, stream, self._err, 4096))

    def spectral(self, k, x, stages=False):
        """FFC k's SpectralTransform alone over x [384][h][w] (lama_hip_spectral);
        with stages=True also (f, spectrum, FU conv output, f + irfft2)."""
        x = _c(x)
        _, h, w = x.shape
        out = np.empty((384, h, w), np.float32)
        arr = None
        st = None
        if stages:
            wh = w // 2 + 1
            st = [np.empty((192, h, w), np.float32), np.empty((384, h, wh), np.float32),
                  np.empty((384, h, wh), np.float32), np.empty((192, h, w), np.float32)]
            arr = (ctypes.POINTER(ctypes.c_float) * 4)(*[_f(a) for a in st])
        self._check(lib().lama_hip_spectral(self.ctx, k, _f(x), h, w, _f(out), arr, self._err, 4096))
        return (out, st) if stages else out

    def spectral_device(self, k, d_x, h, w, d_out, stream=None):
        self._check(lib().lama_hip_spectral_device(self.ctx, k, d_x, h, w, d_out, stream, self._err, 4096))

    # device buffers
    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self._check(lib().lama_hip_malloc(self.ctx, nbytes, ctypes.byref(p), self._err, 4096))
        return p.value

    def free(self, p):
        lib().lama_hip_free(self.ctx, p)

    def upload(self, dptr, a):
        a = np.ascontiguousarray(a)
        self._check(lib().lama_hip_memcpy(self.ctx, dptr, a.ctypes.data, a.nbytes, 1, self._err, 4096))

    def download(self, a, dptr):
        self._check(lib().lama_hip_memcpy(self.ctx, a.ctypes.data, dptr, a.nbytes, 2, self._err, 4096))
        return a

    def copy_d2d(self, dst, src, nbytes):
        self._check(lib().lama_hip_memcpy(self.ctx, dst, src, nbytes, 3, self._err, 4096))

    def synchronize(self):
        self._check(lib().lama_hip_synchronize(self.ctx, self._err, 4096))

    # profiling
    def profile(self, families):
        mask = 0
        for f in families:
            mask |= 1 << FAMILIES.index(f)
        lib().lama_hip_profile(self.ctx, mask)

    def profile_reset(self):
        lib().lama_hip_profile_reset(self.ctx)

    def profile_read(self):
        out = {}
        name = ctypes.create_string_buffer(64)
        n = ctypes.c_uint64()
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        i = 0
        while lib().lama_hip_profile_read(self.ctx, i, name, 64, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl),
                                          ctypes.byref(by)):
            cn, cms = ctypes.c_uint64(), ctypes.c_double()
            lib().lama_hip_profile_read_clock(self.ctx, i, ctypes.byref(cn), ctypes.byref(cms))
            out[name.value.decode()] = dict(launches=n.value, ms=ms.value, flops=fl.value, bytes=by.value,
                                            clock_launches=cn.value, clock_ms=cms.value)
            i += 1
        return out

    def timeline(self, on):
        """Record every launch's kernel-clock window (lama_hip_timeline)."""
        self._check(lib().lama_hip_timeline(self.ctx, int(bool(on))) and "lama_hip_timeline failed")

    def timeline_read(self, max_launches=1 << 16):
        """[(family name, stream, start_us, end_us)] in issue order."""
        buf = (LaunchTime * max_launches)()
        n = lib().lama_hip_timeline_read(self.ctx, buf, max_launches)
        if n < 0:
            raise HipError("lama_hip_timeline_read failed")
        return [(FAMILIES[r.family], r.stream, r.start_us, r.end_us) for r in buf[:n]]

    def print_stats(self):
        lib().lama_hip_print_stats(self.ctx)

    def launch_count(self, h, w):
        return lib().lama_hip_launch_count(self.ctx, h, w)

    def kernel_name(self, h, w, family):
        """The kernel symbol of the first `family` launch of the plan at h x w,
        or None (no such plan or launch)."""
        buf = ctypes.create_string_buffer(128)
        if lib().lama_hip_kernel_name(self.ctx, h, w, FAMILIES.index(family), buf, 128) != 0:
            return None
        return buf.value.decode()

    def plan_bytes(self, h, w):
        """(activation arena bytes at h x w, resident weight bytes)."""
        a, wb = ctypes.c_uint64(), ctypes.c_uint64()
        self._check(lib().lama_hip_plan_bytes(self.ctx, h, w, ctypes.byref(a), ctypes.byref(wb), self._err, 4096))
        return a.value, wb.value

    # single kernel families (parity tests)
    def op_conv2d(self, x, wt, bias=None, stride=1, scale=None, shift=None, relu=False):
        x, wt, bias, scale, shift = map(_c, (x, wt, bias, scale, shift))
        cin, h, w = x.shape
        cout, _, k, _ = wt.shape
        pad = k // 2
        oh, ow = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
        out = np.empty((cout, oh, ow), np.float32)
        self._check(lib().lama_hip_op_conv2d(self.ctx, _f(x), cin, h, w, _f(wt), _f(bias), cout, k, stride,
                                             _f(scale), _f(shift), int(relu), _f(out), self._err, 4096))
        return out

    def op_conv_transpose(self, x, wt, bias, scale=None, shift=None, relu=False):
        x, wt, bias, scale, shift = map(_c, (x, wt, bias, scale, shift))
        cin, h, w = x.shape
        cout = wt.shape[1]
        out = np.empty((cout, 2 * h, 2 * w), np.float32)
        self._check(lib().lama_hip_op_conv_transpose(self.ctx, _f(x), cin, h, w, _f(wt), _f(bias), cout, _f(scale),
                                                     _f(shift), int(relu), _f(out), self._err, 4096))
        return out

    def op_rfft2(self, x):
        x = _c(x)
        c, h, w = x.shape
        out = np.empty((2 * c, h, w // 2 + 1), np.float32)
        self._check(lib().lama_hip_op_rfft2(self.ctx, _f(x), c, h, w, _f(out), self._err, 4096))
        return out

    def op_irfft2(self, spec, w, feat=None):
        spec, feat = _c(spec), _c(feat)
        c2, h, _ = spec.shape
        out = np.empty((c2 // 2, h, w), np.float32)
        self._check(lib().lama_hip_op_irfft2(self.ctx, _f(spec), _f(feat), c2 // 2, h, w, _f(out), self._err, 4096))
        return out

    def op_tail(self, x, wt, bias):
        x, wt, bias = map(_c, (x, wt, bias))
        cin, h, w = x.shape
        out = np.empty((3, h, w), np.float32)
        self._check(lib().lama_hip_op_tail(self.ctx, _f(x), cin, h, w, _f(wt), _f(bias), _f(out), self._err, 4096))
        return out


def step_numel(step, h, w):
    h8, w8 = h // 8, w // 8
    table = {0: 4 * (h + 6) * (w + 6), 1: 64 * h * w, 2: 128 * (h // 2) * (w // 2), 3: 256 * (h // 4) * (w // 4),
             24: 256 * (h // 4) * (w // 4), 25: 128 * (h // 2) * (w // 2), 26: 64 * h * w,
             27: 64 * (h + 6) * (w + 6), 28: 3 * h * w}
    return table.get(step, 512 * h8 * w8 if 4 <= step <= 23 else 0)


def vram():
    """mem.rs device_memory(): (free, total, name) or None."""
    f, t = ctypes.c_uint64(), ctypes.c_uint64()
    name = ctypes.create_string_buffer(256)
    err = ctypes.create_string_buffer(1024)
    if lib().lama_hip_vram(ctypes.byref(f), ctypes.byref(t), name, 256, err, 1024):
        return None
    return f.value, t.value, name.value.decode()


_ENGINE = None


def plan_signature():
    """model::describe (model.rs:260-274) of the plan the backend hard-codes."""
    return lib().lama_hip_plan_signature().decode()


def run(store, model, input, h, w):
    """cuda::run: one forward over [4][h][w] -> [3][h][w] with a
    process-wide engine whose weights stay resident (cuda.rs:222-231).
    `model` is None or the model's describe() line; a line other than the
    backend's plan signature is refused before any device work, as a plan
    mismatch rather than a later tensor-shape error."""
    global _ENGINE
    if model is not None and str(model) != plan_signature():
        raise HipError(f"hip backend: plan mismatch (model: {model}; backend: {plan_signature()})")
    if _ENGINE is None or getattr(_ENGINE, "_store", None) is not store:
        if _ENGINE is None:
            _ENGINE = Engine()
        _ENGINE.load_weights(store)
    x = np.asarray(input, np.float32).reshape(4, h, w)
    return _ENGINE.forward(x)
