"""ctypes binding of liblama_host.so (include/lama_host.h): the weight
container, synthetic fixtures, PNG codec, input builder, composite and the
--tile/--sections window geometry."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HOST_SO = os.path.join(HERE, "lib", "liblama_host.so")

_lib = None


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("ndim", ctypes.c_int32), ("shape", ctypes.c_int64 * 4),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class Tile(ctypes.Structure):
    _fields_ = [("x0", ctypes.c_int64), ("y0", ctypes.c_int64), ("side", ctypes.c_int64),
                ("bbox_w", ctypes.c_int64), ("bbox_h", ctypes.c_int64)]


class Section(ctypes.Structure):
    _fields_ = [("x0", ctypes.c_int64), ("y0", ctypes.c_int64), ("x1", ctypes.c_int64), ("y1", ctypes.c_int64)]

    def astuple(self):
        return (self.x0, self.y0, self.x1, self.y1)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(HOST_SO):
            raise RuntimeError(f"{HOST_SO} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(HOST_SO)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        fp = ctypes.POINTER(ctypes.c_float)
        L.lama_store_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.c_char_p, ctypes.c_size_t]
        L.lama_store_close.argtypes = [ctypes.c_void_p]
        L.lama_store_bytes.restype = ctypes.c_void_p
        L.lama_store_bytes.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
        L.lama_store_count.restype = ctypes.c_size_t
        L.lama_store_count.argtypes = [ctypes.c_void_p]
        L.lama_store_table.restype = ctypes.POINTER(TensorInfo)
        L.lama_store_table.argtypes = [ctypes.c_void_p]
        L.lama_store_total_bytes.restype = ctypes.c_uint64
        L.lama_store_total_bytes.argtypes = [ctypes.c_void_p]
        L.lama_synth_weights.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t]
        L.lama_synth_image.argtypes = [u8p, ctypes.c_int, ctypes.c_int, ctypes.c_uint64]
        L.lama_synth_mask_rect.argtypes = [u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_uint64, ctypes.POINTER(ctypes.c_int),
                                           ctypes.POINTER(ctypes.c_int)]
        L.lama_synth_mask_strokes.restype = ctypes.c_double
        L.lama_synth_mask_strokes.argtypes = [u8p, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_uint64]
        L.lama_reflect_index.restype = ctypes.c_size_t
        L.lama_reflect_index.argtypes = [ctypes.c_long, ctypes.c_size_t]
        L.lama_build_input.argtypes = [u8p, u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp]
        L.lama_composite.argtypes = [u8p, u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, u8p]
        L.lama_window_origin.restype = ctypes.c_int64
        L.lama_window_origin.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
        L.lama_tile_rect.argtypes = [u8p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Tile)]
        L.lama_mask_depth.argtypes = [u8p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint32)]
        L.lama_section_rects.restype = ctypes.c_size_t
        L.lama_section_rects.argtypes = [u8p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Section), ctypes.c_size_t]
        L.lama_png_read_rgb.argtypes = [ctypes.c_char_p, ctypes.POINTER(u8p), ctypes.POINTER(ctypes.c_int),
                                        ctypes.POINTER(ctypes.c_int), ctypes.c_char_p, ctypes.c_size_t]
        L.lama_png_read_gray.argtypes = L.lama_png_read_rgb.argtypes
        L.lama_png_write_rgb.argtypes = [ctypes.c_char_p, u8p, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                         ctypes.c_size_t]
        L.lama_free.argtypes = [ctypes.c_void_p]
        L.lama_estimated_bytes.restype = ctypes.c_uint64
        L.lama_estimated_bytes.argtypes = [ctypes.c_uint64]
        _lib = L
    return _lib


def _u8(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def _f(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Store:
    """WeightStore (weights.rs:80-139): the mapped container and its tensor table."""

    def __init__(self, path, map=True):
        self.handle = None
        err = ctypes.create_string_buffer(1024)
        h = ctypes.c_void_p()
        if lib().lama_store_open(os.fsencode(path), 1 if map else 0, ctypes.byref(h), err, 1024):
            raise RuntimeError(err.value.decode())
        self.handle = h

    def __len__(self):
        return lib().lama_store_count(self.handle)

    def table(self):
        return lib().lama_store_table(self.handle)

    def bytes_ptr(self):
        n = ctypes.c_size_t()
        p = lib().lama_store_bytes(self.handle, ctypes.byref(n))
        return p, n.value

    def info(self):
        t = self.table()
        return [(t[i].name.decode(), tuple(t[i].shape[:t[i].ndim]), t[i].offset, t[i].nbytes)
                for i in range(len(self))]

    def total_bytes(self):
        return lib().lama_store_total_bytes(self.handle)

    def close(self):
        if self.handle:
            lib().lama_store_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


def synth_weights(path, seed=0):
    err = ctypes.create_string_buffer(512)
    if lib().lama_synth_weights(os.fsencode(path), seed, err, 512):
        raise RuntimeError(err.value.decode())


def synth_image(h, w, seed=1):
    out = np.empty((h, w, 3), np.uint8)
    lib().lama_synth_image(_u8(out), h, w, seed)
    return out


def synth_mask_rect(h, w, rect_w, rect_h, seed=2):
    out = np.empty((h, w), np.uint8)
    x0, y0 = ctypes.c_int(), ctypes.c_int()
    lib().lama_synth_mask_rect(_u8(out), h, w, rect_w, rect_h, seed, ctypes.byref(x0), ctypes.byref(y0))
    return out, (x0.value, y0.value)


def synth_mask_strokes(h, w, coverage=0.25, seed=2):
    out = np.empty((h, w), np.uint8)
    cov = lib().lama_synth_mask_strokes(_u8(out), h, w, coverage, seed)
    return out, cov


def reflect_index(i, n):
    return lib().lama_reflect_index(i, n)


def build_input(rgb, mask, pad_h=None, pad_w=None):
    rgb = np.ascontiguousarray(rgb, np.uint8)
    mask = np.ascontiguousarray(mask, np.uint8)
    h, w = mask.shape
    if pad_h is None:
        pad_h = (8 - h % 8) % 8
    if pad_w is None:
        pad_w = (8 - w % 8) % 8
    out = np.empty((4, h + pad_h, w + pad_w), np.float32)
    lib().lama_build_input(_u8(rgb), _u8(mask), h, w, pad_h, pad_w, _f(out))
    return out


def composite(rgb, mask, net, pad_h, pad_w):
    rgb = np.ascontiguousarray(rgb, np.uint8)
    mask = np.ascontiguousarray(mask, np.uint8)
    net = np.ascontiguousarray(net, np.float32)
    h, w = mask.shape
    out = np.empty((h, w, 3), np.uint8)
    lib().lama_composite(_u8(rgb), _u8(mask), h, w, pad_h, pad_w, _f(net), _u8(out))
    return out


def window_origin(c, side, extent):
    return lib().lama_window_origin(c, side, extent)


def tile_rect(mask):
    mask = np.ascontiguousarray(mask, np.uint8)
    t = Tile()
    if lib().lama_tile_rect(_u8(mask), mask.shape[1], mask.shape[0], ctypes.byref(t)):
        return None
    return t


def mask_depth(mask):
    mask = np.ascontiguousarray(mask, np.uint8)
    d = np.empty(mask.shape, np.uint32)
    lib().lama_mask_depth(_u8(mask), mask.shape[1], mask.shape[0],
                          d.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return d


def section_rects(mask):
    mask = np.ascontiguousarray(mask, np.uint8)
    n = lib().lama_section_rects(_u8(mask), mask.shape[1], mask.shape[0], None, 0)
    arr = (Section * max(n, 1))()
    lib().lama_section_rects(_u8(mask), mask.shape[1], mask.shape[0], arr, n)
    return [arr[i].astuple() for i in range(n)]


def png_read_rgb(path):
    p = ctypes.POINTER(ctypes.c_uint8)()
    w, h = ctypes.c_int(), ctypes.c_int()
    err = ctypes.create_string_buffer(512)
    if lib().lama_png_read_rgb(os.fsencode(path), ctypes.byref(p), ctypes.byref(w), ctypes.byref(h), err, 512):
        raise RuntimeError(err.value.decode())
    a = np.ctypeslib.as_array(p, shape=(h.value, w.value, 3)).copy()
    lib().lama_free(p)
    return a


def png_read_gray(path):
    p = ctypes.POINTER(ctypes.c_uint8)()
    w, h = ctypes.c_int(), ctypes.c_int()
    err = ctypes.create_string_buffer(512)
    if lib().lama_png_read_gray(os.fsencode(path), ctypes.byref(p), ctypes.byref(w), ctypes.byref(h), err, 512):
        raise RuntimeError(err.value.decode())
    a = np.ctypeslib.as_array(p, shape=(h.value, w.value)).copy()
    lib().lama_free(p)
    return a


def png_write_rgb(path, rgb):
    rgb = np.ascontiguousarray(rgb, np.uint8)
    err = ctypes.create_string_buffer(512)
    if lib().lama_png_write_rgb(os.fsencode(path), _u8(rgb), rgb.shape[1], rgb.shape[0], err, 512):
        raise RuntimeError(err.value.decode())


def estimated_bytes(px):
    return lib().lama_estimated_bytes(px)
