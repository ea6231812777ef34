"""lama_hip_forward_device_noalloc through the C ABI: the forward on the
device's lama_scratch array equals lama_hip_forward_device's bit for bit, on
two calls in a row whose second input is smaller, and again after another
context used the array; after the first call on the device, which sets the
array up, it allocates no device memory; it rejects an input whose arena
exceeds the array."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _noalloc(pkg, eng, d_in, h, w, d_out):
    L = pkg.hip_engine.lib()
    err = ctypes.create_string_buffer(1024)
    rc = L.lama_hip_forward_device_noalloc(eng.ctx, d_in, h, w, d_out, None, err, 1024)
    return rc, err.value.decode()


def _case(pkg, h, w, seed):
    H = pkg.host_api
    img = H.synth_image(h, w, seed)
    mask, _ = H.synth_mask_strokes(h, w, 0.25, seed + 1)
    return H.build_input(img, mask)


def test_noalloc_matches_forward_device(pkg, weights_dir):
    E = pkg.hip_engine
    eng = E.Engine()
    eng.load_weights(pkg.host_api.Store(weights_dir["cal"]))
    # the first call on the device sets the array up (loads its code object)
    x0 = _case(pkg, 64, 64, 9)
    d0i, d0o = eng.malloc(x0.nbytes), eng.malloc(3 * 64 * 64 * 4)
    eng.upload(d0i, x0)
    print("case noalloc set-up call 64x64", flush=True)
    rc, msg = _noalloc(pkg, eng, d0i, 64, 64, d0o)
    assert rc == 0, msg
    eng.synchronize()
    eng.free(d0i)
    eng.free(d0o)
    free0 = E.vram()[0]
    outs = {}
    for h, w, seed in [(512, 512, 1), (256, 384, 3)]:
        x = _case(pkg, h, w, seed)
        d_in, d_ref, d_out = eng.malloc(x.nbytes), eng.malloc(3 * h * w * 4), eng.malloc(3 * h * w * 4)
        eng.upload(d_in, x)
        eng.forward_device(d_in, h, w, d_ref)
        eng.synchronize()
        ref = np.empty((3, h, w), np.float32)
        eng.download(ref, d_ref)
        outs[(h, w)] = (x, ref)
        free1 = E.vram()[0]
        print(f"case noalloc {h}x{w}", flush=True)
        rc, msg = _noalloc(pkg, eng, d_in, h, w, d_out)
        assert rc == 0, msg
        eng.synchronize()
        got = np.empty((3, h, w), np.float32)
        eng.download(got, d_out)
        assert np.array_equal(got, ref), (h, w)
        # no arena was allocated for the call (one would be >= 60 MiB here)
        assert E.vram()[0] >= free1 - (16 << 20), (h, w)
        for p in (d_in, d_ref, d_out):
            eng.free(p)
    assert free0 > 0

    # another context takes the array, then this one again: its descriptors
    # are uploaded afresh and the result is unchanged
    other = E.Engine()
    other.load_weights(pkg.host_api.Store(weights_dir["plain"]))
    for e in (other, eng):
        x, ref = outs[(256, 384)]
        d_in, d_out = e.malloc(x.nbytes), e.malloc(ref.nbytes)
        e.upload(d_in, x)
        rc, msg = _noalloc(pkg, e, d_in, 256, 384, d_out)
        assert rc == 0, msg
        e.synchronize()
        got = np.empty_like(ref)
        e.download(got, d_out)
        if e is eng:
            assert np.array_equal(got, ref)
        else:
            assert np.isfinite(got).all() and not np.array_equal(got, ref)
        e.free(d_in)
        e.free(d_out)
    other.close()

    # beyond the array: a clear error, and the context still works
    d = eng.malloc(4)
    rc, msg = _noalloc(pkg, eng, d, 600, 600, d)
    assert rc != 0 and "no-allocation" in msg and "MiB" in msg, msg
    eng.free(d)
    x, ref = outs[(512, 512)]
    assert np.array_equal(eng.forward(x), ref)
    eng.close()
