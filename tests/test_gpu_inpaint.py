"""lama_hip_inpaint: the whole-image flow of main.rs:241-307 on the device --
the pad to a multiple of 8, build_input (main.rs:175-196), the forward, and
the 8-bit composite fused into the output convolution's epilogue.

Bit-exact checks against the oracle's restatement of the reference rules:
the device composite equals or_composite applied to the same pass's f32
output (returned beside it), and the device-built input equals
or_build_input (through the pass it feeds, and directly through the
LAMA_DUMP_STEP=0 dump of the padded input)."""
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle_api as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _pad(n):
    return (8 - n % 8) % 8


@pytest.mark.parametrize("h,w,kind", [(597, 590, "rect"), (512, 512, "strokes"), (61, 83, "strokes"),
                                      (13, 21, "rect"), (5, 7, "rect")])
def test_inpaint_composite_is_the_reference_rule(pkg, engine, h, w, kind):
    """597 x 590 pads to 600 x 592 (the --tile window shape); 5 x 7 pads to
    8 x 8 with a pad wider than the image."""
    H = pkg.host_api
    img = H.synth_image(h, w, 3)
    if kind == "rect":
        mask, _ = H.synth_mask_rect(h, w, max(1, w // 3), max(1, h // 4), 4)
    else:
        mask, _ = H.synth_mask_strokes(h, w, 0.25, 4)
    mask[0, :3] = [1, 128, 255]  # non-binary mask bytes are holes too
    print(f"case inpaint {h}x{w} {kind}", flush=True)
    u8, net = engine.inpaint(img, mask, net_out=True)
    ph, pw = _pad(h), _pad(w)
    assert net.shape == (3, h + ph, w + pw)
    # the device input equals the reference rule: the pass equals a forward of the oracle's input
    assert np.array_equal(net, engine.forward(O.build_input(img, mask, ph, pw)))
    # the device composite equals the reference rule on the same f32 output
    assert np.array_equal(u8, O.composite(img, mask, net, ph, pw))
    assert np.array_equal(u8[mask == 0], img[mask == 0])
    # the host-buffer and device-buffer entry points agree
    d_rgb, d_mask, d_out = engine.malloc(img.nbytes), engine.malloc(mask.nbytes), engine.malloc(img.nbytes)
    engine.upload(d_rgb, img)
    engine.upload(d_mask, mask)
    engine.inpaint_device(d_rgb, d_mask, h, w, d_out)
    engine.synchronize()
    u8d = np.empty_like(img)
    engine.download(u8d, d_out)
    for p in (d_rgb, d_mask, d_out):
        engine.free(p)
    assert np.array_equal(u8d, u8)


def test_inpaint_crop_sizes_share_a_padded_plan(pkg, engine):
    """Images of different sizes that pad to one shape share its plan; each
    call composites its own h x w crop."""
    H = pkg.host_api
    outs = []
    for h, w in [(64, 64), (57, 60), (64, 64)]:
        img = H.synth_image(h, w, 5)
        mask, _ = H.synth_mask_rect(h, w, 20, 12, 6)
        u8, net = engine.inpaint(img, mask, net_out=True)
        assert np.array_equal(u8, O.composite(img, mask, net, _pad(h), _pad(w)))
        outs.append(u8)
    assert np.array_equal(outs[0], outs[2])


_DUMP0 = r"""
import os, sys
import numpy as np
sys.path.insert(0, {root!r})
sys.path.insert(0, os.path.join({root!r}, "tests"))
import __graft_entry__
pkg = __graft_entry__.load_package()
H = pkg.host_api
import oracle_api as O
eng = pkg.hip_engine.Engine()
eng.load_weights(H.Store({weights!r}))
h, w = 45, 38
rng = np.random.default_rng(9)
img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
img.reshape(-1)[:256] = np.arange(256, dtype=np.uint8)
mask = rng.integers(0, 256, (h, w), dtype=np.uint8)
mask.reshape(-1)[::2] = 0
eng.inpaint(img, mask)
got = np.fromfile("/tmp/gpu_step_0.f32", dtype="<f4")
want = O.reflect_pad(O.build_input(img, mask, 3, 2), 3).ravel()
print("DUMP0", got.shape == want.shape and bool(np.array_equal(got, want)))
"""


def test_device_build_input_is_bit_exact(weights_dir):
    """LAMA_DUMP_STEP=0 in the inpaint flow dumps the device-built input
    (reflect-padded by 3, the reference's step 0): every byte value of the
    image and of the mask, bottom/right padding, bit-exact with or_build_input."""
    env = dict(os.environ, LAMA_DUMP_STEP="0")
    r = subprocess.run([sys.executable, "-c", _DUMP0.format(root=ROOT, weights=weights_dir["plain"])],
                       capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr
    assert "DUMP0 True" in r.stdout, r.stdout + r.stderr
    assert "gpu dumped step 0: local 4x54x46 global None" in r.stderr
