"""the per-layer conv GEMM suite at the 512x512 shapes,
FP32, batch 1, N(0,1) activations and He-normal weights, each with its fused
BN + ReLU epilogue, kernel by kernel against the CPU oracle's direct sums
(cpu.rs:110-168 for the convolutions, cpu.rs:328-374 for the transposed ones,
cpu.rs:66-76 and 376-382 for BN and ReLU):

- the 7x7 head conv 4 -> 64 at 512x512 (reflect pad 3);
- the three stride-2 3x3 convs 64 -> 128 (512 -> 256), 128 -> 256 (256 -> 128)
  and 256 -> 512 (128 -> 64), reflect pad 1;
- the FFC local 3x3 convs at 64x64: l2l 128 -> 128, l2g 128 -> 384, g2l
  384 -> 128 (Winograd F(4,3) along x, the plan's kernel for that plane);
- the three stride-2 transposed convs 512 -> 256 (64 -> 128), 256 -> 128
  (128 -> 256) and 128 -> 64 (256 -> 512).

Beside them, the FFC 3x3 at the 256-wide planes of a 2048x2048 input
(configs[4]'s bottleneck), which the forward otherwise runs only inside the
whole pass.

Tolerance: 1e-5 relative L2 (FP32 products, FP32 sums in another order than
the oracle's sequential loop), 100x inside the north star's 1e-3 per layer.
"""
import numpy as np
import pytest

import oracle_api as O
from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _bn(rng, c):
    return (rng.uniform(0.5, 1.5, c).astype(np.float32), rng.normal(0, 0.1, c).astype(np.float32))


def _bn_relu(y, s, t):
    y = y * s[:, None, None]
    y = y + t[:, None, None]
    return np.where(y < 0, np.float32(0), y)


def _he(rng, shape, fan_in):
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


CONV_CASES = [
    # name, cin, cout, input side, k, stride
    ("model.1 7x7 4->64 @512", 4, 64, 512, 7, 1),
    ("model.2 s2 64->128 @512", 64, 128, 512, 3, 2),
    ("model.3 s2 128->256 @256", 128, 256, 256, 3, 2),
    ("model.4 s2 256->512 @128", 256, 512, 128, 3, 2),
    ("FFC l2l 128->128 @64", 128, 128, 64, 3, 1),
    ("FFC l2g 128->384 @64", 128, 384, 64, 3, 1),
    ("FFC g2l 384->128 @64", 384, 128, 64, 3, 1),
    ("FFC l2l 128->128 @256 (2048 input)", 128, 128, 256, 3, 1),
    ("FFC g2l 384->128 @256 (2048 input)", 384, 128, 256, 3, 1),
]


@pytest.mark.parametrize("name,cin,cout,side,k,stride", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_config1_conv(engine, name, cin, cout, side, k, stride):
    rng = np.random.default_rng(cin * 100003 + cout * 101 + side * 7 + k + stride)
    x = rng.standard_normal((cin, side, side), np.float32)
    wt = _he(rng, (cout, cin, k, k), cin * k * k)
    s, t = _bn(rng, cout)
    print(f"case {name}", flush=True)
    got = engine.op_conv2d(x, wt, None, stride, s, t, relu=True)
    ref = _bn_relu(O.conv2d(x, wt, None, pad=k // 2, stride=stride, reflect=True), s, t)
    assert got.shape == ref.shape == (cout, side // stride, side // stride)
    e = rel_err(got, ref)
    assert e < TOL, f"{name}: rel err {e:.3e}"


CONVT_CASES = [
    ("model.24 convT 512->256 @64", 512, 256, 64),
    ("model.27 convT 256->128 @128", 256, 128, 128),
    ("model.30 convT 128->64 @256", 128, 64, 256),
]


@pytest.mark.parametrize("name,cin,cout,side", CONVT_CASES, ids=[c[0] for c in CONVT_CASES])
def test_config1_conv_transpose(engine, name, cin, cout, side):
    rng = np.random.default_rng(cin * 7 + cout + side)
    x = rng.standard_normal((cin, side, side), np.float32)
    # PyTorch's fan-in of a ConvTranspose2d weight [cin][cout][3][3]: cout * 9
    wt = _he(rng, (cin, cout, 3, 3), cout * 9)
    b = (rng.standard_normal(cout) * 0.05).astype(np.float32)
    s, t = _bn(rng, cout)
    print(f"case {name}", flush=True)
    got = engine.op_conv_transpose(x, wt, b, s, t, relu=True)
    ref = _bn_relu(O.conv_transpose(x, wt, b), s, t)
    assert got.shape == ref.shape == (cout, 2 * side, 2 * side)
    e = rel_err(got, ref)
    assert e < TOL, f"{name}: rel err {e:.3e}"
