"""Each HIP kernel family against the CPU oracle on seeded random data.

Tolerance: FP32 MFMA products with FP32 accumulation in a different order
than the oracle's sequential sum -- relative L2 error <= 1e-5 for the GEMM
families and the f32 FFT (the oracle's FFT runs in f64), far inside the
1e-3 per-layer bound the north star states.
"""
import numpy as np
import pytest

import oracle_api as O
from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _bn(rng, c):
    return (rng.uniform(0.5, 1.5, c).astype(np.float32), rng.normal(0, 0.1, c).astype(np.float32))


def _oracle_bn_relu(y, s, t):
    # cpu.rs:66-76 then 376-382
    y = y * s[:, None, None]
    y = y + t[:, None, None]
    return np.where(y < 0, np.float32(0), y)


@pytest.mark.parametrize("cin,cout,h,w,k,stride", [
    (40, 72, 13, 37, 3, 1),    # ragged channel chunk, partial tiles, M % 64 != 0
    (128, 128, 16, 16, 3, 1),  # resblock l2l shape at a 128x128 input
    (16, 24, 9, 70, 3, 2),     # stride 2, odd height
    (64, 128, 32, 32, 3, 2),   # model.2 shape at a 64x64 input
    (4, 64, 20, 40, 7, 1),     # model.1 head (cin 4)
    (6, 10, 8, 8, 7, 1),       # 7x7 on a plane barely wider than the kernel
    (384, 192, 8, 8, 1, 1),    # SpectralTransform conv1
    (40, 70, 5, 33, 1, 1),     # 1x1, ragged everything (plane not a multiple of 4: per-element loads)
    (384, 384, 64, 33, 1, 1),  # FourierUnit conv at a 512x512 input (float4 loads)
    (96, 130, 7, 12, 1, 1),    # 1x1 float4 loads: partial last tile, M % 64 != 0
    (50, 64, 2, 2, 1, 1),      # 1x1 plane of exactly one float4 run
    (33, 20, 1, 3, 1, 1),      # 1x1 plane shorter than a float4 run
    (384, 384, 75, 38, 1, 1),  # FourierUnit conv at a 600x600 input (N = 2850: float2 loads)
    (24, 40, 3, 2, 1, 1),      # 1x1 plane of 6 values: float2 loads, last run clamped
    (20, 16, 1, 2, 1, 1),      # 1x1 plane of 2 values: shorter than a run, scalar loads
])
def test_conv2d(engine, cin, cout, h, w, k, stride):
    rng = np.random.default_rng(cin * 1000 + cout + k)
    x = rng.standard_normal((cin, h, w), np.float32)
    wt = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
    s, t = _bn(rng, cout)
    got = engine.op_conv2d(x, wt, None, stride, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv2d(x, wt, None, pad=k // 2, stride=stride, reflect=True), s, t)
    assert got.shape == ref.shape
    assert rel_err(got, ref) < TOL


def test_conv2d_bias_no_bn(engine):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((12, 11, 19), np.float32)
    wt = rng.standard_normal((5, 12, 3, 3)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    got = engine.op_conv2d(x, wt, b, 1)
    ref = O.conv2d(x, wt, b, pad=1, stride=1, reflect=True)
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("cin,cout,h,w", [(32, 16, 5, 7), (512, 256, 8, 8), (64, 64, 3, 40)])
def test_conv_transpose(engine, cin, cout, h, w):
    rng = np.random.default_rng(cin + cout + h)
    x = np.maximum(rng.standard_normal((cin, h, w)), 0).astype(np.float32)  # post-ReLU: zeros are skipped
    wt = (rng.standard_normal((cin, cout, 3, 3)) * np.sqrt(2.0 / (cout * 9))).astype(np.float32)
    b = (rng.standard_normal(cout) * 0.05).astype(np.float32)
    s, t = _bn(rng, cout)
    got = engine.op_conv_transpose(x, wt, b, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv_transpose(x, wt, b), s, t)
    assert rel_err(got, ref) < TOL


@pytest.fixture(scope="module", params=["32", "16"], ids=["tile2x32", "tile4x16"])
def edge_engine(pkg, request):
    """An engine with the stride-2 and transposed convolutions' tile forced:
    2 x 32 pixels (lama_conv3x3s2, lama_convt) or 4 x 16 (the _q kernels)."""
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_EDGE_TILE", request.param)
        eng = pkg.hip_engine.Engine()
    yield eng
    eng.close()


@pytest.mark.parametrize("cin,cout,h,w", [(16, 64, 150, 150), (16, 24, 9, 70), (64, 128, 32, 32), (8, 72, 13, 37)])
def test_conv3x3s2_tile_shapes(edge_engine, cin, cout, h, w):
    """Stride 2 in both tile shapes, against the oracle: a 75 x 75 output
    (the 600 x 600 model.4 plane), odd heights, partial tiles, M % 64 != 0."""
    rng = np.random.default_rng(cin * 7 + cout + h)
    x = rng.standard_normal((cin, h, w), np.float32)
    wt = (rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
    s, t = _bn(rng, cout)
    got = edge_engine.op_conv2d(x, wt, None, 2, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv2d(x, wt, None, pad=1, stride=2, reflect=True), s, t)
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("cin,cout,h,w", [(64, 32, 75, 75), (32, 16, 5, 7), (40, 72, 9, 19)])
def test_conv_transpose_tile_shapes(edge_engine, cin, cout, h, w):
    """The transposed convolution in both tile shapes, against the oracle: a
    75 x 75 input (the 600 x 600 model.24 plane) and ragged shapes."""
    rng = np.random.default_rng(cin + 3 * cout + h)
    x = np.maximum(rng.standard_normal((cin, h, w)), 0).astype(np.float32)
    wt = (rng.standard_normal((cin, cout, 3, 3)) * np.sqrt(2.0 / (cout * 9))).astype(np.float32)
    b = (rng.standard_normal(cout) * 0.05).astype(np.float32)
    s, t = _bn(rng, cout)
    got = edge_engine.op_conv_transpose(x, wt, b, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv_transpose(x, wt, b), s, t)
    assert rel_err(got, ref) < TOL


# (64, 64), (32, 32), (33, 96), (31, 32): padded row-pair stride, odd row counts
SIZES = [(8, 8), (64, 64), (32, 32), (75, 75), (6, 10), (5, 7), (1, 1), (2, 3), (64, 33), (16, 12), (38, 19),
         (33, 96), (31, 32)]


# planes too large for one block's LDS take the row/column split launches;
# the square 256 and 128 planes have split kernels with the shape compiled in
LARGE = [(256, 256), (128, 128), (200, 130), (150, 90)]


@pytest.fixture(params=["single", "split", "generic"])
def fft_mode(request, monkeypatch):
    """'split' forces the row/column launches (LAMA_FFT_SPLIT=1) at every size;
    'generic' keeps the runtime-shaped kernels where a kernel with the plane
    shape compiled in exists (single-block 32x32, 64x64 and 75x75, split
    128x128 and 256x256; LAMA_FFT_GENERIC=1)."""
    monkeypatch.delenv("LAMA_FFT_SPLIT", raising=False)
    monkeypatch.delenv("LAMA_FFT_GENERIC", raising=False)
    if request.param == "split":
        monkeypatch.setenv("LAMA_FFT_SPLIT", "1")
    elif request.param == "generic":
        monkeypatch.setenv("LAMA_FFT_GENERIC", "1")
    return request.param


@pytest.mark.parametrize("h,w", SIZES + LARGE)
def test_rfft2(engine, fft_mode, h, w):
    if fft_mode == "single" and (h, w) in LARGE:
        pytest.skip("large planes always split (the 'split' case)")
    rng = np.random.default_rng(h * 100 + w)
    c = 3
    x = rng.standard_normal((c, h, w), np.float32)
    got = engine.op_rfft2(x)
    ref = np.concatenate([O.rfft2_ortho(x[i]) for i in range(c)], axis=0)
    assert got.shape == ref.shape
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("h,w", SIZES + LARGE)
def test_irfft2(engine, fft_mode, h, w):
    if fft_mode == "single" and (h, w) in LARGE:
        pytest.skip("large planes always split (the 'split' case)")
    rng = np.random.default_rng(h * 100 + w + 1)
    c = 3
    wh = w // 2 + 1
    spec = rng.standard_normal((2 * c, h, wh), np.float32)  # not Hermitian: exercises the completion rule
    feat = rng.standard_normal((c, h, w), np.float32)
    got = engine.op_irfft2(spec, w, feat)
    ref = np.stack([O.irfft2_ortho(spec[2 * i:2 * i + 2], w) for i in range(c)]) + feat
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("inverse", [False, True])
def test_fft64_shuffle_rows(engine, monkeypatch, inverse):
    """The 64 x 64 transforms whose rows run as wavefront-shuffle FFTs in
    registers (lama_rfft2_64s / lama_irfft2_64s, taken with LAMA_FFT64_SHFL=1)
    against the oracle, as test_rfft2 / test_irfft2."""
    monkeypatch.setenv("LAMA_FFT64_SHFL", "1")
    rng = np.random.default_rng(6464 + inverse)
    c = 5
    if not inverse:
        x = rng.standard_normal((c, 64, 64), np.float32)
        got = engine.op_rfft2(x)
        ref = np.concatenate([O.rfft2_ortho(x[i]) for i in range(c)], axis=0)
    else:
        spec = rng.standard_normal((2 * c, 64, 33), np.float32)
        feat = rng.standard_normal((c, 64, 64), np.float32)
        got = engine.op_irfft2(spec, 64, feat)
        ref = np.stack([O.irfft2_ortho(spec[2 * i:2 * i + 2], 64) for i in range(c)]) + feat
    assert got.shape == ref.shape
    assert rel_err(got, ref) < TOL


# cin 7 and 1: odd channel counts leave the kernel's second channel half idle
# in the last step; 9 x 70 spans two column tiles with a partial row tile
@pytest.mark.parametrize("h,w,cin", [(16, 64, 64), (24, 40, 64), (8, 8, 64), (64, 128, 64), (24, 40, 7),
                                     (9, 70, 1), (600 // 8 * 8, 75, 64)])
def test_tail(engine, h, w, cin):
    rng = np.random.default_rng(h + w + cin)
    x = rng.standard_normal((cin, h, w), np.float32)
    wt = (rng.standard_normal((3, cin, 7, 7)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(3) * 0.05).astype(np.float32)
    got = engine.op_tail(x, wt, b)
    z = O.conv2d(O.reflect_pad(x, 3), wt, b, pad=0, stride=1, reflect=False)
    ref = (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    assert rel_err(got, ref) < TOL


@pytest.fixture(scope="module")
def direct_engine(pkg):
    # the engine reads LAMA_FFC_WINO when it opens
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_FFC_WINO", "0")
        eng = pkg.hip_engine.Engine()
    yield eng
    eng.close()


WINO_CASES = [
    (40, 72, 13, 37),     # ragged channel chunk, odd width (last Winograd tile half outside), M % 64 != 0
    (128, 128, 16, 16),   # resblock l2l shape at a 128x128 input
    (384, 128, 64, 64),   # g2l at a 512x512 input
    (12, 9, 3, 1),        # a one-pixel-wide plane (both taps reflect onto column 0); odd chunk count
    (5, 64, 2, 130),      # more than one 64-pixel tile column, partial last one
]


@pytest.mark.parametrize("cin,cout,h,w", WINO_CASES)
def test_conv3x3_winograd(engine, cin, cout, h, w):
    """The FFC 3x3 convolution as the default engine runs it (Winograd F(4,3)
    along x in the block shape the plane selects) against the oracle's direct
    sum.  The transforms round differently from the direct sum, within the same
    1e-5 relative bound."""
    rng = np.random.default_rng(cin * 100 + cout + w)
    x = rng.standard_normal((cin, h, w), np.float32)
    wt = (rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
    s, t = _bn(rng, cout)
    print(f"case wino {cin}x{h}x{w} -> {cout}", flush=True)
    got = engine.op_conv2d(x, wt, None, 1, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv2d(x, wt, None, pad=1, stride=1, reflect=True), s, t)
    assert got.shape == ref.shape
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("cin,cout,h,w", WINO_CASES)
def test_conv3x3_direct(direct_engine, cin, cout, h, w):
    """The same cases on the direct implicit GEMM (LAMA_FFC_WINO=0)."""
    rng = np.random.default_rng(cin * 100 + cout + w)
    x = rng.standard_normal((cin, h, w), np.float32)
    wt = (rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
    s, t = _bn(rng, cout)
    print(f"case direct {cin}x{h}x{w} -> {cout}", flush=True)
    got = direct_engine.op_conv2d(x, wt, None, 1, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv2d(x, wt, None, pad=1, stride=1, reflect=True), s, t)
    assert rel_err(got, ref) < TOL


@pytest.fixture(scope="module", params=[("2", ""), ("4", "64"), ("4", "32"), ("4", "16"), ("42", "")],
                ids=["f23", "f43w64", "f43w32", "f43w16", "f2x4"])
def w4_engine(pkg, request):
    """Each Winograd kernel: F(2,3) (LAMA_FFC_WINO=2, lama_conv3x3w), F(4,3)
    (LAMA_FFC_WINO=4) with 64-, 32- or 16-pixel blocks (LAMA_W4_TILE) and
    F(2x4, 3x3) (LAMA_FFC_WINO=42, lama_conv3x3w42); both are read when the
    context opens."""
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_FFC_WINO", request.param[0])
        mp.setenv("LAMA_W4_TILE", request.param[1])
        eng = pkg.hip_engine.Engine()
    yield eng
    eng.close()


W4_CASES = WINO_CASES + [
    (8, 64, 5, 75),       # the 600x600 bottleneck width: 75 = 2 x 32 + 11 (or 64 + 11)
    (16, 32, 9, 32),      # the 256x256 bottleneck width
    (4, 70, 7, 3),        # narrower than one Winograd tile
    # widths that are multiples of 4 take the 16-byte input loads: a partial
    # last block (36 = 32 + 4, 100 = 64 + 32 + 4) and a plane of one quad
    (12, 40, 6, 36),
    (8, 96, 11, 100),
    (4, 8, 5, 4),
]


@pytest.mark.parametrize("cin,cout,h,w", W4_CASES)
def test_conv3x3_winograd_f43(w4_engine, cin, cout, h, w):
    """The FFC 3x3 convolution as Winograd F(2,3) (lama_conv3x3w), F(4,3)
    along x (lama_conv3x3w4 / w4n / w4q) and F(2x4, 3x3) (lama_conv3x3w42)
    against the oracle's direct sum, the same 1e-5 relative bound: F(4,3)'s
    larger transform constants round a little more than F(2,3)'s."""
    rng = np.random.default_rng(cin * 100 + cout + w)
    x = rng.standard_normal((cin, h, w), np.float32)
    wt = (rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
    s, t = _bn(rng, cout)
    print(f"case wino4 {cin}x{h}x{w} -> {cout}", flush=True)
    got = w4_engine.op_conv2d(x, wt, None, 1, s, t, relu=True)
    ref = _oracle_bn_relu(O.conv2d(x, wt, None, pad=1, stride=1, reflect=True), s, t)
    assert got.shape == ref.shape
    assert rel_err(got, ref) < TOL
