"""Pins the CPU oracle (oracle/lama_oracle.c) before it is trusted as the
parity reference.  Each function is checked against something other than its
own formula: committed golden vectors from torch / numpy (tests/golden),
live torch CPU ops, closed forms (brute-force DFTs, Parseval, round trips),
invariants (thread-count independence) and an independent torch model of the
whole generator.  A plausible mistake -- a transposed weight, a wrong reflect
index, a dropped Hermitian term, a flipped FFT sign -- fails at least one.
"""
import os

import numpy as np
import pytest

import oracle_api as O
from conftest import rel_err

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ops.npz"))


# ---------------------------------------------------------------- reflect

@pytest.mark.parametrize("n", [1, 2, 3, 8])
def test_reflect_index_matches_numpy_reflect_pad(n):
    # image.rs:159-169 is PyTorch's 'reflect' (numpy 'reflect': edge not repeated)
    a = np.arange(n)
    for pad in range(0, 3 * n + 2):
        if n == 1:
            want = np.zeros(n + 2 * pad, int)
        else:
            want = np.pad(a, pad, mode="reflect")
        got = [O.reflect_index(i - pad, n) for i in range(n + 2 * pad)]
        assert list(want) == got, (n, pad)


def test_reflect_pad_matches_torch():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    x = np.random.default_rng(0).standard_normal((3, 7, 9)).astype(np.float32)
    want = F.pad(torch.from_numpy(x)[None], (3, 3, 3, 3), mode="reflect")[0].numpy()
    assert np.array_equal(O.reflect_pad(x, 3), want)


# ------------------------------------------------------------ convolutions

@pytest.mark.parametrize("name,stride", [("c3s1", 1), ("c3s2", 2), ("c7", 1), ("c1", 1)])
def test_conv_golden(name, stride):
    x, w, b, y = (GOLD[f"{name}_{k}"] for k in "xwby")
    k = w.shape[2]
    got = O.conv2d(x, w, b, pad=k // 2, stride=stride, reflect=True) if k > 1 else O.conv1x1(x, w, b)
    assert got.shape == y.shape
    assert rel_err(got, y) < 1e-6


def test_conv_transposed_weight_would_fail():
    # a transposed operand is caught: swapping cout/cin in the golden case errs
    x, w, b, y = (GOLD[f"c3s1_{k}"] for k in "xwby")
    assert rel_err(O.conv2d(x, w, b, 1, 1, True), y) < 1e-6
    w2 = np.ascontiguousarray(w[:, :, ::-1, ::-1])  # flipped kernel = correlation vs convolution
    assert rel_err(O.conv2d(x, w2, b, 1, 1, True), y) > 1e-2


def test_conv_live_torch_random_shapes():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    rng = np.random.default_rng(5)
    for cin, cout, h, w, k, s in [(3, 4, 5, 6, 3, 1), (2, 3, 9, 4, 3, 2), (4, 2, 8, 8, 7, 1), (6, 6, 2, 2, 3, 1)]:
        x = rng.standard_normal((cin, h, w)).astype(np.float32)
        wt = rng.standard_normal((cout, cin, k, k)).astype(np.float32)
        p = k // 2
        want = F.conv2d(F.pad(torch.from_numpy(x)[None], (p,) * 4, mode="reflect"), torch.from_numpy(wt),
                        stride=s)[0].numpy()
        assert rel_err(O.conv2d(x, wt, None, p, s, True), want) < 1e-6


def test_conv_zero_padding_mode():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 6, 5)).astype(np.float32)
    wt = rng.standard_normal((3, 2, 3, 3)).astype(np.float32)
    want = F.conv2d(torch.from_numpy(x)[None], torch.from_numpy(wt), padding=1)[0].numpy()
    assert rel_err(O.conv2d(x, wt, None, 1, 1, False), want) < 1e-6


def test_conv_transpose_golden_and_zero_skip():
    x, w, b, y = (GOLD[f"ct_{k}"] for k in "xwby")
    got = O.conv_transpose(x, w, b)
    assert got.shape == y.shape
    assert rel_err(got, y) < 1e-6
    # the scatter skips exact zeros (cpu.rs:350-352): an all-zero input yields the bias
    z = O.conv_transpose(np.zeros_like(x), w, b)
    assert np.array_equal(z, np.broadcast_to(b[:, None, None], z.shape))


def test_bn_fold_golden():
    s, t = O.bn_fold(GOLD["bn_w"], GOLD["bn_b"], GOLD["bn_m"], GOLD["bn_v"])
    x = GOLD["bn_x"]
    got = x * s[:, None, None] + t[:, None, None]
    assert rel_err(got, GOLD["bn_y"]) < 1e-6
    # the f32 fold order of cpu.rs:58-62, exactly
    w, b, m, v = (GOLD[k].astype(np.float32) for k in ("bn_w", "bn_b", "bn_m", "bn_v"))
    s2 = (w / np.sqrt(v + np.float32(1e-5))).astype(np.float32)
    assert np.array_equal(s, s2)
    assert np.array_equal(t, (b - (m * s2).astype(np.float32)).astype(np.float32))


# --------------------------------------------------------------------- FFT

FFT_SIZES = [(8, 8), (16, 8), (4, 16), (6, 10), (5, 7), (3, 4), (1, 1), (12, 12)]


@pytest.mark.parametrize("h,w", FFT_SIZES)
def test_rfft2_golden(h, w):
    got = O.rfft2_ortho(GOLD[f"fft{h}x{w}_x"])
    assert rel_err(got, GOLD[f"fft{h}x{w}_y"]) < 1e-6


@pytest.mark.parametrize("h,w", FFT_SIZES)
def test_irfft2_golden(h, w):
    got = O.irfft2_ortho(GOLD[f"fft{h}x{w}_spec"], w)
    assert rel_err(got, GOLD[f"fft{h}x{w}_iy"]) < 1e-6


@pytest.mark.parametrize("h,w", [(8, 8), (75, 75), (6, 10), (7, 3), (32, 17)])
def test_fft_round_trip_is_identity(h, w):
    # unitary pair at every size (the sign flip of non-power-of-two lengths
    # applies to both directions and cancels)
    x = np.random.default_rng(h * w).standard_normal((h, w)).astype(np.float32)
    assert rel_err(O.irfft2_ortho(O.rfft2_ortho(x), w), x) < 1e-6


def test_rfft2_parseval_pow2():
    h, w = 16, 16
    x = np.random.default_rng(3).standard_normal((h, w))
    s = O.rfft2_ortho(x).astype(np.float64)
    c = s[0] + 1j * s[1]
    # energy of the half spectrum, counting the mirrored columns twice
    e = np.sum(np.abs(c[:, 0]) ** 2) + np.sum(np.abs(c[:, w // 2]) ** 2) + 2 * np.sum(np.abs(c[:, 1:w // 2]) ** 2)
    assert abs(e - np.sum(x.astype(np.float32).astype(np.float64) ** 2)) / e < 1e-5


def test_non_pow2_sign_convention_is_the_reference_bluestein():
    # For a length that is not a power of two the reference's forward
    # transform equals n * ifft (cpu.rs:954-1011): for real rows, conj(fft).
    x = np.random.default_rng(9).standard_normal((1, 6))
    got = O.rfft2_ortho(x).astype(np.float64)
    want = np.conj(np.fft.rfft(x[0])) / np.sqrt(6)
    assert np.allclose(got[0, 0] + 1j * got[1, 0], want, atol=1e-6)
    assert not np.allclose(got[0, 0] + 1j * got[1, 0], np.conj(want), atol=1e-3)


def test_irfft2_uses_the_2d_hermitian_rule():
    # cpu.rs:786-800: completing only along x would differ on non-Hermitian
    # input; the oracle must agree with torch's irfft2 (2-D rule) instead.
    torch = pytest.importorskip("torch")
    h, w = 8, 8
    spec = np.random.default_rng(11).standard_normal((2, h, w // 2 + 1)).astype(np.float32)
    got = O.irfft2_ortho(spec, w)
    want = torch.fft.irfft2(torch.complex(torch.from_numpy(spec[0]).double(), torch.from_numpy(spec[1]).double()),
                            s=(h, w), norm="ortho").float().numpy()
    assert np.abs(got - want).max() < 1e-5
    # the x-only completion (rows conjugated independently) is measurably different
    c = spec[0] + 1j * spec[1]
    full = np.zeros((h, w), complex)
    full[:, :w // 2 + 1] = c
    for x in range(w // 2 + 1, w):
        full[:, x] = np.conj(c[:, w - x])
    xonly = np.real(np.fft.ifft2(full)) * np.sqrt(h * w)
    assert np.abs(got - xonly).max() > 0.05


# ----------------------------------------------------------- invariants

def test_thread_count_independence():
    L = O.lib()
    L.or_set_threads.argtypes = [O.ctypes.c_int]
    x = np.random.default_rng(2).standard_normal((16, 24, 20)).astype(np.float32)
    w = np.random.default_rng(3).standard_normal((12, 16, 3, 3)).astype(np.float32)
    L.or_set_threads(1)
    a = O.conv2d(x, w, None, 1, 1, True)
    L.or_set_threads(8)
    b = O.conv2d(x, w, None, 1, 1, True)
    assert np.array_equal(a, b)


def test_build_input_and_composite_rules():
    rng = np.random.default_rng(4)
    h, w = 13, 11
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    mask = (rng.random((h, w)) < 0.3).astype(np.uint8) * rng.integers(1, 256, (h, w), dtype=np.uint8)
    x = O.build_input(rgb, mask, 3, 5)
    # main.rs:175-196, restated in numpy
    ys = [O.reflect_index(y, h) for y in range(h + 3)]
    xs = [O.reflect_index(x_, w) for x_ in range(w + 5)]
    m = (mask[np.ix_(ys, xs)].astype(np.float32) / 255.0 > 0).astype(np.float32)
    img = rgb[np.ix_(ys, xs)].astype(np.float32) / 255.0
    want = np.concatenate([np.moveaxis(img * (1 - m)[..., None], -1, 0), m[None]])
    assert np.array_equal(x, want.astype(np.float32))
    net = rng.uniform(-0.2, 1.2, (3, h + 3, w + 5)).astype(np.float32)
    out = O.composite(rgb, mask, net, 3, 5)
    keep = mask == 0
    assert np.array_equal(out[keep], rgb[keep])  # unmasked pixels bit-exact
    v = np.clip(net[:, :h, :w], 0, 1) * np.float32(255.0)
    want_u8 = (v + np.float32(0.5)).astype(np.uint8)
    assert np.array_equal(out[~keep], np.moveaxis(want_u8, 0, -1)[~keep])


# ----------------------------------------------- whole network vs torch

@pytest.fixture(scope="module")
def cal_weights(weights_dir):
    return O.read_safetensors(weights_dir["cal"])


def test_whole_network_matches_independent_torch_model(pkg, cal_weights):
    pytest.importorskip("torch")
    import torch_ffc
    H = pkg.host_api
    img = H.synth_image(64, 64, 1)
    mask, _ = H.synth_mask_rect(64, 64, 24, 16, 2)
    x = H.build_input(img, mask)
    out, steps = O.OracleNet(cal_weights).forward(x, steps=True)
    tout, tsteps = torch_ffc.forward(cal_weights, x)
    for s in range(29):
        assert rel_err(steps[s], tsteps[s]) < 1e-4, s
    assert rel_err(out, tout) < 1e-4


def test_net_load_reports_missing_tensor(cal_weights):
    w = dict(cal_weights)
    del w["model.7.conv2.ffc.convg2g.fu.bn.running_var"]
    with pytest.raises(RuntimeError, match="missing tensor in weight blob: model.7.conv2.ffc.convg2g.fu.bn.running_var"):
        O.OracleNet(w)


@pytest.mark.parametrize("k,hw", [(0, (32, 32)), (7, (16, 32)), (35, (32, 16))])
def test_spectral_block_matches_independent_torch_model(weights_dir, k, hw):
    """or_net_spectral (Spectral::forward, cpu.rs:239-265, the isolated
    SpectralTransform of BASELINE configs[2]) against the torch model's
    SpectralTransform on N(0,1) inputs with the plain fixture weights: every
    LAMA_DUMP_SPECTRAL stage (f, spectrum, FU conv, f + ifft) and the output.
    Power-of-two planes, where torch's FFT sign is the reference's."""
    pytest.importorskip("torch")
    import torch_ffc
    W = O.read_safetensors(weights_dir["plain"])
    h, w = hw
    x = np.random.default_rng(100 + k).standard_normal((384, h, w)).astype(np.float32)
    out, st = O.OracleNet(W).spectral(k, x, stages=True)
    tout, tst = torch_ffc.spectral_block(W, k, x)
    for i in range(4):
        assert rel_err(st[i], tst[i]) < 1e-5, i
    assert rel_err(out, tout) < 1e-5
    # the wrong FFC's weights fail the same comparison
    other = O.OracleNet(W).spectral((k + 1) % 36, x)
    assert rel_err(other, tout) > 0.1


@pytest.mark.parametrize("h,w,pad_h,pad_w", [(13, 11, 3, 5), (16, 8, 0, 0), (3, 5, 5, 3), (1, 1, 7, 7)])
def test_host_build_input_and_composite_equal_the_oracle(pkg, h, w, pad_h, pad_w):
    """The product host rules (liblama_host: lama_build_input, lama_composite,
    main.rs:175-196, 272-307) against the oracle's restatement, bit for bit,
    over every byte value and with bottom/right padding (including a pad
    wider than the image, which wraps the reflection)."""
    H = pkg.host_api
    rng = np.random.default_rng(h * 100 + w)
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    rgb.reshape(-1)[:min(256, rgb.size)] = np.arange(min(256, rgb.size), dtype=np.uint8)
    mask = rng.integers(0, 256, (h, w), dtype=np.uint8)
    mask.reshape(-1)[::3] = 0
    assert np.array_equal(H.build_input(rgb, mask, pad_h, pad_w), O.build_input(rgb, mask, pad_h, pad_w))
    net = rng.uniform(-0.1, 1.1, (3, h + pad_h, w + pad_w)).astype(np.float32)
    net.reshape(-1)[:4] = [0.0, 1.0, np.float32(0.5) / 255, np.float32(254.5) / 255]
    assert np.array_equal(H.composite(rgb, mask, net, pad_h, pad_w), O.composite(rgb, mask, net, pad_h, pad_w))
