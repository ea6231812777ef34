"""The whole forward on the GPU against the CPU oracle: every plan step
within 1e-3 relative L2 error (the north star's per-layer bound), the final
8-bit composite within 1/255 max and 0.1 levels mean, unmasked pixels
bit-exact."""
import numpy as np
import pytest

import oracle_api as O
from conftest import rel_err

pytestmark = pytest.mark.gpu

STEP_TOL = 1e-3


def _case(pkg, h, w, kind="rect"):
    H = pkg.host_api
    img = H.synth_image(h, w, 1)
    if kind == "rect":
        mask, _ = H.synth_mask_rect(h, w, max(1, w // 5), max(1, h // 8), 2)
    else:
        mask, _ = H.synth_mask_strokes(h, w, 0.25, 2)
    return img, mask


@pytest.fixture(scope="module")
def oracle_cal(weights_dir):
    return O.OracleNet(O.read_safetensors(weights_dir["cal"]))


@pytest.mark.parametrize("h,w,kind", [(64, 64, "rect"), (128, 96, "strokes"), (256, 256, "rect")])
def test_forward_steps_calibrated(pkg, engine, oracle_cal, h, w, kind):
    img, mask = _case(pkg, h, w, kind)
    x = pkg.host_api.build_input(img, mask)
    print(f"case {h}x{w} {kind}", flush=True)
    ref, ref_steps = oracle_cal.forward(x, steps=True)
    got, got_steps = engine.forward_steps(x, list(range(29)))
    for s in range(29):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
    assert rel_err(got, ref) < STEP_TOL
    u8g = pkg.host_api.composite(img, mask, got, 0, 0)
    u8r = pkg.host_api.composite(img, mask, ref, 0, 0)
    d = np.abs(u8g.astype(int) - u8r.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())
    keep = mask == 0
    assert np.array_equal(u8g[keep], img[keep])


@pytest.fixture(scope="module")
def direct_engine(pkg, weights_dir):
    # the engine reads LAMA_FFC_WINO when it opens
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_FFC_WINO", "0")
        eng = pkg.hip_engine.Engine()
    eng.load_weights(pkg.host_api.Store(weights_dir["cal"]))
    yield eng
    eng.close()


@pytest.mark.parametrize("h,w,kind", [(64, 64, "rect"), (128, 96, "strokes"), (512, 512, "strokes")])
def test_forward_direct_3x3_matches_winograd(pkg, direct_engine, engine, oracle_cal, h, w, kind):
    """The forward with the FFC 3x3 convolutions as direct implicit GEMMs
    (LAMA_FFC_WINO=0): every plan step within the per-layer bound of the
    oracle (where it runs in seconds), and the output within float rounding
    of the default Winograd forward, its composite within 1/255."""
    img, mask = _case(pkg, h, w, kind)
    x = pkg.host_api.build_input(img, mask)
    print(f"case direct {h}x{w} {kind}", flush=True)
    got, got_steps = direct_engine.forward_steps(x, list(range(29)))
    if h * w <= 128 * 128:
        ref, ref_steps = oracle_cal.forward(x, steps=True)
        for s in range(29):
            e = rel_err(got_steps[s], ref_steps[s])
            assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
        assert rel_err(got, ref) < STEP_TOL
    wino = engine.forward(x)
    assert rel_err(got, wino) < 1e-4
    u8g = pkg.host_api.composite(img, mask, got, 0, 0)
    u8w = pkg.host_api.composite(img, mask, wino, 0, 0)
    d = np.abs(u8g.astype(int) - u8w.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())
    keep = mask == 0
    assert np.array_equal(u8g[keep], img[keep])


@pytest.mark.parametrize("h,w", [(512, 512), (256, 384)])
def test_g2l_stream_matches_single_order(pkg, engine, monkeypatch, h, w):
    """The FFC's g2l launch B(k) on a stream of its own (LAMA_B_STREAM=1),
    overlapping A(k+1), ordered by events (B waits for x_g, finalize waits
    for B) and with the g2l partials double-buffered by FFC parity: three
    passes with different inputs queued back to back, each into its own
    output, all bit-identical to the default schedule's forward."""
    H = pkg.host_api
    xs = []
    for seed in range(3):
        img = H.synth_image(h, w, seed + 1)
        mask, _ = H.synth_mask_strokes(h, w, 0.25, seed + 2)
        xs.append(H.build_input(img, mask))
    monkeypatch.setenv("LAMA_B_STREAM", "0")
    eng0 = pkg.hip_engine.Engine()
    eng0.load_weights(engine._cal_store)
    ref = [eng0.forward(x) for x in xs]
    eng0.close()
    monkeypatch.setenv("LAMA_B_STREAM", "1")
    eng1 = pkg.hip_engine.Engine()
    eng1.load_weights(engine._cal_store)
    d_in = [eng1.malloc(x.nbytes) for x in xs]
    d_out = [eng1.malloc(3 * h * w * 4) for _ in xs]
    for d, x in zip(d_in, xs):
        eng1.upload(d, x)
    print(f"case {h}x{w} g2l stream, 2 x 3 queued passes", flush=True)
    for rep in range(2):
        for d, o in zip(d_in, d_out):
            eng1.forward_device(d, h, w, o)
        eng1.synchronize()
        for i, o in enumerate(d_out):
            out = np.empty((3, h, w), np.float32)
            eng1.download(out, o)
            assert np.array_equal(out, ref[i]), f"rep {rep} pass {i}"
    assert np.array_equal(eng1.forward(xs[1]), ref[1])
    for d in d_in + d_out:
        eng1.free(d)
    eng1.close()


def test_forward_plain_weights(pkg, weights_dir):
    """The BASELINE fixture as specified (uncalibrated BN statistics, so the
    activations grow by ~1e10 through the resblocks): per-step relative error
    still within 1e-3."""
    eng = pkg.hip_engine.Engine()
    store = pkg.host_api.Store(weights_dir["plain"])
    eng.load_weights(store)
    net = O.OracleNet(O.read_safetensors(weights_dir["plain"]))
    img, mask = _case(pkg, 64, 64)
    x = pkg.host_api.build_input(img, mask)
    ref, ref_steps = net.forward(x, steps=True)
    got, got_steps = eng.forward_steps(x, list(range(29)))
    for s in range(28):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
    # saturated sigmoid: compare where the oracle is not saturated
    assert rel_err(got, ref) < STEP_TOL
    eng.close()


def test_forward_repeatable_and_shapes(pkg, engine):
    img, mask = _case(pkg, 64, 128)
    x = pkg.host_api.build_input(img, mask)
    a = engine.forward(x)
    b = engine.forward(x)
    assert a.shape == (3, 64, 128)
    assert np.array_equal(a, b)
    # head, 3 downsamplers, 36 FFCs x (2 grouped GEMMs, finalize, conv1, rfft2, FU conv, irfft2, conv2),
    # 3 upsamplers, tail
    assert engine.launch_count(64, 128) == 1 + 3 + 36 * 8 + 3 + 1


def test_forward_split_fft_1024(pkg, engine, oracle_cal):
    """1024x1024: the 128x128 bottleneck planes exceed one block's 64 KB LDS
    budget, so every rfft2/irfft2 runs as row + column launches."""
    h = w = 1024
    img, mask = _case(pkg, h, w, "strokes")
    x = pkg.host_api.build_input(img, mask)
    print(f"case {h}x{w} strokes (split FFT)", flush=True)
    got, got_steps = engine.forward_steps(x, list(range(29)))
    assert engine.launch_count(h, w) == 1 + 3 + 36 * 10 + 3 + 1
    ref, ref_steps = oracle_cal.forward(x, steps=True)
    for s in range(29):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
    u8g = pkg.host_api.composite(img, mask, got, 0, 0)
    u8r = pkg.host_api.composite(img, mask, ref, 0, 0)
    d = np.abs(u8g.astype(int) - u8r.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())


def test_forward_split_forced_matches_single(pkg, engine, monkeypatch):
    """The split launches compute the same transform as the single-block
    kernels: at 128x96 the whole forward agrees to float rounding."""
    img, mask = _case(pkg, 128, 96, "strokes")
    x = pkg.host_api.build_input(img, mask)
    a = engine.forward(x)
    monkeypatch.setenv("LAMA_FFT_SPLIT", "1")
    eng2 = pkg.hip_engine.Engine()
    eng2.load_weights(engine._store)
    b = eng2.forward(x)
    assert eng2.launch_count(128, 96) == 1 + 3 + 36 * 10 + 3 + 1
    eng2.close()
    assert rel_err(b, a) < 1e-5


@pytest.mark.parametrize("size", [256, 512, 600, 1024, 2048])
def test_compiled_shape_fft_equals_generic(pkg, engine, monkeypatch, size):
    """The 32x32 / 64x64 / 75x75 bottleneck planes (256, 512 and 600 inputs) use
    single-block FFT kernels with the shape compiled in, the 128x128 / 256x256 planes (1024
    and 2048 inputs) split row/column kernels with the shape compiled in; they
    run the same radix plan as the runtime-shaped kernels (LAMA_FFT_GENERIC=1),
    so the whole forward agrees to float rounding (the compiler contracts a few
    multiply-adds differently)."""
    print(f"case {size}x{size} strokes (compiled-shape vs generic FFT)", flush=True)
    img, mask = _case(pkg, size, size, "strokes")
    x = pkg.host_api.build_input(img, mask)
    a = engine.forward(x)
    monkeypatch.setenv("LAMA_FFT_GENERIC", "1")
    eng2 = pkg.hip_engine.Engine()
    eng2.load_weights(engine._store)
    b = eng2.forward(x)
    eng2.close()
    assert rel_err(b, a) < 1e-5


def test_forward_512_shuffle_row_fft(pkg, engine, monkeypatch):
    """With LAMA_FFT64_SHFL=1 the 512x512 plan takes the 64 x 64 transforms
    whose rows are wavefront-shuffle FFTs in registers; the forward agrees
    with the default (LDS-pass) transforms to float rounding."""
    print("case 512x512 strokes (shuffle-row vs LDS-pass 64x64 FFT)", flush=True)
    img, mask = _case(pkg, 512, 512, "strokes")
    x = pkg.host_api.build_input(img, mask)
    a = engine.forward(x)
    monkeypatch.setenv("LAMA_FFT64_SHFL", "1")
    eng2 = pkg.hip_engine.Engine()
    eng2.load_weights(engine._store)
    b = eng2.forward(x)
    assert eng2.kernel_name(512, 512, "rfft2") == "lama_rfft2_64s"
    assert eng2.kernel_name(512, 512, "irfft2") == "lama_irfft2_64s"
    eng2.close()
    assert rel_err(b, a) < 1e-5


def test_forward_2048_whole_image(pkg, engine):
    """configs[4] at its full size (bottleneck 512 x 256 x 256): checked by
    size-independent properties -- finite, bitwise repeatable, sigmoid range,
    unmasked pixels of the composite bit-exact."""
    h = w = 2048
    H = pkg.host_api
    img = H.synth_image(h, w, 1)
    mask, _ = H.synth_mask_rect(h, w, 300, 300, 2)
    x = H.build_input(img, mask)
    print(f"case {h}x{w} rect 300", flush=True)
    a = engine.forward(x)
    b = engine.forward(x)
    assert np.array_equal(a, b)
    assert np.isfinite(a).all() and a.min() >= 0 and a.max() <= 1
    u8 = H.composite(img, mask, a, 0, 0)
    keep = mask == 0
    assert np.array_equal(u8[keep], img[keep])
    assert engine.launch_count(h, w) == 1 + 3 + 36 * 10 + 3 + 1


@pytest.mark.timeout(900)
def test_forward_2048_whole_image_against_the_oracle(pkg, engine, oracle_cal):
    """configs[4] whole image at its full size against the CPU oracle
    (main.rs:212-313 through cpu.rs:741-751): a 2048 x 2048 blurred-noise
    image with a seeded 300 x 300 hole; every plan step within the per-layer
    bound, the composite within 1/255 max and 0.1 levels mean, unmasked pixels
    bit-exact.  The oracle pass takes about a minute on 16 host threads."""
    h = w = 2048
    H = pkg.host_api
    img = H.synth_image(h, w, 1)
    mask, _ = H.synth_mask_rect(h, w, 300, 300, 2)
    x = H.build_input(img, mask)
    print(f"case oracle {h}x{w} rect 300", flush=True)
    got, got_steps = engine.forward_steps(x, list(range(29)))
    ref, ref_steps = oracle_cal.forward(x, steps=True)
    for s in range(29):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
        got_steps[s] = ref_steps[s] = None
    assert rel_err(got, ref) < STEP_TOL
    u8g = H.composite(img, mask, got, 0, 0)
    u8r = H.composite(img, mask, ref, 0, 0)
    d = np.abs(u8g.astype(int) - u8r.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())
    assert np.array_equal(u8g[mask == 0], img[mask == 0])


@pytest.mark.parametrize("h,w", [(128, 96), (256, 256), (512, 512)])
def test_graph_replays_match_eager(pkg, engine, monkeypatch, h, w):
    """The forward captured as one HIP graph and replayed (the default at
    256 x 256 and below, LAMA_GRAPH=1 above): every replay, with eager work and
    synchronisations in between, equals the per-launch path bit for bit."""
    img, mask = _case(pkg, h, w, "strokes")
    x = pkg.host_api.build_input(img, mask)
    monkeypatch.setenv("LAMA_GRAPH", "0")
    eng0 = pkg.hip_engine.Engine()
    eng0.load_weights(engine._store)
    eager = eng0.forward(x)
    eng0.close()
    monkeypatch.setenv("LAMA_GRAPH", "1")
    eng1 = pkg.hip_engine.Engine()
    eng1.load_weights(engine._store)
    rng = np.random.default_rng(3)
    d_in = eng1.malloc(x.nbytes)
    d_out = eng1.malloc(3 * h * w * 4)
    eng1.upload(d_in, x)
    for i in range(4):
        out = eng1.forward(x) if i % 2 == 0 else None
        if out is None:
            eng1.forward_device(d_in, h, w, d_out)
            eng1.synchronize()
            out = np.empty((3, h, w), np.float32)
            eng1.download(out, d_out)
        assert np.array_equal(out, eager), f"replay {i}"
        # eager work between replays
        eng1.op_conv2d(rng.standard_normal((8, 9, 11), np.float32), rng.standard_normal((16, 8, 3, 3), np.float32))
    eng1.free(d_in)
    eng1.free(d_out)
    eng1.close()


@pytest.mark.parametrize("h,w", [(600, 600), (600, 592)])
def test_forward_600_tile_window_non_pow2_bottleneck(pkg, engine, oracle_cal, h, w):
    """configs[4]'s --tile window: 600 x 600 (75 x 75 bottleneck, FFT lengths
    75 and 38 through the reference's opposite-sign rule) against the oracle,
    every step.  600 x 592 gives bottleneck planes of 5550 and spectral planes
    of 2850 values: even but not multiples of 4, so every 1x1 convolution
    (conv1, FourierUnit, conv2 with its epilogue) takes the float2 loads."""
    img, mask = _case(pkg, h, w, "rect")
    x = pkg.host_api.build_input(img, mask)
    print(f"case {h}x{w} rect", flush=True)
    got, got_steps = engine.forward_steps(x, list(range(29)))
    ref, ref_steps = oracle_cal.forward(x, steps=True)
    for s in range(29):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
    u8g = pkg.host_api.composite(img, mask, got, 0, 0)
    u8r = pkg.host_api.composite(img, mask, ref, 0, 0)
    d = np.abs(u8g.astype(int) - u8r.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())
    assert np.array_equal(u8g[mask == 0], img[mask == 0])


@pytest.mark.parametrize("h,w", [(8, 8), (8, 24), (16, 24), (24, 56)])
def test_forward_tiny_bottleneck_planes(pkg, engine, oracle_cal, h, w):
    """Bottleneck planes of 1, 3, 6 and 21 pixels against the oracle, every
    step: the local branch's finish (sum of the K-range partials, BN, ReLU,
    residual) takes its one-element path below 4 pixels and its clamped
    4-element window at the plane's end otherwise."""
    img, mask = _case(pkg, h, w, "rect")
    x = pkg.host_api.build_input(img, mask)
    print(f"case {h}x{w} rect", flush=True)
    got, got_steps = engine.forward_steps(x, list(range(29)))
    ref, ref_steps = oracle_cal.forward(x, steps=True)
    for s in range(29):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
    assert rel_err(got, ref) < STEP_TOL


@pytest.fixture(scope="module", params=[("2", ""), ("4", "64"), ("4", "32"), ("4", "16"), ("42", "")],
                ids=["f23", "f43w64", "f43w32", "f43w16", "f2x4"])
def w4_forward_engine(pkg, weights_dir, request):
    """The forward with each Winograd kernel forced: F(2,3) (LAMA_FFC_WINO=2),
    F(4,3) in 64-, 32- or 16-pixel blocks (LAMA_W4_TILE) and F(2x4, 3x3)
    (LAMA_FFC_WINO=42)."""
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_FFC_WINO", request.param[0])
        mp.setenv("LAMA_W4_TILE", request.param[1])
        eng = pkg.hip_engine.Engine()
    eng.load_weights(pkg.host_api.Store(weights_dir["cal"]))
    yield eng
    eng.close()


@pytest.mark.parametrize("h,w,kind", [(128, 96, "strokes"), (256, 256, "rect"), (600, 600, "rect")])
def test_forward_winograd_f43_steps(pkg, w4_forward_engine, oracle_cal, h, w, kind):
    """The forward with the FFC 3x3 convolutions as Winograd F(2,3) and as
    F(4,3) in 64-pixel blocks (the default, F(4,3) in 32-pixel blocks, runs
    every other forward test): every plan step within the per-layer bound of
    the oracle, the composite within 1/255."""
    img, mask = _case(pkg, h, w, kind)
    x = pkg.host_api.build_input(img, mask)
    print(f"case f43 {h}x{w} {kind}", flush=True)
    got, got_steps = w4_forward_engine.forward_steps(x, list(range(29)))
    ref, ref_steps = oracle_cal.forward(x, steps=True)
    for s in range(29):
        e = rel_err(got_steps[s], ref_steps[s])
        assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"
    assert np.array_equal(w4_forward_engine.forward(x), got)
    u8g = pkg.host_api.composite(img, mask, got, 0, 0)
    u8r = pkg.host_api.composite(img, mask, ref, 0, 0)
    d = np.abs(u8g.astype(int) - u8r.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())


def test_forward_winograd_f43_matches_f23_512(pkg, w4_forward_engine, engine):
    """At the bench shape, the default forward within float rounding of the
    other Winograd variants'."""
    img, mask = _case(pkg, 512, 512, "strokes")
    x = pkg.host_api.build_input(img, mask)
    a = w4_forward_engine.forward(x)
    b = engine.forward(x)
    assert rel_err(a, b) < 1e-4


def test_forward_f2x4_matches_f43_1536(pkg, weights_dir, engine):
    """At 1536 x 1536 the bottleneck planes are 192 wide, three of the
    F(2x4, 3x3) kernel's 64-pixel block columns: the default forward, which
    takes that kernel there, within float rounding of the F(4,3) one
    (LAMA_W42=0), with the composite within 1/255."""
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_W42", "0")
        e43 = pkg.hip_engine.Engine()
    try:
        e43.load_weights(pkg.host_api.Store(weights_dir["cal"]))
        img, mask = _case(pkg, 1536, 1536, "strokes")
        x = pkg.host_api.build_input(img, mask)
        print("case f2x4 vs f43 1536x1536", flush=True)
        a = engine.forward(x)
        assert engine.kernel_name(1536, 1536, "conv3x3") == "lama_conv3x3w42"
        b = e43.forward(x)
        assert e43.kernel_name(1536, 1536, "conv3x3").startswith("lama_conv3x3w4")
        assert e43.kernel_name(1536, 1536, "conv3x3") != "lama_conv3x3w42"
        assert rel_err(a, b) < 1e-4
        ua = pkg.host_api.composite(img, mask, a, 0, 0)
        ub = pkg.host_api.composite(img, mask, b, 0, 0)
        d = np.abs(ua.astype(int) - ub.astype(int))
        assert d.max() <= 1, d.max()
    finally:
        e43.close()


def test_device_packed_weights_match_host_packed(pkg, weights_dir, engine):
    """The FFC 3x3 weights packed for the Winograd kernels on the device
    (lama_pack_wino, the default) and on the host (LAMA_HOST_PACK=1): the same
    floats, so forwards through the F(4,3) packs (128 x 96) and through the
    F(2x4, 3x3) packs (1024 x 1024) are bit-identical."""
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("LAMA_HOST_PACK", "1")
        eh = pkg.hip_engine.Engine()
    try:
        eh.load_weights(pkg.host_api.Store(weights_dir["cal"]))
        for (h, w), f2x4 in (((128, 96), False), ((1024, 1024), True)):
            img, mask = _case(pkg, h, w, "strokes")
            x = pkg.host_api.build_input(img, mask)
            print(f"case device vs host packs {h}x{w}", flush=True)
            a = engine.forward(x)
            b = eh.forward(x)
            kern = engine.kernel_name(h, w, "conv3x3")
            assert kern == eh.kernel_name(h, w, "conv3x3")
            assert kern.startswith("lama_conv3x3w4") and (kern == "lama_conv3x3w42") == f2x4, kern
            assert np.array_equal(a, b)
    finally:
        eh.close()


def test_timeline_records_every_launch(pkg, engine):
    """lama_hip_timeline: one pass's 296 launches in issue order, each with a
    kernel-clock window; launches on one stream never overlap, and the
    timeline leaves the result unchanged."""
    img, mask = _case(pkg, 128, 96, "strokes")
    x = pkg.host_api.build_input(img, mask)
    ref = engine.forward(x)
    engine.timeline(True)
    got = engine.forward(x)
    tl = engine.timeline_read()
    engine.timeline(False)
    assert np.array_equal(got, ref)
    assert len(tl) == 1 + 3 + 36 * 8 + 3 + 1
    assert tl[0][0] == "conv7x7" and tl[-1][0] == "tail"
    assert all(0 <= s <= e for _, _, s, e in tl)
    for stream in (0, 1, 2):
        own = [(s, e) for _, st, s, e in tl if st == stream]
        assert own and all(b[0] >= a[1] - 0.05 for a, b in zip(own, own[1:])), stream
    # FFC k's conv2 (stream 1) starts after its l2l + l2g launch (stream 0) ends
    a_ends = [e for f, st, s, e in tl if f == "conv3x3"]
    c2_starts = [s for f, st, s, e in tl if f == "conv1x1res"]
    assert len(a_ends) == len(c2_starts) == 36
    assert all(c >= a - 0.05 for a, c in zip(a_ends, c2_starts))


@pytest.mark.parametrize("ks", ["1", "2"])
def test_forward_ksplit_variants_256(pkg, engine, oracle_cal, monkeypatch, ks):
    """The FFC GEMMs' K split (LAMA_KSPLIT, read at open): at 256 x 256 the
    default splits K in 4 (its raw partials summed by finalize and by conv2's
    epilogue); 1 and 2 slices give the same forward within float rounding,
    and every plan step of the 2-slice forward is within the per-layer bound
    of the oracle."""
    img, mask = _case(pkg, 256, 256, "rect")
    x = pkg.host_api.build_input(img, mask)
    default = engine.forward(x)
    monkeypatch.setenv("LAMA_KSPLIT", ks)
    eng = pkg.hip_engine.Engine()
    eng.load_weights(engine._cal_store)
    print(f"case 256x256 ksplit {ks}", flush=True)
    got, got_steps = eng.forward_steps(x, list(range(29)))
    eng.close()
    assert rel_err(got, default) < 1e-4
    if ks == "2":
        ref, ref_steps = oracle_cal.forward(x, steps=True)
        for s in range(29):
            e = rel_err(got_steps[s], ref_steps[s])
            assert e < STEP_TOL, f"step {s}: rel err {e:.3e}"


@pytest.mark.parametrize("h,w,kernel,fft", [(512, 512, "lama_conv3x3w4", "lama_rfft2_64"),
                                            (600, 600, "lama_conv3x3w4q", "lama_rfft2_75"),
                                            (600, 592, "lama_conv3x3w4q", "lama_rfft2"),
                                            (256, 256, "lama_conv3x3w4n", "lama_rfft2_32"),
                                            (16, 1024, "lama_conv3x3w4", "lama_rfft2"),
                                            (1024, 1024, "lama_conv3x3w42", "lama_rfft2_rows_128")])
def test_ffc_block_shape_per_plane(pkg, engine, h, w, kernel, fft):
    """The FFC GEMMs take the F(4,3) block shape that covers the bottleneck
    plane with the fewest blocks of 32 tiles (2 x 64 px on a tie): 75-rows
    planes 10 x 5 blocks of 8 x 16 instead of 19 x 3 of 4 x 32; a plane of 2
    rows and 128 columns 2 blocks of 2 x 64 instead of 4 of 4 x 32.  From
    128 x 128 bottleneck planes (1024 x 1024 inputs) on they run as F(2x4,
    3x3).  Square 32, 64 and 75 planes take the FFT kernels with the shape
    compiled in."""
    print(f"case block shape {h}x{w}", flush=True)
    x = np.zeros((4, h, w), np.float32)
    engine.forward(x)
    assert engine.kernel_name(h, w, "conv3x3") == kernel
    assert engine.kernel_name(h, w, "conv3x3g2l") == kernel
    assert engine.kernel_name(h, w, "rfft2") == fft
