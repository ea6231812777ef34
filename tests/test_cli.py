"""The lama-inpaint command line (lama-inpaint-rs_amd/bin/lama-inpaint), the
reference's CLI (lama-rs/src/main.rs:49-566) over the MI355X engine.

CPU tests cover argument handling and the error policy (no CPU engine in
this build, so --cpu and a failed GPU are errors with a message).  GPU tests
run the whole-image, --tile and --sections flows end to end and compare them
bit for bit with the same flows restated in Python over the engine
(main.rs:213-313, 378-443, 465-566) -- including the reference's own claim
that --tile equals cropping the window out, running it and pasting the hole
back -- and the whole-image output with the CPU oracle."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "lama-inpaint-rs_amd", "bin", "lama-inpaint")


# The reference's own inputs (testdata/in.png and testdata/mask.png), kept as fixtures:
# a 512 x 512 photograph with a 38,000-pixel hole inside the box x 150-469, y 60-329.
TD_IMG = os.path.join(ROOT, "tests", "golden", "testdata_in.png")
TD_MASK = os.path.join(ROOT, "tests", "golden", "testdata_mask.png")


def run_cli(*args, stdin=None, timeout=300):
    return subprocess.run([CLI, *args], capture_output=True, timeout=timeout, input=stdin)


@pytest.fixture(scope="module")
def H(pkg):
    return pkg.host_api


def write_case(H, d, img, mask):
    ip, mp = os.path.join(d, "in.png"), os.path.join(d, "mask.png")
    H.png_write_rgb(ip, img)
    H.png_write_rgb(mp, np.repeat(mask[..., None], 3, -1))
    return ip, mp


# ------------------------------------------------------------------ CPU

def test_help_and_usage_errors():
    r = run_cli("--help")
    assert r.returncode == 0 and b"usage: lama-inpaint" in r.stdout
    for args, msg in [((), b"--image is required"), (("--image", "a"), b"--mask is required"),
                      (("--image", "a", "--mask", "b"), b"--output is required"),
                      (("--bogus",), b"unknown argument --bogus"), (("--image",), b"--image needs a value"),
                      (("--image", "-", "--mask", "-", "--output", "o"), b"cannot both be '-'"),
                      (("--image", "a", "--mask", "b", "--output", "o", "--tile", "--sections"),
                       b"mutually exclusive")]:
        r = run_cli(*args)
        assert r.returncode == 2, args
        assert msg in r.stderr and b"usage:" in r.stderr, (args, r.stderr)


def test_input_errors(H, tmp_path):
    img = H.synth_image(24, 32, 1)
    ip = str(tmp_path / "i.png")
    H.png_write_rgb(ip, img)
    mp = str(tmp_path / "m.png")
    H.png_write_rgb(mp, np.zeros((16, 32, 3), np.uint8))
    r = run_cli("--image", ip, "--mask", mp, "--output", str(tmp_path / "o.png"))
    assert r.returncode == 1 and b"mask is 32x16 but image is 32x24" in r.stderr
    r = run_cli("--image", str(tmp_path / "nope.png"), "--mask", mp, "--output", str(tmp_path / "o.png"))
    assert r.returncode == 1 and b"error:" in r.stderr
    H.png_write_rgb(mp, np.zeros((24, 32, 3), np.uint8))
    r = run_cli("--image", ip, "--mask", mp, "--output", str(tmp_path / "o.png"), "--weights", "/nonexistent.st")
    assert r.returncode == 1 and b"/nonexistent.st" in r.stderr


def test_cpu_flag_is_refused_without_fallback(H, tmp_path, weights_dir):
    img = H.synth_image(24, 32, 1)
    mask, _ = H.synth_mask_rect(24, 32, 8, 8, 2)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    r = run_cli("--image", ip, "--mask", mp, "--output", str(tmp_path / "o.png"), "--weights", weights_dir["plain"],
                "--cpu")
    assert r.returncode == 1 and b"no CPU engine" in r.stderr
    assert not (tmp_path / "o.png").exists()


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK),
                    reason="a GPU is present")
def test_gpu_failure_is_an_error_not_a_fallback(H, tmp_path, weights_dir):
    img = H.synth_image(24, 32, 1)
    mask, _ = H.synth_mask_rect(24, 32, 8, 8, 2)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    r = run_cli("--image", ip, "--mask", mp, "--output", str(tmp_path / "o.png"), "--weights", weights_dir["plain"])
    assert r.returncode == 1 and b"gpu unavailable" in r.stderr and b"no CPU engine" in r.stderr
    r = run_cli("--image", ip, "--mask", mp, "--output", str(tmp_path / "o.png"), "--weights", weights_dir["plain"],
                "--gpu")
    assert r.returncode == 1 and b"gpu inference failed" in r.stderr


def test_empty_mask_tile_and_sections_copy_the_input(H, tmp_path, weights_dir):
    # main.rs:393-398, 486-490: an empty mask needs no network at all
    img = H.synth_image(600, 640, 3)
    ip, mp = write_case(H, str(tmp_path), img, np.zeros((600, 640), np.uint8))
    for flag in ("--tile", "--sections"):
        out = str(tmp_path / f"o{flag}.png")
        r = run_cli("--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["plain"], flag)
        assert r.returncode == 0, r.stderr
        assert b"mask is empty" in r.stderr
        assert np.array_equal(H.png_read_rgb(out), img)


def test_reference_testdata_geometry(H):
    """The --tile and --sections geometry on the reference's own inputs.
    --tile wants a window twice the 320-pixel box, which the 512-pixel image
    caps, so the window is the whole image (main.rs:740-790).  --sections cuts
    the box into 256-pixel cells from its top-left corner, clipped to the box,
    keeps those holding hole pixels and orders them by the shallowest hole
    pixel's 4-connected distance to the rim, then y0, x0 (main.rs:597-659).
    The distance is the taxicab distance transform of the zero-padded mask
    less one: the nearest unmasked pixel in L1 is reached by a monotone path
    through masked pixels, so the breadth-first depth equals it."""
    from scipy.ndimage import distance_transform_cdt
    img, mask = H.png_read_rgb(TD_IMG), H.png_read_gray(TD_MASK)
    assert img.shape == (512, 512, 3) and mask.shape == (512, 512)
    ys, xs = np.nonzero(mask)
    assert len(xs) == 38000 and (xs.min(), xs.max(), ys.min(), ys.max()) == (150, 469, 60, 329)
    t = H.tile_rect(mask)
    assert (t.x0, t.y0, t.side) == (0, 0, 512)

    hole = mask > 0
    depth = distance_transform_cdt(np.pad(hole, 1), metric="taxicab")[1:-1, 1:-1] - 1
    assert np.array_equal(H.mask_depth(mask)[hole], depth[hole])
    cells = [(x0, y0, min(x0 + 256, 470), min(y0 + 256, 330)) for y0 in (60, 316) for x0 in (150, 406)]
    cells = [c for c in cells if hole[c[1]:c[3], c[0]:c[2]].any()]
    secs = H.section_rects(mask)
    assert len(secs) == 3 and sorted(secs) == sorted(cells)
    cover = np.zeros(mask.shape, int)
    for x0, y0, x1, y1 in secs:
        cover[y0:y1, x0:x1] += 1
    assert np.all(cover[hole] == 1)
    keys = [(int(depth[y0:y1, x0:x1][hole[y0:y1, x0:x1]].min()), y0, x0) for x0, y0, x1, y1 in secs]
    assert keys == sorted(keys)


# ------------------------------------------------------------------ GPU

def _tile_by_hand(H, engine, img, mask):
    t = H.tile_rect(mask)
    s = t.side
    sub, sm = img[t.y0:t.y0 + s, t.x0:t.x0 + s], mask[t.y0:t.y0 + s, t.x0:t.x0 + s]
    pad = (8 - s % 8) % 8
    out = engine.forward(H.build_input(sub, sm, pad, pad))
    res = img.copy()
    u8 = H.composite(sub, sm, out, pad, pad)
    hole = sm > 0
    res[t.y0:t.y0 + s, t.x0:t.x0 + s][hole] = u8[hole]
    return res


def _sections_by_hand(H, engine, img, mask):
    h, w = mask.shape
    side = max(1, min(512, w, h))
    pad = (8 - side % 8) % 8
    work = img.copy()
    for x0, y0, x1, y1 in H.section_rects(mask):
        wx = H.window_origin((x0 + x1) // 2, side, w)
        wy = H.window_origin((y0 + y1) // 2, side, h)
        sub = work[wy:wy + side, wx:wx + side]
        sm = mask[wy:wy + side, wx:wx + side].copy()
        own = np.zeros_like(sm, bool)
        own[y0 - wy:y1 - wy, x0 - wx:x1 - wx] = True
        sm[~own] = 0
        out = engine.forward(H.build_input(sub, sm, pad, pad))
        u8 = H.composite(sub, sm, out, pad, pad)
        # the section's own hole pixels, which lie inside the window
        sel = np.zeros((h, w), bool)
        sel[y0:y1, x0:x1] = mask[y0:y1, x0:x1] > 0
        work[sel] = u8[sel[wy:wy + side, wx:wx + side]]
    return work


@pytest.mark.gpu
def test_cli_whole_image_matches_engine_and_oracle(H, engine, tmp_path, weights_dir):
    import oracle_api as O
    img = H.synth_image(76, 100, 1)  # pads to 80 x 104
    mask, _ = H.synth_mask_rect(76, 100, 30, 20, 2)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    out = str(tmp_path / "o.png")
    r = run_cli("--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["cal"], "--gpu")
    assert r.returncode == 0, r.stderr
    got = H.png_read_rgb(out)
    x = H.build_input(img, mask)
    want = H.composite(img, mask, engine.forward(x), 4, 4)
    assert np.array_equal(got, want)
    ref = H.composite(img, mask, O.OracleNet(O.read_safetensors(weights_dir["cal"])).forward(x), 4, 4)
    d = np.abs(got.astype(int) - ref.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1
    assert np.array_equal(got[mask == 0], img[mask == 0])


@pytest.mark.gpu
def test_cli_tile_equals_crop_run_paste(H, engine, tmp_path, weights_dir):
    img = H.synth_image(900, 1100, 4)
    mask, _ = H.synth_mask_rect(900, 1100, 120, 90, 5)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    out = str(tmp_path / "o.png")
    r = run_cli("--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["cal"], "--tile")
    assert r.returncode == 0, r.stderr
    assert b"tile: 512x512 window" in r.stderr
    assert np.array_equal(H.png_read_rgb(out), _tile_by_hand(H, engine, img, mask))


@pytest.mark.gpu
def test_cli_sections_equal_the_restated_pass_loop(H, engine, tmp_path, weights_dir):
    img = H.synth_image(1000, 1100, 6)
    mask = np.zeros((1000, 1100), np.uint8)
    mask[200:800, 300:900] = 255  # 600 x 600 -> 3 x 3 sections
    ip, mp = write_case(H, str(tmp_path), img, mask)
    out = str(tmp_path / "o.png")
    dump = tmp_path / "dump"
    dump.mkdir()
    env = dict(os.environ, LAMA_DUMP_SECTIONS=str(dump))
    r = subprocess.run([CLI, "--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["cal"],
                        "--sections"], capture_output=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr
    assert b"sections: 9 passes, 512x512 window each" in r.stderr
    got = H.png_read_rgb(out)
    assert np.array_equal(got, _sections_by_hand(H, engine, img, mask))
    assert np.array_equal(got[mask == 0], img[mask == 0])
    assert len(list(dump.iterdir())) == 9


@pytest.mark.gpu
def test_cli_reference_testdata_whole_tile_sections(H, engine, tmp_path, weights_dir):
    """The reference's own image and mask through the whole-image, --tile and
    --sections flows.  Unmasked pixels come back bit-exact in all three.  The
    --tile window is the whole image, so its output equals the whole-image
    pass; --sections on an image whose short side is at most 512 runs the
    whole image (main.rs:244-251).  The whole-image pass is within 1/255 (max)
    and 0.1 (mean) of the CPU oracle's."""
    import oracle_api as O
    img, mask = H.png_read_rgb(TD_IMG), H.png_read_gray(TD_MASK)
    outs = {}
    for flag in ("", "--tile", "--sections"):
        print(f"case testdata 512x512 {flag or 'whole image'}", flush=True)
        out = str(tmp_path / f"o{flag}.png")
        r = run_cli("--image", TD_IMG, "--mask", TD_MASK, "--output", out, "--weights", weights_dir["cal"], "--gpu",
                    *([flag] if flag else []))
        assert r.returncode == 0, r.stderr
        got = H.png_read_rgb(out)
        assert np.array_equal(got[mask == 0], img[mask == 0])
        outs[flag] = (got, r.stderr)
    assert b"tile: 512x512 window at (0,0) covering a 320x270 mask" in outs["--tile"][1]
    assert np.array_equal(outs["--tile"][0], outs[""][0])
    assert b"at or below 512px on its short side; running the whole image" in outs["--sections"][1]
    assert np.array_equal(outs["--sections"][0], outs[""][0])
    x = O.build_input(img, mask, 0, 0)
    ref = O.composite(img, mask, O.OracleNet(O.read_safetensors(weights_dir["cal"])).forward(x), 0, 0)
    d = np.abs(outs[""][0].astype(int) - ref.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1


@pytest.mark.gpu
def test_cli_reference_testdata_in_a_larger_frame(H, engine, tmp_path, weights_dir):
    """The reference's image and mask set into a 700 x 660 frame (so that
    --sections cuts the real hole into its 3 sections): --sections equals the
    restated pass loop and --tile the crop-run-paste, bit for bit, with the
    frame's pixels and the unmasked image pixels untouched."""
    img, mask = H.png_read_rgb(TD_IMG), H.png_read_gray(TD_MASK)
    big = H.synth_image(700, 660, 9)
    bmask = np.zeros((700, 660), np.uint8)
    big[100:612, 80:592], bmask[100:612, 80:592] = img, mask
    ip, mp = write_case(H, str(tmp_path), big, bmask)
    for flag, want in (("--sections", lambda: _sections_by_hand(H, engine, big, bmask)),
                       ("--tile", lambda: _tile_by_hand(H, engine, big, bmask))):
        print(f"case testdata in 700x660 {flag}", flush=True)
        out = str(tmp_path / f"o{flag}.png")
        r = run_cli("--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["cal"], flag)
        assert r.returncode == 0, r.stderr
        got = H.png_read_rgb(out)
        assert np.array_equal(got[bmask == 0], big[bmask == 0])
        assert np.array_equal(got, want())
        if flag == "--sections":
            assert b"sections: 3 passes, 512x512 window each" in r.stderr


@pytest.mark.gpu
def test_cli_stdin_stdout(H, tmp_path, weights_dir):
    img = H.synth_image(64, 72, 7)
    mask, _ = H.synth_mask_rect(64, 72, 20, 12, 8)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    a = run_cli("--image", "-", "--mask", mp, "--output", "-", "--weights", weights_dir["cal"],
                stdin=open(ip, "rb").read())
    assert a.returncode == 0, a.stderr
    b_out = str(tmp_path / "b.png")
    b = run_cli("--image", ip, "--mask", mp, "--output", b_out, "--weights", weights_dir["cal"])
    assert b.returncode == 0
    assert a.stdout == open(b_out, "rb").read()


@pytest.mark.gpu
def test_plan_bytes_is_the_allocated_arena(pkg, engine):
    x = np.zeros((4, 136, 200), np.float32)
    predicted, weights = engine.plan_bytes(136, 200)
    engine.forward(x)
    actual, _ = engine.plan_bytes(136, 200)
    assert predicted == actual > 0 and weights > 200e6


@pytest.mark.gpu
def test_plan_rejects_unsupported_shapes(pkg, engine):
    # not padded to 8 (the caller pads, main.rs:241-242), and beyond the 2^27-pixel
    # bound of the kernels' 32-bit staging offsets
    for h, w, msg in [(100, 64, "multiple of 8"), (16384, 8200, "2\\^27 pixels")]:
        with pytest.raises(pkg.hip_engine.HipError, match=msg):
            engine.plan_bytes(h, w)
    assert engine.plan_bytes(8192, 16384)[0] > 0  # exactly 2^27 pixels plans


@pytest.mark.gpu
def test_cli_sections_config4_2048_with_1024_hole(H, engine, tmp_path, weights_dir):
    """BASELINE configs[4] --sections as specified: a 2048 x 2048 image with a
    seeded 1024 x 1024 hole, filled as 16 sections of 256 x 256 in 512 x 512
    windows, rim inward; bit-exact with the restated pass loop."""
    img = H.synth_image(2048, 2048, 1)
    mask, (x0, y0) = H.synth_mask_rect(2048, 2048, 1024, 1024, 2)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    out = str(tmp_path / "o.png")
    print("case sections 2048 / 1024 hole", flush=True)
    r = run_cli("--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["cal"], "--sections",
                timeout=600)
    assert r.returncode == 0, r.stderr
    assert b"sections: 16 passes, 512x512 window each" in r.stderr
    got = H.png_read_rgb(out)
    assert np.array_equal(got, _sections_by_hand(H, engine, img, mask))
    assert np.array_equal(got[mask == 0], img[mask == 0])


@pytest.mark.gpu
def test_cli_tile_config4_2048_with_300_hole(H, engine, tmp_path, weights_dir):
    """BASELINE configs[4] --tile as specified: a 2048 x 2048 image with a
    seeded 300 x 300 hole runs one 600 x 600 window (tile_rect, main.rs:740-777;
    the README's --tile timing is this window).  The output is bit-exact with
    crop-run-paste (main.rs:378-443) restated over the engine; the window's
    composite is within 1/255 max and 0.1 levels mean of the CPU oracle's on
    the same window; every pixel outside the hole keeps its source bytes."""
    import oracle_api as O
    img = H.synth_image(2048, 2048, 1)
    mask, _ = H.synth_mask_rect(2048, 2048, 300, 300, 2)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    out = str(tmp_path / "o.png")
    print("case tile 2048 / 300 hole", flush=True)
    r = run_cli("--image", ip, "--mask", mp, "--output", out, "--weights", weights_dir["cal"], "--gpu", "--tile",
                timeout=600)
    assert r.returncode == 0, r.stderr
    t = H.tile_rect(mask)
    assert t.side == 600, t.side
    assert f"tile: 600x600 window at ({t.x0},{t.y0})".encode() in r.stderr, r.stderr
    got = H.png_read_rgb(out)
    assert np.array_equal(got, _tile_by_hand(H, engine, img, mask))
    assert np.array_equal(got[mask == 0], img[mask == 0])
    # the window against the oracle: the same crop, build_input and composite
    sub, sm = img[t.y0:t.y0 + 600, t.x0:t.x0 + 600], mask[t.y0:t.y0 + 600, t.x0:t.x0 + 600]
    x = H.build_input(sub, sm, 0, 0)
    ref = H.composite(sub, sm, O.OracleNet(O.read_safetensors(weights_dir["cal"])).forward(x), 0, 0)
    win = got[t.y0:t.y0 + 600, t.x0:t.x0 + 600]
    d = np.abs(win.astype(int) - ref.astype(int))
    assert d.max() <= 1 and d.mean() <= 0.1, (d.max(), d.mean())


@pytest.mark.gpu
def test_cli_dump_step_matches_the_oracle(H, tmp_path, weights_dir):
    """LAMA_DUMP_STEP=<n> (cuda.rs:1572-1574, 1647-1662): the CLI's pass
    writes /tmp/gpu_step_<n>.f32 in the reference's layout (local planes, then
    global); it matches the oracle's step n within the per-layer bound.
    LAMA_PROFILE adds the per-step lines (cuda.rs:1663-1686)."""
    import oracle_api as O
    img = H.synth_image(64, 80, 2)
    mask, _ = H.synth_mask_rect(64, 80, 24, 16, 3)
    ip, mp = write_case(H, str(tmp_path), img, mask)
    ref, ref_steps = O.OracleNet(O.read_safetensors(weights_dir["cal"])).forward(H.build_input(img, mask),
                                                                                 steps=True)
    for n in (7, 26):
        path = f"/tmp/gpu_step_{n}.f32"
        if os.path.exists(path):
            os.remove(path)
        env = dict(os.environ, LAMA_DUMP_STEP=str(n), LAMA_PROFILE="1", LAMA_PROFILE_SYNC="1")
        r = subprocess.run([CLI, "--image", ip, "--mask", mp, "--output", str(tmp_path / "o.png"), "--weights",
                            weights_dir["cal"]], capture_output=True, timeout=300, env=env)
        assert r.returncode == 0, r.stderr
        got = np.fromfile(path, dtype="<f4")
        assert got.shape == ref_steps[n].shape
        assert float(np.linalg.norm(got - ref_steps[n]) / np.linalg.norm(ref_steps[n])) < 1e-3
        assert f"gpu dumped step {n}:".encode() in r.stderr
        assert b"gpu step 28:" in r.stderr and b"gpu step  0:" in r.stderr
        assert b"gpu step  7:" in r.stderr and b"global Some((384, 8, 10))" in r.stderr
        assert b"gpu totals:" in r.stderr
