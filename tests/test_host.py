"""Host-side logic of liblama_host.so on the CPU: the --tile / --sections
window geometry (the 21 tests of lama-rs/src/main.rs:800-1160, restated), the
memory guard (mem.rs:103-150), the weight container reader/writer, the PNG
codec and the synthetic fixtures.  Geometry is integer work: bit-exact."""
import os
import struct
import json

import numpy as np
import pytest

TILE_MIN = 512
PAD_MOD = 8
SECTION_BLOCK = 256


@pytest.fixture(scope="module")
def H(pkg):
    return pkg.host_api


def mask_of(w, h, rect=None):
    m = np.zeros((h, w), np.uint8)
    if rect is not None:
        x0, y0, x1, y1 = rect
        m[y0:y1 + 1, x0:x1 + 1] = 255
    return m


# ------------------------------------------------------------ --tile window

def assert_contains(t, m):
    h, w = m.shape
    ys, xs = np.nonzero(m)
    assert (xs >= t.x0).all() and (xs < t.x0 + t.side).all()
    assert (ys >= t.y0).all() and (ys < t.y0 + t.side).all()
    assert t.x0 + t.side <= w and t.y0 + t.side <= h
    if min(w, h) >= PAD_MOD:
        assert t.side % PAD_MOD == 0


def test_empty_mask_has_no_window(H):
    assert H.tile_rect(mask_of(256, 256)) is None


def test_small_mask_gets_the_minimum_window(H):
    m = mask_of(1024, 1024, (500, 500, 515, 515))
    t = H.tile_rect(m)
    assert t.side == TILE_MIN
    assert_contains(t, m)


def test_window_is_twice_the_bounding_box(H):
    m = mask_of(2048, 2048, (900, 800, 1199, 1099))
    t = H.tile_rect(m)
    assert t.side == 600
    assert (t.bbox_w, t.bbox_h) == (300, 300)
    assert_contains(t, m)


def test_wider_than_tall_uses_the_longer_side(H):
    m = mask_of(2048, 2048, (100, 1000, 799, 1099))
    t = H.tile_rect(m)
    assert t.side == 1400
    assert_contains(t, m)


@pytest.mark.parametrize("x0,y0", [(0, 0), (824, 0), (0, 824), (824, 924)])
def test_window_stays_inside_the_image_at_every_corner(H, x0, y0):
    m = mask_of(1024, 1024, (x0, y0, x0 + 199, y0 + 99))
    assert_contains(H.tile_rect(m), m)


def test_window_is_capped_at_the_image_size(H):
    m = mask_of(300, 500, (0, 0, 299, 499))
    t = H.tile_rect(m)
    assert t.side == 296
    assert (t.x0, t.y0) == (2, 102)
    assert t.x0 + t.side <= 300 and t.y0 + t.side <= 500


def test_oversized_bounding_box_is_clamped_not_clipped(H):
    m = mask_of(2048, 2048, (1700, 1700, 1999, 1999))
    t = H.tile_rect(m)
    assert t.side == 600
    assert (t.x0, t.y0) == (1448, 1448)
    assert_contains(t, m)


def test_tiny_images_do_not_panic(H):
    for side in range(1, 9):
        t = H.tile_rect(mask_of(side, side, (0, 0, side - 1, side - 1)))
        assert 1 <= t.side <= side
        assert t.x0 + t.side <= side and t.y0 + t.side <= side


def test_window_origin_stays_inside(H):
    assert H.window_origin(0, 512, 1024) == 0
    assert H.window_origin(1023, 512, 1024) == 512
    assert H.window_origin(500, 512, 1024) == 244
    assert H.window_origin(600, 512, 300) == 0
    assert H.window_origin(0, 4096, 1024) == 0


# ----------------------------------------------------------- --sections

def assert_covers(sections, m):
    hits = np.zeros(m.shape, np.int32)
    for x0, y0, x1, y1 in sections:
        sub = m[y0:y1, x0:x1] > 0
        assert sub.any(), f"empty section at ({x0},{y0})"
        assert x1 - x0 <= SECTION_BLOCK and y1 - y0 <= SECTION_BLOCK
        hits[y0:y1, x0:x1] += sub
    assert (hits[m > 0] == 1).all(), "every masked pixel in exactly one section"
    assert (hits[m == 0] == 0).all()


def section_depth(s, m, depth):
    x0, y0, x1, y1 = s
    sub = m[y0:y1, x0:x1] > 0
    return int(depth[y0:y1, x0:x1][sub].min()) if sub.any() else 2**32 - 1


def test_sections_of_a_small_mask_are_single_and_cover_it(H):
    m = mask_of(1024, 1024, (500, 500, 700, 700))
    s = H.section_rects(m)
    assert s == [(500, 500, 701, 701)]
    assert_covers(s, m)


def test_a_300x300_mask_becomes_four_sections(H):
    m = mask_of(1024, 1024, (300, 300, 598, 598))
    s = H.section_rects(m)
    assert len(s) == 4
    assert_covers(s, m)
    for i, a in enumerate(s):
        for b in s[i + 1:]:
            assert a[2] <= b[0] or b[2] <= a[0] or a[3] <= b[1] or b[3] <= a[1], (a, b)
    assert (s[0][0], s[0][2], s[2][0], s[2][2]) == (300, 556, 300, 556)


def test_the_rim_is_filled_before_the_interior(H):
    m = mask_of(2048, 2048, (500, 500, 1099, 1099))
    s = H.section_rects(m)
    assert_covers(s, m)
    d = H.mask_depth(m)
    ds = [section_depth(x, m, d) for x in s]
    assert ds[0] == 0 and ds[-1] > 0
    assert ds == sorted(ds)


def test_mask_depth_is_zero_on_the_rim_and_grows_inward(H):
    m = mask_of(512, 512, (100, 100, 299, 299))
    d = H.mask_depth(m)
    assert d[100, 100] == 0 and d[299, 299] == 0
    assert d[200, 200] >= 99
    assert d[0, 0] == 2**32 - 1


def test_mask_depth_is_the_4_neighbour_distance_to_the_hole_boundary(H):
    # brute force on a small irregular mask: depth = 4-connected steps from the
    # nearest masked pixel that touches an unmasked pixel or the image border
    rng = np.random.default_rng(0)
    m = (rng.random((24, 31)) < 0.7).astype(np.uint8) * 255
    d = H.mask_depth(m)
    h, w = m.shape
    rim = np.zeros_like(m, bool)
    for y in range(h):
        for x in range(w):
            if m[y, x]:
                for dy, dx in ((-1, 0), (1, 0), (0, -1), (0, 1)):
                    yy, xx = y + dy, x + dx
                    if not (0 <= yy < h and 0 <= xx < w) or not m[yy, xx]:
                        rim[y, x] = True
    want = np.full(m.shape, 2**32 - 1, np.uint64)
    want[rim] = 0
    changed = True
    while changed:  # Bellman-Ford relaxation inside the mask
        changed = False
        for y in range(h):
            for x in range(w):
                if not m[y, x]:
                    continue
                for dy, dx in ((-1, 0), (1, 0), (0, -1), (0, 1)):
                    yy, xx = y + dy, x + dx
                    if 0 <= yy < h and 0 <= xx < w and m[yy, xx] and want[yy, xx] + 1 < want[y, x]:
                        want[y, x] = want[yy, xx] + 1
                        changed = True
    assert np.array_equal(d.astype(np.uint64), want)


def test_order_is_deterministic(H):
    a = mask_of(2048, 2048, (100, 100, 699, 399))
    b = mask_of(2048, 2048, (100, 100, 699, 399))
    assert H.section_rects(a) == H.section_rects(b)
    assert H.section_rects(a)


def test_a_wide_mask_is_sectioned_and_ordered_by_depth(H):
    m = mask_of(2048, 2048, (100, 100, 699, 399))
    s = H.section_rects(m)
    assert len(s) == 6
    assert_covers(s, m)
    d = H.mask_depth(m)
    ds = [section_depth(x, m, d) for x in s]
    assert ds == sorted(ds)


def test_empty_mask_has_no_sections(H):
    assert H.section_rects(mask_of(256, 256)) == []


def test_a_single_pixel_mask_is_one_small_piece(H):
    m = mask_of(1024, 1024, (800, 900, 800, 900))
    s = H.section_rects(m)
    assert s == [(800, 900, 801, 901)]


def test_passes_fill_the_hole_monotonically_and_completely(H):
    m = mask_of(1024, 1024, (300, 300, 598, 598))
    s = H.section_rects(m)
    total = int((m > 0).sum())
    filled = np.zeros(m.shape, bool)
    seen = []
    for x0, y0, x1, y1 in s:
        filled[y0:y1, x0:x1] |= m[y0:y1, x0:x1] > 0
        seen.append(total - int(filled.sum()))
    assert seen[-1] == 0 and seen[0] < total
    assert all(b <= a for a, b in zip(seen, seen[1:]))
    d = H.mask_depth(m)
    x0, y0, x1, y1 = s[0]
    assert ((m[y0:y1, x0:x1] > 0) & (d[y0:y1, x0:x1] == 0)).any()


def test_every_section_fits_in_a_512_window_inside_a_large_image(H):
    m = mask_of(1024, 1024, (0, 0, 1023, 1023))
    for x0, y0, x1, y1 in H.section_rects(m):
        ox = H.window_origin((x0 + x1) // 2, TILE_MIN, 1024)
        oy = H.window_origin((y0 + y1) // 2, TILE_MIN, 1024)
        assert ox <= x0 and x1 <= ox + TILE_MIN
        assert oy <= y0 and y1 <= oy + TILE_MIN


def test_sections_of_a_ragged_stroke_mask_partition_the_hole(H):
    m, _ = H.synth_mask_strokes(700, 900, 0.3, 5)
    s = H.section_rects(m)
    assert_covers(s, m)
    d = H.mask_depth(m)
    ds = [section_depth(x, m, d) for x in s]
    assert ds == sorted(ds)


# --------------------------------------------------------- memory guard

def test_estimate_matches_the_measured_points(H):
    for side, mib in [(1536, 2933), (2048, 5051), (2560, 7619)]:
        got = H.estimated_bytes(side * side) >> 20
        assert abs(got - mib) <= mib // 50, (side, got, mib)


def test_the_failing_window_is_out_of_range_and_a_section_is_not(H):
    gb8 = 8192 << 20
    assert H.estimated_bytes(3472 * 3472) > gb8
    assert H.estimated_bytes(3072 * 3072) > gb8
    assert H.estimated_bytes(2560 * 2560) < gb8
    assert H.estimated_bytes(512 * 512) < gb8 // 8


def test_estimate_is_monotone_and_saturating(H):
    last = 0
    for side in [1, 64, 512, 1024, 2048, 4096]:
        v = H.estimated_bytes(side * side)
        assert v > last
        last = v
    assert H.estimated_bytes(2**63 - 1) >= last


# ------------------------------------------------------ weight container

def read_header(path):
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        return n, json.loads(f.read(n))


@pytest.fixture(scope="module")
def synth_path(weights_dir):
    return weights_dir["plain"]


def test_synth_container_layout(H, synth_path):
    n, hdr = read_header(synth_path)
    names = [k for k in hdr if k != "__metadata__"]
    assert len(names) == 989
    assert (8 + n) % 8 == 0
    size = os.path.getsize(synth_path)
    spans = sorted(tuple(hdr[k]["data_offsets"]) for k in names)
    assert spans[0][0] == 0 and spans[-1][1] == size - 8 - n
    for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
        # each payload starts at the next 8-byte boundary (safetensors_light.py:35-37)
        assert b0 == a1 + (-a1) % 8 and b0 % 8 == 0
    for k in names:
        assert hdr[k]["dtype"] == "F32"
        assert hdr[k]["data_offsets"][1] - hdr[k]["data_offsets"][0] == 4 * int(np.prod(hdr[k]["shape"]))
    # the state-dict names of the architecture (lama-rs/export_weights.py)
    for k in ["model.1.ffc.convl2l.weight", "model.4.ffc.convl2g.weight", "model.4.bn_g.running_var",
              "model.22.conv2.ffc.convg2g.fu.conv_layer.weight", "model.24.weight", "model.34.bias"]:
        assert k in hdr, k
    assert hdr["model.5.conv1.ffc.convl2l.weight"]["shape"] == [128, 128, 3, 3]
    assert hdr["model.5.conv1.ffc.convg2g.fu.conv_layer.weight"]["shape"] == [384, 384, 1, 1]
    assert hdr["model.24.weight"]["shape"] == [512, 256, 3, 3]


def test_store_matches_an_independent_reader(H, synth_path):
    import oracle_api as O
    ref = O.read_safetensors(synth_path)
    st = H.Store(synth_path)
    info = st.info()
    assert len(info) == 989
    raw = np.fromfile(synth_path, np.uint8)
    total = 0
    offs = [o for _, _, o, _ in info]
    assert offs == sorted(offs)  # container order = data order
    for name, shape, off, nb in info:
        assert shape == ref[name].shape
        assert np.array_equal(raw[off:off + nb].view(np.float32).reshape(shape), ref[name])
        total += nb
    assert st.total_bytes() == total
    st.close()
    st2 = H.Store(synth_path, map=False)
    assert st2.info() == info


def test_synth_weights_are_deterministic_and_seeded(H, tmp_path):
    a, b, c = (str(tmp_path / f"{n}.safetensors") for n in "abc")
    H.synth_weights(a, 7)
    H.synth_weights(b, 7)
    H.synth_weights(c, 8)
    ra, rb, rc = (open(p, "rb").read() for p in (a, b, c))
    assert ra == rb and ra != rc


def test_synth_weight_statistics(H, synth_path):
    import oracle_api as O
    W = O.read_safetensors(synth_path)
    w = W["model.5.conv1.ffc.convl2l.weight"]
    std = np.sqrt(2.0 / (w.shape[1] * 9))
    assert abs(w.std() / std - 1) < 0.05 and abs(w.mean()) < 0.01
    g = W["model.5.conv1.bn_l.weight"]
    assert g.min() >= 0.8 and g.max() <= 1.2
    v = W["model.5.conv1.bn_l.running_var"]
    assert v.min() >= 0.5 and v.max() <= 1.5
    assert W["model.5.conv1.bn_l.num_batches_tracked"].size == 1


def _write_st(path, tensors, dtype="F32", header_extra=None):
    hdr, blobs, off = {}, [], 0
    for k, a in tensors.items():
        b = a.tobytes()
        hdr[k] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if header_extra:
        hdr.update(header_extra)
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_store_rejects_non_f32_and_bad_offsets(H, tmp_path):
    p = str(tmp_path / "bad.safetensors")
    _write_st(p, {"a": np.zeros(4, np.float32)}, dtype="F16")
    with pytest.raises(RuntimeError, match="F16|dtype"):
        H.Store(p)
    q = str(tmp_path / "trunc.safetensors")
    _write_st(q, {"a": np.zeros(4, np.float32)})
    with open(q, "r+b") as f:
        f.truncate(os.path.getsize(q) - 4)
    with pytest.raises(RuntimeError):
        H.Store(q)
    with pytest.raises(RuntimeError):
        H.Store(str(tmp_path / "missing.safetensors"))


def _raw_st(path, header_bytes, payload=b""):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header_bytes)) + header_bytes + payload)


def test_store_rejects_malformed_headers(H, tmp_path):
    """A header whose last token is a number running up to the end of the file
    (no NUL after it), negative or overflowing dimensions, and integers beyond
    int64: each is an error with a message, read within the header's bytes."""
    p = str(tmp_path / "h.safetensors")
    cases = [
        b'{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,16',  # truncated inside a number
        b'{"a":{"dtype":"F32","shape":[-4],"data_offsets":[0,16]}}',
        b'{"a":{"dtype":"F32","shape":[4611686018427387904,4],"data_offsets":[0,16]}}',
        b'{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,99999999999999999999999]}}',
        b'{"a":{"dtype":"F32","shape":[-1,-4],"data_offsets":[0,16]}}',
    ]
    for hdr in cases:
        _raw_st(p, hdr, b"\0" * 16)
        with pytest.raises(RuntimeError):
            H.Store(p)
    # the well-formed version of the same header loads
    _raw_st(p, b'{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}', b"\0" * 16)
    assert len(H.Store(p)) == 1


def test_store_reads_metadata_and_orders_by_offset(H, tmp_path):
    p = str(tmp_path / "meta.safetensors")
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.arange(4, dtype=np.float32)
    _write_st(p, {"z": a, "y": b}, header_extra={"__metadata__": {"format": "pt"}})
    st = H.Store(p)
    info = st.info()
    assert [i[0] for i in info] == ["z", "y"]
    raw = np.fromfile(p, np.uint8)
    assert np.array_equal(raw[info[0][2]:info[0][2] + 24].view(np.float32).reshape(2, 3), a)


# ----------------------------------------------------------------- PNG

def test_png_round_trip_and_pil_agreement(H, tmp_path):
    PIL = pytest.importorskip("PIL.Image")
    img = H.synth_image(37, 53, 3)
    p = str(tmp_path / "a.png")
    H.png_write_rgb(p, img)
    assert np.array_equal(H.png_read_rgb(p), img)
    assert np.array_equal(np.asarray(PIL.open(p).convert("RGB")), img)


@pytest.mark.parametrize("mode", ["L", "LA", "RGB", "RGBA", "P", "I;16", "interlace"])
def test_png_decodes_pil_variants(H, tmp_path, mode):
    PIL = pytest.importorskip("PIL.Image")
    rng = np.random.default_rng(1)
    rgb = rng.integers(0, 256, (19, 23, 3), dtype=np.uint8)
    p = str(tmp_path / "v.png")
    base = PIL.fromarray(rgb, "RGB")
    if mode == "interlace":
        base.save(p, interlace=1)
        want = rgb
    elif mode == "P":
        im = base.quantize(64)
        im.save(p)
        want = np.asarray(im.convert("RGB"))
    elif mode == "I;16":
        g16 = rng.integers(0, 65536, (19, 23), dtype=np.uint16)
        PIL.fromarray(g16).save(p)
        hi = (g16 >> 8).astype(np.uint8)
        want = np.repeat(hi[..., None], 3, -1)
    else:
        im = base.convert(mode)
        im.save(p)
        want = np.asarray(im.convert("RGB")) if mode in ("RGB", "RGBA") else \
            np.repeat(np.asarray(im.convert("L"))[..., None], 3, -1)
    got = H.png_read_rgb(p)
    assert np.array_equal(got, want)
    gray = H.png_read_gray(p)
    assert np.array_equal(gray, want[..., 0])  # the mask is the red channel


def _png_filtered(rgb, filters, bpp=3):
    """An RGB8 PNG whose row y uses filter filters[y % len(filters)] (PNG spec
    section 9), built here with zlib."""
    import struct
    import zlib

    h, w, _ = rgb.shape
    rows = rgb.reshape(h, w * bpp).astype(np.int32)
    out = bytearray()
    prev = np.zeros(w * bpp, np.int32)
    for y in range(h):
        ft = filters[y % len(filters)]
        cur = rows[y]
        a = np.concatenate([np.zeros(bpp, np.int32), cur[:-bpp]])
        c = np.concatenate([np.zeros(bpp, np.int32), prev[:-bpp]])
        if ft == 0:
            f = cur
        elif ft == 1:
            f = cur - a
        elif ft == 2:
            f = cur - prev
        elif ft == 3:
            f = cur - (a + prev) // 2
        else:
            p = a + prev - c
            pa, pb, pc = np.abs(p - a), np.abs(p - prev), np.abs(p - c)
            f = cur - np.where((pa <= pb) & (pa <= pc), a, np.where(pb <= pc, prev, c))
        out.append(ft)
        out += (f & 0xFF).astype(np.uint8).tobytes()
        prev = cur

    def chunk(t, d):
        return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xFFFFFFFF)

    ihdr = struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0)
    return b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", ihdr) + chunk(b"IDAT", zlib.compress(bytes(out), 6)) + \
        chunk(b"IEND", b"")


@pytest.mark.parametrize("filters", [[0], [1], [2], [3], [4], [0, 1, 2, 3, 4], [4, 3, 2, 1, 0]])
def test_png_decodes_every_scanline_filter(H, tmp_path, filters):
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (23, 31, 3), dtype=np.uint8)
    img[5:15, 4:20] = H.synth_image(10, 16, 2)  # smooth patch beside noise
    p = tmp_path / "f.png"
    p.write_bytes(_png_filtered(img, filters))
    assert np.array_equal(H.png_read_rgb(str(p)), img)


def test_png_writer_bands_read_back(H, tmp_path):
    """The writer deflates 1 MiB bands on several threads into one zlib
    stream: images of one band, several bands and a ragged last band read
    back exactly, through this decoder and PIL's."""
    PIL = pytest.importorskip("PIL.Image")
    rng = np.random.default_rng(4)
    for h, w in ((1, 1), (600, 700), (1100, 1000)):
        img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
        img[: h // 2] = H.synth_image(h // 2, w, 5) if h > 1 else img[: h // 2]
        p = str(tmp_path / f"b{h}.png")
        H.png_write_rgb(p, img)
        assert np.array_equal(H.png_read_rgb(p), img)
        assert np.array_equal(np.asarray(PIL.open(p).convert("RGB")), img)


def test_png_rejects_garbage(H, tmp_path):
    p = tmp_path / "x.png"
    p.write_bytes(b"not a png at all")
    with pytest.raises(RuntimeError):
        H.png_read_rgb(str(p))


# ------------------------------------------------------- synthetic inputs

def test_synth_image_and_masks(H):
    a = H.synth_image(64, 80, 1)
    assert a.shape == (64, 80, 3) and np.array_equal(a, H.synth_image(64, 80, 1))
    assert not np.array_equal(a, H.synth_image(64, 80, 2))
    m, (x0, y0) = H.synth_mask_rect(100, 120, 30, 20, 3)
    assert int((m == 255).sum()) == 600 and set(np.unique(m)) == {0, 255}
    assert (m[y0:y0 + 20, x0:x0 + 30] == 255).all()
    s, cov = H.synth_mask_strokes(256, 256, 0.25, 2)
    assert abs(cov - (s > 0).mean()) < 1e-12
    assert cov >= 0.25


def test_build_input_pads_to_multiple_of_8(H):
    img = H.synth_image(13, 21, 1)
    m, _ = H.synth_mask_rect(13, 21, 5, 5, 1)
    x = H.build_input(img, m)
    assert x.shape == (4, 16, 24)
    assert set(np.unique(x[3])) <= {0.0, 1.0}
