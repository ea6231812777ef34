#!/usr/bin/env python3
"""Writes tests/golden/ops.npz: seeded inputs and library outputs that pin the
CPU oracle's functions (test infrastructure).

Every expected output comes from a routine other than the oracle:
  * torch 2.10 CPU ops (F.conv2d after F.pad(mode='reflect'), F.conv_transpose2d,
    F.batch_norm in eval, torch.fft.rfft2 / irfft2 with norm='ortho'),
  * numpy f64 direct DFTs for lengths that are not powers of two, with the
    sign convention the reference CPU engine uses there (its Bluestein path,
    lama-rs/src/cpu.rs:931-1011, computes the opposite-sign DFT).
Regenerate with:  python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def dft_axis(x, axis, sign):
    n = x.shape[axis]
    k = np.arange(n)
    m = np.exp(sign * 2j * np.pi * np.outer(k, k) / n)
    return np.moveaxis(np.tensordot(m, np.moveaxis(x, axis, 0), axes=(1, 0)), 0, axis)


def ref_sign(n, inverse):
    """Exponent sign the reference CPU engine uses for a length-n transform."""
    base = 1 if inverse else -1
    pow2 = n > 0 and (n & (n - 1)) == 0
    return base if pow2 else -base


def rfft2_ref(x):
    """cpu.rs rfft2_ortho semantics (rows then columns, per-length sign)."""
    h, w = x.shape
    y = dft_axis(x.astype(np.complex128), 1, ref_sign(w, False))
    y = dft_axis(y, 0, ref_sign(h, False)) / np.sqrt(h * w)
    y = y[:, : w // 2 + 1]
    return np.stack([y.real, y.imag]).astype(np.float32)


def irfft2_ref(spec, w):
    """cpu.rs irfft2_ortho semantics: 2-D Hermitian completion, real part."""
    h, wh = spec.shape[1:]
    full = np.zeros((h, w), np.complex128)
    full[:, :wh] = spec[0] + 1j * spec[1]
    for y in range(h):
        for x in range(wh, w):
            xm = w - x
            if xm >= wh:
                continue
            full[y, x] = np.conj(full[(h - y) % h, xm])
    r = dft_axis(full, 1, ref_sign(w, True))
    r = dft_axis(r, 0, ref_sign(h, True)) / np.sqrt(h * w)
    return r.real.astype(np.float32)


def main():
    rng = np.random.default_rng(1234)
    out = {}
    t = torch.from_numpy
    # 3x3 reflect convolutions, stride 1 and 2 (model.rs:146-165)
    for name, (cin, cout, h, w, k, s) in {"c3s1": (5, 7, 9, 11, 3, 1), "c3s2": (6, 4, 10, 12, 3, 2),
                                          "c7": (4, 6, 12, 10, 7, 1), "c1": (9, 5, 6, 7, 1, 1)}.items():
        x = rng.standard_normal((cin, h, w)).astype(np.float32)
        wt = rng.standard_normal((cout, cin, k, k)).astype(np.float32)
        b = rng.standard_normal(cout).astype(np.float32)
        p = k // 2
        xp = F.pad(t(x)[None], (p, p, p, p), mode="reflect") if p else t(x)[None]
        y = F.conv2d(xp, t(wt), t(b), stride=s)[0].numpy()
        out.update({f"{name}_x": x, f"{name}_w": wt, f"{name}_b": b, f"{name}_y": y})
    # ConvTranspose2d k3 s2 p1 op1 (model.rs:172-201)
    x = np.maximum(rng.standard_normal((6, 5, 7)), 0).astype(np.float32)
    wt = rng.standard_normal((6, 4, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y = F.conv_transpose2d(t(x)[None], t(wt), t(b), stride=2, padding=1, output_padding=1)[0].numpy()
    out.update({"ct_x": x, "ct_w": wt, "ct_b": b, "ct_y": y})
    # eval BatchNorm (cpu.rs:45-76)
    c = 8
    bw = rng.uniform(0.8, 1.2, c).astype(np.float32)
    bb = rng.normal(0, 0.05, c).astype(np.float32)
    bm = rng.normal(0, 0.1, c).astype(np.float32)
    bv = rng.uniform(0.5, 1.5, c).astype(np.float32)
    x = rng.standard_normal((c, 4, 5)).astype(np.float32)
    y = F.batch_norm(t(x)[None], t(bm), t(bv), t(bw), t(bb), False, 0.0, 1e-5)[0].numpy()
    out.update({"bn_w": bw, "bn_b": bb, "bn_m": bm, "bn_v": bv, "bn_x": x, "bn_y": y})
    # FFTs: torch for powers of two, direct DFT (reference sign rule) otherwise
    for h, w in [(8, 8), (16, 8), (4, 16), (6, 10), (5, 7), (3, 4), (1, 1), (12, 12)]:
        x = rng.standard_normal((h, w)).astype(np.float32)
        spec = rng.standard_normal((2, h, w // 2 + 1)).astype(np.float32)
        pow2 = all(n & (n - 1) == 0 for n in (h, w))
        if pow2:
            f = torch.fft.rfft2(t(x).double(), norm="ortho")
            fy = np.stack([f.real.numpy(), f.imag.numpy()]).astype(np.float32)
            iy = torch.fft.irfft2(torch.complex(t(spec[0]).double(), t(spec[1]).double()), s=(h, w),
                                  norm="ortho").float().numpy()
        else:
            fy = rfft2_ref(x)
            iy = irfft2_ref(spec, w)
        out.update({f"fft{h}x{w}_x": x, f"fft{h}x{w}_y": fy, f"fft{h}x{w}_spec": spec, f"fft{h}x{w}_iy": iy})
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **out)
    print("wrote", os.path.join(HERE, "ops.npz"), len(out), "arrays")


if __name__ == "__main__":
    main()
