"""Writes the golden fixtures in this directory (run from the repository root:
`python tests/golden/make_golden.py`).

The reference (sam-rs) ships no golden vectors, so these are build-owned: small inputs drawn with
fixed seeds, rounded so that every value is exactly representable in bf16, f16 and f32 (bf16
rounding, magnitudes below 2^-14 flushed to zero), and expected outputs computed in float64 by the
brute-force formulations in tests/refimpl.py (which share no code with the oracle). The same fixture
therefore pins the CPU oracle and every GPU dtype.

Cases follow the shapes the reference's tests use: the rel-pos geometries of tests/kernels.rs:23 and
tests/cpu_gemm.rs:37 (reduced in batch), the deform shapes of tests/dino.rs:46-55, and small flash /
memory-attention cases (Lq 5, Lk 7, hd 16 and 256).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import refimpl  # noqa: E402


def exact(x):
    """Round to bf16 (nearest even) and flush |x| < 2^-14, so the value is exact in bf16, f16 and f32."""
    x = np.asarray(x, np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    y = b.astype(np.uint32).view(np.float32)
    y = np.where(np.abs(y) < 2.0 ** -14, np.float32(0), y)
    return y.astype(np.float32)


def relpos_case(name, h, w, bh, hd, seed, table_std=0.5):
    r = np.random.default_rng(seed)
    n = h * w
    q = exact(r.standard_normal((bh, n, hd)))
    kt = exact(r.standard_normal((bh, hd, n)))
    v = exact(r.standard_normal((bh, n, hd)))
    table = exact(table_std * r.standard_normal((2 * h - 1 + 2 * w - 1, hd)))
    scale = np.float32(hd ** -0.5)
    s = np.asarray(q, np.float64) @ np.asarray(kt, np.float64)
    p = refimpl.relpos_softmax64(s, q, table, h, w, float(scale))
    out = p @ np.asarray(v, np.float64)
    np.savez_compressed(os.path.join(HERE, f"relpos_{name}.npz"), q=q, kt=kt, v=v, table=table,
                        geom=np.array([h, w, bh, hd], np.int32), scale=np.array([scale], np.float32),
                        s=s if n <= 8 else np.zeros(0), probs=p if n <= 8 else np.zeros(0), out=out)


def deform_case(name, shapes, b, q, h, d, p, seed, spread=0.5):
    r = np.random.default_rng(seed)
    s = sum(hh * ww for hh, ww in shapes)
    l = len(shapes)
    value = exact(r.standard_normal((b, s, h, d)))
    loc = exact(0.5 + spread * (r.random((b, q, h, l, p, 2)) * 2 - 1))
    logits = r.standard_normal((b, q, h, l * p))
    attn = exact((np.exp(logits) / np.exp(logits).sum(-1, keepdims=True)).reshape(b, q, h, l, p))
    out = refimpl.deform_naive64(value, loc, attn, shapes)
    np.savez_compressed(os.path.join(HERE, f"deform_{name}.npz"), value=value, loc=loc, attn=attn,
                        shapes=np.array(shapes, np.int32), out=out)


def flash_case(name, b, lq, lk, h, d, seed):
    r = np.random.default_rng(seed)
    q = exact(r.standard_normal((b, lq, h, d)))
    k = exact(r.standard_normal((b, lk, h, d)))
    v = exact(r.standard_normal((b, lk, h, d)))
    t = lambda x: np.asarray(x, np.float64).transpose(0, 2, 1, 3)
    out = refimpl.sdpa64(t(q), t(k), t(v)).transpose(0, 2, 1, 3)
    np.savez_compressed(os.path.join(HERE, f"flash_{name}.npz"), q=q, k=k, v=v, out=out)


def rope_case(name, side, hd, rows, seed):
    r = np.random.default_rng(seed)
    x = exact(r.standard_normal((rows, hd)))
    cis = refimpl.axial_rope_cis64(side, hd, 10000.0)
    reps = rows // (side * side)
    out = refimpl.rope_complex64(x, np.concatenate([cis] * reps))
    np.savez_compressed(os.path.join(HERE, f"rope_{name}.npz"), x=x, side=np.array([side], np.int32), out=out)


def main():
    relpos_case("2x3_hd8", 2, 3, 2, 8, 101)
    relpos_case("7x11_hd80", 7, 11, 1, 80, 102)
    relpos_case("14x14_hd64", 14, 14, 1, 64, 103)
    deform_case("dino_spec", [(7, 9), (4, 5), (2, 3)], 1, 13, 4, 8, 3, 201, spread=0.7)
    deform_case("kernels_rs", [(9, 12), (5, 6), (3, 3), (2, 2)], 1, 37, 8, 32, 4, 202, spread=0.6)
    flash_case("lq5_lk7_hd16", 1, 5, 7, 2, 16, 301)
    flash_case("lq5_lk7_hd256", 1, 5, 7, 1, 256, 302)
    flash_case("lq33_lk130_hd64", 1, 33, 130, 2, 64, 303)
    rope_case("side4_hd16", 4, 16, 32, 401)
    rope_case("side8_hd256", 8, 256, 64, 402)


if __name__ == "__main__":
    main()
