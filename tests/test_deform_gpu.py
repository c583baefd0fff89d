"""Parity of the multi-scale deformable attention (libsam_hip.so) with the CPU oracle, on an MI355X.

Cases: the reference's own test shapes (tests/kernels.rs:65-83, tests/dino.rs:46-63) with sampling
locations spread beyond [0, 1] so the zero padding is exercised, shapes that take each of the two
kernels (16-byte lanes when D allows, scalar lanes otherwise) and multi-batch grids of hundreds of
workgroups, plus the Grounding DINO-tiny encoder and decoder layers at full size. Bars (tests/parity.py,
the attention bars): f32 max|gpu - cpu| / max|cpu| <= 1e-5; f16 max-abs 2e-3 and bf16 max-abs 2e-3
beyond the output's own rounding, against the f32 oracle on the same rounded inputs. These are tighter
than the reference test's own (f32 1e-4, bf16 5e-2; tests/kernels.rs:65-83).
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle
from parity import check

pytestmark = pytest.mark.gpu
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}

DINO_LEVELS = [(100, 167), (50, 84), (25, 42), (13, 21)]


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def inputs(shapes, b, q, h, d, p, seed, spread=0.5, dtype="f32"):
    r = np.random.default_rng(seed)
    s = sum(hh * ww for hh, ww in shapes)
    l = len(shapes)
    value = r.standard_normal((b, s, h, d)).astype(np.float32)
    loc = (r.standard_normal((b, q, h, l, p, 2)) * spread + 0.5).astype(np.float32)
    logits = r.standard_normal((b, q, h, l * p))
    attn = np.exp(logits - logits.max(-1, keepdims=True))
    attn = (attn / attn.sum(-1, keepdims=True)).reshape(b, q, h, l, p).astype(np.float32)
    return [oracle.round_to(x, dtype) for x in (value, loc, attn)]


def run(hip, arrays, shapes, dtype):
    dev = [torch.from_numpy(a).to("cuda", TORCH_DT[dtype]) for a in arrays]
    out = hip.deform_attn(*dev, shapes)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    ("kernels.rs", [(9, 12), (5, 6), (3, 3), (2, 2)], 1, 37, 8, 32, 4, 0.5),
    ("dino.rs", [(7, 9), (4, 5), (2, 3)], 1, 13, 4, 8, 3, 0.6),
    ("batch2-odd-d", [(6, 5), (3, 3)], 2, 11, 3, 20, 2, 0.7),
    ("single-level", [(16, 16)], 1, 64, 2, 64, 8, 0.4),
    ("d-not-multiple-of-4", [(5, 7), (2, 4)], 1, 9, 2, 6, 3, 0.5),
    # hundreds of workgroups: the head-major, per-XCD work order crosses head and batch boundaries
    ("batch2-many-blocks", [(30, 40), (15, 20), (8, 10), (4, 5)], 2, 3001, 8, 32, 4, 0.6),
    ("five-heads-d16", [(12, 10), (6, 5)], 1, 777, 5, 16, 3, 0.5),
]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name,shapes,b,q,h,d,p,spread", CASES, ids=[c[0] for c in CASES])
def test_deform_matches_oracle(hip, name, shapes, b, q, h, d, p, spread, dtype):
    print(f"deform {name} {dtype}", flush=True)
    arrays = inputs(shapes, b, q, h, d, p, 20 + q, spread, dtype)
    want = oracle.deform_attn(*arrays, shapes)
    got = run(hip, arrays, shapes, dtype)
    check(got, want, dtype, f"deform {name} {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("q", [22223, 900], ids=["encoder", "decoder"])
def test_dino_tiny_full_size(hip, q, dtype):
    """Grounding DINO-tiny: 800x1333 input -> 4 levels, 22223 value tokens, 8 heads x 32, 4 points."""
    print(f"deform dino-tiny q={q} {dtype}", flush=True)
    r = np.random.default_rng(q)
    s = sum(a * b for a, b in DINO_LEVELS)
    value = r.standard_normal((1, s, 8, 32)).astype(np.float32)
    ref = r.uniform(0, 1, (1, q, 1, 1, 1, 2))
    wh = np.array([[w, h] for h, w in DINO_LEVELS], np.float64).reshape(1, 1, 1, 4, 1, 2)
    loc = (ref + r.normal(0, 2, (1, q, 8, 4, 4, 2)) / wh).astype(np.float32)  # offsets ~N(0,2) px
    logits = r.standard_normal((1, q, 8, 16))
    attn = np.exp(logits - logits.max(-1, keepdims=True))
    attn = (attn / attn.sum(-1, keepdims=True)).reshape(1, q, 8, 4, 4).astype(np.float32)
    value, loc, attn = (oracle.round_to(x, dtype) for x in (value, loc, attn))
    want = oracle.deform_attn(value, loc, attn, DINO_LEVELS)
    got = run(hip, [value, loc, attn], DINO_LEVELS, dtype)
    check(got, want, dtype, f"deform dino-tiny q={q} {dtype}")


def test_pixel_centres_are_exact_gathers(hip):
    """Locations at pixel centres with one-hot weights return the value rows bit for bit (power-of-two
    level sizes, so (x + 0.5) / W * W - 0.5 is exact in f32)."""
    shapes = [(8, 8), (4, 4)]
    r = np.random.default_rng(3)
    value = r.standard_normal((1, 80, 2, 16)).astype(np.float32)
    xs, ys = r.integers(0, 4, (1, 5, 2, 2, 2)), r.integers(0, 4, (1, 5, 2, 2, 2))
    loc = np.stack([(xs + 0.5) / np.array([8, 4]).reshape(1, 1, 1, 2, 1),
                    (ys + 0.5) / np.array([8, 4]).reshape(1, 1, 1, 2, 1)], -1).astype(np.float32)
    attn = np.zeros((1, 5, 2, 2, 2), np.float32)
    attn[..., 1, 1] = 1.0
    got = run(hip, [value, loc, attn], shapes, "f32").reshape(1, 5, 2, 16)
    for qi in range(5):
        for hi in range(2):
            s_idx = 64 + ys[0, qi, hi, 1, 1] * 4 + xs[0, qi, hi, 1, 1]
            assert np.array_equal(got[0, qi, hi], value[0, s_idx, hi])


def test_deform_errors(hip):
    v = torch.zeros(1, 30, 2, 8, device="cuda")
    loc = torch.zeros(1, 3, 2, 5, 2, 2, device="cuda")
    a = torch.zeros(1, 3, 2, 5, 2, device="cuda")
    with pytest.raises(hip.SamHipError, match="at most 4 levels, got 5"):
        hip.deform_attn(v, loc, a, [(2, 3)] * 5)
    loc = torch.zeros(1, 3, 2, 2, 2, 2, device="cuda")
    a = torch.zeros(1, 3, 2, 2, 2, device="cuda")
    with pytest.raises(hip.SamHipError, match="pixels"):
        hip.deform_attn(v, loc, a, [(2, 3), (2, 3)])


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("d", [32, 6])
def test_degenerate_sampling_locations(hip, d, dtype):
    """Sampling locations the reference takes without complaint: exactly on the edges (0 and 1), far
    outside the levels (+-3, +-1e10) and NaN. The reference's `x.floor() as i64` (kernels.rs:799-800)
    saturates and maps NaN to 0, so a far-out point adds nothing and a NaN point's corner (0, 0) is
    read with a NaN weight: the output columns of that query and head are NaN. The oracle follows
    that cast; the kernel must give the same NaN pattern and the usual bars elsewhere. Both the
    16-byte-lane kernel (d 32) and the scalar-lane kernel (d 6) run."""
    shapes = [(20, 30), (10, 15), (5, 8), (3, 4)]
    value, loc, attn = inputs(shapes, 1, 300, 8, d, 4, 8800 + d, 0.5, dtype)
    flat = loc.reshape(-1, 2)
    r = np.random.default_rng(8801)
    idx = r.permutation(flat.shape[0])
    for k, val in enumerate([0.0, 1.0, 3.0, -3.0, 1e10, -1e10, np.nan]):
        sel = idx[k * 40:(k + 1) * 40]
        flat[sel, k % 2] = val
    loc = oracle.round_to(loc, dtype)  # f16 takes +-1e10 as +-inf: still outside every level
    print(f"deform degenerate locations d={d} {dtype}", flush=True)
    got = run(hip, [value, loc, attn], shapes, dtype)
    want = oracle.deform_attn(value, loc, attn, shapes)
    assert np.isnan(want).any() and (np.isnan(got) == np.isnan(want)).all(), "NaN pattern differs"
    check(np.nan_to_num(got), np.nan_to_num(want), dtype, f"deform degenerate locations d={d} {dtype}")
