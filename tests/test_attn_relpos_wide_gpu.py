"""Parity of the fused rel-pos attention on grids past 64 rows or columns (attn_relpos_wide.hip, up to
128 x 128, f16 / bf16) with the CPU oracle, on an MI355X.

The reference's GPU sequence reaches these shapes through bmm -> relpos_softmax -> bmm, and only up to
h*w <= 8192 (kernels.rs:14, 1078-1083); its CPU TiledAttention takes any size (kernels.rs:116-225),
which the oracle restates. Shapes: one and two column passes (W = 64, 65, 100, 128), row counts that end
a 32-row bias chunk early or late (65, 70, 96, 100, 128), thin grids (1 x 128, 128 x 1), every K-load
width (W a multiple of 8, even, odd), head dims 8 to 128, grids beyond 8192 keys (96 x 96, 128 x 128),
the reference test's sharp N(0, 1) draws, and a non-positive scale (the plain-Rw path). Bars as in
tests/parity.py. f32 stays limited to 64 x 64 and is refused past it.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle
from parity import check, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def make_inputs(h, w, bh, hd, seed, dtype, qkv_std=0.5, table_std=0.5):
    n = h * w
    r = np.random.default_rng(seed)
    q = (qkv_std * r.standard_normal((bh, n, hd))).astype(np.float32)
    kt = (qkv_std * r.standard_normal((bh, hd, n))).astype(np.float32)
    v = r.standard_normal((bh, n, hd)).astype(np.float32)
    table = (table_std * r.standard_normal((2 * h - 1 + 2 * w - 1, hd))).astype(np.float32)
    return [oracle.round_to(x, dtype) for x in (q, kt, v, table)]


def run(hip, arrays, h, w, scale, dtype):
    q, kt, v, table = (to_dev(a, dtype) for a in arrays)
    out = hip.attention_relpos(q, kt, v, table, h, w, scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


# (h, w, bh, hd)
WIDE = [(65, 64, 2, 64), (64, 65, 2, 80), (100, 90, 1, 80), (70, 70, 2, 128), (1, 128, 3, 32), (128, 1, 2, 16),
        (77, 100, 1, 24), (67, 99, 1, 8), (96, 96, 1, 64), (128, 128, 1, 64), (3, 100, 2, 80), (128, 20, 1, 80)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("h,w,bh,hd", WIDE)
def test_wide_grids(hip, h, w, bh, hd, dtype):
    print(f"attn_relpos wide {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 500 + h * w + hd, dtype)
    scale = hd ** -0.5
    want = oracle.attention_relpos(*arrays, h, w, scale)
    got = run(hip, arrays, h, w, scale, dtype)
    check(got, want, dtype, f"wide {h}x{w} bh={bh} hd={hd} {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("h,w,bh,hd", [(96, 96, 1, 64), (65, 128, 1, 80)])
def test_wide_grids_sharp_logits(hip, h, w, bh, hd, dtype):
    """The reference test's draws (q, k, v and both tables ~ N(0, 1)): sharp rows, undamped errors."""
    print(f"attn_relpos wide sharp {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 700 + h * w + hd, dtype, qkv_std=1.0, table_std=1.0)
    scale = hd ** -0.5
    want = oracle.attention_relpos(*arrays, h, w, scale)
    got = run(hip, arrays, h, w, scale, dtype)
    check(got, want, dtype, f"wide sharp {h}x{w} bh={bh} hd={hd} {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_wide_grid_non_positive_scale(hip, dtype):
    """scale <= 0 takes the plain-Rw path (bias added after the MFMA instead of as its start value)."""
    h, w, bh, hd = 66, 70, 1, 16
    print(f"attn_relpos wide scale<0 {dtype}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 901, dtype)
    want = oracle.attention_relpos(*arrays, h, w, -0.1)
    got = run(hip, arrays, h, w, -0.1, dtype)
    check(got, want, dtype, f"wide {h}x{w} scale -0.1 {dtype}")


def test_wide_grid_heads_are_independent(hip):
    """Each head of a wide grid only reads its own rows: a head run alone equals the same head in a
    batch of three, bit for bit."""
    h, w, hd = 80, 72, 64
    arrays = make_inputs(h, w, 3, hd, 77, "f16")
    scale = hd ** -0.5
    all3 = run(hip, arrays, h, w, scale, "f16")
    q, kt, v, table = arrays
    one = run(hip, [q[1:2], kt[1:2], v[1:2], table], h, w, scale, "f16")
    assert np.array_equal(all3[1:2], one)


def test_f32_past_64_is_refused(hip):
    h, w, hd = 65, 64, 16
    q, kt, v, table = (to_dev(a, "f32") for a in make_inputs(h, w, 1, hd, 3, "f32"))
    with pytest.raises(hip.SamHipError, match="64x64 in f32"):
        hip.attention_relpos(q, kt, v, table, h, w, hd ** -0.5)
