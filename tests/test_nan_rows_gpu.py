"""A NaN in one query row reaches that row's output and no other, on an MI355X.

The oracle, like the reference's CPU softmax (f32::max passes over a NaN score, but its exponential and
so the row's sum and every weight are NaN: kernels.rs:85-100, 198-212), returns NaN for that row and
the ordinary values elsewhere. The kernels must do the same: no NaN may leak into other rows through
the lane-pair reductions, the bias scratch in LDS or the K/V buffers, and the poisoned row must not
come out finite. Every other row is held to the usual bars (tests/parity.py). No address in these
kernels depends on a value, so the NaN is data only. relpos_softmax is also given -inf scores (masked
keys), which must get weight 0 and leave their rows finite.
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


def split_rows(got, want, row, what):
    """Assert the poisoned row is all NaN in both, and every other value finite; return both arrays
    with that row zeroed for the parity check."""
    assert np.isnan(want[row]).all(), f"{what}: the oracle's poisoned row is not NaN"
    assert np.isnan(got[row]).all(), f"{what}: the poisoned row came out (partly) finite"
    got, want = got.copy(), want.copy()
    got[row] = 0.0
    want[row] = 0.0
    assert np.isfinite(got).all(), f"{what}: a NaN leaked into another row"
    return got, want


# every fused rel-pos kernel family: the 14x14 windows and the 64x64 global grid at hd 80 and 64, the
# generic kernel (7x11), the wide-grid kernel (65x64, f16/bf16 only) and the f32 kernels
RELPOS = [(14, 14, 4, 80), (14, 14, 4, 64), (64, 64, 2, 80), (64, 64, 2, 64), (7, 11, 3, 80), (65, 64, 1, 64)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,bh,hd", RELPOS)
def test_attention_relpos_nan_query_row(hip, h, w, bh, hd, dtype):
    if dtype == "f32" and max(h, w) > 64:
        pytest.skip("f32 rel-pos attention stops at 64 x 64 (larger f32 grids take the reference's sequence)")
    n = h * w
    print(f"attn_relpos nan row {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    r = np.random.default_rng(7000 + n + hd)
    q, kt, v = (oracle.round_to(r.standard_normal(s).astype(np.float32), dtype)
                for s in ((bh, n, hd), (bh, hd, n), (bh, n, hd)))
    table = oracle.round_to((0.02 * r.standard_normal((2 * h - 1 + 2 * w - 1, hd))).astype(np.float32), dtype)
    row = (bh - 1, n // 3)
    q[row][hd // 2] = np.nan
    got = hip.attention_relpos(to_dev(q, dtype), to_dev(kt, dtype), to_dev(v, dtype), to_dev(table, dtype), h, w,
                               hd ** -0.5)
    torch.cuda.synchronize()
    want = oracle.attention_relpos(q, kt, v, table, h, w, hd ** -0.5)
    what = f"nan row {h}x{w} bh={bh} hd={hd} {dtype}"
    got, want = split_rows(got.float().cpu().numpy(), want, row, what)
    check(got, want, dtype, what)


# the generic flash kernel (head dims 64 and 96, with and without a key split) and the head-dim-256
# kernel with its key-split combine
FLASH = [(1, 300, 700, 2, 64), (2, 130, 200, 4, 96), (1, 17, 3000, 1, 64), (2, 130, 517, 3, 256)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("b,lq,lk,h,d", FLASH)
def test_flash_attn_nan_query_row(hip, b, lq, lk, h, d, dtype):
    print(f"flash nan row {dtype} b={b} lq={lq} lk={lk} h={h} d={d}", flush=True)
    r = np.random.default_rng(7100 + lq + lk + d)
    q, k, v = (oracle.round_to(r.standard_normal((b, n_, h, d)).astype(np.float32), dtype) for n_ in (lq, lk, lk))
    row = (b - 1, lq // 2, h - 1)
    q[row][d // 3] = np.nan
    got = hip.flash_attn(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    want = oracle.mha_blhd(q, k, v)
    what = f"flash nan row b{b} lq{lq} lk{lk} h{h} d{d} {dtype}"
    got, want = split_rows(got.float().cpu().numpy(), want, row, what)
    check(got, want, dtype, what)


# relpos_softmax over materialised scores: a window grid, a global grid (vector kernel) and a short-row
# grid (16 lanes per row)
SOFTMAX = [(14, 14, 3, 80), (64, 64, 1, 80), (5, 9, 4, 64)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,bh,hd", SOFTMAX)
def test_relpos_softmax_nan_score_row(hip, h, w, bh, hd, dtype):
    n = h * w
    print(f"relpos_softmax nan row {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    r = np.random.default_rng(7200 + n + hd)
    s = oracle.round_to(r.standard_normal((bh, n, n)).astype(np.float32), dtype)
    q = oracle.round_to(r.standard_normal((bh, n, hd)).astype(np.float32), dtype)
    t = oracle.round_to(r.standard_normal((2 * h - 1 + 2 * w - 1, hd)).astype(np.float32), dtype)
    row = (0, n - 2)
    s[row][n // 2] = np.nan
    got = hip.relpos_softmax(to_dev(s, dtype), to_dev(q, dtype), to_dev(t, dtype), h, w, 0.125)
    torch.cuda.synchronize()
    want = oracle.relpos_softmax(s, q, t, h, w, 0.125)
    what = f"relpos_softmax nan row {h}x{w} bh={bh} hd={hd} {dtype}"
    got, want = split_rows(got.float().cpu().numpy(), want, row, what)
    check(got, want, dtype, what)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,bh,hd", SOFTMAX)
def test_relpos_softmax_neg_inf_scores(hip, h, w, bh, hd, dtype):
    """-inf scores (masked keys) get weight 0 and leave the row finite, as exp(-inf - max) = 0 does in the
    reference (kernels.rs:95); the first row also starts with a run of them, so a lane of the scalar
    kernel sees nothing but -inf."""
    n = h * w
    print(f"relpos_softmax -inf scores {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    r = np.random.default_rng(7300 + n + hd)
    s = oracle.round_to(r.standard_normal((bh, n, n)).astype(np.float32), dtype)
    q = oracle.round_to(r.standard_normal((bh, n, hd)).astype(np.float32), dtype)
    t = oracle.round_to(r.standard_normal((2 * h - 1 + 2 * w - 1, hd)).astype(np.float32), dtype)
    s[0, 0, : n // 2] = -np.inf
    s[bh - 1, n - 1, 1::3] = -np.inf
    got = hip.relpos_softmax(to_dev(s, dtype), to_dev(q, dtype), to_dev(t, dtype), h, w, 0.125)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    want = oracle.relpos_softmax(s, q, t, h, w, 0.125)
    assert np.isfinite(want).all() and np.isfinite(got).all()
    assert (got[0, 0, : n // 2] == 0).all() and (got[bh - 1, n - 1, 1::3] == 0).all()
    check(got, want, dtype, f"relpos_softmax -inf scores {h}x{w} bh={bh} hd={hd} {dtype}")
