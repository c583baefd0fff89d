"""Parity of relpos_softmax and qkv_split (libsam_hip.so) with the CPU oracle, on an MI355X.

relpos_softmax follows the reference's own test (tests/kernels.rs:19-37): geometries (14,14,6,64),
(64,64,2,64), (7,11,3,80), N(0,1) scores, q and table, scale 0.125, inputs rounded to the kernel dtype
and the oracle run on the rounded values; max-abs 1e-3 on the probabilities (f16, the reference's bar),
1e-5 relative for f32, and for bf16 1e-3 beyond the half-ulp rounding of the bf16 output itself.
qkv_split is a permutation plus one rounded addition: bit-exact against the oracle.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle

pytestmark = pytest.mark.gpu
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", TORCH_DT[dtype])


def half_ulp_bf16(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 8)


# The reference test's geometries, then shapes that take each of the kernel's paths: whole-row
# 16-byte vectors (64-column grids, and 8192-long rows), 8-byte vectors (14x14 windows in f16), vectors
# that straddle grid rows (33 and 14 columns), narrow grids (2 columns), the scalar two-pass kernel
# (odd row lengths, and 8192 f32 columns), and row counts that leave a wave's 32 rows ragged. 16-bit
# rows of at most 64 vectors run 16 lanes per row: one, two or four vectors per lane (64 columns;
# 10x12 and 12x12 grids, whose 8-element vectors wrap into the next grid row; 14x14).
RELPOS_SHAPES = [(14, 14, 6, 64), (64, 64, 2, 64), (7, 11, 3, 80), (2, 3, 2, 8), (16, 33, 1, 32),
                 (64, 64, 2, 80), (14, 14, 40, 80), (13, 2, 5, 16), (5, 33, 3, 16), (128, 64, 1, 16),
                 (91, 90, 1, 8), (1, 64, 7, 24), (10, 12, 3, 16), (12, 12, 2, 16)]


LONG_ROWS = {(128, 64, 1, 16), (91, 90, 1, 8)}  # f32 over ~8192 keys: test_relpos_softmax_long_rows_f32


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,bh,hd", RELPOS_SHAPES)
def test_relpos_softmax_matches_oracle(hip, h, w, bh, hd, dtype):
    if dtype == "f32" and (h, w, bh, hd) in LONG_ROWS:
        pytest.skip("f32 rows of ~8192 keys: checked against the float64 value in test_relpos_softmax_long_rows_f32")
    print(f"relpos_softmax {dtype} {h}x{w} bh={bh} hd={hd}", flush=True)
    n = h * w
    r = np.random.default_rng(h * 100 + w)
    s = oracle.round_to(r.standard_normal((bh, n, n)), dtype)
    q = oracle.round_to(r.standard_normal((bh, n, hd)), dtype)
    t = oracle.round_to(r.standard_normal((2 * h - 1 + 2 * w - 1, hd)), dtype)
    want = oracle.relpos_softmax(s, q, t, h, w, 0.125)
    got = hip.relpos_softmax(dev(s, dtype), dev(q, dtype), dev(t, dtype), h, w, 0.125)
    got = got.float().cpu().numpy()
    err = np.abs(got - want).max()
    print(f"parity relpos_softmax {h}x{w} bh={bh} hd={hd} {dtype}: max-abs {err:.3g}", flush=True)
    if dtype == "f32":
        assert np.abs(got - want).max() / np.abs(want).max() <= 1e-5
    elif dtype == "bf16":
        assert (np.abs(got - want) - half_ulp_bf16(want)).max() <= 1e-3
    else:
        assert np.abs(got - want).max() <= 1e-3
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=2e-2 if dtype == "bf16" else 2e-3)


@pytest.mark.parametrize("h,w,bh,hd", sorted(LONG_ROWS))
def test_relpos_softmax_long_rows_f32(hip, h, w, bh, hd):
    """f32 rows of 8190 and 8192 keys with the reference test's N(0,1) draws. Over that many keys the
    reference's own f32 arithmetic (sequential sums, kernels.rs:84-103, which the oracle restates) is
    1.3e-5 to 1.8e-5 away from the float64 value of the formula on these draws, so the kernel is held to
    the 1e-5 relative bar against a float64 evaluation on sampled rows; its distance to the oracle is
    reported beside the oracle's own distance to the float64 value."""
    n = h * w
    r = np.random.default_rng(h * 100 + w)
    s = oracle.round_to(r.standard_normal((bh, n, n)), "f32")
    q = oracle.round_to(r.standard_normal((bh, n, hd)), "f32")
    t = oracle.round_to(r.standard_normal((2 * h - 1 + 2 * w - 1, hd)), "f32")
    got = hip.relpos_softmax(dev(s, "f32"), dev(q, "f32"), dev(t, "f32"), h, w, 0.125).cpu().numpy()[0]
    want = oracle.relpos_softmax(s, q, t, h, w, 0.125)[0]
    rows = np.arange(0, n, 61)
    th, tw = t[:2 * h - 1].astype(np.float64), t[2 * h - 1:].astype(np.float64)
    exact = []
    for rr in rows:
        i, j = rr // w, rr % w
        qq = q[0, rr].astype(np.float64)
        rh = np.array([qq @ th[i - kh + h - 1] for kh in range(h)])
        rw = np.array([qq @ tw[j - kw + w - 1] for kw in range(w)])
        x = s[0, rr].astype(np.float64) * 0.125 + (rh[:, None] + rw[None, :]).reshape(-1)
        e = np.exp(x - x.max())
        exact.append(e / e.sum())
    exact = np.array(exact)
    e64 = np.abs(got[rows] - exact).max() / np.abs(exact).max()
    eor = np.abs(got - want).max() / np.abs(want).max()
    own = np.abs(want[rows] - exact).max() / np.abs(exact).max()
    print(f"parity relpos_softmax {h}x{w} f32: vs float64 {e64:.3g}, vs oracle {eor:.3g} (oracle vs float64 "
          f"{own:.3g})", flush=True)
    assert e64 <= 1e-5


def test_relpos_softmax_rejects_grids_past_128(hip):
    h, w = 129, 2
    n = h * w
    s = torch.zeros(1, n, n, device="cuda", dtype=torch.float16)
    q = torch.zeros(1, n, 8, device="cuda", dtype=torch.float16)
    t = torch.zeros(2 * h - 1 + 2 * w - 1, 8, device="cuda", dtype=torch.float16)
    with pytest.raises(hip.SamHipError, match="h, w <= 128"):
        hip.relpos_softmax(s, q, t, h, w, 0.1)


# Rows past the reference GPU kernel's 8192 keys (kernels.rs:1078-1083), where the reference takes its
# tensor path and this library its two-pass scalar kernel: 96 x 96 (9216 keys) in every dtype, and the
# 128 x 128 maximum (16384 keys) in f16. N(0,1) scores, q and table as above.
@pytest.mark.parametrize("dtype,h,w", [("f16", 96, 96), ("bf16", 96, 96), ("f16", 128, 128), ("bf16", 90, 128)])
def test_relpos_softmax_past_8192_keys(hip, dtype, h, w):
    print(f"relpos_softmax long {dtype} {h}x{w}", flush=True)
    n, hd = h * w, 8
    r = np.random.default_rng(h * 1000 + w)
    s = oracle.round_to(r.standard_normal((1, n, n), dtype=np.float32), dtype)
    q = oracle.round_to(r.standard_normal((1, n, hd), dtype=np.float32), dtype)
    t = oracle.round_to(r.standard_normal((2 * h - 1 + 2 * w - 1, hd), dtype=np.float32), dtype)
    want = oracle.relpos_softmax(s, q, t, h, w, 0.125)
    got = hip.relpos_softmax(dev(s, dtype), dev(q, dtype), dev(t, dtype), h, w, 0.125).float().cpu().numpy()
    err = float(np.abs(got - want).max())
    print(f"parity relpos_softmax {h}x{w} {dtype}: max-abs {err:.3g}", flush=True)
    if dtype == "bf16":
        assert (np.abs(got - want) - half_ulp_bf16(want)).max() <= 1e-3
    else:
        assert err <= 1e-3
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=2e-2 if dtype == "bf16" else 4e-3)


def test_relpos_softmax_past_8192_keys_f32(hip):
    """f32 rows of 9216 keys against a float64 evaluation on sampled rows, as for the 8192-key rows."""
    h = w = 96
    n, hd = h * w, 8
    r = np.random.default_rng(4242)
    s = r.standard_normal((1, n, n), dtype=np.float32)
    q = r.standard_normal((1, n, hd), dtype=np.float32)
    t = r.standard_normal((2 * h - 1 + 2 * w - 1, hd), dtype=np.float32)
    got = hip.relpos_softmax(dev(s, "f32"), dev(q, "f32"), dev(t, "f32"), h, w, 0.125).cpu().numpy()[0]
    rows = np.arange(0, n, 97)
    th, tw = t[:2 * h - 1].astype(np.float64), t[2 * h - 1:].astype(np.float64)
    exact = []
    for rr in rows:
        i, j = rr // w, rr % w
        qq = q[0, rr].astype(np.float64)
        rh = np.array([qq @ th[i - kh + h - 1] for kh in range(h)])
        rw = np.array([qq @ tw[j - kw + w - 1] for kw in range(w)])
        x = s[0, rr].astype(np.float64) * 0.125 + (rh[:, None] + rw[None, :]).reshape(-1)
        e = np.exp(x - x.max())
        exact.append(e / e.sum())
    exact = np.array(exact)
    e64 = np.abs(got[rows] - exact).max() / np.abs(exact).max()
    print(f"parity relpos_softmax 96x96 f32: vs float64 {e64:.3g}", flush=True)
    assert e64 <= 1e-5


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("n,nh,hd,win", [(196, 12, 64, 3), (196, 16, 80, 25), (4096, 16, 80, 1), (77, 3, 8, 2),
                                         (5, 2, 6, 3), (130, 1, 256, 2), (64, 4, 16, 2), (65, 2, 24, 1),
                                         (50, 2, 128, 2)])
def test_qkv_split_is_bit_exact(hip, n, nh, hd, win, dtype):
    print(f"qkv_split {dtype} n={n} nh={nh} hd={hd} win={win}", flush=True)
    r = np.random.default_rng(n + hd)
    y = oracle.round_to(r.standard_normal((win * n, 3 * nh * hd)), dtype)
    b = oracle.round_to(r.standard_normal(3 * nh * hd), dtype)
    q0, k0, v0 = (oracle.round_to(x, dtype) for x in oracle.qkv_split(y, b, n, nh, hd))
    q1, k1, v1 = hip.qkv_split(dev(y, dtype), dev(b, dtype), n, nh, hd)
    for a, want in ((q1, q0), (k1, k0), (v1, v0)):
        assert tuple(a.shape) == want.shape
        assert np.array_equal(a.float().cpu().numpy(), want)


def partition_np(y, batch, gh, gw, ws):
    """The reference's window partition (sam1/encoder.rs:129-137) of grid rows [batch*gh*gw, c]: zero
    padding to multiples of ws, windows (b, wi, wj) in order, tokens (ti, tj) row-major."""
    c = y.shape[1]
    ph, pw = -gh % ws, -gw % ws
    g = np.pad(y.reshape(batch, gh, gw, c), ((0, 0), (0, ph), (0, pw), (0, 0)))
    hp, wp = gh + ph, gw + pw
    return g.reshape(batch, hp // ws, ws, wp // ws, ws, c).transpose(0, 1, 3, 2, 4, 5).reshape(-1, c)


# (batch, gh, gw, ws, nh, hd): the ViT-H windowed block (64x64 grid, 14x14 windows, 16 heads x 80), a
# grid already a multiple of the window, one with padding on both sides and odd head dims, the global
# block as one 64x64 window, and a window larger than the grid
GRID_SHAPES = [(1, 64, 64, 14, 16, 80), (2, 28, 28, 14, 2, 64), (2, 20, 13, 7, 3, 12), (1, 64, 64, 64, 2, 80),
               (1, 5, 6, 8, 1, 16)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("batch,gh,gw,ws,nh,hd", GRID_SHAPES)
def test_qkv_split_grid_equals_partition_then_split(hip, batch, gh, gw, ws, nh, hd, dtype):
    """qkv_split_grid on the grid's projection = qkv_split on the projection of the zero-padded windows
    (whose padding rows are 0), bit for bit."""
    print(f"qkv_split_grid {dtype} batch={batch} grid={gh}x{gw} ws={ws} nh={nh} hd={hd}", flush=True)
    r = np.random.default_rng(gh * 31 + gw + hd)
    y = oracle.round_to(r.standard_normal((batch * gh * gw, 3 * nh * hd)), dtype)
    b = oracle.round_to(r.standard_normal(3 * nh * hd), dtype)
    q0, k0, v0 = (oracle.round_to(x, dtype) for x in oracle.qkv_split(partition_np(y, batch, gh, gw, ws), b, ws * ws,
                                                                         nh, hd))
    q1, k1, v1 = hip.qkv_split_grid(dev(y, dtype), dev(b, dtype), batch, gh, gw, ws, nh, hd)
    for a, want in ((q1, q0), (k1, k0), (v1, v0)):
        assert tuple(a.shape) == want.shape
        assert np.array_equal(a.float().cpu().numpy(), want)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("batch,gh,gw,ws,nh,hd", GRID_SHAPES)
def test_window_merge_is_unpartition_of_merged_heads(hip, batch, gh, gw, ws, nh, hd, dtype):
    """window_merge(ctx) = window_unpartition (sam1/encoder.rs:140-143) of the heads merged as
    sam1/encoder.rs:83 merges them, cropped to the grid: a copy, bit for bit."""
    print(f"window_merge {dtype} batch={batch} grid={gh}x{gw} ws={ws} nh={nh} hd={hd}", flush=True)
    nwh, nww = -(-gh // ws), -(-gw // ws)
    bh, n = batch * nwh * nww * nh, ws * ws
    r = np.random.default_rng(gh * 7 + gw + hd)
    ctx = oracle.round_to(r.standard_normal((bh, n, hd)), dtype)
    merged = ctx.reshape(batch * nwh * nww, nh, n, hd).transpose(0, 2, 1, 3).reshape(batch, nwh, nww, ws, ws, nh * hd)
    want = merged.transpose(0, 1, 3, 2, 4, 5).reshape(batch, nwh * ws, nww * ws, nh * hd)[:, :gh, :gw]
    got = hip.window_merge(dev(ctx, dtype), batch, gh, gw, ws, nh).float().cpu().numpy()
    assert got.shape == want.shape
    assert np.array_equal(got, want)
