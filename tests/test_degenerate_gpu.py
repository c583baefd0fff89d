"""Degenerate shapes on an MI355X: one-token grids, one-key attention, and grids of a single row or
column, through every dtype.

With one key the softmax weight is exactly 1 (exp(0) / exp(0)), so the reference's sequence
(bmm -> relpos_softmax -> bmm, sam1/encoder.rs:79-82, kernels.rs:12-43) and its flash attention return
v itself: these cases are checked bit for bit. Single-row and single-column grids (1 x w, h x 1, up to
the wide kernel's 128) are checked against the oracle at the usual bars (tests/parity.py).
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


def draw(r, shape, dtype, std=1.0):
    return oracle.round_to((std * r.standard_normal(shape)).astype(np.float32), dtype)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("hd", [16, 64, 80])
def test_one_token_grid_returns_v(hip, hd, dtype):
    print(f"one-token grid {dtype} hd={hd}", flush=True)
    r = np.random.default_rng(7400 + hd)
    bh = 5
    q, kt, v = draw(r, (bh, 1, hd), dtype), draw(r, (bh, hd, 1), dtype), draw(r, (bh, 1, hd), dtype)
    table = draw(r, (2, hd), dtype, 0.02)
    got = hip.attention_relpos(to_dev(q, dtype), to_dev(kt, dtype), to_dev(v, dtype), to_dev(table, dtype), 1, 1,
                               hd ** -0.5)
    torch.cuda.synchronize()
    assert np.array_equal(got.float().cpu().numpy(), v)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
def test_one_token_relpos_softmax_is_one(hip, dtype):
    r = np.random.default_rng(7410)
    s, q, t = draw(r, (3, 1, 1), dtype), draw(r, (3, 1, 64), dtype), draw(r, (2, 64), dtype)
    got = hip.relpos_softmax(to_dev(s, dtype), to_dev(q, dtype), to_dev(t, dtype), 1, 1, 0.125)
    torch.cuda.synchronize()
    assert (got.float().cpu().numpy() == 1.0).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("lq,h,d", [(1, 1, 64), (300, 2, 64), (70, 3, 96), (33, 1, 256)])
def test_one_key_attention_returns_v(hip, lq, h, d, dtype):
    print(f"one-key flash {dtype} lq={lq} h={h} d={d}", flush=True)
    r = np.random.default_rng(7420 + lq + d)
    q, k, v = draw(r, (2, lq, h, d), dtype), draw(r, (2, 1, h, d), dtype), draw(r, (2, 1, h, d), dtype)
    got = hip.flash_attn(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    assert np.array_equal(got.float().cpu().numpy(), np.broadcast_to(v, (2, lq, h, d)))


# single-row and single-column grids: the generic kernel's shortest rows and columns, a 64-column row
# (the global kernel's width), and the wide kernel's 128 x 1 and 1 x 128
LINES = [(1, 2, 64), (2, 1, 64), (1, 64, 80), (64, 1, 80), (1, 64, 64), (64, 1, 64), (1, 128, 64), (128, 1, 64),
         (1, 100, 80), (100, 1, 80)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,hd", LINES)
def test_single_row_and_column_grids(hip, h, w, hd, dtype):
    if dtype == "f32" and max(h, w) > 64:
        pytest.skip("f32 rel-pos attention stops at 64 x 64 (larger f32 grids take the reference's sequence)")
    n = h * w
    print(f"line grid {dtype} h={h} w={w} hd={hd}", flush=True)
    r = np.random.default_rng(7430 + 7 * h + w + hd)
    bh = 3
    q, kt, v = draw(r, (bh, n, hd), dtype), draw(r, (bh, hd, n), dtype), draw(r, (bh, n, hd), dtype)
    table = draw(r, (2 * h - 1 + 2 * w - 1, hd), dtype, 0.02)
    got = hip.attention_relpos(to_dev(q, dtype), to_dev(kt, dtype), to_dev(v, dtype), to_dev(table, dtype), h, w,
                               hd ** -0.5)
    torch.cuda.synchronize()
    want = oracle.attention_relpos(q, kt, v, table, h, w, hd ** -0.5)
    check(got.float().cpu().numpy(), want, dtype, f"line grid {h}x{w} hd={hd} {dtype}")


# scales other than hd^-0.5: a sharp 1.0, 0.2 (the f16 global kernel pre-scales q only up to hd^-0.5),
# a flat 0.03, 0 (uniform weights over the bias) and a negative one (the dedicated window and global
# kernels take scale > 0; the others go to the general kernel); the wide-grid kernel at 65 x 64
SCALES = [1.0, 0.2, 0.03, 0.0, -0.1]
SCALE_GRIDS = [(14, 14, 80), (64, 64, 80), (14, 14, 64), (64, 64, 64), (7, 11, 64), (65, 64, 64)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,hd", SCALE_GRIDS)
@pytest.mark.parametrize("scale", SCALES)
def test_attention_relpos_other_scales(hip, h, w, hd, scale, dtype):
    if dtype == "f32" and max(h, w) > 64:
        pytest.skip("f32 rel-pos attention stops at 64 x 64 (larger f32 grids take the reference's sequence)")
    n = h * w
    print(f"scale {scale} {dtype} h={h} w={w} hd={hd}", flush=True)
    r = np.random.default_rng(7500 + n + hd)
    bh = 2
    q, kt, v = draw(r, (bh, n, hd), dtype), draw(r, (bh, hd, n), dtype), draw(r, (bh, n, hd), dtype)
    table = draw(r, (2 * h - 1 + 2 * w - 1, hd), dtype, 0.02)
    got = hip.attention_relpos(to_dev(q, dtype), to_dev(kt, dtype), to_dev(v, dtype), to_dev(table, dtype), h, w,
                               scale)
    torch.cuda.synchronize()
    want = oracle.attention_relpos(q, kt, v, table, h, w, scale)
    check(got.float().cpu().numpy(), want, dtype, f"scale {scale} {h}x{w} hd={hd} {dtype}")


# larger activations at the model's own scale hd^-0.5: q and k of standard deviation 2 and 3 (logits 4
# and 9 times those of unit inputs), v of 1. In f32 the oracle's own sequential f32 arithmetic (the
# reference's, kernels.rs:197-214) is itself up to 1.3e-5 from the exact value on these draws (64 x 64,
# standard deviation 2), so f32 is held to the 1e-5 bar against a float64 evaluation of the formula and
# its distance to the oracle is printed beside the oracle's own.
MAGNITUDES = [2.0, 3.0]


def attention_relpos_f64(q, kt, v, table, h, w, scale):
    """The fused rel-pos attention in float64 (textbook form, for the f32 bar)."""
    n = h * w
    th, tw = table[: 2 * h - 1].astype(np.float64), table[2 * h - 1:].astype(np.float64)
    ri, rj = np.arange(n) // w, np.arange(n) % w
    rows = np.arange(n)[:, None]
    out = np.empty(q.shape, np.float64)
    for b in range(q.shape[0]):
        qq = q[b].astype(np.float64)
        s = qq @ kt[b].astype(np.float64) * scale
        s += (qq @ th.T)[rows, ri[:, None] - ri[None, :] + h - 1] + (qq @ tw.T)[rows, rj[:, None] - rj[None, :] + w - 1]
        p = np.exp(s - s.max(1, keepdims=True))
        out[b] = (p / p.sum(1, keepdims=True)) @ v[b].astype(np.float64)
    return out


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,hd", [(14, 14, 80), (64, 64, 80), (64, 64, 64), (7, 11, 64), (65, 64, 64), (96, 96, 80)])
@pytest.mark.parametrize("std", MAGNITUDES)
def test_attention_relpos_larger_activations(hip, h, w, hd, std, dtype):
    if dtype == "f32" and max(h, w) > 64:
        pytest.skip("f32 rel-pos attention stops at 64 x 64 (larger f32 grids take the reference's sequence)")
    n = h * w
    print(f"std {std} {dtype} h={h} w={w} hd={hd}", flush=True)
    r = np.random.default_rng(7600 + n + hd + int(10 * std))
    bh = 2
    q, kt = draw(r, (bh, n, hd), dtype, std), draw(r, (bh, hd, n), dtype, std)
    v = draw(r, (bh, n, hd), dtype)
    table = draw(r, (2 * h - 1 + 2 * w - 1, hd), dtype, 0.02)
    got = hip.attention_relpos(to_dev(q, dtype), to_dev(kt, dtype), to_dev(v, dtype), to_dev(table, dtype), h, w,
                               hd ** -0.5)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    want = oracle.attention_relpos(q, kt, v, table, h, w, hd ** -0.5)
    if dtype == "f32":
        exact = attention_relpos_f64(q, kt, v, table, h, w, hd ** -0.5)
        e64 = np.abs(got - exact).max() / np.abs(exact).max()
        eor = np.abs(got - want).max() / np.abs(want).max()
        own = np.abs(want - exact).max() / np.abs(exact).max()
        print(f"parity std {std} {h}x{w} hd={hd} f32: vs float64 {e64:.3g}, vs oracle {eor:.3g} (oracle vs "
              f"float64 {own:.3g})", flush=True)
        assert e64 <= 1e-5
    else:
        check(got, want, dtype, f"std {std} {h}x{w} hd={hd} {dtype}")


# flash attention with larger activations: q and k of standard deviation 3 at the default scale d^-0.5,
# through the generic kernel (head dims 64 and 96) and the head-dim-256 kernel with a key split
@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("b,lq,lk,h,d", [(1, 576, 576, 4, 64), (1, 300, 1000, 2, 96), (1, 130, 4096, 1, 256)])
def test_flash_attn_larger_activations(hip, b, lq, lk, h, d, dtype):
    """f32 is held to 1e-5 against a float64 evaluation, as for the rel-pos attention above."""
    print(f"flash std 3 {dtype} b={b} lq={lq} lk={lk} h={h} d={d}", flush=True)
    r = np.random.default_rng(7700 + lq + lk + d)
    q, k = draw(r, (b, lq, h, d), dtype, 3.0), draw(r, (b, lk, h, d), dtype, 3.0)
    v = draw(r, (b, lk, h, d), dtype)
    got = hip.flash_attn(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    want = oracle.mha_blhd(q, k, v)
    if dtype == "f32":
        q64, k64, v64 = (x.astype(np.float64).transpose(0, 2, 1, 3) for x in (q, k, v))
        s = q64 @ k64.transpose(0, 1, 3, 2) * d ** -0.5
        p = np.exp(s - s.max(-1, keepdims=True))
        exact = ((p / p.sum(-1, keepdims=True)) @ v64).transpose(0, 2, 1, 3)
        e64 = np.abs(got - exact).max() / np.abs(exact).max()
        own = np.abs(want - exact).max() / np.abs(exact).max()
        print(f"parity flash std 3 b{b} lq{lq} lk{lk} h{h} d{d} f32: vs float64 {e64:.3g} (oracle vs float64 "
              f"{own:.3g})", flush=True)
        assert e64 <= 1e-5
    else:
        check(got, want, dtype, f"flash std 3 b{b} lq{lq} lk{lk} h{h} d{d} {dtype}")


# relpos_softmax over large scores (standard deviation 10: rows dominated by a few keys) on the window
# grid (16 lanes per row), the global grid (vector kernel) and an odd-length row (scalar kernel)
@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,hd", [(14, 14, 80), (64, 64, 80), (5, 9, 64)])
def test_relpos_softmax_large_scores(hip, h, w, hd, dtype):
    n = h * w
    print(f"relpos_softmax std 10 {dtype} h={h} w={w} hd={hd}", flush=True)
    r = np.random.default_rng(7800 + n + hd)
    bh = 2
    s = draw(r, (bh, n, n), dtype, 10.0)
    q = draw(r, (bh, n, hd), dtype)
    t = draw(r, (2 * h - 1 + 2 * w - 1, hd), dtype)
    got = hip.relpos_softmax(to_dev(s, dtype), to_dev(q, dtype), to_dev(t, dtype), h, w, 0.125)
    torch.cuda.synchronize()
    want = oracle.relpos_softmax(s, q, t, h, w, 0.125)
    check(got.float().cpu().numpy(), want, dtype, f"relpos_softmax std 10 {h}x{w} hd={hd} {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("c", [1280, 768, 1024])
def test_bias_residual_ln_constant_rows(hip, c, dtype):
    """Rows whose residual sum is constant have zero variance: the LayerNorm gives (x - mean) = 0 times
    1/sqrt(eps), so the normed row is ln_b exactly, and x itself is the constant."""
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    g = torch.Generator(device="cuda").manual_seed(7900 + c)
    rows = 300
    res = torch.full((rows, c), 0.75, dtype=tdt, device="cuda")
    y = torch.full((rows, c), -0.25, dtype=tdt, device="cuda")
    bias = torch.zeros(c, dtype=tdt, device="cuda")
    ln_w = torch.randn(c, device="cuda", generator=g).to(tdt)
    ln_b = torch.randn(c, device="cuda", generator=g).to(tdt)
    x, normed = hip.bias_residual_ln(res, y, bias, ln_w, ln_b)
    torch.cuda.synchronize()
    assert (x == 0.5).all()
    assert torch.equal(normed, ln_b.expand(rows, c))


def offset_view(x):
    """x copied into a buffer one element past a 16-byte boundary: a contiguous view with a storage
    offset, as candle's narrow of a packed tensor produces."""
    buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=x.device)
    v = buf[1:].view(x.shape)
    v.copy_(x)
    assert v.data_ptr() % 16 != 0
    return v


def test_views_off_a_16_byte_boundary(hip):
    """The reference's kernels take views with a storage offset. The front end copies such an input to
    an aligned buffer for the kernels that need 16-byte alignment (their C ABI entry points refuse it);
    bias_residual and bias_gelu take it as it is, through a scalar loop that rounds as their vector loop
    does. Either way the results equal those of aligned inputs bit for bit."""
    g = torch.Generator(device="cuda").manual_seed(8100)
    f16 = torch.float16
    q, kt, v = (torch.randn(s, device="cuda", generator=g).to(f16) for s in ((50, 196, 80), (50, 80, 196), (50, 196, 80)))
    t = (0.02 * torch.randn(54, 80, device="cuda", generator=g)).to(f16)
    want = hip.attention_relpos(q, kt, v, t, 14, 14, 80 ** -0.5)
    got = hip.attention_relpos(offset_view(q), offset_view(kt), offset_view(v), offset_view(t), 14, 14, 80 ** -0.5)
    assert torch.equal(got, want)
    fq, fk, fv = (torch.randn(s, device="cuda", generator=g).to(f16) for s in ((1, 300, 2, 64), (1, 900, 2, 64), (1, 900, 2, 64)))
    assert torch.equal(hip.flash_attn(offset_view(fq), offset_view(fk), offset_view(fv)), hip.flash_attn(fq, fk, fv))
    s = torch.randn(2, 196, 196, device="cuda", generator=g).to(f16)
    sq = torch.randn(2, 196, 64, device="cuda", generator=g).to(f16)
    st = torch.randn(54, 64, device="cuda", generator=g).to(f16)
    assert torch.equal(hip.relpos_softmax(offset_view(s), offset_view(sq), offset_view(st), 14, 14, 0.125),
                       hip.relpos_softmax(s, sq, st, 14, 14, 0.125))
    y, b = torch.randn(196 * 4, 3 * 4 * 64, device="cuda", generator=g).to(f16), torch.randn(3 * 4 * 64, device="cuda", generator=g).to(f16)
    for got_, want_ in zip(hip.qkv_split(offset_view(y), offset_view(b), 196, 4, 64), hip.qkv_split(y, b, 196, 4, 64)):
        assert torch.equal(got_, want_)
    assert torch.equal(hip.bias_gelu(offset_view(y), offset_view(b)), hip.bias_gelu(y, b))
    assert torch.equal(hip.bias_residual(offset_view(y), offset_view(y), offset_view(b)), hip.bias_residual(y, y, b))
