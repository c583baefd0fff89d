"""Parity of the flash-attention, RoPE and memory-attention entry points (libsam_hip.so) with the CPU
oracle, on an MI355X.

The oracle restates the reference's attention back ends on the same seeded inputs, pre-rounded to the
kernel dtype (as tests/kernels.rs:28-31 does): sdpa (sam3/nn.rs:26-34) for the [B, H, L, D] layout,
the per-(batch, query, head) scalar attention for the [B, L, H, D] layout that flash_attn_cpu and
candle_flash_attn take (kernels.rs:416-434), rope (sam3/video.rs:106-113) and RopeAttn's core
(sam3/video.rs:129-145). Bars: f32 max|gpu - cpu| / max|cpu| <= 1e-5 (the reference's f32 GPU path is
sdpa as candle matmuls); f16/bf16 max-abs 2e-3 against the f32 oracle, measured beyond the
output's own rounding where that rounding alone reaches the bar (bf16 |out| >= 0.5, f16 |out| >= 4;
tests/parity.py); RoPE bit-exact.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle
from parity import TORCH_DT, check, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def rounded(r, shape, dtype, std=1.0):
    return oracle.round_to((std * r.standard_normal(shape)).astype(np.float32), dtype)


# (b, lq, lk, h, d): tiny and ragged shapes (partial key tiles, partial query blocks, one key), the
# head dims of the reference's callers (Hiera 96 at its widest stage, SAM 3 ViT 64, memory attention
# 256), and shapes whose few query blocks force the key-split path. Up to head dim 64, and at 96 and 128
# for up to 1024 keys, a workgroup holds 128 queries (256 past that): several query blocks with a
# partial last one (576 queries: 4.5 blocks, two idle waves), with and without key splits, and both
# sides of the 1024-key line.
BLHD = [(1, 5, 7, 2, 16), (2, 33, 65, 3, 64), (1, 40, 100, 1, 256), (2, 130, 200, 4, 96), (1, 64, 64, 8, 64),
        (1, 300, 1000, 2, 128), (1, 1, 1, 1, 8), (1, 17, 3000, 1, 64), (3, 49, 49, 2, 32), (1, 257, 129, 1, 256),
        (2, 130, 517, 3, 256), (1, 70, 33, 2, 256), (1, 128, 64, 1, 256), (2, 576, 576, 3, 64),
        (1, 1000, 1000, 2, 64), (1, 300, 700, 2, 32), (1, 260, 1100, 2, 96), (2, 300, 1024, 1, 128)]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("b,lq,lk,h,d", BLHD)
def test_flash_attn_matches_oracle(hip, b, lq, lk, h, d, dtype):
    r = np.random.default_rng(1000 + lq + lk + d)
    q, k, v = (rounded(r, (b, n, h, d), dtype) for n in (lq, lk, lk))
    got = hip.flash_attn(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    want = oracle.mha_blhd(q, k, v)
    check(got.float().cpu().numpy(), want, dtype, f"flash_attn b{b} lq{lq} lk{lk} h{h} d{d} {dtype}")


# SAM 3 ViT's own attention calls (sam3/vision.rs:113-121), full size: the 24 x 24 windows of a 72 x 72
# grid (9 windows of 576 tokens) and the global grid (5184 tokens), 16 heads of 64. The GPU runs every
# window and head; the oracle checks two windows and two heads.
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("case", ["window", "global"])
def test_sam3_vit_attention_full_size(hip, case, dtype):
    b, l = (9, 576) if case == "window" else (1, 5184)
    h, d = 16, 64
    print(f"sam3 vit {case} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(31 if case == "window" else 32)
    q, k, v = (torch.randn(b, l, h, d, device="cuda", generator=g).to(TORCH_DT[dtype]) for _ in range(3))
    got = hip.flash_attn(q, k, v)
    torch.cuda.synchronize()
    host = lambda t: t.float().cpu().numpy()
    if case == "window":
        sel = [0, 8]
        want = oracle.mha_blhd(host(q[sel]), host(k[sel]), host(v[sel]))
        check(host(got[sel]), want, dtype, f"sam3 vit window {dtype}")
    else:
        sel = [0, 15]
        want = oracle.mha_blhd(host(q[:, :, sel]), host(k[:, :, sel]), host(v[:, :, sel]))
        check(host(got[:, :, sel]), want, dtype, f"sam3 vit global {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("b,h,lq,lk,d", [(1, 1, 5, 7, 16), (2, 3, 33, 65, 64), (1, 1, 40, 100, 256),
                                         (1, 2, 200, 700, 256)])
def test_sdpa_bhld_layout(hip, b, h, lq, lk, d, dtype):
    r = np.random.default_rng(7 + lq)
    q, k, v = (rounded(r, (b, h, n, d), dtype) for n in (lq, lk, lk))
    got = hip.sdpa(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    check(got.float().cpu().numpy(), oracle.sdpa(q, k, v), dtype, f"sdpa {b}x{h}x{lq}x{lk}x{d} {dtype}")


def masked_inputs(r, kind, b, h, lq, lk, d, dtype):
    q, k, v = (rounded(r, (b, h, n, d), dtype) for n in (lq, lk, lk))
    if kind == "bias":  # TinyViT's attention biases, one [N, N] table per head (sam1/tinyvit.rs:216)
        mask = oracle.round_to(r.standard_normal((1, h, lq, lk)).astype(np.float32), dtype)
    else:  # a key-padding mask of 0 / -inf per batch (sam3/detr.rs:55, 191, 272)
        mask = np.zeros((b, 1, 1, lk), np.float32)
        for bi in range(b):
            mask[bi, ..., lk - 5 - 3 * bi:] = -np.inf
    return q, k, v, mask


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("kind,b,h,lq,lk,d", [("bias", 3, 4, 49, 49, 32), ("padding", 2, 8, 200, 37, 32),
                                              ("padding", 1, 2, 100, 130, 256), ("bias", 1, 2, 70, 300, 64),
                                              ("padding", 2, 3, 33, 65, 128)])
def test_sdpa_additive_mask(hip, kind, b, h, lq, lk, d, dtype):
    """sdpa with Some(mask) (sam3/nn.rs:26-34): the mask broadcasts from its own shape (stride 0 on the
    broadcast dimensions), is added to the scaled scores, and -inf drops a key."""
    r = np.random.default_rng(11 + lk + d)
    q, k, v, mask = masked_inputs(r, kind, b, h, lq, lk, d, dtype)
    print(f"sdpa mask {kind} b={b} h={h} lq={lq} lk={lk} d={d} {dtype}", flush=True)
    got = hip.sdpa(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(mask, dtype))
    torch.cuda.synchronize()
    check(got.float().cpu().numpy(), oracle.sdpa(q, k, v, mask), dtype, f"sdpa mask {kind} {b}x{h}x{lq}x{lk}x{d}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("where", ["tail", "head"])
def test_sdpa_mask_whole_key_splits_masked(hip, where, dtype):
    """One query block and 3000 keys split across many workgroups (16 splits of 3 tiles), with every key
    past 150 ("tail") or before 2850 ("head") at -inf: most splits see only masked keys, and their
    partials must weigh nothing in the combine, also when more than its first chunk of 8 splits is
    masked. One query whose keys are all -inf comes out NaN, as the reference's softmax gives, and no
    other row does."""
    r = np.random.default_rng(5)
    b, h, lq, lk, d = 1, 1, 40, 3000, 64
    q, k, v = (rounded(r, (b, h, n, d), dtype) for n in (lq, lk, lk))
    mask = np.zeros((1, 1, lq, lk), np.float32)
    if where == "tail":
        mask[..., 150:] = -np.inf
    else:
        mask[..., :2850] = -np.inf
    mask[0, 0, 7, :] = -np.inf
    got = hip.sdpa(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(mask, dtype))
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    want = oracle.sdpa(q, k, v, mask)
    assert np.isnan(got[0, 0, 7]).all() and np.isnan(want[0, 0, 7]).all()
    rows = [i for i in range(lq) if i != 7]
    check(got[:, :, rows], want[:, :, rows], dtype, f"sdpa mask, split keys, {where} masked {dtype}")


def test_sdpa_mask_rejects_bad_arguments(hip):
    """A mask of another dtype, or one that does not broadcast to [B, H, Lq, Lk], is refused."""
    q = torch.zeros(1, 2, 8, 32, device="cuda", dtype=torch.float16)
    with pytest.raises(hip.SamHipError):
        hip.sdpa(q, q, q, torch.zeros(1, 1, 1, 8, device="cuda", dtype=torch.float32))
    with pytest.raises(hip.SamHipError):
        hip.sdpa(q, q, q, torch.zeros(1, 3, 8, 8, device="cuda", dtype=torch.float16))


def test_strided_views_are_read_in_place(hip):
    """A [B, L, H, D] slice of a wider packed projection (row stride > H*D) gives the same result as
    its contiguous copy."""
    r = np.random.default_rng(3)
    b, l, h, d = 2, 90, 2, 64
    packed = to_dev(rounded(r, (b, l, 3, h, d), "f16"), "f16")
    q, k, v = packed[:, :, 0], packed[:, :, 1], packed[:, :, 2]
    got = hip.flash_attn(q, k, v)
    ref = hip.flash_attn(q.contiguous(), k.contiguous(), v.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_strided_views_d256(hip):
    """Head dim 256 read in place from a packed [B, L, 3, H, D] projection (row stride 6 x 256)."""
    r = np.random.default_rng(4)
    b, l, h, d = 1, 150, 2, 256
    packed = to_dev(rounded(r, (b, l, 3, h, d), "bf16"), "bf16")
    q, k, v = packed[:, :, 0], packed[:, :, 1], packed[:, :, 2]
    got = hip.flash_attn(q, k, v)
    ref = hip.flash_attn(q.contiguous(), k.contiguous(), v.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_flash_d256_growing_scores(hip, dtype):
    """Key norms growing along the sequence (0.03 to 10) push each query's running max past the lazy
    rescale's slack 2 to 4 times, mid-loop: b x h = 256 query blocks leave the keys unsplit, so every
    workgroup walks all 10 key tiles and rescales its accumulated O on the way."""
    r = np.random.default_rng(77)
    b, h, lq, lk, d = 2, 128, 32, 640, 256
    q = rounded(r, (b, lq, h, d), dtype)
    grow = (np.linspace(0.1, 10.0, lk, dtype=np.float32) ** 1.5 / np.float32(10.0 ** 0.5))[None, :, None, None]
    k = oracle.round_to((r.standard_normal((b, lk, h, d)).astype(np.float32) * grow), dtype)
    v = rounded(r, (b, lk, h, d), dtype)
    got = hip.flash_attn(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    check(got.float().cpu().numpy(), oracle.mha_blhd(q, k, v), dtype, f"flash_attn growing scores {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_rope_is_bit_exact(hip, dtype):
    """rope rounds like the reference: f32 products and sum, then one rounding to the dtype."""
    side, d = 8, 256
    cos, sin = oracle.rope_tables(side, 1.0, d, 10000.0)
    r = np.random.default_rng(5)
    x = rounded(r, (3 * side * side, d), dtype)
    got = hip.rope(to_dev(x, dtype).unsqueeze(0), torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda())
    torch.cuda.synchronize()
    want = oracle.round_to(np.concatenate([oracle.rope(x[i * 64:(i + 1) * 64], cos, sin) for i in range(3)]), dtype)
    assert np.array_equal(got[0].float().cpu().numpy(), want)


def test_rope_leaves_excluded_rows(hip):
    side, d = 4, 64
    cos, sin = oracle.rope_tables(side, 1.0, d, 10000.0)
    r = np.random.default_rng(6)
    x = rounded(r, (2 * 16 + 5, d), "f16")
    got = hip.rope(to_dev(x, "f16").unsqueeze(0), torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(),
                   n_rot=32)[0].float().cpu().numpy()
    assert np.array_equal(got[32:], x[32:])
    want = oracle.round_to(np.concatenate([oracle.rope(x[:16], cos, sin), oracle.rope(x[16:32], cos, sin)]), "f16")
    assert np.array_equal(got[:32], want)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("side,l,n_rot", [(2, 37, 30), (4, 37, 30), (4, 70, 70)])
def test_rope_batches_heads_and_tiled_tables(hip, side, l, n_rot, dtype):
    """Several batches and heads, a [B, H, L, D] view (strided rows), tables of side*side rows reused by
    up to 8 rows each (row r takes table row r % T), and rows past n_rot copied: bit-exact against the
    oracle's rope row by row."""
    b, h, d = 2, 3, 64
    cos, sin = oracle.rope_tables(side, 1.0, d, 10000.0)
    trows = side * side
    r = np.random.default_rng(7 + l + side)
    x = rounded(r, (b, h, l, d), dtype)
    xd = to_dev(x, dtype).permute(0, 2, 1, 3)  # [B, L, H, D] view of the [B, H, L, D] tensor
    print(f"rope b={b} h={h} l={l} trows={trows} n_rot={n_rot} {dtype}", flush=True)
    got = hip.rope(xd, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), n_rot=n_rot)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()  # [B, L, H, D]
    for bi in range(b):
        for hi in range(h):
            rows = x[bi, hi]
            want = rows.copy()
            for rr in range(n_rot):
                t = rr % trows
                want[rr] = oracle.rope(rows[rr:rr + 1], cos[t:t + 1], sin[t:t + 1])[0]
            want = oracle.round_to(want, dtype)
            assert np.array_equal(got[bi, :, hi], want), (bi, hi)


def memory_inputs(side, frames, n_ptr, d, dtype, seed):
    r = np.random.default_rng(seed)
    n = side * side
    m = frames * n + n_ptr
    q = rounded(r, (n, d), dtype)
    k = rounded(r, (m, d), dtype)
    v = rounded(r, (m, d), dtype)
    cos, sin = oracle.rope_tables(side, 1.0, d, 10000.0)
    return q, k, v, cos, sin


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("side,frames,n_ptr", [(8, 1, 0), (8, 3, 8), (6, 2, 4)])
def test_rope_attention_small(hip, side, frames, n_ptr, dtype):
    """RopeAttn's attention core: self-attention (frames 1, no pointers) and cross-attention over tiled
    memory frames plus unrotated object-pointer tokens."""
    q, k, v, cos, sin = memory_inputs(side, frames, n_ptr, 256, dtype, 11 + side + frames)
    got = hip.rope_attention(to_dev(q, dtype)[None], to_dev(k, dtype)[None], to_dev(v, dtype)[None],
                             torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), n_ptr)
    torch.cuda.synchronize()
    # the reference rounds the rotated q and k to the dtype before sdpa (rope converts back, video.rs:112)
    qr = oracle.round_to(oracle.rope(q, cos, sin), dtype)
    rot = k.shape[0] - n_ptr
    kr = np.concatenate([oracle.round_to(oracle.rope(k[i:i + len(cos)], cos, sin), dtype)
                         for i in range(0, rot, len(cos))] + [k[rot:]])
    want = oracle.sdpa(qr[None, None], kr[None, None], v[None, None])[0, 0]
    check(got[0].float().cpu().numpy(), want, dtype, f"rope_attention side{side} frames{frames} ptr{n_ptr}")
    # and, in f16, against the oracle's own f32 RopeAttn core (rotated q/k kept in f32): f16 rounding of
    # the rotated q/k stays inside the bar; bf16's (2^-9 of each score) does not, as in the reference
    if dtype == "f16":
        want32 = oracle.rope_attention(q, k, v, cos, sin, n_ptr)
        check(got[0].float().cpu().numpy(), want32, dtype, "rope_attention vs f32 rotation")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("d,lq,n_rope_q", [(256, 200, 150), (64, 130, 130)])
def test_rope_on_queries_only(hip, d, lq, n_rope_q, dtype):
    """Queries rotated and keys not (n_rope_k = 0): the rotation then happens while the attention kernel
    loads Q, with the same rounding as the separate pass (f32 products and sum, one rounding)."""
    side, lk = 8, 300
    cos, sin = oracle.rope_tables(side, 1.0, d, 10000.0)
    r = np.random.default_rng(31 + d)
    q, k, v = (rounded(r, (1, n, 1, d), dtype) for n in (lq, lk, lk))
    got = hip._flash(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), torch.empty(1, lq, 1, d, device="cuda",
                     dtype=TORCH_DT[dtype]), "blhd", d ** -0.5, torch.from_numpy(cos).cuda(),
                     torch.from_numpy(sin).cuda(), n_rope_q=n_rope_q, n_rope_k=0)
    torch.cuda.synchronize()
    qr = q[0, :, 0].copy()
    for i in range(0, n_rope_q, len(cos)):
        j = min(n_rope_q, i + len(cos))
        qr[i:j] = oracle.round_to(oracle.rope(q[0, i:j, 0], cos[:j - i], sin[:j - i]), dtype)
    want = oracle.sdpa(qr[None, None], k[0, :, 0][None, None], v[0, :, 0][None, None])[0, 0]
    check(got[0, :, 0].float().cpu().numpy(), want, dtype, f"rope on queries only d{d} {dtype}")


@pytest.mark.parametrize("case", ["self", "cross"])
def test_sam2_memory_attention_full_size(hip, case):
    """SAM 2.1 memory attention at its real size (f16, d 256, 64x64 grid): self-attention over 4096
    tokens, cross-attention over 7 memory frames x 4096 + 64 pointer tokens = 28736 keys. The oracle
    checks 96 query rows spread over the grid (each output row depends only on its own query)."""
    frames, n_ptr = (1, 0) if case == "self" else (7, 64)
    q, k, v, cos, sin = memory_inputs(64, frames, n_ptr, 256, "f16", 21 if case == "self" else 22)
    got = hip.rope_attention(to_dev(q, "f16")[None], to_dev(k, "f16")[None], to_dev(v, "f16")[None],
                             torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), n_ptr)
    torch.cuda.synchronize()
    got = got[0].float().cpu().numpy()
    assert np.isfinite(got).all()
    rows = np.linspace(0, 4095, 96).astype(int)
    qr = oracle.round_to(oracle.rope(q, cos, sin), "f16")[rows]
    rot = k.shape[0] - n_ptr
    kr = np.concatenate([oracle.round_to(oracle.rope(k[i:i + 4096], cos, sin), "f16") for i in range(0, rot, 4096)]
                        + [k[rot:]])
    want = oracle.sdpa(qr[None, None], kr[None, None], v[None, None])[0, 0]
    check(got[rows], want, "f16", f"memory attention {case}")


def test_full_size_properties(hip):
    """Size-independent properties at the cross-attention size: identical keys give the mean of v
    (uniform softmax), and permuting keys together with values leaves the output unchanged."""
    g = torch.Generator(device="cuda").manual_seed(4)
    lq, lk, d = 4096, 28736, 256
    q = torch.randn(1, lq, 1, d, device="cuda", generator=g).half()
    v = torch.randn(1, lk, 1, d, device="cuda", generator=g).half()
    k1 = torch.randn(1, 1, 1, d, device="cuda", generator=g).half().expand(1, lk, 1, d).contiguous()
    out = hip.flash_attn(q, k1, v)
    mean = v.float().mean(dim=1, keepdim=True)
    assert (out.float() - mean).abs().max().item() <= 2e-3
    k = torch.randn(1, lk, 1, d, device="cuda", generator=g).half()
    perm = torch.randperm(lk, device="cuda", generator=g)
    o1 = hip.flash_attn(q, k, v)
    o2 = hip.flash_attn(q, k[:, perm].contiguous(), v[:, perm].contiguous())
    assert (o1.float() - o2.float()).abs().max().item() <= 2e-3


def test_flash_errors(hip):
    x16 = torch.zeros(1, 8, 1, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(hip.SamHipError, match="unsupported dtype"):
        hip.flash_attn(x16.double(), x16.double(), x16.double())
    with pytest.raises(hip.SamHipError, match="multiple of 8"):
        y = torch.zeros(1, 8, 1, 20, device="cuda", dtype=torch.float16)
        hip.flash_attn(y, y, y)
    with pytest.raises(hip.SamHipError, match="incompatible"):
        hip.flash_attn(x16, torch.zeros(1, 8, 2, 64, device="cuda", dtype=torch.float16), x16)
    with pytest.raises(hip.SamHipError, match="mask"):
        hip.sdpa(x16, x16, x16, mask=x16)
    with pytest.raises(hip.SamHipError, match="dtype mismatch"):
        hip.flash_attn(x16, x16.bfloat16(), x16)
    assert TORCH_DT["f16"] == torch.float16
