"""The SAM image encoder forward on this library's kernels (sam-rs_amd/sam_encoder.py) against a plain
torch float32 implementation of the same architecture (sam1/encoder.rs: windowed and global blocks with
decomposed rel-pos attention, MLP with exact GELU, neck), on an MI355X.

The reference here is the textbook form: full score matrices with get_rel_pos tables and an einsum
bias, torch's softmax, conv2d for the patch embedding and the neck, no fused kernels. The small
configurations (2 heads x hd 80 or hd 64, one windowed block on the 64x64 grid padded to 70x70, one
global block) run the same dedicated window and global kernels as ViT-H (hd 80) and ViT-B / ViT-L
(hd 64).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def enc():
    import sam_encoder
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_encoder


def ref_attention(x, p, heads):
    """Textbook SAM attention (float32): softmax(scale q k^T + rel_h + rel_w) v, then the projection
    without its bias."""
    nw, h, w, c = x.shape
    hd, n = c // heads, h * w
    qkv = (x.reshape(nw, n, c) @ p.qkv_w.float().t() + p.qkv_b.float()).view(nw, n, 3, heads, hd)
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3).contiguous() for i in range(3))  # [nw, heads, n, hd]
    rel = p.rel.float()
    rel_h, rel_w = rel[: 2 * h - 1], rel[2 * h - 1:]
    ih = torch.arange(h, device=x.device)
    iw = torch.arange(w, device=x.device)
    rh = rel_h[ih[:, None] - ih[None, :] + h - 1]  # [h, h, hd]
    rw = rel_w[iw[:, None] - iw[None, :] + w - 1]  # [w, w, hd]
    qg = q.view(nw, heads, h, w, hd)
    bias_h = torch.einsum("bnijc,ikc->bnijk", qg, rh)  # [.., h, w, kh]
    bias_w = torch.einsum("bnijc,jkc->bnijk", qg, rw)  # [.., h, w, kw]
    s = (q * hd ** -0.5) @ k.transpose(-1, -2).contiguous()
    s = s.view(nw, heads, h, w, h, w) + bias_h[..., :, None] + bias_w[..., None, :]
    a = torch.softmax(s.view(nw, heads, n, n), -1)
    o = (a @ v).permute(0, 2, 1, 3).reshape(nw, n, c)
    return (o @ p.proj_w.float().t()).view(nw, h, w, c)


def ref_forward(img, w, enc):
    cfg = w.cfg
    c, k, o = cfg.embed_dim, cfg.patch, cfg.out_chans
    wconv = w.patch_w.float().reshape(c, 3, k, k)
    # convolutions on the CPU: torch's own conv2d, independent of the GEMM forms the encoder uses
    x = F.conv2d(img.float().cpu(), wconv.cpu(), w.patch_b.float().cpu(), stride=k).cuda()
    x = x.permute(0, 2, 3, 1) + w.pos.float()
    for p in w.blocks:
        b, h, ww, _ = x.shape
        y = F.layer_norm(x, (c,), p.norm1_w.float(), p.norm1_b.float(), 1e-6)
        if p.window:
            parts, hp, wp = enc.window_partition(y, p.window)
            y = enc.window_unpartition(ref_attention(parts, p, cfg.heads), p.window, hp, wp, (h, ww), b, c)
        else:
            y = ref_attention(y, p, cfg.heads)
        x = x + y + p.proj_b.float()
        m = F.layer_norm(x, (c,), p.norm2_w.float(), p.norm2_b.float(), 1e-6)
        m = m @ p.lin1_w.float().t() + p.lin1_b.float()
        x = x + F.gelu(m) @ p.lin2_w.float().t() + p.lin2_b.float()
    x = x.permute(0, 3, 1, 2)
    y = F.conv2d(x.cpu(), w.neck0_w.float().reshape(o, c, 1, 1).cpu()).cuda()
    y = F.layer_norm(y.permute(0, 2, 3, 1), (o,), w.neck1_w.float(), w.neck1_b.float(), 1e-6).permute(0, 3, 1, 2)
    y = F.conv2d(y.cpu(), w.neck2_w.float().reshape(o, o, 3, 3).cpu(), padding=1).cuda()
    return F.layer_norm(y.permute(0, 2, 3, 1), (o,), w.neck3_w.float(), w.neck3_b.float(), 1e-6).permute(0, 3, 1, 2)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-4), (torch.float16, 2e-2), (torch.bfloat16, 6e-2)],
                         ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("dim", [160, 128], ids=["hd80", "hd64"])
def test_small_encoder_matches_torch_float32(enc, dim, dtype, tol):
    print(f"encoder dim {dim} {dtype}", flush=True)
    cfg = enc.EncoderConfig(dim, 2, 2, (1,))
    w = enc.random_weights(cfg, dtype=dtype, seed=3, std=0.05)
    g = torch.Generator(device="cuda").manual_seed(4)
    img = torch.randn(1, 3, 1024, 1024, generator=g, device="cuda").to(dtype)
    got = enc.encoder_forward(img, w).float()
    torch.cuda.synchronize()
    with torch.no_grad():
        want = ref_forward(img, w, enc)
    assert got.shape == (1, 256, 64, 64)
    err = ((got - want).abs().max() / want.abs().max()).item()
    assert np.isfinite(err) and err < tol, err


def test_window_partition_round_trip(enc):
    x = torch.randn(2, 64, 64, 8, device="cuda")
    parts, hp, wp = enc.window_partition(x, 14)
    assert parts.shape == (2 * 25, 14, 14, 8) and (hp, wp) == (70, 70)
    assert torch.equal(enc.window_unpartition(parts, 14, hp, wp, (64, 64), 2, 8), x)
    assert not parts.view(2, 5, 5, 14, 14, 8)[:, 4, :, 8:].any()  # rows 64..69 are the zero padding
