"""SAM ViT image encoder forward on this library's kernels: the caller of the attention path.

Mirrors sam1::encoder::ImageEncoder (sam1/encoder.rs:1-200): patch embedding, absolute position
embedding, `depth` blocks (windowed 14x14 or global attention with decomposed rel-pos, MLP with exact
GELU) and the neck. Per block, the reference's kernel calls map to:
- window_partition + qkv_split (encoder.rs:129-137, kernels.rs:872) -> sam_hip.qkv_split_grid;
- attention_relpos / relpos_softmax + bmm (encoder.rs:79-82) -> sam_hip.attention_relpos (fused);
- the head merge and window_unpartition (encoder.rs:83, 140-143) -> sam_hip.window_merge;
- bias_residual (kernels.rs:1040) and the LayerNorm after it (the block's norm2, or the next
  block's norm1) -> sam_hip.bias_residual_ln, one pass; the last block's bias_residual ->
  sam_hip.bias_residual;
- bias_gelu (kernels.rs:1052) -> sam_hip.bias_gelu.

The linears run as torch's F.linear (hipBLASLt) and LayerNorm as torch's layer_norm. Their weights
are held as [out, in], the layout in which hipBLASLt runs these shapes fastest on gfx950 (10-25%
faster than [in, out] for the four ViT-H linears); a loader of the reference's weights, whose Linear
holds weight^T as [in, out] (encoder.rs:64), transposes each once. The two
convolutions are exact GEMMs: the 16x16 stride-16 patch embedding over non-overlapping patches, and
the neck's 3x3 conv as an unfold. The reference's window partition zero-pads the token grid to a
multiple of the window (encoder.rs:134-138): the padded tokens are real keys with no mask, whose
q/k/v equal the qkv bias. The linears act on each token alone, so here they run on the grid's tokens
and qkv_split_grid writes the padded windows' q/k/v (the bias for padding tokens), which is the
same. window_partition / window_unpartition below are the reference's steps, kept for the tests.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

import sam_hip


@dataclass(frozen=True)
class EncoderConfig:
    """encoder.rs:9-23."""
    embed_dim: int
    depth: int
    heads: int
    global_attn: tuple
    window: int = 14
    out_chans: int = 256
    img_size: int = 1024
    patch: int = 16


VIT_B = EncoderConfig(768, 12, 12, (2, 5, 8, 11))
VIT_L = EncoderConfig(1024, 24, 16, (5, 11, 17, 23))
VIT_H = EncoderConfig(1280, 32, 16, (7, 15, 23, 31))


@dataclass
class BlockWeights:
    norm1_w: torch.Tensor
    norm1_b: torch.Tensor
    qkv_w: torch.Tensor  # [3C, C], [out, in]
    qkv_b: torch.Tensor
    proj_w: torch.Tensor  # [C, C]
    proj_b: torch.Tensor
    rel: torch.Tensor  # rel_pos_h rows then rel_pos_w rows, [2 (2 input - 1), hd]
    norm2_w: torch.Tensor
    norm2_b: torch.Tensor
    lin1_w: torch.Tensor  # [4C, C]
    lin1_b: torch.Tensor
    lin2_w: torch.Tensor  # [C, 4C]
    lin2_b: torch.Tensor
    window: int  # 0 = global attention


@dataclass
class EncoderWeights:
    cfg: EncoderConfig
    patch_w: torch.Tensor  # [C, 3 * 16 * 16], columns in (channel, ky, kx) order of the conv weight
    patch_b: torch.Tensor
    pos: torch.Tensor  # [1, 64, 64, C]
    blocks: list = field(default_factory=list)
    neck0_w: torch.Tensor = None  # [out, C]
    neck1_w: torch.Tensor = None
    neck1_b: torch.Tensor = None
    neck2_w: torch.Tensor = None  # [out, out * 9], columns in (channel, ky, kx) order
    neck3_w: torch.Tensor = None
    neck3_b: torch.Tensor = None


def random_weights(cfg: EncoderConfig, dtype=torch.float16, device="cuda", seed: int = 0, std: float = 0.02):
    """Random-init weights of the architecture: N(0, std) for weights, tables and biases, LayerNorm
    weight 1 and bias 0."""
    g = torch.Generator(device=device).manual_seed(seed)
    c, hd = cfg.embed_dim, cfg.embed_dim // cfg.heads
    grid = cfg.img_size // cfg.patch

    def rn(*shape):
        return (std * torch.randn(*shape, generator=g, device=device, dtype=torch.float32)).to(dtype)

    def ones(n):
        return torch.ones(n, device=device, dtype=dtype)

    def zeros(n):
        return torch.zeros(n, device=device, dtype=dtype)

    w = EncoderWeights(cfg, rn(c, 3 * cfg.patch * cfg.patch), rn(c), rn(1, grid, grid, c))
    for i in range(cfg.depth):
        glob = i in cfg.global_attn
        inp = grid if glob else cfg.window
        w.blocks.append(BlockWeights(ones(c), zeros(c), rn(3 * c, c), rn(3 * c), rn(c, c), rn(c),
                                     rn(2 * (2 * inp - 1), hd), ones(c), zeros(c), rn(4 * c, c), rn(4 * c),
                                     rn(c, 4 * c), rn(c), 0 if glob else cfg.window))
    o = cfg.out_chans
    w.neck0_w, w.neck1_w, w.neck1_b = rn(o, c), ones(o), zeros(o)
    w.neck2_w, w.neck3_w, w.neck3_b = rn(o, o * 9), ones(o), zeros(o)
    return w


def window_partition(x: torch.Tensor, ws: int):
    """encoder.rs:129-137: [B, H, W, C] zero-padded to multiples of ws -> [B * nH * nW, ws, ws, C]."""
    b, h, w, c = x.shape
    ph, pw = (ws - h % ws) % ws, (ws - w % ws) % ws
    if ph or pw:
        x = F.pad(x, (0, 0, 0, pw, 0, ph))
    hp, wp = h + ph, w + pw
    x = x.view(b, hp // ws, ws, wp // ws, ws, c).permute(0, 1, 3, 2, 4, 5).reshape(-1, ws, ws, c)
    return x, hp, wp


def window_unpartition(x: torch.Tensor, ws: int, hp: int, wp: int, hw, b: int, c: int):
    """encoder.rs:140-143."""
    x = x.view(b, hp // ws, wp // ws, ws, ws, c).permute(0, 1, 3, 2, 4, 5).reshape(b, hp, wp, c)
    return x[:, : hw[0], : hw[1], :].contiguous()


def attention(x: torch.Tensor, p: BlockWeights, heads: int) -> torch.Tensor:
    """encoder.rs:73-85 with the window partition and unpartition of encoder.rs:129-143 around it:
    [B, H, W, C] -> the output projection without its bias, [B, H, W, C].

    The qkv and proj linears act on each token alone, so they run on the H*W grid tokens instead of
    the zero-padded windows: sam_hip.qkv_split_grid cuts the windows from the grid's projection (a
    padding token's q, k and v are the bias alone, as the padded zeros give), and
    sam_hip.window_merge puts the attention output back on the grid with the heads merged. A global
    block is one window of the whole grid."""
    b, h, w, c = x.shape
    ws = p.window if p.window > 0 else h
    wsw = p.window if p.window > 0 else w
    if ws != wsw:
        raise ValueError("square windows only")
    hd = c // heads
    y = F.linear(x.reshape(b * h * w, c), p.qkv_w)
    q, kt, v = sam_hip.qkv_split_grid(y, p.qkv_b, b, h, w, ws, heads, hd)
    ctx = sam_hip.attention_relpos(q, kt, v, p.rel, ws, ws, hd ** -0.5)
    out = sam_hip.window_merge(ctx, b, h, w, ws, heads).reshape(b * h * w, c)
    return F.linear(out, p.proj_w).view(b, h, w, c)


def block(x: torch.Tensor, xn: torch.Tensor, p: BlockWeights, heads: int, nxt: BlockWeights = None):
    """encoder.rs:112-126: x and xn = norm1(x) -> the block's output and, when a next block follows,
    its norm1 of that output (each residual and the norm after it run as one pass)."""
    b, h, w, c = x.shape
    y = attention(xn, p, heads)
    x, xn2 = sam_hip.bias_residual_ln(x, y, p.proj_b, p.norm2_w, p.norm2_b, 1e-6)
    t = b * h * w
    m = sam_hip.bias_gelu(F.linear(xn2.reshape(t, c), p.lin1_w), p.lin1_b)
    y = F.linear(m, p.lin2_w).view(b, h, w, c)
    if nxt is None:
        return sam_hip.bias_residual(x, y, p.lin2_b), None
    return sam_hip.bias_residual_ln(x, y, p.lin2_b, nxt.norm1_w, nxt.norm1_b, 1e-6)


def encoder_forward(img: torch.Tensor, w: EncoderWeights) -> torch.Tensor:
    """encoder.rs:181-190: [1, 3, S, S] (the preprocess output) -> [1, out_chans, S/16, S/16]."""
    cfg = w.cfg
    b, _, s, _ = img.shape
    g, k, c = s // cfg.patch, cfg.patch, cfg.embed_dim
    patches = img.view(b, 3, g, k, g, k).permute(0, 2, 4, 1, 3, 5).reshape(b * g * g, 3 * k * k)
    x = (F.linear(patches, w.patch_w) + w.patch_b).view(b, g, g, c) + w.pos
    xn = F.layer_norm(x, (c,), w.blocks[0].norm1_w, w.blocks[0].norm1_b, 1e-6)
    for i, p in enumerate(w.blocks):
        x, xn = block(x, xn, p, cfg.heads, w.blocks[i + 1] if i + 1 < len(w.blocks) else None)
    o = cfg.out_chans
    y = F.linear(x.reshape(b * g * g, c), w.neck0_w)  # 1x1 conv, tokens x out
    y = F.layer_norm(y, (o,), w.neck1_w, w.neck1_b, 1e-6)  # LayerNorm2d over channels
    cols = F.unfold(y.view(b, g, g, o).permute(0, 3, 1, 2), 3, padding=1)  # [b, o * 9, g * g]
    y = F.linear(cols.transpose(1, 2).reshape(b * g * g, o * 9), w.neck2_w)
    y = F.layer_norm(y, (o,), w.neck3_w, w.neck3_b, 1e-6)
    return y.view(b, g, g, o).permute(0, 3, 1, 2).contiguous()
