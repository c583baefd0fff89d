"""Independent float64 formulations used to pin the oracle and to write the golden fixtures.

Each function states the mathematics in a form that does NOT share code or index arithmetic with the
oracle's restatement of the reference:

* rel-pos attention follows the textbook decomposed relative-position form of the SAM ViT
  (``Rh = rel_pos_h[q_coord - k_coord + (k_size - 1)]``, einsum over channels, bias broadcast over the
  other key axis), evaluated by brute force in float64;
* the alternative index form of the reference's tensor fallback (kernels.rs:20-42) is kept as a second
  formulation so the two can be compared exactly;
* deformable attention is the scalar ``grid_sample(align_corners=False, padding_mode="zeros")`` loop of
  the reference's own test (tests/dino.rs:9-40) and, separately, torch's ``grid_sample``;
* the deformable-attention module's sampling locations and weights (Deform::forward) follow the
  Deformable-DETR formulation with torch broadcasting (offset normaliser stacked as (W, H), box refs as
  ``xy + off / P * wh * 0.5``), in float64;
* attention without bias uses torch's ``scaled_dot_product_attention`` in float64;
* RoPE uses the complex-number (polar) formulation of 2-D axial rotary embeddings.
"""
from __future__ import annotations

import numpy as np


def softmax64(x: np.ndarray, axis: int = -1) -> np.ndarray:
    x = np.asarray(x, np.float64)
    m = x.max(axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def _get_rel_pos(q_size: int, k_size: int, rel_pos: np.ndarray) -> np.ndarray:
    q_coords = np.arange(q_size)[:, None]
    k_coords = np.arange(k_size)[None, :]
    rel = (q_coords - k_coords) + (k_size - 1)
    return rel_pos[rel]  # [q_size, k_size, C]


def relpos_logits64(s_raw: np.ndarray, q: np.ndarray, table: np.ndarray, h: int, w: int, scale: float) -> np.ndarray:
    """Textbook decomposed rel-pos logits: scale * s + rel_h[..., kh, None] + rel_w[..., None, kw]."""
    s_raw = np.asarray(s_raw, np.float64)
    q = np.asarray(q, np.float64)
    table = np.asarray(table, np.float64)
    bh, n, hd = q.shape
    rel_pos_h, rel_pos_w = table[: 2 * h - 1], table[2 * h - 1:]
    Rh = _get_rel_pos(h, h, rel_pos_h)
    Rw = _get_rel_pos(w, w, rel_pos_w)
    r_q = q.reshape(bh, h, w, hd)
    rel_h = np.einsum("bhwc,hkc->bhwk", r_q, Rh)
    rel_w = np.einsum("bhwc,wkc->bhwk", r_q, Rw)
    a = (scale * s_raw).reshape(bh, h, w, h, w) + rel_h[:, :, :, :, None] + rel_w[:, :, :, None, :]
    return a.reshape(bh, n, n)


def relpos_softmax64(s_raw, q, table, h, w, scale) -> np.ndarray:
    return softmax64(relpos_logits64(s_raw, q, table, h, w, scale))


def attention_relpos64(q, kt, v, table, h, w, scale) -> np.ndarray:
    """softmax(scale * q k^T + relpos(q)) v in float64; kt is [BH, hd, N] as the reference passes it."""
    q64 = np.asarray(q, np.float64)
    s = q64 @ np.asarray(kt, np.float64)
    p = relpos_softmax64(s, q64, table, h, w, scale)
    return p @ np.asarray(v, np.float64)


def relpos_logits_fallback_index64(s_raw, q, table, h, w, scale) -> np.ndarray:
    """Second formulation: the reference's tensor fallback index form (kernels.rs:20-42),
    idx[qi*size + ki] = qi + size - 1 - ki, gathered tables, batched matmuls and permutes."""
    s_raw = np.asarray(s_raw, np.float64)
    q = np.asarray(q, np.float64)
    table = np.asarray(table, np.float64)
    bh, n, hd = q.shape

    def idx(size):
        return np.array([qi + size - 1 - ki for qi in range(size) for ki in range(size)], np.int64)

    th, tw = table[: 2 * h - 1], table[2 * h - 1: 2 * h - 1 + 2 * w - 1]
    rh = th[idx(h)].reshape(h, h, hd)
    rw = tw[idx(w)].reshape(w, w, hd)
    rq = q.reshape(bh, h, w, hd)
    rel_h = (rq.transpose(1, 0, 2, 3).reshape(h, bh * w, hd) @ rh.transpose(0, 2, 1)).reshape(h, bh, w, h)
    rel_h = rel_h.transpose(1, 0, 2, 3)
    rel_w = (rq.transpose(2, 0, 1, 3).reshape(w, bh * h, hd) @ rw.transpose(0, 2, 1)).reshape(w, bh, h, w)
    rel_w = rel_w.transpose(1, 2, 0, 3)
    a = (scale * s_raw).reshape(bh, h, w, h, w) + rel_h[..., None] + rel_w[:, :, :, None, :]
    return a.reshape(bh, n, n)


def deform_naive64(value, loc, attn, shapes) -> np.ndarray:
    """Scalar grid_sample(align_corners=False, zeros) loop (tests/dino.rs:9-40), float64, any batch."""
    value = np.asarray(value, np.float64)
    loc = np.asarray(loc, np.float64)
    attn = np.asarray(attn, np.float64)
    b, s, h, d = value.shape
    q = loc.shape[1]
    p = loc.shape[4]
    out = np.zeros((b, q, h, d))
    for bi in range(b):
        for qi in range(q):
            for hi in range(h):
                start = 0
                for li, (hl, wl) in enumerate(shapes):
                    for pi in range(p):
                        x = loc[bi, qi, hi, li, pi, 0] * wl - 0.5
                        y = loc[bi, qi, hi, li, pi, 1] * hl - 0.5
                        x0, y0 = int(np.floor(x)), int(np.floor(y))
                        fx, fy = x - x0, y - y0

                        def at(yy, xx):
                            if yy < 0 or xx < 0 or yy >= hl or xx >= wl:
                                return np.zeros(d)
                            return value[bi, start + yy * wl + xx, hi]

                        val = (at(y0, x0) * (1 - fx) * (1 - fy) + at(y0, x0 + 1) * fx * (1 - fy)
                               + at(y0 + 1, x0) * (1 - fx) * fy + at(y0 + 1, x0 + 1) * fx * fy)
                        out[bi, qi, hi] += attn[bi, qi, hi, li, pi] * val
                    start += hl * wl
    return out.reshape(b, q, h * d)


def deform_grid_sample64(value, loc, attn, shapes) -> np.ndarray:
    """The same operator through torch.nn.functional.grid_sample (float64): the multi-scale deformable
    attention core with sampling grid 2*loc - 1, align_corners=False, zero padding."""
    import torch
    import torch.nn.functional as F

    value = torch.as_tensor(np.asarray(value, np.float64))
    loc = torch.as_tensor(np.asarray(loc, np.float64))
    attn = torch.as_tensor(np.asarray(attn, np.float64))
    b, s, h, d = value.shape
    q, l, p = loc.shape[1], loc.shape[3], loc.shape[4]
    splits = value.split([hh * ww for hh, ww in shapes], dim=1)
    grids = 2 * loc - 1
    samples = []
    for li, (hh, ww) in enumerate(shapes):
        v_l = splits[li].flatten(2).transpose(1, 2).reshape(b * h, d, hh, ww)
        g_l = grids[:, :, :, li].transpose(1, 2).flatten(0, 1)  # [b*h, q, p, 2]
        samples.append(F.grid_sample(v_l, g_l, mode="bilinear", padding_mode="zeros", align_corners=False))
    a = attn.transpose(1, 2).reshape(b * h, 1, q, l * p)
    out = (torch.stack(samples, dim=-2).flatten(-2) * a).sum(-1).view(b, h * d, q)
    return out.transpose(1, 2).contiguous().numpy()


def deform_prep64(off, logits, refs, shapes):
    """Sampling locations and attention weights of a multi-scale deformable attention module, float64:
    weights = softmax over the L*P points; 2-coordinate refs: ref + off / (W_l, H_l); 4-coordinate
    (box) refs: xy + off / P * wh * 0.5. off [B,Q,H,L,P,2], logits [B,Q,H,L,P], refs [B,Q,L,2|4]."""
    import torch

    off = torch.as_tensor(np.asarray(off, np.float64))
    logits = torch.as_tensor(np.asarray(logits, np.float64))
    refs = torch.as_tensor(np.asarray(refs, np.float64))
    b, q, h, l, p, _ = off.shape
    attn = torch.softmax(logits.reshape(b, q, h, l * p), -1).reshape(b, q, h, l, p)
    shp = torch.as_tensor(np.asarray(shapes, np.float64))  # (H_l, W_l)
    if refs.shape[-1] == 2:
        norm = torch.stack([shp[:, 1], shp[:, 0]], -1)  # (W_l, H_l)
        loc = refs[:, :, None, :, None, :] + off / norm[None, None, None, :, None, :]
    else:
        loc = refs[:, :, None, :, None, :2] + off / p * refs[:, :, None, :, None, 2:] * 0.5
    return loc.numpy(), attn.numpy()


def sdpa64(q, k, v, scale: float | None = None, attn_mask=None) -> np.ndarray:
    """torch scaled_dot_product_attention in float64 on [..., L, D] tensors; a float attn_mask is added to
    the scaled scores."""
    import torch
    import torch.nn.functional as F

    qt = torch.as_tensor(np.asarray(q, np.float64))
    kt = torch.as_tensor(np.asarray(k, np.float64))
    vt = torch.as_tensor(np.asarray(v, np.float64))
    mt = None if attn_mask is None else torch.as_tensor(np.asarray(attn_mask, np.float64))
    return F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mt, scale=scale).numpy()


def axial_rope_cis64(side: int, hd: int, theta: float) -> np.ndarray:
    """Complex rotation factors for 2-D axial RoPE [side*side, hd/2]: the first hd/4 follow the
    column (x), the next hd/4 the row (y), frequency theta^(-4i/hd)."""
    t = np.arange(side * side)
    tx = (t % side).astype(np.float64)
    ty = (t // side).astype(np.float64)
    freqs = 1.0 / theta ** (np.arange(0, hd, 4)[: hd // 4].astype(np.float64) / hd)
    cx = np.exp(1j * np.outer(tx, freqs))
    cy = np.exp(1j * np.outer(ty, freqs))
    return np.concatenate([cx, cy], axis=-1)


def rope_complex64(x, cis) -> np.ndarray:
    """Rotate interleaved pairs (x0 + i x1) by cis: x [L, D], cis [L, D/2]."""
    x = np.asarray(x, np.float64)
    z = x[:, 0::2] + 1j * x[:, 1::2]
    r = z * cis
    out = np.empty_like(x)
    out[:, 0::2] = r.real
    out[:, 1::2] = r.imag
    return out
