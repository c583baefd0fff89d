"""Grounding DINO's multi-scale deformable attention module on this library's kernels: the caller
Deform::forward (dino/mod.rs:137-182) and the encoder's reference points (dino/mod.rs:660-678).

The four projections (sampling_offsets, attention_weights, value_proj, output_proj) are torch linears
(hipBLASLt), as candle_nn::Linear computes them (x @ W^T + b). Everything between them, the softmax of
the attention logits over a head's L*P points, the sampling locations and the bilinear gather, is one
sam_hip_deform_core launch. There is no CPU fallback.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

import sam_hip


def encoder_reference_points(shapes, device="cuda", dtype=torch.float32) -> torch.Tensor:
    """Every position's centre ((x + 0.5) / W, (y + 0.5) / H), level by level in row-major order,
    repeated for each level: [N, L, 2] (dino/mod.rs:660-678; valid ratios are 1)."""
    pts = []
    for h, w in shapes:
        ys, xs = torch.meshgrid(torch.arange(h, dtype=torch.float32), torch.arange(w, dtype=torch.float32),
                                indexing="ij")
        pts.append(torch.stack([(xs.reshape(-1) + 0.5) / w, (ys.reshape(-1) + 0.5) / h], -1))
    p = torch.cat(pts, 0)
    return p[:, None, :].expand(p.shape[0], len(shapes), 2).contiguous().to(device=device, dtype=dtype)


class Deform:
    """dino::Deform (dino/mod.rs:137-158): weights as candle_nn::Linear holds them, W [out, in] and
    b [out]: sampling_offsets (C -> heads*levels*points*2), attention_weights (C ->
    heads*levels*points), value_proj and output_proj (C -> C)."""

    def __init__(self, offsets, weights, value, out, heads: int, levels: int, points: int):
        self.offsets, self.weights, self.value, self.out = offsets, weights, value, out
        self.heads, self.levels, self.points = heads, levels, points

    @staticmethod
    def random(c: int, heads: int, levels: int, points: int, std: float = 0.02, device="cuda",
               dtype=torch.float32, generator=None) -> "Deform":
        """Random-init N(0, std) weights and biases of the module's shapes."""
        def lin(o, i):
            w = std * torch.randn(o, i, device=device, generator=generator)
            b = std * torch.randn(o, device=device, generator=generator)
            return w.to(dtype), b.to(dtype)

        return Deform(lin(heads * levels * points * 2, c), lin(heads * levels * points, c), lin(c, c), lin(c, c),
                      heads, levels, points)

    def forward(self, query: torch.Tensor, value_in: torch.Tensor, refs: torch.Tensor, shapes) -> torch.Tensor:
        """query [Q, C] (position embedding already added), value_in [S, C], refs [Q, L, 2 or 4] ->
        [Q, C] (dino/mod.rs:161-181)."""
        q, c = query.shape
        s = value_in.shape[0]
        h, l, p = self.heads, self.levels, self.points
        value = F.linear(value_in, *self.value).reshape(1, s, h, c // h)
        off = F.linear(query, *self.offsets).reshape(1, q, h, l, p, 2)
        logits = F.linear(query, *self.weights).reshape(1, q, h, l, p)
        if refs.dim() != 3 or refs.shape[:2] != (q, l) or refs.shape[2] not in (2, 4):
            raise sam_hip.SamHipError(f"Deform: refs must be [Q, L, 2 or 4], got {tuple(refs.shape)}")
        o = sam_hip.deform_core(value, off, logits, refs.reshape(1, q, l, refs.shape[2]), shapes).reshape(q, c)
        return F.linear(o, *self.out)
