"""Python front end of libsam_hip.so, mirroring the reference's `src/kernels.rs` entry points.

Functions take and return torch tensors that live on a HIP device; outputs are allocated here (as
candle allocates them inside each op) and every launch is asynchronous on torch's current stream.
Names, argument meaning and errors follow the reference:

    relpos_softmax(scores, q, table, h, w, scale)        kernels.rs:12-43
    attention_relpos(q, kt, v, table, h, w, scale)       kernels.rs:899-906 (GPU: the fused kernel)
    qkv_split(y, bias, n, nh, hd)                        kernels.rs:872-894
    deform_attn(value, loc, attn, shapes)                kernels.rs:824-835
    flash_attn(q, k, v, scale=None)                      kernels.rs:910-915 / candle_flash_attn::flash_attn
    sdpa(q, k, v, mask=None)                             sam3/nn.rs:26-34

There is no CPU fallback: on a machine without the built library or a GPU every call raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsam_hip.so")
_lib = None

_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float


class SamHipError(RuntimeError):
    """An error reported by libsam_hip.so (the message is the library's own)."""


def load():
    """Load libsam_hip.so and declare the C ABI (include/sam_hip.h)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SamHipError(f"libsam_hip.so is not built ({LIB_PATH}); run python sam-rs_amd/build_lib.py")
        L = ctypes.CDLL(LIB_PATH)
        L.sam_hip_last_error.restype = ctypes.c_char_p
        L.sam_hip_abi_version.restype = _i
        L.sam_hip_attn_relpos.argtypes = [_vp] * 5 + [_i] * 5 + [_f, _vp]
        L.sam_hip_attn_relpos.restype = _i
        L.sam_hip_deform_attn.argtypes = [_vp] * 4 + [_i] * 8 + [ctypes.POINTER(ctypes.c_int), _vp]
        L.sam_hip_deform_attn.restype = _i
        L.sam_hip_relpos_softmax.argtypes = [_vp] * 4 + [_i, ctypes.c_long, _i, _i, _i, _f, _vp]
        L.sam_hip_relpos_softmax.restype = _i
        L.sam_hip_qkv_split.argtypes = [_vp] * 3 + [_i, ctypes.c_long, _i, _i, _i, _vp]
        L.sam_hip_qkv_split.restype = _i
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise SamHipError(load().sam_hip_last_error().decode())


def _stream():
    return _vp(torch.cuda.current_stream().cuda_stream)


def _dtype(*ts: torch.Tensor) -> int:
    dt = ts[0].dtype
    for t in ts:
        if t.dtype != dt:
            raise SamHipError(f"dtype mismatch: {t.dtype} vs {dt}")
    if dt not in _DTYPES:
        raise SamHipError(f"unsupported dtype {dt} for a sam-rs HIP kernel")
    return _DTYPES[dt]


def _contig(*ts: torch.Tensor):
    for t in ts:
        if not t.is_cuda:
            raise SamHipError("sam-rs HIP kernels need device tensors")
        if not t.is_contiguous():
            raise SamHipError("sam-rs kernels need contiguous inputs")  # kernels.rs:1100


def attention_relpos(q: torch.Tensor, kt: torch.Tensor, v: torch.Tensor, table: torch.Tensor, h: int, w: int,
                     scale: float) -> torch.Tensor:
    """softmax(scale * q k^T + relpos(q)) v in one kernel.

    q, v: [BH, h*w, hd]; kt: [BH, hd, h*w]; table: rel_pos_h rows followed by rel_pos_w rows,
    [(2h-1)+(2w-1), hd]. Returns [BH, h*w, hd] in the inputs' dtype.
    """
    _contig(q, kt, v, table)
    dt = _dtype(q, kt, v, table)
    bh, n, hd = q.shape
    if n != h * w or kt.shape != (bh, hd, n) or v.shape != (bh, n, hd) or table.shape != (2 * h - 1 + 2 * w - 1, hd):
        raise SamHipError(f"attention_relpos: inconsistent shapes q{tuple(q.shape)} kt{tuple(kt.shape)} "
                          f"v{tuple(v.shape)} table{tuple(table.shape)} for a {h}x{w} grid")
    out = torch.empty_like(q)
    _check(load().sam_hip_attn_relpos(q.data_ptr(), kt.data_ptr(), v.data_ptr(), table.data_ptr(), out.data_ptr(),
                                      dt, bh, h, w, hd, scale, _stream()))
    return out


def deform_attn(value: torch.Tensor, loc: torch.Tensor, attn: torch.Tensor, shapes) -> torch.Tensor:
    """Multi-scale deformable attention: value [B, S, H, D] (the levels' pixels concatenated),
    loc [B, Q, H, L, P, 2] sampling locations in [0, 1] as (x, y), attn [B, Q, H, L, P] weights ->
    [B, Q, H*D]. Bilinear sampling with zero padding, like grid_sample(align_corners=False).
    shapes: (height, width) of each of the (at most 4) levels. Inputs are made contiguous first, as
    the reference does (kernels.rs:825).
    """
    value, loc, attn = value.contiguous(), loc.contiguous(), attn.contiguous()
    _contig(value, loc, attn)
    dt = _dtype(value, loc, attn)
    b, s, h, d = value.shape
    if loc.dim() != 6 or loc.shape[0] != b or loc.shape[2] != h or loc.shape[5] != 2:
        raise SamHipError(f"deform_attn: loc must be [B, Q, H, L, P, 2], got {tuple(loc.shape)}")
    q, l, p = loc.shape[1], loc.shape[3], loc.shape[4]
    if attn.shape != (b, q, h, l, p):
        raise SamHipError(f"deform_attn: attn must be {(b, q, h, l, p)}, got {tuple(attn.shape)}")
    if len(shapes) != l:
        raise SamHipError(f"deform_attn: {len(shapes)} level shapes for {l} levels")
    flat = (ctypes.c_int * (2 * l))(*[int(x) for hw in shapes for x in hw])
    out = torch.empty((b, q, h * d), dtype=value.dtype, device=value.device)
    _check(load().sam_hip_deform_attn(value.data_ptr(), loc.data_ptr(), attn.data_ptr(), out.data_ptr(), dt, b, s, q,
                                      h, d, l, p, flat, _stream()))
    return out


def relpos_softmax(scores: torch.Tensor, q: torch.Tensor, table: torch.Tensor, h: int, w: int,
                   scale: float) -> torch.Tensor:
    """softmax_{kh,kw}(scale * scores[bh, i*w+j, kh*w+kw] + q.rel_h[i-kh+h-1] + q.rel_w[j-kw+w-1]).

    scores: [BH, h*w, h*w] raw q.k^T; q: [BH, h*w, hd]; table: rel_pos_h rows then rel_pos_w rows,
    [(2h-1)+(2w-1), hd]. Returns [BH, h*w, h*w].
    """
    _contig(scores, q, table)
    dt = _dtype(scores, q, table)
    bh, n, hd = q.shape
    if n != h * w or scores.shape != (bh, n, n) or table.shape != (2 * h - 1 + 2 * w - 1, hd):
        raise SamHipError(f"relpos_softmax: inconsistent shapes scores{tuple(scores.shape)} q{tuple(q.shape)} "
                          f"table{tuple(table.shape)} for a {h}x{w} grid")
    out = torch.empty_like(scores)
    _check(load().sam_hip_relpos_softmax(scores.data_ptr(), q.data_ptr(), table.data_ptr(), out.data_ptr(), dt,
                                         bh * n, h, w, hd, scale, _stream()))
    return out


def qkv_split(y: torch.Tensor, bias: torch.Tensor, n: int, nh: int, hd: int):
    """y: [T, 3*nh*hd] (bias-free qkv projection of T = windows * n tokens) + bias[3*nh*hd] ->
    (q [BH, n, hd], kT [BH, hd, n], v [BH, n, hd]) with BH = windows * nh, views of one packed buffer."""
    y = y.contiguous()
    _contig(y, bias)
    dt = _dtype(y, bias)
    t = y.shape[0]
    if y.shape != (t, 3 * nh * hd) or bias.shape != (3 * nh * hd,):
        raise SamHipError(f"qkv_split: y must be [T, {3 * nh * hd}] and bias [{3 * nh * hd}], "
                          f"got {tuple(y.shape)} and {tuple(bias.shape)}")
    bh = t // n * nh
    packed = torch.empty((3, t * nh * hd), dtype=y.dtype, device=y.device)
    _check(load().sam_hip_qkv_split(y.data_ptr(), bias.data_ptr(), packed.data_ptr(), dt, t, n, nh, hd, _stream()))
    return packed[0].view(bh, n, hd), packed[1].view(bh, hd, n), packed[2].view(bh, n, hd)
