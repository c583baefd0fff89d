"""Python front end of libsam_hip.so, mirroring the reference's `src/kernels.rs` entry points.

Functions take and return torch tensors that live on a HIP device; outputs are allocated here (as
candle allocates them inside each op) and every launch is asynchronous on torch's current stream.
Names, argument meaning and errors follow the reference:

    relpos_softmax(scores, q, table, h, w, scale)        kernels.rs:12-43
    attention_relpos(q, kt, v, table, h, w, scale)       kernels.rs:899-906 (GPU: the fused kernel)
    qkv_split(y, bias, n, nh, hd)                        kernels.rs:872-894
    deform_attn(value, loc, attn, shapes)                kernels.rs:824-835
    deform_core(value, offsets, logits, refs, shapes)    dino/mod.rs:166-179 (Deform::forward's core)
    flash_attn(q, k, v, scale=None)                      kernels.rs:910-915 / candle_flash_attn::flash_attn
    sdpa(q, k, v, mask=None)                             sam3/nn.rs:26-34
    rope(x, cos, sin)                                    sam3/video.rs:106-113
    rope_attention(q, k, v, cos, sin, n_exclude)         sam3/video.rs:129-145 (after the projections)
    set_enabled(on), enabled()                           cpu_gemm.rs:11, 25-32 (the process-wide switch)

There is no CPU fallback: on a machine without the built library or a GPU every call raises. While the
switch is off every call raises SamHipDisabled without touching the device; the caller then takes its
own path, as the reference's callers do when cpu_gemm::enabled() is false.
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


class SamHipDisabled(SamHipError):
    """The HIP path is switched off (set_enabled(False) or SAM_HIP_DISABLE); nothing was done."""


_EDISABLED = 5  # SAM_HIP_EDISABLED


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
        L.sam_hip_deform_core.argtypes = [_vp] * 5 + [_i] * 9 + [ctypes.POINTER(ctypes.c_int), _vp]
        L.sam_hip_deform_core.restype = _i
        L.sam_hip_bias_residual.argtypes = [_vp] * 4 + [_i, ctypes.c_long, _i, _vp]
        L.sam_hip_bias_residual.restype = _i
        L.sam_hip_bias_gelu.argtypes = [_vp] * 3 + [_i, ctypes.c_long, _i, _vp]
        L.sam_hip_bias_gelu.restype = _i
        L.sam_hip_bias_residual_ln.argtypes = [_vp] * 7 + [_i, ctypes.c_long, _i, ctypes.c_float, _vp]
        L.sam_hip_bias_residual_ln.restype = _i
        _fp = ctypes.POINTER(ctypes.c_float)
        L.sam_hip_preprocess.argtypes = [_vp, _vp] + [_i] * 6 + [_fp, _fp, _vp]
        L.sam_hip_preprocess.restype = _i
        L.sam_hip_deform_attn.restype = _i
        L.sam_hip_relpos_softmax.argtypes = [_vp] * 4 + [_i, ctypes.c_long, _i, _i, _i, _f, _vp]
        L.sam_hip_relpos_softmax.restype = _i
        L.sam_hip_qkv_split.argtypes = [_vp] * 3 + [_i, ctypes.c_long, _i, _i, _i, _vp]
        L.sam_hip_qkv_split.restype = _i
        L.sam_hip_qkv_split_grid.argtypes = [_vp] * 3 + [_i] * 7 + [_vp]
        L.sam_hip_qkv_split_grid.restype = _i
        L.sam_hip_window_merge.argtypes = [_vp] * 2 + [_i] * 7 + [_vp]
        L.sam_hip_window_merge.restype = _i
        _lp = ctypes.POINTER(ctypes.c_long)
        L.sam_hip_flash_attn_workspace_size.argtypes = [_i] * 7
        L.sam_hip_flash_attn_workspace_size.restype = ctypes.c_long
        L.sam_hip_flash_attn.argtypes = [_vp] * 4 + [_i] * 6 + [_lp] * 4 + [_f, _vp, _vp, _i, _i, _i, _vp,
                                                                        ctypes.c_long, _vp]
        L.sam_hip_flash_attn.restype = _i
        L.sam_hip_flash_attn_noalloc.argtypes = [_vp] * 4 + [_i] * 6 + [_lp] * 4 + [_f, _vp, _vp, _i, _i, _i, _vp]
        L.sam_hip_flash_attn_noalloc.restype = _i
        L.sam_hip_rope.argtypes = [_vp] * 4 + [_i] * 5 + [_lp] * 2 + [_i, _i, _vp]
        L.sam_hip_rope.restype = _i
        L.sam_hip_qkv_rope.argtypes = [_vp] * 5 + [_i, ctypes.c_long, _i, _i, _i, _vp]
        L.sam_hip_qkv_rope.restype = _i
        L.sam_hip_sdpa_mask.argtypes = [_vp] * 5 + [_i] * 6 + [_lp] * 5 + [_f, _vp, ctypes.c_long, _vp]
        L.sam_hip_sdpa_mask.restype = _i
        L.sam_hip_set_enabled.argtypes = [_i]
        L.sam_hip_set_enabled.restype = None
        L.sam_hip_enabled.argtypes = []
        L.sam_hip_enabled.restype = _i
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        msg = load().sam_hip_last_error().decode()
        raise (SamHipDisabled if rc == _EDISABLED else SamHipError)(msg)


def set_enabled(on: bool) -> None:
    """Turn the HIP path on or off for the whole process (cpu_gemm::set_enabled, cpu_gemm.rs:25-28)."""
    load().sam_hip_set_enabled(1 if on else 0)


def enabled() -> bool:
    """Whether the HIP path is on (cpu_gemm::enabled, cpu_gemm.rs:30-32)."""
    return bool(load().sam_hip_enabled())


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


def _aligned16(*ts: torch.Tensor):
    """The tensors, with any that starts off a 16-byte boundary (a view with a storage offset) replaced by
    a copy: the kernels move 16-byte vectors, and a fresh allocation is always aligned. The reference's
    kernels take such views, so the copy keeps the call a drop-in instead of an error."""
    return tuple(t if t.data_ptr() % 16 == 0 else t.clone() for t in ts)


def _contig(*ts: torch.Tensor):
    for t in ts:
        if not t.is_cuda:
            raise SamHipError("sam-rs HIP kernels need device tensors")
        if t.device != ts[0].device:
            raise SamHipError(f"sam-rs HIP kernels need all operands on one device: {t.device} vs {ts[0].device}")
        if not t.is_contiguous():
            raise SamHipError("sam-rs kernels need contiguous inputs")  # kernels.rs:1100


def attention_relpos(q: torch.Tensor, kt: torch.Tensor, v: torch.Tensor, table: torch.Tensor, h: int, w: int,
                     scale: float) -> torch.Tensor:
    """softmax(scale * q k^T + relpos(q)) v in one kernel.

    q, v: [BH, h*w, hd]; kt: [BH, hd, h*w]; table: rel_pos_h rows followed by rel_pos_w rows,
    [(2h-1)+(2w-1), hd]. Returns [BH, h*w, hd] in the inputs' dtype.
    """
    q, kt, v, table = _aligned16(q, kt, v, table)
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
    value, loc, attn = _aligned16(value, loc, attn)
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


def deform_core(value: torch.Tensor, offsets: torch.Tensor, logits: torch.Tensor, refs: torch.Tensor,
                shapes) -> torch.Tensor:
    """Deform::forward between its projections (dino/mod.rs:166-179) in one kernel: logits
    [B, Q, H, L, P] softmaxed over the L*P points, sampling locations from offsets [B, Q, H, L, P, 2]
    and reference points refs [B, Q, L, 2] (encoder: ref + off / (W, H)) or [B, Q, L, 4] (decoder:
    xy + off / P * wh * 0.5), then the bilinear gather of value [B, S, H, D] -> [B, Q, H*D]."""
    value, offsets, logits, refs = (t.contiguous() for t in (value, offsets, logits, refs))
    value, offsets, logits, refs = _aligned16(value, offsets, logits, refs)
    _contig(value, offsets, logits, refs)
    dt = _dtype(value, offsets, logits, refs)
    b, s, h, d = value.shape
    if offsets.dim() != 6 or offsets.shape[0] != b or offsets.shape[2] != h or offsets.shape[5] != 2:
        raise SamHipError(f"deform_core: offsets must be [B, Q, H, L, P, 2], got {tuple(offsets.shape)}")
    q, l, p = offsets.shape[1], offsets.shape[3], offsets.shape[4]
    if logits.shape != (b, q, h, l, p):
        raise SamHipError(f"deform_core: logits must be {(b, q, h, l, p)}, got {tuple(logits.shape)}")
    if refs.dim() != 4 or refs.shape[:3] != (b, q, l) or refs.shape[3] not in (2, 4):
        raise SamHipError(f"deform_core: refs must be [B, Q, L, 2 or 4], got {tuple(refs.shape)}")
    if len(shapes) != l:
        raise SamHipError(f"deform_core: {len(shapes)} level shapes for {l} levels")
    flat = (ctypes.c_int * (2 * l))(*[int(x) for hw in shapes for x in hw])
    out = torch.empty((b, q, h * d), dtype=value.dtype, device=value.device)
    _check(load().sam_hip_deform_core(value.data_ptr(), offsets.data_ptr(), logits.data_ptr(), refs.data_ptr(),
                                      out.data_ptr(), dt, b, s, q, h, d, l, p, refs.shape[3], flat, _stream()))
    return out


def bias_residual(res: torch.Tensor, y: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """kernels::bias_residual (kernels.rs:1040-1049): res + y + bias, bias broadcast over the last
    dimension; res and y of one shape, made contiguous first as the reference does."""
    res, y, bias = res.contiguous(), y.contiguous(), bias.contiguous()
    _contig(res, y, bias)
    dt = _dtype(res, y, bias)
    if res.shape != y.shape:
        raise SamHipError(f"bias-residual: shape mismatch {tuple(res.shape)} vs {tuple(y.shape)}")
    if bias.dim() != 1 or res.shape[-1] != bias.shape[0]:
        raise SamHipError(f"bias-residual: bias {tuple(bias.shape)} does not match the last dimension of "
                          f"{tuple(res.shape)}")
    out = torch.empty_like(res)
    _check(load().sam_hip_bias_residual(res.data_ptr(), y.data_ptr(), bias.data_ptr(), out.data_ptr(), dt,
                                        res.numel(), bias.numel(), _stream()))
    return out


def bias_residual_ln(res: torch.Tensor, y: torch.Tensor, bias: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor,
                     eps: float = 1e-6):
    """bias_residual (kernels.rs:1040-1049) and then LayerNorm over the last dimension of its result
    (candle_nn::LayerNorm as the encoder block applies it after each residual, sam1/encoder.rs:118-124),
    in one pass: -> (x = res + y + bias, LayerNorm(x) * ln_w + ln_b), the norm taken over x as rounded
    to the dtype."""
    res, y, bias, ln_w, ln_b = (t.contiguous() for t in (res, y, bias, ln_w, ln_b))
    res, y, bias, ln_w, ln_b = _aligned16(res, y, bias, ln_w, ln_b)
    _contig(res, y, bias, ln_w, ln_b)
    dt = _dtype(res, y, bias, ln_w, ln_b)
    c = res.shape[-1]
    if res.shape != y.shape:
        raise SamHipError(f"bias-residual-ln: shape mismatch {tuple(res.shape)} vs {tuple(y.shape)}")
    if any(t.shape != (c,) for t in (bias, ln_w, ln_b)):
        raise SamHipError(f"bias-residual-ln: bias, ln_w and ln_b must be [{c}], got "
                          f"{[tuple(t.shape) for t in (bias, ln_w, ln_b)]}")
    out, ln = torch.empty_like(res), torch.empty_like(res)
    _check(load().sam_hip_bias_residual_ln(res.data_ptr(), y.data_ptr(), bias.data_ptr(), ln_w.data_ptr(),
                                           ln_b.data_ptr(), out.data_ptr(), ln.data_ptr(), dt, res.numel() // c, c,
                                           eps, _stream()))
    return out, ln


def bias_gelu(y: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """kernels::bias_gelu (kernels.rs:1051-1061): gelu_erf(y + bias), bias broadcast over the last
    dimension."""
    y, bias = y.contiguous(), bias.contiguous()
    _contig(y, bias)
    dt = _dtype(y, bias)
    if bias.dim() != 1 or y.shape[-1] != bias.shape[0]:
        raise SamHipError(f"bias-gelu: bias {tuple(bias.shape)} does not match the last dimension of "
                          f"{tuple(y.shape)}")
    out = torch.empty_like(y)
    _check(load().sam_hip_bias_gelu(y.data_ptr(), bias.data_ptr(), out.data_ptr(), dt, y.numel(), bias.numel(),
                                    _stream()))
    return out


IMG_SIZE = 1024  # image_proc.rs:6
SAM_MEAN = (123.675, 116.28, 103.53)  # image_proc.rs:7-8
SAM_STD = (58.395, 57.12, 57.375)


def preprocess(src: torch.Tensor, new_hw, size: int, mean=SAM_MEAN, std=SAM_STD,
               dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """kernels::preprocess (kernels.rs:1063-1070): src u8 [h, w, 3] on the device -> [1, 3, size, size]
    of `dtype`: antialiased resize to new_hw = (nh, nw), (x - mean) / std, zero padding."""
    if not src.is_cuda or src.dtype != torch.uint8 or src.dim() != 3 or src.shape[2] != 3:
        raise SamHipError(f"preprocess: src must be a u8 [h, w, 3] device tensor, got {src.dtype} "
                          f"{tuple(src.shape)}")
    _contig(src)
    if dtype not in _DTYPES:
        raise SamHipError(f"unsupported dtype {dtype} for a sam-rs HIP kernel")
    h, w, _ = src.shape
    nh, nw = (int(x) for x in new_hw)
    out = torch.empty((1, 3, size, size), dtype=dtype, device=src.device)
    m = (ctypes.c_float * 3)(*[float(x) for x in mean])
    sd = (ctypes.c_float * 3)(*[float(x) for x in std])
    _check(load().sam_hip_preprocess(src.data_ptr(), out.data_ptr(), _DTYPES[dtype], h, w, nh, nw, size, m, sd,
                                     _stream()))
    return out


def resized_hw(h: int, w: int, size: int = IMG_SIZE):
    """image_proc.rs:22-25: the longest side scaled to `size`, computed in f32, rounded half up."""
    import numpy as np

    f = np.float32
    scale = f(size) / f(max(w, h))
    nw = int(f(w) * scale + f(0.5))
    nh = int(f(h) * scale + f(0.5))
    return nh, nw, float(scale)


def prepare(src: torch.Tensor, size: int = IMG_SIZE, mean=SAM_MEAN, std=SAM_STD, dtype: torch.dtype = torch.float32):
    """image_proc::prepare (image_proc.rs:21-36) for an image already on the device: resize the longest
    side to `size`, normalise, pad. Returns (tensor [1, 3, size, size], orig (h, w), resized (nh, nw),
    scale)."""
    h, w = int(src.shape[0]), int(src.shape[1])
    nh, nw, scale = resized_hw(h, w, size)
    return preprocess(src, (nh, nw), size, mean, std, dtype), (h, w), (nh, nw), scale


def prepare_square(src: torch.Tensor, size: int, mean=SAM_MEAN, std=SAM_STD, dtype: torch.dtype = torch.float32):
    """image_proc::prepare_square (image_proc.rs:43-53): squash to size x size (no padding)."""
    return preprocess(src, (size, size), size, mean, std, dtype)


def relpos_softmax(scores: torch.Tensor, q: torch.Tensor, table: torch.Tensor, h: int, w: int,
                   scale: float) -> torch.Tensor:
    """softmax_{kh,kw}(scale * scores[bh, i*w+j, kh*w+kw] + q.rel_h[i-kh+h-1] + q.rel_w[j-kw+w-1]).

    scores: [BH, h*w, h*w] raw q.k^T; q: [BH, h*w, hd]; table: rel_pos_h rows then rel_pos_w rows,
    [(2h-1)+(2w-1), hd]. Returns [BH, h*w, h*w].
    """
    scores, q, table = _aligned16(scores, q, table)
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
    y, bias = _aligned16(y, bias)
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


def qkv_split_grid(y: torch.Tensor, bias: torch.Tensor, batch: int, gh: int, gw: int, ws: int, nh: int, hd: int):
    """y: [batch*gh*gw, 3*nh*hd] (bias-free qkv projection of the unpadded grid tokens) + bias ->
    (q [BH, ws*ws, hd], kT [BH, hd, ws*ws], v [BH, ws*ws, hd]) for the windows of the grid zero-padded to
    multiples of ws (padding tokens: the bias alone), BH = batch * ceil(gh/ws) * ceil(gw/ws) * nh."""
    y = y.contiguous()
    y, bias = _aligned16(y, bias)
    _contig(y, bias)
    dt = _dtype(y, bias)
    if y.shape != (batch * gh * gw, 3 * nh * hd) or bias.shape != (3 * nh * hd,):
        raise SamHipError(f"qkv_split_grid: y must be [{batch * gh * gw}, {3 * nh * hd}] and bias [{3 * nh * hd}], "
                          f"got {tuple(y.shape)} and {tuple(bias.shape)}")
    n = ws * ws
    bh = batch * (-(-gh // ws)) * (-(-gw // ws)) * nh
    packed = torch.empty((3, bh * n * hd), dtype=y.dtype, device=y.device)
    _check(load().sam_hip_qkv_split_grid(y.data_ptr(), bias.data_ptr(), packed.data_ptr(), dt, batch, gh, gw, ws, nh,
                                         hd, _stream()))
    return packed[0].view(bh, n, hd), packed[1].view(bh, hd, n), packed[2].view(bh, n, hd)


def window_merge(ctx: torch.Tensor, batch: int, gh: int, gw: int, ws: int, nh: int) -> torch.Tensor:
    """ctx [BH, ws*ws, hd] in qkv_split_grid's window order -> [batch, gh, gw, nh*hd] (heads merged,
    windows back on the grid without their padding)."""
    ctx = ctx.contiguous()
    ctx, = _aligned16(ctx)
    _contig(ctx)
    dt = _dtype(ctx)
    bh, n, hd = ctx.shape
    if n != ws * ws or bh != batch * (-(-gh // ws)) * (-(-gw // ws)) * nh:
        raise SamHipError(f"window_merge: ctx {tuple(ctx.shape)} does not hold the windows of a {gh}x{gw} grid")
    out = torch.empty((batch, gh, gw, nh * hd), dtype=ctx.dtype, device=ctx.device)
    _check(load().sam_hip_window_merge(ctx.data_ptr(), out.data_ptr(), dt, batch, gh, gw, ws, nh, hd, _stream()))
    return out


def _strides_blhd(t: torch.Tensor, layout: str):
    """(batch, row, head) element strides of a 4-d tensor in the [B, L, H, D] or [B, H, L, D] layout;
    the head dimension must be contiguous."""
    if t.stride(3) != 1:
        raise SamHipError("sam-rs kernels need contiguous inputs")  # kernels.rs:1100
    if layout == "blhd":
        s = (t.stride(0), t.stride(1), t.stride(2))
    else:
        s = (t.stride(0), t.stride(2), t.stride(1))
    return (ctypes.c_long * 3)(*s)


def _flash(q, k, v, out, layout: str, scale: float, cos=None, sin=None, n_rope_q: int = 0, n_rope_k: int = 0,
           noalloc: bool = False):
    # the kernel writes q.shape elements of q's dtype through out's pointer: anything else is refused
    if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise SamHipError(f"flash-attn: out must match q (shape {tuple(q.shape)}, {q.dtype}, {q.device}), got "
                          f"{tuple(out.shape)}, {out.dtype}, {out.device}")
    for t in (q, k, v, out):
        if not t.is_cuda:
            raise SamHipError("sam-rs HIP kernels need device tensors")
        if t.device != q.device:
            raise SamHipError(f"sam-rs HIP kernels need all operands on one device: {t.device} vs {q.device}")
    q, k, v = _aligned16(q, k, v)
    dt = _dtype(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise SamHipError(f"flash-attn: incompatible q/k/v shapes {tuple(q.shape)}/{tuple(k.shape)}/{tuple(v.shape)}")
    if layout == "blhd":
        b, lq, h, d = q.shape
        kb, lk, kh, kd = k.shape
    else:
        b, h, lq, d = q.shape
        kb, kh, lk, kd = k.shape
    if (kb, kh, kd) != (b, h, d):  # kernels.rs:425-427
        raise SamHipError(f"flash-attn: incompatible q/k/v shapes {tuple(q.shape)}/{tuple(k.shape)}/{tuple(v.shape)}")
    L = load()
    cs = cos.data_ptr() if cos is not None else None
    sn = sin.data_ptr() if sin is not None else None
    rows = cos.shape[0] if cos is not None else 0
    if noalloc:
        # the library's own workspace array: no device allocation for this call
        _check(L.sam_hip_flash_attn_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dt, b, lq, lk,
                                            h, d, _strides_blhd(q, layout), _strides_blhd(k, layout),
                                            _strides_blhd(v, layout), _strides_blhd(out, layout), scale, cs, sn, rows,
                                            n_rope_q, n_rope_k, _stream()))
        return out
    ws_bytes = L.sam_hip_flash_attn_workspace_size(dt, b, lq, lk, h, d, n_rope_k)
    if ws_bytes < 0:
        raise SamHipError(L.sam_hip_last_error().decode())
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    rc = L.sam_hip_flash_attn(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dt, b, lq, lk, h, d,
                              _strides_blhd(q, layout), _strides_blhd(k, layout), _strides_blhd(v, layout),
                              _strides_blhd(out, layout), scale, cs, sn, rows, n_rope_q, n_rope_k, ws.data_ptr(),
                              ws_bytes, _stream())
    _check(rc)
    return out


def flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None,
               out: torch.Tensor | None = None, noalloc: bool = False) -> torch.Tensor:
    """softmax(scale * q k^T) v without a mask on q [B, Lq, H, D], k/v [B, Lk, H, D] -> [B, Lq, H, D]
    (f16 / bf16), as candle_flash_attn::flash_attn(q, k, v, scale, false) and kernels::flash_attn_cpu
    compute it. scale defaults to D^-0.5, the value every reference caller passes. With noalloc the call
    goes through sam_hip_flash_attn_noalloc (the library's fixed workspace array; no allocation when
    `out` is given)."""
    d = q.shape[-1]
    scale = float(d) ** -0.5 if scale is None else float(scale)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    return _flash(q, k, v, out, "blhd", scale, noalloc=noalloc)


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask=None) -> torch.Tensor:
    """sam3::nn::sdpa on [B, H, L, D] tensors (sam3/nn.rs:26-34): softmax(q k^T * D^-0.5 + mask) v, with
    an optional additive mask that broadcasts to [B, H, Lq, Lk] and has q's dtype, as candle's
    broadcast_add needs. mask None goes through sam_hip_flash_attn, a mask through sam_hip_sdpa_mask."""
    d = q.shape[-1]
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    if mask is None:
        return _flash(q, k, v, out, "bhld", float(d) ** -0.5)
    for t in (q, k, v, mask):
        if not t.is_cuda:
            raise SamHipError("sam-rs HIP kernels need device tensors")
        if t.device != q.device:
            raise SamHipError(f"sam-rs HIP kernels need all operands on one device: {t.device} vs {q.device}")
    q, k, v = _aligned16(q, k, v)
    dt = _dtype(q, k, v)
    if mask.dtype != q.dtype:
        raise SamHipError(f"sdpa: the mask must have q's dtype {q.dtype}, got {mask.dtype}")
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise SamHipError(f"sdpa: incompatible q/k/v shapes {tuple(q.shape)}/{tuple(k.shape)}/{tuple(v.shape)}")
    b, h, lq, _ = q.shape
    lk = k.shape[2]
    if (k.shape[0], k.shape[1], k.shape[3]) != (b, h, d):
        raise SamHipError(f"sdpa: incompatible q/k/v shapes {tuple(q.shape)}/{tuple(k.shape)}/{tuple(v.shape)}")
    try:
        m4 = mask.expand(b, h, lq, lk)  # broadcast dimensions get stride 0
    except RuntimeError as e:
        raise SamHipError(f"sdpa: mask {tuple(mask.shape)} does not broadcast to {(b, h, lq, lk)}") from e
    L = load()
    ws_bytes = L.sam_hip_flash_attn_workspace_size(dt, b, lq, lk, h, d, 0)
    if ws_bytes < 0:
        raise SamHipError(L.sam_hip_last_error().decode())
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    sm = (ctypes.c_long * 4)(*m4.stride())
    rc = L.sam_hip_sdpa_mask(q.data_ptr(), k.data_ptr(), v.data_ptr(), m4.data_ptr(), out.data_ptr(), dt, b, lq, lk,
                             h, d, _strides_blhd(q, "bhld"), _strides_blhd(k, "bhld"), _strides_blhd(v, "bhld"), sm,
                             _strides_blhd(out, "bhld"), float(d) ** -0.5, ws.data_ptr(), ws_bytes, _stream())
    _check(rc)
    return out


def _rope_tables(cos: torch.Tensor, sin: torch.Tensor, d: int, device):
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != d:
        raise SamHipError(f"rope: tables must be [rows, {d}], got {tuple(cos.shape)} and {tuple(sin.shape)}")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise SamHipError("rope: the cos/sin tables are f32 (sam3/vision.rs:26-46)")
    if cos.device != device or sin.device != device:
        raise SamHipError("rope: the tables must be on the same device as x")
    return _aligned16(cos.contiguous(), sin.contiguous())


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_rot: int | None = None) -> torch.Tensor:
    """x * cos + rotate_pairwise(x) * sin in f32 over x [B, L, D] (or [B, L, H, D]), tables [T, D];
    row r uses table row r % T. Rows r >= n_rot (default: all rotated) are copied unchanged."""
    squeeze = x.dim() == 3
    x4 = x.unsqueeze(2) if squeeze else x
    if x4.dim() != 4:
        raise SamHipError(f"rope: x must be [B, L, D] or [B, L, H, D], got {tuple(x.shape)}")
    b, l, h, d = x4.shape
    cos, sin = _rope_tables(cos, sin, d, x.device)
    n_rot = l if n_rot is None else int(n_rot)
    dt = _dtype(x4)
    out = torch.empty((b, l, h, d), dtype=x.dtype, device=x.device)
    _check(load().sam_hip_rope(x4.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(), dt, b, l, h, d,
                               _strides_blhd(x4, "blhd"), None, cos.shape[0], n_rot, _stream()))
    return out.squeeze(2) if squeeze else out


def qkv_rope(y: torch.Tensor, bias: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n: int, heads: int,
             hd: int) -> torch.Tensor:
    """kernels::qkv_rope (kernels.rs:1013-1037): y [T, 3*heads*hd] (bias-free fused qkv projection) + bias,
    2-D RoPE on q and k with f32 tables [n, hd] (token t uses row t % n) -> packed [3, T, heads, hd]."""
    y = y.contiguous()
    y, bias = _aligned16(y, bias)
    _contig(y, bias)
    dt = _dtype(y, bias)
    t = y.shape[0]
    if y.dim() != 2 or y.shape[1] != 3 * heads * hd or bias.shape != (3 * heads * hd,):
        raise SamHipError(f"qkv_rope: y must be [T, {3 * heads * hd}] and bias [{3 * heads * hd}], "
                          f"got {tuple(y.shape)} and {tuple(bias.shape)}")
    cos, sin = _rope_tables(cos, sin, hd, y.device)
    if cos.shape[0] != n:
        raise SamHipError(f"qkv_rope: tables must have n = {n} rows, got {cos.shape[0]}")
    out = torch.empty((3, t, heads, hd), dtype=y.dtype, device=y.device)
    _check(load().sam_hip_qkv_rope(y.data_ptr(), bias.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(), dt,
                                   t, n, heads, hd, _stream()))
    return out


def rope_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                   n_exclude: int, noalloc: bool = False) -> torch.Tensor:
    """The attention core of RopeAttn::forward (sam3/video.rs:129-145) after the projections, one head:
    q [B, Lq, D] rotated with the tables, the first M - n_exclude keys of k [B, M, D] rotated with the
    tables tiled to their length, the last n_exclude (object pointers) not, then sdpa with v [B, M, D].
    Returns [B, Lq, D]."""
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape:
        raise SamHipError(f"rope_attention: q [B, Lq, D] and k, v [B, M, D], got {tuple(q.shape)}, "
                          f"{tuple(k.shape)}, {tuple(v.shape)}")
    b, lq, d = q.shape
    m = k.shape[1]
    cos, sin = _rope_tables(cos, sin, d, q.device)
    rot = m - n_exclude
    if n_exclude < 0 or rot < 0 or rot % cos.shape[0] != 0:
        raise SamHipError(f"rope_attention: {rot} rotated keys is not a whole number of {cos.shape[0]}-row tables")
    if lq > cos.shape[0]:
        raise SamHipError(f"rope_attention: {lq} queries but the tables have {cos.shape[0]} rows")
    out = torch.empty((b, lq, d), dtype=q.dtype, device=q.device)
    _flash(q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2), out.unsqueeze(2), "blhd", float(d) ** -0.5, cos, sin,
           lq, rot, noalloc=noalloc)
    return out
