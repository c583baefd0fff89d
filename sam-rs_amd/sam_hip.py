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
