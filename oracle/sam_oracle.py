"""ctypes front end of the CPU oracle (liboracle.so).

Test infrastructure only: the test suite, the smoke check and the CPU-baseline leg of the benchmark
use it as the checker. The product (libsam_hip.so and sam_hip.py) never imports it.

Every function takes and returns contiguous float32 numpy arrays and cites the reference lines its C
implementation restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_relpos_softmax.argtypes = [_F, _F, _F, _F, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_float, ctypes.c_int]
        L.oracle_attention_relpos.argtypes = [_F, _F, _F, _F, _F, ctypes.c_long, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.oracle_qkv_split.argtypes = [_F, _F, _F, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int]
        L.oracle_qkv_rope.argtypes = [_F] * 5 + [ctypes.c_long] + [ctypes.c_int] * 4
        L.oracle_deform_attn.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 7 + [_I, ctypes.c_int]
        L.oracle_deform_prep.argtypes = [_F] * 5 + [ctypes.c_int] * 6 + [_I, ctypes.c_int, ctypes.c_int]
        L.oracle_sdpa.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 6
        L.oracle_sdpa_mask.argtypes = [_F, _F, _F, _F, ctypes.POINTER(ctypes.c_long), _F] + [ctypes.c_int] * 6
        L.oracle_mha_blhd.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int]
        L.oracle_rope_tables.argtypes = [ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_float, _F, _F]
        L.oracle_rope.argtypes = [_F, _F, _F, _F, ctypes.c_long, ctypes.c_int]
        L.oracle_rope_attention.argtypes = [_F, _F, _F, _F, _F, ctypes.c_int, _F] + [ctypes.c_int] * 5
        L.oracle_preprocess.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 5 + [_F, _F, _F, ctypes.c_int]
        L.oracle_bias_residual.argtypes = [_F, _F, _F, _F, ctypes.c_long, ctypes.c_int]
        L.oracle_bias_gelu.argtypes = [_F, _F, _F, ctypes.c_long, ctypes.c_int]
        L.oracle_bf16_available.restype = ctypes.c_int
        _U16 = ctypes.POINTER(ctypes.c_uint16)
        L.oracle_bf16_round.argtypes = [_F, _U16, ctypes.c_long]
        L.oracle_bf16_exp.argtypes = [_F, _F, ctypes.c_long]
        L.oracle_bf16_matmul.argtypes = [_F, _F, _F] + [ctypes.c_int] * 4
        L.oracle_bf16_attention_relpos.argtypes = [_F] * 5 + [ctypes.c_long] + [ctypes.c_int] * 3 + [ctypes.c_float,
                                                                                                   ctypes.c_int]
        L.oracle_bf16_flash_attention.argtypes = [_F] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int]
        L.oracle_round_f16.argtypes = [_F, ctypes.c_long]
        L.oracle_round_bf16.argtypes = [_F, ctypes.c_long]
        L.oracle_randn.argtypes = [ctypes.c_ulonglong, _F, ctypes.c_long, ctypes.c_float, ctypes.c_float]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_F)


def relpos_softmax(s, q, table, h: int, w: int, scale: float, nthreads: int = 0) -> np.ndarray:
    """kernels.rs:62-105. s [BH, N, N], q [BH, N, hd], table [(2h-1)+(2w-1), hd] -> [BH, N, N]."""
    s, q, table = _f32(s), _f32(q), _f32(table)
    bh, n, hd = q.shape
    assert n == h * w and s.shape == (bh, n, n) and table.shape == (2 * h - 1 + 2 * w - 1, hd)
    out = np.empty_like(s)
    lib().oracle_relpos_softmax(_p(s), _p(q), _p(table), _p(out), bh, h, w, hd, scale, nthreads)
    return out


def attention_relpos(q, kt, v, table, h: int, w: int, scale: float, nthreads: int = 0) -> np.ndarray:
    """kernels.rs:181-220 (exact f32 TiledAttention). q [BH,N,hd], kt [BH,hd,N], v [BH,N,hd] -> [BH,N,hd]."""
    q, kt, v, table = _f32(q), _f32(kt), _f32(v), _f32(table)
    bh, n, hd = q.shape
    assert n == h * w and kt.shape == (bh, hd, n) and v.shape == (bh, n, hd)
    assert table.shape == (2 * h - 1 + 2 * w - 1, hd)
    out = np.empty_like(q)
    lib().oracle_attention_relpos(_p(q), _p(kt), _p(v), _p(table), _p(out), bh, h, w, hd, scale, nthreads)
    return out


def qkv_split(y, bias, n: int, nh: int, hd: int, nthreads: int = 0):
    """kernels.rs:239-263. y [T, 3*nh*hd], bias [3*nh*hd] -> (q [BH,n,hd], kT [BH,hd,n], v [BH,n,hd])."""
    y, bias = _f32(y), _f32(bias)
    t = y.shape[0]
    assert y.shape == (t, 3 * nh * hd) and bias.shape == (3 * nh * hd,) and t % n == 0
    out = np.empty((3, t * nh * hd), np.float32)
    lib().oracle_qkv_split(_p(y), _p(bias), _p(out), t, n, nh, hd, nthreads)
    bh = t // n * nh
    return out[0].reshape(bh, n, hd), out[1].reshape(bh, hd, n), out[2].reshape(bh, n, hd)


def qkv_rope(y, bias, cos, sin, n: int, nh: int, hd: int, dtype: str = "f32", nthreads: int = 0) -> np.ndarray:
    """kernels.rs:321-362 (and the GPU op sam.cu:210-235). y [T, 3*nh*hd] and bias [3*nh*hd] holding
    values of `dtype`, cos/sin f32 [n, hd] -> packed [3, T, nh, hd]: the f32 result of the reference's
    arithmetic, converted to `dtype` once at the end as the GPU op stores it."""
    y, bias, cos, sin = _f32(y), _f32(bias), _f32(cos), _f32(sin)
    t = y.shape[0]
    assert y.shape == (t, 3 * nh * hd) and bias.shape == (3 * nh * hd,) and hd % 2 == 0
    assert cos.shape == (n, hd) and sin.shape == (n, hd)
    out = np.empty((3, t, nh, hd), np.float32)
    lib().oracle_qkv_rope(_p(y), _p(bias), _p(cos), _p(sin), _p(out), t, n, nh, hd, nthreads)
    return out if dtype == "f32" else round_to(out, dtype)


def deform_attn(value, loc, attn, shapes, nthreads: int = 0) -> np.ndarray:
    """kernels.rs:776-818. value [B,S,H,D], loc [B,Q,H,L,P,2], attn [B,Q,H,L,P] -> [B,Q,H*D]."""
    value, loc, attn = _f32(value), _f32(loc), _f32(attn)
    b, s, h, d = value.shape
    q, l, p = loc.shape[1], loc.shape[3], loc.shape[4]
    assert loc.shape == (b, q, h, l, p, 2) and attn.shape == (b, q, h, l, p) and len(shapes) == l
    assert sum(hh * ww for hh, ww in shapes) == s
    sh = np.ascontiguousarray(np.array(shapes, np.int32).reshape(-1))
    out = np.empty((b, q, h * d), np.float32)
    lib().oracle_deform_attn(_p(value), _p(loc), _p(attn), _p(out), b, s, q, h, d, l, p, sh.ctypes.data_as(_I),
                             nthreads)
    return out


_ROUND_DT = {"f32": 0, "f16": 1, "bf16": 2}


def deform_prep(off, logits, refs, shapes, nthreads: int = 0, dtype: str = "f32"):
    """dino/mod.rs:166-178. off [B,Q,H,L,P,2], logits [B,Q,H,L,P], refs [B,Q,L,2|4] -> (loc, attn).
    dtype "f16" / "bf16": the candle ops run in that dtype, so every step's result (and the softmax
    output) is rounded to it, as the reference computes them for a query of that dtype."""
    off, logits, refs = _f32(off), _f32(logits), _f32(refs)
    b, q, h, l, p, two = off.shape
    nc = refs.shape[-1]
    assert two == 2 and logits.shape == (b, q, h, l, p) and refs.shape == (b, q, l, nc) and nc in (2, 4)
    assert len(shapes) == l
    sh = np.ascontiguousarray(np.array(shapes, np.int32).reshape(-1))
    loc = np.empty_like(off)
    attn = np.empty_like(logits)
    lib().oracle_deform_prep(_p(off), _p(logits), _p(refs), _p(loc), _p(attn), b, q, h, l, p, nc,
                             sh.ctypes.data_as(_I), _ROUND_DT[dtype], nthreads)
    return loc, attn


def deform_forward_core(value, off, logits, refs, shapes, nthreads: int = 0, dtype: str = "f32") -> np.ndarray:
    """Deform::forward between its projections (dino/mod.rs:166-179): deform_prep (its steps rounded to
    `dtype`), then deform_attn (which reads loc and attn as the dtype's values and computes in f32)."""
    loc, attn = deform_prep(off, logits, refs, shapes, nthreads, dtype)
    return deform_attn(value, loc, attn, shapes, nthreads)


def bf16_available() -> bool:
    """Whether this CPU has AVX-512F and AVX-512 BF16, the condition for the reference's bf16 CPU path
    (cpu_gemm.rs:14-32)."""
    return bool(lib().oracle_bf16_available())


def _need_bf16():
    if not bf16_available():
        raise RuntimeError("the bf16 CPU path needs AVX-512 BF16 (cpu_gemm.rs:14-24)")


def bf16_bits(x) -> np.ndarray:
    """cpu_gemm.rs:38-45: f32 -> bf16 bits (round to nearest even)."""
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_bf16_round(_p(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return out


def bf16_exp(x) -> np.ndarray:
    """cpu_gemm.rs:272-286 (exp_ps) elementwise."""
    _need_bf16()
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_bf16_exp(_p(x), _p(y), x.size)
    return y


def bf16_matmul(x, w, nthreads: int = 0) -> np.ndarray:
    """cpu_gemm.rs:100-178: x [M, K] @ w [K, N] with bf16 operands and f32 accumulation (vdpbf16ps)."""
    _need_bf16()
    x, w = _f32(x), _f32(w)
    m, k = x.shape
    k2, n = w.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().oracle_bf16_matmul(_p(x), _p(w), _p(c), m, k, n, nthreads)
    return c


def bf16_attention_relpos(q, kt, v, table, h: int, w: int, scale: float, nthreads: int = 0) -> np.ndarray:
    """kernels.rs:139-179 (TiledAttention, bf16 branch): the reference's default CPU attention."""
    _need_bf16()
    q, kt, v, table = _f32(q), _f32(kt), _f32(v), _f32(table)
    bh, n, hd = q.shape
    assert n == h * w and kt.shape == (bh, hd, n) and v.shape == (bh, n, hd)
    out = np.empty_like(q)
    lib().oracle_bf16_attention_relpos(_p(q), _p(kt), _p(v), _p(table), _p(out), bh, h, w, hd, scale, nthreads)
    return out


def bf16_flash_attention(q, k, v, scale: float | None = None, nthreads: int = 0) -> np.ndarray:
    """cpu_gemm.rs:361-417: q [B, Lq, H, D], k/v [B, Lk, H, D] -> [B, Lq, H, D] on the bf16 kernels."""
    _need_bf16()
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, lq, h, d = q.shape
    lk = k.shape[1]
    assert k.shape == (b, lk, h, d) and v.shape == k.shape
    scale = d ** -0.5 if scale is None else scale
    out = np.empty_like(q)
    lib().oracle_bf16_flash_attention(_p(q), _p(k), _p(v), _p(out), b, lq, lk, h, d, scale, nthreads)
    return out


def sdpa(q, k, v, mask=None, nthreads: int = 0) -> np.ndarray:
    """sam3/nn.rs:26-34. q [B,H,Lq,D], k/v [B,H,Lk,D] -> [B,H,Lq,D]; mask None, or an additive mask that
    broadcasts to [B,H,Lq,Lk]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, h, lq, d = q.shape
    lk = k.shape[2]
    assert k.shape == (b, h, lk, d) and v.shape == k.shape
    out = np.empty_like(q)
    if mask is None:
        lib().oracle_sdpa(_p(q), _p(k), _p(v), _p(out), b, h, lq, lk, d, nthreads)
        return out
    m = _f32(mask)
    mb = np.broadcast_to(m, (b, h, lq, lk))  # stride 0 on the broadcast dimensions
    sm = (ctypes.c_long * 4)(*[st // 4 for st in mb.strides])
    lib().oracle_sdpa_mask(_p(q), _p(k), _p(v), _p(m), sm, _p(out), b, h, lq, lk, d, nthreads)
    return out


def mha_blhd(q, k, v, scale: float | None = None, nthreads: int = 0) -> np.ndarray:
    """kernels.rs:416-434 / 502-548 semantics on [B, L, H, D] (the flash-attention layout)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, lq, h, d = q.shape
    lk = k.shape[1]
    assert k.shape == (b, lk, h, d) and v.shape == k.shape
    if scale is None:
        scale = float(d) ** -0.5
    out = np.empty_like(q)
    lib().oracle_mha_blhd(_p(q), _p(k), _p(v), _p(out), b, lq, lk, h, d, scale, nthreads)
    return out


def rope_tables(side: int, scale: float, hd: int, theta: float):
    """sam3/vision.rs:26-46 -> (cos, sin), each [side*side, hd]."""
    cos = np.empty((side * side, hd), np.float32)
    sin = np.empty((side * side, hd), np.float32)
    lib().oracle_rope_tables(side, scale, hd, theta, _p(cos), _p(sin))
    return cos, sin


def rope(x, cos, sin) -> np.ndarray:
    """sam3/video.rs:106-113 on x [L, D] with cos/sin [L, D]."""
    x, cos, sin = _f32(x), _f32(cos), _f32(sin)
    l, d = x.shape
    assert cos.shape == (l, d) and sin.shape == (l, d)
    out = np.empty_like(x)
    lib().oracle_rope(_p(x), _p(cos), _p(sin), _p(out), l, d)
    return out


def rope_attention(q, k, v, cos, sin, n_exclude: int, nthreads: int = 0) -> np.ndarray:
    """sam3/video.rs:129-145 after the projections: q [Lq, D], k/v [M, D]; one head."""
    q, k, v, cos, sin = _f32(q), _f32(k), _f32(v), _f32(cos), _f32(sin)
    lq, d = q.shape
    mk = k.shape[0]
    trows = cos.shape[0]
    assert lq == trows and (mk - n_exclude) % trows == 0
    out = np.empty_like(q)
    lib().oracle_rope_attention(_p(q), _p(k), _p(v), _p(cos), _p(sin), trows, _p(out), lq, mk, d, n_exclude,
                                nthreads)
    return out


SAM_MEAN = (123.675, 116.28, 103.53)  # image_proc.rs:7-8
SAM_STD = (58.395, 57.12, 57.375)


def resized_hw(h: int, w: int, size: int):
    """image_proc.rs:22-25: the longest side scaled to `size`, rounded half up, in f32."""
    scale = np.float32(size) / np.float32(max(w, h))
    nw = int(np.float32(np.float32(w) * scale) + np.float32(0.5))
    nh = int(np.float32(np.float32(h) * scale) + np.float32(0.5))
    return nh, nw


def preprocess(img, nh: int, nw: int, size: int, mean=SAM_MEAN, std=SAM_STD, nthreads: int = 0) -> np.ndarray:
    """image_proc.rs:57-96: u8 [h, w, 3] -> f32 [3, size, size] (resize to nh x nw, normalise, zero pad)."""
    img = np.ascontiguousarray(img, dtype=np.uint8)
    h, w, c = img.shape
    assert c == 3 and 1 <= nh <= size and 1 <= nw <= size
    out = np.empty((3, size, size), np.float32)
    m, sd = _f32(mean), _f32(std)
    lib().oracle_preprocess(img.ctypes.data, h, w, nh, nw, size, _p(m), _p(sd), _p(out), nthreads)
    return out


def bias_residual(res, y, bias) -> np.ndarray:
    """kernels.rs:618-640: res + y + bias, bias broadcast over the last dimension."""
    res, y, bias = _f32(res), _f32(y), _f32(bias).ravel()
    assert res.shape == y.shape and res.size % bias.size == 0
    out = np.empty_like(res)
    lib().oracle_bias_residual(_p(res), _p(y), _p(bias), _p(out), res.size, bias.size)
    return out


def bias_gelu(y, bias) -> np.ndarray:
    """kernels.rs:642-663: gelu_erf(y + bias), bias broadcast over the last dimension."""
    y, bias = _f32(y), _f32(bias).ravel()
    assert y.size % bias.size == 0
    out = np.empty_like(y)
    lib().oracle_bias_gelu(_p(y), _p(bias), _p(out), y.size, bias.size)
    return out


def round_to(x, dtype: str) -> np.ndarray:
    """Round f32 values to f16 or bf16 (round-to-nearest-even) and return them as f32."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    if dtype == "f16":
        lib().oracle_round_f16(_p(x), x.size)
    elif dtype == "bf16":
        lib().oracle_round_bf16(_p(x), x.size)
    elif dtype != "f32":
        raise ValueError(dtype)
    return x


def randn(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """SplitMix64 + Box-Muller normals: the seeded synthetic-input generator."""
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().oracle_randn(seed, _p(out), n, mean, std)
    return out.reshape(shape)
