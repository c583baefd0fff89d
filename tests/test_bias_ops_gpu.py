"""Parity of bias_residual and bias_gelu (libsam_hip.so) with the CPU oracle, on an MI355X.

bias_residual is (res + y) + bias in f32 rounded once: bit-identical to the oracle in f32 and to the
oracle's value rounded to nearest even in f16 / bf16. bias_gelu evaluates erf through a Chebyshev fit
of erfc (fractional error below 1.2e-7) where the reference calls the `libm` crate's erf and the
oracle the C library's; the formula amplifies such differences for negative inputs, so gelu is held to
a relative bar with an absolute floor (below). Cases: the ViT-H shapes (tokens x
1280 after attention, tokens x 5120 in the MLP), odd channel counts that take the scalar loop,
misaligned views, in-place use and the argument errors.

bias_residual_ln fuses bias_residual with the LayerNorm that follows it in an encoder block: its x is
held bit for bit to the oracle's bias_residual rounded to the dtype, and its norm to a float64
LayerNorm of that rounded x (mean, biased variance, (x - mean) / sqrt(var + eps) * w + b) within one
rounding step of the dtype (f32: 10^-5 relative), with a 10^-5 absolute floor.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle

pytestmark = pytest.mark.gpu
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def data(shape, seed, dtype, scale=1.0):
    x = (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)
    return oracle.round_to(x, dtype)


def dev(x, dtype):
    return torch.from_numpy(x).to("cuda", TORCH_DT[dtype])


SHAPES = [(4096, 1280), (2, 70, 70, 768), (33, 12), (5, 7, 3), (1, 1)]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_bias_residual_matches_oracle(hip, shape, dtype):
    print(f"bias_residual {shape} {dtype}", flush=True)
    res, y, b = data(shape, 1, dtype), data(shape, 2, dtype), data(shape[-1:], 3, dtype)
    want = oracle.round_to(oracle.bias_residual(res, y, b), dtype)
    got = hip.bias_residual(dev(res, dtype), dev(y, dtype), dev(b, dtype)).float().cpu().numpy()
    assert np.array_equal(got, want)


# gelu_erf(x) = 0.5 x (1 + erf(x / sqrt 2)) cancels for negative x: one ulp of erf there is many ulps of
# the result (near x = -2 about 15, and more as the result goes to 0). So the bar is relative with an
# absolute floor, 1e-5 for f32 (the path's f32 bar) and one rounding step of the output type for f16 /
# bf16.
GELU_RTOL = {"f32": 1e-5, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(4096, 5120), (63, 20), (2, 3, 9)], ids=["4096x5120", "63x20", "2x3x9"])
def test_bias_gelu_matches_oracle(hip, shape, dtype):
    print(f"bias_gelu {shape} {dtype}", flush=True)
    y, b = data(shape, 4, dtype, 2.0), data(shape[-1:], 5, dtype)
    want = oracle.round_to(oracle.bias_gelu(y, b), dtype)
    got = hip.bias_gelu(dev(y, dtype), dev(b, dtype)).float().cpu().numpy()
    assert np.isfinite(got).all()
    assert np.allclose(got, want, rtol=GELU_RTOL[dtype], atol=1e-6), np.abs(got - want).max()


def test_in_place_and_misaligned_views(hip):
    y = torch.randn(4097, device="cuda")
    res = torch.randn(4097, device="cuda")
    b = torch.randn(1, device="cuda")
    want = oracle.bias_residual(res.cpu().numpy(), y.cpu().numpy(), b.cpu().numpy())
    # element offset 1 leaves the data 4-byte but not 16-byte aligned: the scalar loop
    got = hip.bias_residual(res[1:].view(4096, 1), y[1:].view(4096, 1), b).cpu().numpy()
    assert np.array_equal(got.ravel(), want[1:])
    lib = hip.load()
    r2 = res.clone()
    assert lib.sam_hip_bias_residual(r2.data_ptr(), y.data_ptr(), b.data_ptr(), r2.data_ptr(), 0, r2.numel(), 1,
                                     hip._stream()) == 0
    assert np.array_equal(r2.cpu().numpy(), want)


def test_bias_op_errors(hip):
    x = torch.zeros(4, 6, device="cuda")
    with pytest.raises(hip.SamHipError, match="shape mismatch"):
        hip.bias_residual(x, torch.zeros(4, 5, device="cuda"), torch.zeros(6, device="cuda"))
    with pytest.raises(hip.SamHipError, match="last dimension"):
        hip.bias_gelu(x, torch.zeros(5, device="cuda"))
    lib = hip.load()
    assert lib.sam_hip_bias_gelu(x.data_ptr(), x.data_ptr(), x.data_ptr(), 0, 24, 5, None) == 1
    assert b"whole rows" in lib.sam_hip_last_error()
    assert lib.sam_hip_bias_gelu(x.data_ptr(), x.data_ptr(), x.data_ptr(), 0, 0, 6, None) == 0  # empty


LN_SHAPES = [(4096, 1280), (2, 33, 768), (3, 1024), (5, 8), (2, 2048), (7, 4)]
LN_RTOL = {"f32": 1e-5, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}


def ln_want(res, y, b, w, lb, dtype, eps):
    x = oracle.round_to(oracle.bias_residual(res, y, b), dtype)
    x64 = x.astype(np.float64)
    mean = x64.mean(-1, keepdims=True)
    var = ((x64 - mean) ** 2).mean(-1, keepdims=True)
    return x, (x64 - mean) / np.sqrt(var + eps) * w.astype(np.float64) + lb.astype(np.float64)


# rows must be whole 16-byte vectors: 4 f32 or 8 f16/bf16 elements
LN_CASES = [(s, d) for s in LN_SHAPES for d in ("f32", "f16", "bf16") if s[-1] % (4 if d == "f32" else 8) == 0]


@pytest.mark.parametrize("shape,dtype", LN_CASES, ids=["x".join(map(str, s)) + "-" + d for s, d in LN_CASES])
def test_bias_residual_ln_matches_float64_layer_norm(hip, shape, dtype):
    c = shape[-1]
    print(f"bias_residual_ln {shape} {dtype}", flush=True)
    res, y = data(shape, 21, dtype), data(shape, 22, dtype, 0.5)
    b = data((c,), 23, dtype, 0.1)
    w = oracle.round_to(1.0 + 0.2 * np.random.default_rng(24).standard_normal(c).astype(np.float32), dtype)
    lb = data((c,), 25, dtype, 0.1)
    x_want, ln64 = ln_want(res, y, b, w, lb, dtype, 1e-6)
    x, ln = hip.bias_residual_ln(dev(res, dtype), dev(y, dtype), dev(b, dtype), dev(w, dtype), dev(lb, dtype), 1e-6)
    assert np.array_equal(x.float().cpu().numpy(), x_want)
    got = ln.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ln64)
    assert (err <= LN_RTOL[dtype] * np.abs(ln64) + 1e-5).all(), err.max()


def test_bias_residual_ln_in_place_and_errors(hip):
    res = torch.randn(64, 1280, device="cuda").half()
    y = torch.randn(64, 1280, device="cuda").half()
    b, w, lb = (torch.randn(1280, device="cuda").half() for _ in range(3))
    x_ref, ln_ref = hip.bias_residual_ln(res, y, b, w, lb)
    lib = hip.load()
    r2, ln2 = res.clone(), torch.empty_like(res)
    # out over res: every element is read and then written by the same thread
    assert lib.sam_hip_bias_residual_ln(r2.data_ptr(), y.data_ptr(), b.data_ptr(), w.data_ptr(), lb.data_ptr(),
                                        r2.data_ptr(), ln2.data_ptr(), 1, 64, 1280, 1e-6, hip._stream()) == 0
    assert torch.equal(r2, x_ref) and torch.equal(ln2, ln_ref)
    args = [r2.data_ptr(), y.data_ptr(), b.data_ptr(), w.data_ptr(), lb.data_ptr(), r2.data_ptr(), ln2.data_ptr()]
    assert lib.sam_hip_bias_residual_ln(*args, 1, 64 * 1280 // 1284, 1284, 1e-6, None) == 3  # not whole vectors
    assert b"multiple of 8" in lib.sam_hip_last_error()
    assert lib.sam_hip_bias_residual_ln(*args, 1, 1, 8192, 1e-6, None) == 3  # longer than 512 vectors
    assert lib.sam_hip_bias_residual_ln(*args, 1, 64, 1280, -1.0, None) == 1  # negative eps
    mis = args[:]
    mis[1] = y.data_ptr() + 2
    assert lib.sam_hip_bias_residual_ln(*mis, 1, 63, 1280, 1e-6, None) == 3
    assert b"16-byte aligned" in lib.sam_hip_last_error()
    assert lib.sam_hip_bias_residual_ln(*args, 1, 0, 1280, 1e-6, None) == 0  # no rows
