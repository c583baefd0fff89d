"""Parity of bias_residual and bias_gelu (libsam_hip.so) with the CPU oracle, on an MI355X.

bias_residual is (res + y) + bias in f32 rounded once: bit-identical to the oracle in f32 and to the
oracle's value rounded to nearest even in f16 / bf16. bias_gelu calls the device erff where the
reference calls the `libm` crate's and the oracle the C library's; all are faithful to about an ulp,
and the formula amplifies that for negative inputs, so gelu is held to a relative bar with an absolute
floor (below). Cases: the ViT-H shapes (tokens x
1280 after attention, tokens x 5120 in the MLP), odd channel counts that take the scalar loop,
misaligned views, in-place use and the argument errors.
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
