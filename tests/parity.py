"""Parity bars shared by the GPU tests (the bars the reference's numerics call for).

f32: max|gpu - cpu| / max|cpu| <= 1e-5. f16 / bf16: max-abs <= 2e-3 on attention outputs against the
f32 oracle run on inputs pre-rounded to the kernel dtype (as tests/kernels.rs:28-31 does). Where the
output's own rounding alone can exceed the bar, the error is measured beyond that rounding (its
half-ulp): every bf16 output of magnitude 0.5 or more, and f16 outputs of magnitude 4 or more (f16
half-ulp 2^-9 ~ 1.95e-3 there). The raw max-abs is always reported beside the figure the bar applies to.
"""
import numpy as np
import torch

F32_REL_TOL = 1e-5
HALF_ABS_TOL = 2e-3
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device="cuda", dtype=TORCH_DT[dtype])


def bf16_half_ulp(x):
    """Half the spacing of bf16 numbers at |x| (8 significant bits): the rounding any bf16 output has."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 8)


def f16_half_ulp(x):
    """Half the spacing of f16 numbers at |x| (11 significant bits, subnormal spacing below 2^-14)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 11)


def check(got, want, dtype, what):
    """f32: max|gpu-cpu| / max|cpu| <= 1e-5. f16: max-abs <= 2e-3, measured beyond the output's own
    half-ulp where |out| >= 4 (f16 spacing 2^-8 there, so rounding alone can reach 1.95e-3). bf16:
    max-abs <= 2e-3 beyond the half-ulp rounding of the bf16 output itself (|out| >= 0.5 has a half-ulp
    of 2e-3 or more, so no bf16 result can meet a bare 2e-3 there). The raw max-abs is printed and
    carried in the message. Returns the figure the bar applies to."""
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    raw = float(np.abs(got - want).max())
    if dtype == "f32":
        err = raw / float(np.abs(want).max())
        print(f"parity {what}: max|gpu-cpu|/max|cpu| {err:.3g} (max-abs {raw:.3g})", flush=True)
        assert err <= F32_REL_TOL, f"{what}: max|gpu-cpu|/max|cpu| = {err:.3g}"
    elif dtype == "bf16":
        err = float((np.abs(got - want) - bf16_half_ulp(want)).max())
        print(f"parity {what}: raw max-abs {raw:.3g}, beyond bf16 output rounding {err:.3g}", flush=True)
        assert err <= HALF_ABS_TOL, f"{what}: max abs diff beyond bf16 output rounding {err:.3g} (raw max-abs {raw:.3g})"
    else:
        d = np.abs(got - want)
        big = np.abs(want) >= 4.0  # f16 spacing 2^-8 there: rounding alone reaches 1.95e-3
        err = float(np.where(big, d - f16_half_ulp(want), d).max())
        own = float((d - f16_half_ulp(want)).max())
        print(f"parity {what}: max-abs {raw:.3g}, bar figure {err:.3g} (beyond f16 output rounding {own:.3g})",
              flush=True)
        assert err <= HALF_ABS_TOL, f"{what}: max abs diff {err:.3g} (raw max-abs {raw:.3g})"
    return err
