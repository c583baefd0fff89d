"""Parity of sam_hip_qkv_rope (libsam_hip.so) with the CPU oracle, on an MI355X.

qkv_rope is one addition, two products and a sum per element in f32, then one rounding to the element
type: bit-exact against the oracle (kernels.rs:321-362) in f32, f16 and bf16. Shapes: SAM 3 ViT's windowed
layer (9 windows of 24x24 tokens, 16 heads x 64) and its global layer (72x72 tokens), token counts that
are not multiples of the table's rows or of the kernel's 1024-vector workgroup step, a single token, and
head dims that are not multiples of 8 (the per-pair kernel). The tables are those of rope_tables_hd
(sam3/vision.rs:26-46); one case gives tables whose odd columns are NaN, which the reference never reads.
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


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", TORCH_DT[dtype])


# (tokens, side of the table's token grid (n = side^2), heads, hd)
SHAPES = [(9 * 576, 24, 16, 64), (5184, 72, 16, 64), (1000, 8, 3, 16), (1, 4, 2, 8), (77, 3, 5, 24),
          (100, 5, 2, 12), (33, 2, 3, 20), (2, 1, 1, 4), (130, 6, 1, 256)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("tokens,side,nh,hd", SHAPES)
def test_qkv_rope_is_bit_exact(hip, tokens, side, nh, hd, dtype):
    print(f"qkv_rope {dtype} tokens={tokens} n={side * side} nh={nh} hd={hd}", flush=True)
    n = side * side
    r = np.random.default_rng(tokens + 7 * hd + nh)
    y = oracle.round_to(r.standard_normal((tokens, 3 * nh * hd)), dtype)
    b = oracle.round_to(r.standard_normal(3 * nh * hd), dtype)
    cos, sin = oracle.rope_tables(side, 1.0, hd, 10000.0)
    want = oracle.qkv_rope(y, b, cos, sin, n, nh, hd, dtype=dtype)
    got = hip.qkv_rope(dev(y, dtype), dev(b, dtype), dev(cos, "f32"), dev(sin, "f32"), n, nh, hd)
    assert tuple(got.shape) == (3, tokens, nh, hd) and got.dtype == TORCH_DT[dtype]
    g = got.float().cpu().numpy()
    if not np.array_equal(g, want):
        bad = np.argwhere(g != want)
        raise AssertionError(f"{len(bad)} elements differ, first at {tuple(bad[0])}: {g[tuple(bad[0])]} vs "
                             f"{want[tuple(bad[0])]}")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("hd", [64, 6])
def test_qkv_rope_reads_only_the_even_table_columns(hip, dtype, hd):
    """Both elements of a pair take the table's even column (kernels.rs:348, sam.cu:222): with N(0,1)
    tables whose odd columns are NaN the output is finite and equals the oracle's."""
    print(f"qkv_rope even columns {dtype} hd={hd}", flush=True)
    tokens, n, nh = 300, 50, 2
    r = np.random.default_rng(5 + hd)
    y = oracle.round_to(r.standard_normal((tokens, 3 * nh * hd)), dtype)
    b = oracle.round_to(r.standard_normal(3 * nh * hd), dtype)
    cos = r.standard_normal((n, hd)).astype(np.float32)
    sin = r.standard_normal((n, hd)).astype(np.float32)
    cos[:, 1::2] = np.nan
    sin[:, 1::2] = np.nan
    want = oracle.qkv_rope(y, b, cos, sin, n, nh, hd, dtype=dtype)
    assert np.all(np.isfinite(want))
    got = hip.qkv_rope(dev(y, dtype), dev(b, dtype), dev(cos, "f32"), dev(sin, "f32"), n, nh, hd)
    assert np.array_equal(got.float().cpu().numpy(), want)
