"""The HIP kernels against the committed golden fixtures (float64 brute force, inputs exact in every
dtype), in every dtype each entry point takes, at the parity bars of tests/parity.py."""
import numpy as np
import pytest
import torch

import golden_io
from parity import check, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name", golden_io.names("relpos"))
def test_attention_relpos_golden(hip, name, dtype):
    g = golden_io.load("relpos", name)
    h, w, bh, hd = (int(x) for x in g["geom"])
    out = hip.attention_relpos(*(to_dev(g[k], dtype) for k in ("q", "kt", "v", "table")), h, w, float(g["scale"][0]))
    check(host(out), g["out"], dtype, f"attention_relpos golden {name} {dtype}")


def test_relpos_softmax_golden(hip):
    """f32 only: the golden scores are an input here and are not exact in f16/bf16 (the rounded-input
    cases of those dtypes are in test_relpos_softmax_qkv_gpu.py)."""
    g = golden_io.load("relpos", "2x3_hd8")
    h, w, bh, hd = (int(x) for x in g["geom"])
    s = g["s"].astype(np.float32)
    p = hip.relpos_softmax(to_dev(s, "f32"), to_dev(g["q"], "f32"), to_dev(g["table"], "f32"), h, w,
                           float(g["scale"][0]))
    assert np.abs(host(p) - g["probs"]).max() <= 1e-6


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name", golden_io.names("deform"))
def test_deform_golden(hip, name, dtype):
    g = golden_io.load("deform", name)
    out = hip.deform_attn(to_dev(g["value"], dtype), to_dev(g["loc"], dtype), to_dev(g["attn"], dtype),
                          [tuple(x) for x in g["shapes"].tolist()])
    check(host(out), g["out"], dtype, f"deform golden {name} {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("name", golden_io.names("flash"))
def test_flash_golden(hip, name, dtype):
    g = golden_io.load("flash", name)
    out = hip.flash_attn(*(to_dev(g[k], dtype) for k in ("q", "k", "v")))
    check(host(out), g["out"], dtype, f"flash golden {name} {dtype}")
    t = lambda x: x.transpose(1, 2)
    out2 = hip.sdpa(*(t(to_dev(g[k], dtype)) for k in ("q", "k", "v")))
    check(host(t(out2)), g["out"], dtype, f"sdpa golden {name} {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name", golden_io.names("rope"))
def test_rope_golden(hip, name, dtype):
    import sam_oracle

    g = golden_io.load("rope", name)
    side = int(g["side"][0])
    x = g["x"]
    cos, sin = sam_oracle.rope_tables(side, 1.0, x.shape[1], 10000.0)
    out = host(hip.rope(to_dev(x, dtype)[None], torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda())[0])
    want = g["out"]
    tol = {"f32": 1e-5, "f16": 2.0 ** -11, "bf16": 2.0 ** -8}[dtype]  # one rounding to the dtype
    assert (np.abs(out - want) <= tol * np.maximum(np.abs(want), 1.0) + 1e-5).all()
