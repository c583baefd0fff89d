"""Parity of Grounding DINO's Deform::forward on the GPU (sam_hip_deform_core and the sam_dino.Deform
module) with the CPU oracle, on an MI355X.

sam_hip_deform_core is the part of Deform::forward between its projections (dino/mod.rs:166-179): the
softmax of the attention logits over a head's L*P points, the sampling locations from the offsets and
the reference points, encoder form ref + off / (W, H) (2 coordinates) and decoder form
xy + off / P * wh * 0.5 (4 coordinates), and the bilinear gather. The oracle runs its restatement
(oracle_deform_prep, then oracle_deform_attn) on the same inputs, pre-rounded to the kernel dtype; for
f16 / bf16 the restatement rounds each step to that dtype, as the reference's candle ops do.
Bars: f32 max|gpu - cpu| / max|cpu| <= 1e-5; f16 max-abs 2e-3; bf16 2e-3 beyond its output rounding.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle
from parity import check

pytestmark = pytest.mark.gpu
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
DINO_LEVELS = [(100, 167), (50, 84), (25, 42), (13, 21)]


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def core_inputs(shapes, b, q, h, d, p, nc, seed, dtype):
    """value ~ N(0,1); offsets ~ N(0,2) (pixels for the encoder form); logits ~ N(0,1); refs ~ U(0,1)
    (2 coordinates) or boxes with centres in [0.1, 0.9] and sizes in [0.05, 0.6] (4 coordinates)."""
    r = np.random.default_rng(seed)
    s = sum(hh * ww for hh, ww in shapes)
    l = len(shapes)
    value = r.standard_normal((b, s, h, d))
    off = 2.0 * r.standard_normal((b, q, h, l, p, 2))
    logits = r.standard_normal((b, q, h, l, p))
    if nc == 2:
        refs = r.uniform(0, 1, (b, q, l, 2))
    else:
        refs = np.concatenate([r.uniform(0.1, 0.9, (b, q, 1, 2)), r.uniform(0.05, 0.6, (b, q, 1, 2))], -1)
        refs = np.broadcast_to(refs, (b, q, l, 4))  # the decoder repeats its box over the levels
    return [oracle.round_to(np.ascontiguousarray(x, dtype=np.float32), dtype) for x in (value, off, logits, refs)]


def run_core(hip, arrays, shapes, dtype):
    dev = [torch.from_numpy(a).to("cuda", TORCH_DT[dtype]) for a in arrays]
    out = hip.deform_core(*dev, shapes)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    ("kernels.rs", [(9, 12), (5, 6), (3, 3), (2, 2)], 1, 37, 8, 32, 4),  # tests/kernels.rs:65-83
    ("dino.rs", [(7, 9), (4, 5), (2, 3)], 1, 13, 4, 8, 3),  # tests/dino.rs:46-63
    ("batch2-odd-d", [(6, 5), (3, 3)], 2, 11, 3, 20, 2),  # scalar lanes
    ("many-blocks", [(30, 40), (15, 20), (8, 10), (4, 5)], 2, 1501, 8, 32, 4),
    ("sixteen-points", [(12, 10), (6, 5)], 1, 97, 5, 16, 8),  # 16 points per level: lanes own 2+ points
]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("nc", [2, 4], ids=["encoder-refs", "decoder-refs"])
@pytest.mark.parametrize("name,shapes,b,q,h,d,p", CASES, ids=[c[0] for c in CASES])
def test_deform_core_matches_oracle(hip, name, shapes, b, q, h, d, p, nc, dtype):
    print(f"deform core {name} nc={nc} {dtype}", flush=True)
    arrays = core_inputs(shapes, b, q, h, d, p, nc, 60 + q + nc, dtype)
    want = oracle.deform_forward_core(*arrays, shapes, dtype=dtype)
    got = run_core(hip, arrays, shapes, dtype)
    check(got, want, dtype, f"deform core {name} nc={nc} {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("q,nc", [(22223, 2), (900, 4)], ids=["encoder", "decoder"])
def test_deform_core_dino_tiny(hip, q, nc, dtype):
    """Grounding DINO-tiny at full size: 4 levels of an 800x1333 input (22223 value tokens), 8 heads x
    32, 4 points; the encoder's queries are its value tokens with the centre reference points of
    encoder_reference_points (dino/mod.rs:660-678), the decoder has 900 queries with box references."""
    import sam_dino

    print(f"deform core dino-tiny q={q} {dtype}", flush=True)
    arrays = core_inputs(DINO_LEVELS, 1, q, 8, 32, 4, nc, 7 + q, dtype)
    if nc == 2:
        refs = sam_dino.encoder_reference_points(DINO_LEVELS, device="cpu").numpy()[None]
        arrays[3] = oracle.round_to(refs, dtype)
    want = oracle.deform_forward_core(*arrays, DINO_LEVELS, dtype=dtype)
    got = run_core(hip, arrays, DINO_LEVELS, dtype)
    check(got, want, dtype, f"deform core dino-tiny q={q} {dtype}")


def test_encoder_reference_points_match_the_reference_loop():
    """encoder_reference_points against the reference's own loop order (level, y, x; then level)."""
    import sam_dino

    shapes = [(3, 4), (2, 2)]
    got = sam_dino.encoder_reference_points(shapes, device="cpu").numpy()
    pts = [((x + 0.5) / w, (y + 0.5) / h) for h, w in shapes for y in range(h) for x in range(w)]
    want = np.array([[p] * len(shapes) for p in pts], np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("q,nc", [(900, 4), (2000, 2)], ids=["decoder", "encoder-slice"])
def test_deform_module_forward(hip, q, nc):
    """The whole Deform::forward (dino/mod.rs:161-181) in f32 at DINO-tiny's width (C 256, 8 heads,
    4 levels, 4 points) with N(0, 0.02) weights: the four projections run as torch linears
    (hipBLASLt), the middle as sam_hip_deform_core. The oracle composes float64 projections with its
    restated core. Bar: the f32 bar, max|gpu - cpu| / max|cpu| <= 1e-5, which the f32 GEMM rounding
    of the projections (K = 256) stays well inside."""
    import sam_dino

    g = torch.Generator(device="cuda").manual_seed(5 + q)
    mod = sam_dino.Deform.random(256, 8, 4, 4, generator=g)
    s = sum(a * b for a, b in DINO_LEVELS)
    query = torch.randn(q, 256, device="cuda", generator=g)
    value_in = torch.randn(s, 256, device="cuda", generator=g)
    if nc == 2:
        refs = torch.rand(q, 1, 2, device="cuda", generator=g).expand(q, 4, 2).contiguous()
    else:
        box = torch.cat([0.1 + 0.8 * torch.rand(q, 1, 2, device="cuda", generator=g),
                         0.05 + 0.55 * torch.rand(q, 1, 2, device="cuda", generator=g)], -1)
        refs = box.expand(q, 4, 4).contiguous()
    got = mod.forward(query, value_in, refs, DINO_LEVELS)
    torch.cuda.synchronize()

    h64 = lambda t: t.double().cpu().numpy()
    lin = lambda x, wb: x @ h64(wb[0]).T + h64(wb[1])
    xq, xv = h64(query), h64(value_in)
    value = lin(xv, mod.value).reshape(1, s, 8, 32)
    off = lin(xq, mod.offsets).reshape(1, q, 8, 4, 4, 2)
    logits = lin(xq, mod.weights).reshape(1, q, 8, 4, 4)
    core = oracle.deform_forward_core(value, off, logits, h64(refs)[None], DINO_LEVELS).reshape(q, 256)
    want = lin(core.astype(np.float64), mod.out)
    err = np.abs(got.cpu().numpy() - want).max() / np.abs(want).max()
    print(f"parity deform module q={q} nc={nc}: max|gpu-cpu|/max|cpu| {err:.3g}", flush=True)
    assert err <= 1e-5


def test_deform_core_errors(hip):
    v = torch.zeros(1, 30, 2, 8, device="cuda")
    off = torch.zeros(1, 3, 2, 2, 2, 2, device="cuda")
    lg = torch.zeros(1, 3, 2, 2, 2, device="cuda")
    with pytest.raises(hip.SamHipError, match="refs must be"):
        hip.deform_core(v, off, lg, torch.zeros(1, 3, 2, 3, device="cuda"), [(2, 3), (4, 6)])
    with pytest.raises(hip.SamHipError, match="pixels"):
        hip.deform_core(v, off, lg, torch.zeros(1, 3, 2, 2, device="cuda"), [(2, 3), (2, 3)])
    L = hip.load()
    flat = (__import__("ctypes").c_int * 4)(2, 3, 4, 6)
    rc = L.sam_hip_deform_core(v.data_ptr(), off.data_ptr(), lg.data_ptr(), lg.data_ptr(), v.data_ptr(), 0, 1, 30,
                               3, 2, 8, 2, 2, 3, flat, None)
    assert rc != 0 and b"2 or 4 coordinates" in L.sam_hip_last_error()
