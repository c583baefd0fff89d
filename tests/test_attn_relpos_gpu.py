"""Parity of the fused rel-pos attention (libsam_hip.so) with the CPU oracle, on an MI355X.

Inputs are drawn with a fixed seed, rounded to the kernel dtype, and the oracle runs on the rounded
values, so only the kernel's own error is measured (the reference's test does the same,
tests/kernels.rs:28-31). Bars: f32 max|gpu - cpu| / max|cpu| <= 1e-5; f16/bf16 max-abs <= 2e-3 on
the attention outputs against the f32 oracle.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle
from parity import F32_REL_TOL, HALF_ABS_TOL, TORCH_DT, check, to_dev

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def make_inputs(h, w, bh, hd, seed, dtype, qkv_std=1.0, table_std=0.02):
    n = h * w
    r = np.random.default_rng(seed)
    q = (qkv_std * r.standard_normal((bh, n, hd))).astype(np.float32)
    kt = (qkv_std * r.standard_normal((bh, hd, n))).astype(np.float32)
    v = (qkv_std * r.standard_normal((bh, n, hd))).astype(np.float32)
    table = (table_std * r.standard_normal((2 * h - 1 + 2 * w - 1, hd))).astype(np.float32)
    return [oracle.round_to(x, dtype) for x in (q, kt, v, table)]


def run_gpu(hip, arrays, h, w, scale, dtype):
    q, kt, v, table = (to_dev(a, dtype) for a in arrays)
    out = hip.attention_relpos(q, kt, v, table, h, w, scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


# The reference test geometries (tests/kernels.rs:23, tests/cpu_gemm.rs:37) with its N(0,1) tables,
# plus small and ragged shapes: a 2x3 grid with hd 8, a single grid row, and odd sizes; 64-column
# grids with hd 80 and hd 64 of 1, 2, 3, 6 and 37 rows (ring shorter than its depth, odd tile counts, a
# partial last query block); window grids with hd 80 and hd 64 of 13..16 rows (a full or half-empty
# last key tile, idle query blocks), and narrow window grids of 2..8 columns, whose 8-slot DMA groups
# span several grid rows; at hd 64 the f32 window kernel's one- to three-tile grids of fewer than 128
# queries (3x7, 1x16, 5x9).
SMALL = [(14, 14, 6, 64), (64, 64, 2, 64), (7, 11, 3, 80), (2, 3, 2, 8), (1, 5, 2, 16), (5, 33, 2, 32),
         (3, 40, 2, 128), (9, 17, 2, 48), (1, 64, 2, 80), (2, 64, 1, 80), (3, 64, 2, 80), (6, 64, 2, 80),
         (37, 64, 3, 80), (16, 16, 2, 80), (13, 12, 3, 80), (15, 14, 2, 80), (14, 10, 2, 80),
         (1, 64, 2, 64), (2, 64, 1, 64), (3, 64, 2, 64), (37, 64, 3, 64), (16, 16, 2, 64), (13, 12, 3, 64),
         (15, 14, 2, 64), (14, 10, 2, 64),
         (13, 2, 3, 80), (14, 4, 2, 80), (16, 6, 2, 80), (15, 8, 2, 80),
         (13, 2, 3, 64), (14, 4, 2, 64), (16, 6, 2, 64), (15, 8, 2, 64),
         (3, 7, 2, 64), (1, 16, 2, 64), (5, 9, 2, 64)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,bh,hd", SMALL)
def test_attention_relpos_reference_geometries(hip, h, w, bh, hd, dtype):
    print(f"attn_relpos {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    # q, k ~ N(0, 0.5) keeps N(0,1)-table logits in the range the reference's f16 test exercises
    arrays = make_inputs(h, w, bh, hd, 100 + h * w + hd, dtype, qkv_std=0.5, table_std=0.5)
    scale = hd ** -0.5
    want = oracle.attention_relpos(*arrays, h, w, scale)
    got = run_gpu(hip, arrays, h, w, scale, dtype)
    check(got, want, dtype, f"{h}x{w} bh={bh} hd={hd} {dtype}")


# The reference test's own draws (tests/kernels.rs:20-37): q, k, v and both tables ~ N(0, 1). Each bias
# term then has a standard deviation of about sqrt(hd) (8 to 9), so the logits are sharp: a row's
# softmax is dominated by a few keys and any error in the exp2 argument (the f16 path's pre-scaled q,
# the bias split into f16 hi / lo halves) shows up undamped. The reference geometries plus the hd-80
# window and global kernels of ViT-H.
SHARP = [(14, 14, 6, 64), (64, 64, 2, 64), (7, 11, 3, 80), (14, 14, 4, 80), (64, 64, 2, 80)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("h,w,bh,hd", SHARP)
def test_attention_relpos_sharp_logits(hip, h, w, bh, hd, dtype):
    print(f"attn_relpos sharp {dtype} h={h} w={w} bh={bh} hd={hd}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 300 + h * w + hd, dtype, qkv_std=1.0, table_std=1.0)
    scale = hd ** -0.5
    want = oracle.attention_relpos(*arrays, h, w, scale)
    got = run_gpu(hip, arrays, h, w, scale, dtype)
    check(got, want, dtype, f"sharp {h}x{w} bh={bh} hd={hd} {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_vit_b_l_global_layer(hip, dtype):
    """ViT-B / ViT-L global attention layer shape: 64x64 tokens, hd 64 (12 or 16 heads; 16 here),
    q/k/v ~ N(0,1), rel_pos ~ N(0, 0.02). The GPU runs all 16 heads; the oracle checks heads 0, 9, 15."""
    h = w = 64
    bh, hd = 16, 64
    print(f"vit-b/l global {dtype}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 17, dtype)
    scale = hd ** -0.5
    got = run_gpu(hip, arrays, h, w, scale, dtype)
    heads = [0, 9, 15]
    q, kt, v, table = arrays
    want = oracle.attention_relpos(q[heads], kt[heads], v[heads], table, h, w, scale)
    check(got[heads], want, dtype, f"vit-b/l global {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_vit_h_global_layer(hip, dtype):
    """ViT-H global attention layer: BH 16, 64x64 tokens, hd 80, q/k/v ~ N(0,1), rel_pos ~ N(0, 0.02).
    The GPU runs all 16 heads; the oracle checks heads 0, 7 and 15."""
    h = w = 64
    bh, hd = 16, 80
    print(f"vit-h global {dtype}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 7, dtype)
    scale = hd ** -0.5
    got = run_gpu(hip, arrays, h, w, scale, dtype)
    heads = [0, 7, 15]
    q, kt, v, table = arrays
    want = oracle.attention_relpos(q[heads], kt[heads], v[heads], table, h, w, scale)
    check(got[heads], want, dtype, f"vit-h global {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_vit_h_window_layer(hip, dtype):
    """ViT-H windowed layer at batch 1: 25 windows x 16 heads of 14x14 tokens, hd 80, (27, 80) tables."""
    h = w = 14
    bh, hd = 400, 80
    print(f"vit-h window {dtype}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 8, dtype)
    scale = hd ** -0.5
    want = oracle.attention_relpos(*arrays, h, w, scale)
    got = run_gpu(hip, arrays, h, w, scale, dtype)
    check(got, want, dtype, f"vit-h window {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("bh", [300, 400], ids=["vit_b", "vit_l"])
def test_vit_b_l_window_layer(hip, bh, dtype):
    """ViT-B (12 heads) and ViT-L (16 heads) windowed layers at batch 1: 25 windows x heads of 14x14
    tokens, hd 64, (27, 64) tables."""
    h = w = 14
    hd = 64
    print(f"vit-b/l window {dtype} bh={bh}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 9 + bh, dtype)
    scale = hd ** -0.5
    want = oracle.attention_relpos(*arrays, h, w, scale)
    got = run_gpu(hip, arrays, h, w, scale, dtype)
    check(got, want, dtype, f"vit-b/l window {dtype} bh={bh}")


def device_inputs(h, w, bh, hd, seed, dtype, table_std=0.02):
    """q, k, v ~ N(0,1) and a table ~ N(0, table_std), drawn on the device in the kernel dtype (the
    large launches would take long to draw and move on the host)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dt = TORCH_DT[dtype]
    n = h * w
    q = torch.randn(bh, n, hd, device="cuda", generator=g).to(dt)
    kt = torch.randn(bh, hd, n, device="cuda", generator=g).to(dt)
    v = torch.randn(bh, n, hd, device="cuda", generator=g).to(dt)
    table = (table_std * torch.randn(2 * h - 1 + 2 * w - 1, hd, device="cuda", generator=g)).to(dt)
    return q, kt, v, table


def sampled_units(bh, period):
    """The first and last units, those around every multiple of `period` and a spread in between."""
    units = set(np.linspace(0, bh - 1, 12).astype(int).tolist())
    for m in range(0, bh + 1, period):
        units.update(u for u in (m - 1, m, m + 1) if 0 <= u < bh)
    return sorted(units)


def check_units(hip, tensors, units, h, w, dtype, what):
    q, kt, v, table = tensors
    hd = q.shape[2]
    got = hip.attention_relpos(q, kt, v, table, h, w, hd ** -0.5)
    torch.cuda.synchronize()
    idx = torch.tensor(units, device="cuda")
    host = lambda t: t.float().cpu().numpy()
    want = oracle.attention_relpos(host(q[idx]), host(kt[idx]), host(v[idx]), host(table), h, w, hd ** -0.5)
    check(host(got[idx]), want, dtype, what)


# Window launches with more half-unit workgroups than the chip holds at once (two per CU at hd 80,
# three at hd 64), so the hardware schedules them in several rounds: 257 units (a few workgroups in a
# second round), 768 and 1024 at hd 80, and the encoder sweep's batch 4 and 8: ViT-B 1200 and 2400
# units, ViT-L 1600 and 3200 (hd 64), ViT-H 1600 and 3200 (hd 80).
MANY_UNITS = [(80, 257), (80, 768), (80, 1024), (80, 1600), (80, 3200), (64, 1200), (64, 1600), (64, 2400),
              (64, 3200)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("hd,bh", MANY_UNITS)
def test_window_kernel_many_units(hip, hd, bh, dtype):
    """Every unit runs on the GPU; the oracle checks the first and last units, those around each
    multiple of 256 and a spread in between."""
    h = w = 14
    print(f"window many units {dtype} hd={hd} bh={bh}", flush=True)
    tensors = device_inputs(h, w, bh, hd, 50 + bh + hd, dtype)
    check_units(hip, tensors, sampled_units(bh, 256), h, w, dtype, f"window kernel hd={hd} bh={bh} {dtype}")


# Global launches of the encoder sweep beyond one head block per CU: ViT-B batch 4 and 8 (48, 96
# heads), ViT-L batch 4 and 8 (64, 128) at hd 64, ViT-H batch 4 (64) at hd 80. The oracle checks the
# first and last heads and a few between.
MANY_HEADS = [(64, 48), (64, 64), (64, 96), (64, 128), (80, 64)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("hd,bh", MANY_HEADS)
def test_global_kernel_many_heads(hip, hd, bh, dtype):
    h = w = 64
    print(f"global many heads {dtype} hd={hd} bh={bh}", flush=True)
    tensors = device_inputs(h, w, bh, hd, 70 + bh + hd, dtype)
    heads = sorted({0, 1, bh // 2, bh - 2, bh - 1})
    check_units(hip, tensors, heads, h, w, dtype, f"global kernel hd={hd} bh={bh} {dtype}")


# Padding keys (grid columns past W, rows past H, the slots of the last key tile) make the kernels'
# tile loads reach past the last unit's kT and V; the loads go through buffer descriptors of the unit
# (window kernels) or stay inside the tensor, so nothing past the end may reach a result. kT and v
# here are views of buffers whose tails hold NaN: a load past the end that was not zeroed would put NaN
# into S or into P.V (0 * NaN). The last units of every kernel family are checked against the oracle.
PAST_END = [(14, 14, 80), (13, 12, 80), (14, 14, 64), (15, 8, 64), (7, 11, 80), (37, 64, 80), (65, 64, 64)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("h,w,hd", PAST_END)
def test_loads_past_the_last_unit_read_no_data(hip, h, w, hd, dtype):
    bh = 6
    n = h * w
    print(f"past-end {dtype} h={h} w={w} hd={hd}", flush=True)
    arrays = make_inputs(h, w, bh, hd, 900 + n + hd, dtype)
    q, kt, v, table = (to_dev(a, dtype) for a in arrays)
    tail = 64 * 1024  # elements of NaN after each tensor
    def nan_tailed(x):
        buf = torch.full((x.numel() + tail,), float("nan"), device="cuda", dtype=x.dtype)
        buf[: x.numel()].copy_(x.reshape(-1))
        return buf[: x.numel()].view(x.shape)
    kt2, v2 = nan_tailed(kt), nan_tailed(v)
    got = hip.attention_relpos(q, kt2, v2, table, h, w, hd ** -0.5)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), "a load past the end reached the output"
    want = oracle.attention_relpos(*arrays, h, w, hd ** -0.5)
    check(got, want, dtype, f"past-end {h}x{w} hd={hd} {dtype}")


def test_window_kernel_units_are_independent(hip):
    """At 1600 units the windowed kernel's workgroups run several half units each: permuting the units
    moves them to other workgroups and pipeline positions, and the output rows move with them exactly."""
    h = w = 14
    bh, hd = 1600, 80
    g = torch.Generator(device="cuda").manual_seed(13)
    q = torch.randn(bh, h * w, hd, device="cuda", generator=g).half()
    kt = torch.randn(bh, hd, h * w, device="cuda", generator=g).half()
    v = torch.randn(bh, h * w, hd, device="cuda", generator=g).half()
    table = (0.02 * torch.randn(2 * h - 1 + 2 * w - 1, hd, device="cuda", generator=g)).half()
    perm = torch.randperm(bh, device="cuda", generator=g)
    a = hip.attention_relpos(q, kt, v, table, h, w, hd ** -0.5)
    b = hip.attention_relpos(q[perm].contiguous(), kt[perm].contiguous(), v[perm].contiguous(), table, h, w,
                             hd ** -0.5)
    assert torch.equal(a[perm], b)


def test_vit_b_f32_layers(hip):
    """ViT-B f32: windowed layer (300 x 14x14, hd 64, (27,64) tables) and global layer (12 x 64x64,
    (127,64) tables) at scale 64^-0.5; q/k/v ~ N(0, 0.3) as the qkv projection of N(0,1) tokens
    with N(0, 0.02) weights gives. The oracle checks every window and global heads 0 and 11."""
    print("vit-b f32 window", flush=True)
    arrays = make_inputs(14, 14, 300, 64, 9, "f32", qkv_std=0.55)
    want = oracle.attention_relpos(*arrays, 14, 14, 0.125)
    got = run_gpu(hip, arrays, 14, 14, 0.125, "f32")
    check(got, want, "f32", "vit-b window f32")
    print("vit-b f32 global", flush=True)
    arrays = make_inputs(64, 64, 12, 64, 10, "f32", qkv_std=0.55)
    got = run_gpu(hip, arrays, 64, 64, 0.125, "f32")
    heads = [0, 11]
    q, kt, v, table = arrays
    want = oracle.attention_relpos(q[heads], kt[heads], v[heads], table, 64, 64, 0.125)
    check(got[heads], want, "f32", "vit-b global f32")


def test_vit_l_f32_global_layer(hip):
    """ViT-L f32 global layer (16 x 64x64, hd 64): its 1024 workgroups of 64 queries would take 1.33
    rounds of the 16-queries-per-wave kernel, so it runs on the 32-queries-per-wave kernel; the oracle
    checks heads 0, 8 and 15."""
    print("vit-l f32 global", flush=True)
    arrays = make_inputs(64, 64, 16, 64, 12, "f32", qkv_std=0.55)
    got = run_gpu(hip, arrays, 64, 64, 0.125, "f32")
    heads = [0, 8, 15]
    q, kt, v, table = arrays
    want = oracle.attention_relpos(q[heads], kt[heads], v[heads], table, 64, 64, 0.125)
    check(got[heads], want, "f32", "vit-l global f32")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_full_size_properties(hip, dtype):
    """Size-independent checks over every row of a batch-8 ViT-H global layer (BH 128): a constant
    value vector comes back unchanged (softmax rows sum to 1), and the map is linear in v."""
    h = w = 64
    bh, hd = 128, 80
    print(f"full-size properties {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    dt = TORCH_DT[dtype]
    q = torch.randn(bh, h * w, hd, device="cuda", generator=g).to(dt)
    kt = torch.randn(bh, hd, h * w, device="cuda", generator=g).to(dt)
    table = (0.02 * torch.randn(2 * h - 1 + 2 * w - 1, hd, device="cuda", generator=g)).to(dt)
    const = torch.linspace(-2, 2, hd, device="cuda").to(dt)
    v = const.expand(bh, h * w, hd).contiguous()
    out = hip.attention_relpos(q, kt, v, table, h, w, hd ** -0.5).float()
    tol = 1e-5 * 2.0 if dtype == "f32" else 2e-3  # f32: the 1e-5 parity bar relative to max|v| = 2
    assert (out - const.float()).abs().max().item() <= tol
    v1 = torch.randn(bh, h * w, hd, device="cuda", generator=g).to(dt)
    v2 = torch.randn(bh, h * w, hd, device="cuda", generator=g).to(dt)
    o1 = hip.attention_relpos(q, kt, v1, table, h, w, hd ** -0.5).float()
    o2 = hip.attention_relpos(q, kt, v2, table, h, w, hd ** -0.5).float()
    o12 = hip.attention_relpos(q, kt, (v1.float() + v2.float()).to(dt), table, h, w, hd ** -0.5).float()
    lin_tol = 1e-4 if dtype == "f32" else 1e-2  # v1 + v2 is rounded once more in f16
    assert (o12 - o1 - o2).abs().max().item() <= lin_tol


def test_heads_are_independent(hip):
    """Permuting the batch-head axis permutes the output rows exactly (bit-identical)."""
    h = w = 14
    bh, hd = 40, 64
    g = torch.Generator(device="cuda").manual_seed(12)
    q = torch.randn(bh, h * w, hd, device="cuda", generator=g).half()
    kt = torch.randn(bh, hd, h * w, device="cuda", generator=g).half()
    v = torch.randn(bh, h * w, hd, device="cuda", generator=g).half()
    table = torch.randn(2 * h - 1 + 2 * w - 1, hd, device="cuda", generator=g).half()
    perm = torch.randperm(bh, device="cuda", generator=g)
    a = hip.attention_relpos(q, kt, v, table, h, w, 0.125)
    b = hip.attention_relpos(q[perm].contiguous(), kt[perm].contiguous(), v[perm].contiguous(), table, h, w, 0.125)
    assert torch.equal(a[perm], b)


def test_argument_errors_are_reported(hip):
    x = torch.zeros(2, 129 * 2, 16, device="cuda", dtype=torch.float16)
    kt = torch.zeros(2, 16, 129 * 2, device="cuda", dtype=torch.float16)
    t = torch.zeros(2 * 129 - 1 + 3, 16, device="cuda", dtype=torch.float16)
    with pytest.raises(hip.SamHipError, match="128x128"):
        hip.attention_relpos(x, kt, x, t, 129, 2, 0.25)
    with pytest.raises(hip.SamHipError, match="contiguous"):
        hip.attention_relpos(x.transpose(1, 2), kt, x, t, 129, 2, 0.25)
    y = torch.zeros(1, 6, 12, device="cuda", dtype=torch.float16)
    with pytest.raises(hip.SamHipError, match="multiple of 8"):
        hip.attention_relpos(y, torch.zeros(1, 12, 6, device="cuda", dtype=torch.float16), y,
                             torch.zeros(3 + 5, 12, device="cuda", dtype=torch.float16), 2, 3, 0.3)
    with pytest.raises(hip.SamHipError, match="dtype"):
        z = torch.zeros(1, 6, 8, device="cuda", dtype=torch.float64)
        hip.attention_relpos(z, torch.zeros(1, 8, 6, device="cuda", dtype=torch.float64), z,
                             torch.zeros(8, 8, device="cuda", dtype=torch.float64), 2, 3, 0.3)


def test_the_switch_on_device_tensors(hip):
    """set_enabled(False) (cpu_gemm::set_enabled's counterpart): a call raises SamHipDisabled and
    launches nothing, so the output buffer keeps what it held; set_enabled(True) gives the ordinary
    result again, equal to a call made before the switch."""
    g = torch.Generator(device="cuda").manual_seed(8)
    h = w = 14
    q = torch.randn(4, h * w, 80, device="cuda", generator=g).half()
    kt = torch.randn(4, 80, h * w, device="cuda", generator=g).half()
    v = torch.randn(4, h * w, 80, device="cuda", generator=g).half()
    table = (0.02 * torch.randn(4 * h - 2, 80, device="cuda", generator=g)).half()
    want = hip.attention_relpos(q, kt, v, table, h, w, 80 ** -0.5)
    L = hip.load()
    out = torch.full_like(q, 7.0)
    try:
        hip.set_enabled(False)
        assert not hip.enabled()
        with pytest.raises(hip.SamHipDisabled, match="switched off"):
            hip.attention_relpos(q, kt, v, table, h, w, 80 ** -0.5)
        rc = L.sam_hip_attn_relpos(q.data_ptr(), kt.data_ptr(), v.data_ptr(), table.data_ptr(), out.data_ptr(), 1, 4,
                                   h, w, 80, 80 ** -0.5, None)
        assert rc == 5
        torch.cuda.synchronize()
        assert bool((out == 7.0).all())
    finally:
        hip.set_enabled(True)
    assert hip.enabled()
    got = hip.attention_relpos(q, kt, v, table, h, w, 80 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_misaligned_operands_are_rejected(hip):
    """The kernels move q, kT, v, the table and out in 16-byte vectors, so the C ABI rejects pointers
    that are not 16-byte aligned instead of running on them. A view that starts one element into a
    buffer is contiguous but misaligned. (The Python front end copies such a view to an aligned buffer
    first, as a binding would; tests/test_degenerate_gpu.py checks that path.)"""
    import ctypes
    h = w = 14
    bh, hd = 2, 64
    n = h * w
    buf = torch.zeros(bh * n * hd + 8, device="cuda", dtype=torch.float16)
    ok = buf[: bh * n * hd].view(bh, n, hd)
    bad = buf[1: 1 + bh * n * hd].view(bh, n, hd)
    kt = torch.zeros(bh, hd, n, device="cuda", dtype=torch.float16)
    t = torch.zeros(2 * h - 1 + 2 * w - 1, hd, device="cuda", dtype=torch.float16)
    out = torch.empty(bh, n, hd, device="cuda", dtype=torch.float16)
    lib = hip.load()
    call = lambda q_, v_: lib.sam_hip_attn_relpos(q_.data_ptr(), kt.data_ptr(), v_.data_ptr(), t.data_ptr(),
                                                  out.data_ptr(), 1, bh, h, w, hd, ctypes.c_float(0.125),
                                                  hip._stream())
    assert call(ok, ok) == 0
    torch.cuda.synchronize()
    for args in [(bad, ok), (ok, bad)]:
        assert call(*args) == 3  # SAM_HIP_EUNSUPPORTED, before any launch
        assert b"16-byte aligned" in lib.sam_hip_last_error()


_THREADS_CHILD = r"""
import sys, threading
sys.path.insert(0, sys.argv[1])
import torch
import sam_hip
sam_hip.load()
g = torch.Generator(device="cuda").manual_seed(21)
cases = []
for h, w, bh, hd in [(14, 14, 50, 80), (64, 64, 2, 64), (64, 64, 2, 80), (14, 14, 30, 64)]:
    q = torch.randn(bh, h * w, hd, device="cuda", generator=g).half()
    kt = torch.randn(bh, hd, h * w, device="cuda", generator=g).half()
    v = torch.randn(bh, h * w, hd, device="cuda", generator=g).half()
    table = (0.02 * torch.randn(2 * h - 1 + 2 * w - 1, hd, device="cuda", generator=g)).half()
    cases.append((q, kt, v, table, h, w, hd ** -0.5))
torch.cuda.synchronize()
outs, errs = {}, []
start = threading.Barrier(2)

def work(i):
    try:
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            start.wait()
            # both threads make the first call of every kernel instance at about the same time
            order = range(len(cases)) if i == 0 else reversed(range(len(cases)))
            for _ in range(10):
                for c in order:
                    outs[(i, c)] = sam_hip.attention_relpos(*cases[c])
        s.synchronize()
    except Exception as e:
        errs.append(repr(e))

threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
for t in threads: t.start()
for t in threads: t.join(timeout=60)
assert not any(t.is_alive() for t in threads), "a thread did not finish"
assert not errs, errs
for c in range(len(cases)):
    ref = sam_hip.attention_relpos(*cases[c])
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(outs[(i, c)], ref), (i, c)
print("threads ok", flush=True)
"""


def test_calls_from_two_host_threads(hip):
    """The C ABI is safe to call from several host threads, including the first call of each kernel
    (its once-per-device LDS opt-in). A fresh child process, whose first calls into the library come
    from two threads on their own streams at once, runs the window and global kernels at hd 64 and 80
    ten times each; every output equals the same call made afterwards from the main thread."""
    import os
    import subprocess
    import sys

    pkg = os.path.dirname(hip.__file__)
    r = subprocess.run([sys.executable, "-c", _THREADS_CHILD, pkg], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "threads ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
