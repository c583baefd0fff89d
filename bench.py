"""Benchmark: SAM ViT-H image-encoder attention on one MI355X.

One step = the attention core of every encoder layer of ViT-H for one batch of 1024x1024 images:
28 windowed layers (25 windows x 16 heads per image, 14x14 tokens, hd 80, (27, 80) rel-pos tables) and
4 global layers (16 heads per image, 64x64 tokens, hd 80, (127, 80) tables), each one launch of the
fused rel-pos attention kernel on inputs already resident in HBM (fresh q/kT/v per layer).

Prints one JSON line: ms per image, the global-layer kernel's achieved TFLOP/s against the f16 MFMA
peak (timed live with HIP events on the launch stream), and the CPU oracle timed on this host. A
"secondary" object times the other kernels of the path at their workload shapes: the SAM encoder
attention sweep (ViT-B/L/H, batch 1/4/8), the ViT-B f32 layers, the ViT-H layers in bf16, SAM 3 ViT's
flash attention, SAM 2.1 memory attention (4 layers, f16), Grounding DINO-tiny deformable attention
(f32), relpos_softmax, qkv_split, qkv_rope, the bias ops, preprocessing, the image-encoder forwards,
and the platform's own GEMM and flash attention as references.

    python bench.py [--steps K] [--warmup W] [--batch B] [--dtype f16|bf16] [--no-cpu-baseline]
                    [--no-secondary] [--layers all|global|window] [--copy-probe]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sam-rs_amd"))

MFMA_PEAK_TFLOPS = {"f16": 2516.6, "bf16": 2516.6, "f32": 157.3}
HBM_PEAK_GBS = 8000.0
GLOBAL_LAYERS = (7, 15, 23, 31)
DEPTH, HEADS, HD = 32, 16, 80
WINDOWS = 25  # 64x64 tokens padded to 70x70 -> 5 x 5 windows of 14x14
CODE = {"f32": 0, "f16": 1, "bf16": 2}
WARM_MS = 100.0  # minimum GPU time of the headline's warmup, whatever --warmup says


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the GPU takes tens of milliseconds of load to reach its steady clock: 100 untimed steps (about
    # 0.1 s) come first, so the timed steps measure the steady state
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--dtype", default="f16", choices=["f16", "bf16"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--layers", default="all", choices=["all", "global", "window"],
                    help="restrict the step to one layer kind (for profiling one kernel)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a device copy of 256 MiB five times (the PMC byte-counter calibration)")
    return ap.parse_args()


def layer_shapes(batch):
    """(bh, h, w) of every encoder layer in order."""
    out = []
    for i in range(DEPTH):
        if i in GLOBAL_LAYERS:
            out.append((batch * HEADS, 64, 64))
        else:
            out.append((batch * WINDOWS * HEADS, 14, 14))
    return out


def flops(bh, n, hd=HD):
    return 4.0 * bh * n * n * hd


def window_bytes(bh, n, elem=2, hd=HD):
    return float(bh) * n * hd * elem * 4  # q, kT, v read once, out written once


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import sam_oracle

    return sam_oracle


def cpu_cores():
    return int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            return next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        return ""


def best_of(fn, reps):
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def cpu_baseline():
    """The reference's CPU attention, restated (oracle/), on the host threads, for one image's windowed
    layer and one image's global layer; ms/image = 28 x window + 4 x global. The reference runs its
    bf16 branch (TiledAttention with vdpbf16ps GEMMs, kernels.rs:166-179) by default when the CPU has
    AVX-512 BF16, and its exact-f32 branch (kernels.rs:181-220) otherwise; the default branch is the
    value, and the f32 branch is reported beside it."""
    import numpy as np

    sam_oracle = _oracle()
    cores = cpu_cores()
    r = np.random.default_rng(1)
    bf16 = sam_oracle.bf16_available()

    def layer(bh, h, w):
        n = h * w
        q = r.standard_normal((bh, n, HD), dtype=np.float32)
        kt = r.standard_normal((bh, HD, n), dtype=np.float32)
        v = r.standard_normal((bh, n, HD), dtype=np.float32)
        table = (0.02 * r.standard_normal((2 * h - 1 + 2 * w - 1, HD))).astype(np.float32)
        return q, kt, v, table, h, w, HD ** -0.5

    win, glob = layer(WINDOWS * HEADS, 14, 14), layer(HEADS, 64, 64)
    nw, ng = DEPTH - len(GLOBAL_LAYERS), len(GLOBAL_LAYERS)
    t32 = (best_of(lambda: sam_oracle.attention_relpos(*win, nthreads=cores), 3),
           best_of(lambda: sam_oracle.attention_relpos(*glob, nthreads=cores), 2))
    ms32 = 1e3 * (nw * t32[0] + ng * t32[1])
    out = {"unit": "ms/image", "cores": cores, "kind": "port", "cpu_model": cpu_model(), "nproc": os.cpu_count(),
           "f32_branch_ms": round(ms32, 1)}
    if bf16:
        tb = (best_of(lambda: sam_oracle.bf16_attention_relpos(*win, nthreads=cores), 3),
              best_of(lambda: sam_oracle.bf16_attention_relpos(*glob, nthreads=cores), 2))
        out.update(value=round(1e3 * (nw * tb[0] + ng * tb[1]), 1), branch="bf16 (the reference's default on "
                   "AVX-512 BF16 hosts: cpu_gemm.rs PackedB/vdpbf16ps, softmax_row/exp_ps)",
                   sample=f"one windowed layer (400 x 14x14) and one global layer (16 x 64x64) of one image, best "
                          f"of 3 and 2 runs (bf16 {tb[0]:.3f} s, {tb[1]:.3f} s; f32 {t32[0]:.3f} s, {t32[1]:.3f} s), "
                          "scaled by 28 and 4 layers")
    else:
        out.update(value=round(ms32, 1), branch="exact f32 (the reference's default without AVX-512 BF16)",
                   sample=f"one windowed layer (400 x 14x14) and one global layer (16 x 64x64) of one image, f32, "
                          f"best of 3 and 2 runs ({t32[0]:.3f} s, {t32[1]:.3f} s) scaled by 28 and 4 layers")
    return out


def cpu_leg(seconds, scale, unit_value, unit, sample, kind="port"):
    """A secondary leg's CPU baseline: `seconds` for the sample, times `scale` to the leg's workload."""
    return {"value": round(seconds * scale * unit_value, 4), "unit": unit, "cores": cpu_cores(), "kind": kind,
            "sample": sample}


def traffic_from_profiles():
    p = os.path.join(ROOT, "profiles", "attn_relpos_vit_h_global_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


class Timer:
    """One pair of HIP events on the launch stream around reps back-to-back calls; the average call
    time in ms (no markers between the calls).

    Before timing, fn runs at least `warmup` times and for at least `warm_s` seconds of GPU time: the
    chip reaches its steady clock only after tens of milliseconds of load, and a leg timed right after
    host-side work (the CPU baselines) would otherwise run its few timed calls on the ramp."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def avg_ms(self, fn, reps, warmup=2, warm_s=0.05):
        t0 = time.perf_counter()
        n = 0
        while n < warmup or time.perf_counter() - t0 < warm_s:
            for _ in range(max(warmup, 1)):
                fn()
            n += max(warmup, 1)
            self.torch.cuda.synchronize()
        a, b = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
        a.record(self.stream)
        for _ in range(reps):
            fn()
        b.record(self.stream)
        self.torch.cuda.synchronize()
        return a.elapsed_time(b) / reps


LLC_SPAN = 768 << 20  # three times MI355X's 256 MB last-level cache


def cold_sets(nbytes, *tensors):
    """Copies of a leg's operands (inputs and outputs) to cycle through: enough that more than the
    last-level cache is touched between two uses of one copy, so that an HBM-bound leg reads its
    operands from HBM on every timed call, as a model step does, and not from the cache that a
    repeated call on one set leaves them in."""
    n = max(1, -(-LLC_SPAN // int(nbytes)))
    return [tensors] + [tuple(t.clone() for t in tensors) for _ in range(n - 1)]


class Cycle:
    """A leg's timed call: fn on the next operand set each time."""

    def __init__(self, sets, fn):
        self.sets, self.fn, self.i = sets, fn, 0

    def __call__(self):
        self.fn(*self.sets[self.i])
        self.i = (self.i + 1) % len(self.sets)


def check(lib, rc):
    if rc:
        raise RuntimeError(lib.sam_hip_last_error().decode())


def secondary(torch, sam_hip, lib, dev, sp, timer, cpu=True):
    """The other kernels of the path at their workload shapes (synthetic inputs resident in HBM). With
    cpu, each leg also carries the reference's CPU path for it (restated in oracle/) timed on a bounded
    sample on the host threads."""
    res = {}
    g = torch.Generator(device=dev).manual_seed(7)
    vp = ctypes.c_void_p
    if cpu:
        import numpy as np

        orc = _oracle()
        cores = cpu_cores()
    host = lambda t: t.float().cpu().numpy()

    # SAM 2.1 memory attention: per layer self-attention (4096 x 4096) and cross-attention
    # (4096 x 7*4096 + 64 pointer tokens), one head, d 256, 2-D RoPE (theta 1e4) on a 64x64 grid.
    sys.path.insert(0, os.path.join(ROOT, "sam-rs_amd"))
    import math

    side, d, lq, mk, nptr = 64, 256, 4096, 7 * 4096 + 64, 64
    sp_ = d // 2
    inv = torch.tensor([1.0 / 10000.0 ** (2.0 * i / sp_) for i in range(sp_ // 2)], dtype=torch.float32)
    t = torch.arange(side * side)
    pos = torch.stack([(t % side).float(), (t // side).float()], 1)  # (col, row)
    ang = torch.cat([pos[:, :1] * inv, pos[:, 1:] * inv], 1)  # [N, sp]
    cos = torch.cos(ang).repeat_interleave(2, 1).contiguous().to(dev)
    sin = torch.sin(ang).repeat_interleave(2, 1).contiguous().to(dev)
    layers = []
    for _ in range(4):
        q = torch.randn(1, lq, 1, d, device=dev, generator=g).half()
        ks = torch.randn(1, lq, 1, d, device=dev, generator=g).half()
        vs = torch.randn(1, lq, 1, d, device=dev, generator=g).half()
        kc = torch.randn(1, mk, 1, d, device=dev, generator=g).half()
        vc = torch.randn(1, mk, 1, d, device=dev, generator=g).half()
        layers.append((q, ks, vs, kc, vc, torch.empty_like(q)))
    ws_bytes = max(lib.sam_hip_flash_attn_workspace_size(1, 1, lq, mk, 1, d, mk - nptr),
                   lib.sam_hip_flash_attn_workspace_size(1, 1, lq, lq, 1, d, lq))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    scale = d ** -0.5

    def attn(q, k, v, out, lk, nrk):
        check(lib, lib.sam_hip_flash_attn(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 1, 1, lq, lk, 1,
                                          d, None, None, None, None, scale, vp(cos.data_ptr()), vp(sin.data_ptr()),
                                          side * side, lq, nrk, vp(ws.data_ptr()), ws_bytes, sp))

    def mem_step():
        for q, ks, vs, kc, vc, out in layers:
            attn(q, ks, vs, out, lq, lq)
            attn(q, kc, vc, out, mk, mk - nptr)

    self_ms = timer.avg_ms(lambda: attn(*layers[0][:3], layers[0][5], lq, lq), 20)
    cross_ms = timer.avg_ms(lambda: attn(layers[0][0], layers[0][3], layers[0][4], layers[0][5], mk, mk - nptr), 20)
    total_ms = timer.avg_ms(mem_step, 5)
    f_self, f_cross = 4.0 * lq * lq * d, 4.0 * lq * mk * d
    res["sam2_memory_attention_f16"] = {
        "workload": "SAM 2.1 memory attention, 4 layers x (self 4096x4096 + cross 4096x28736), 1 head, d 256, "
                    "2-D RoPE on q and the 28672 memory keys (64 pointer keys unrotated)",
        "ms_4_layers": round(total_ms, 4),
        "self_us": round(self_ms * 1e3, 2), "cross_us": round(cross_ms * 1e3, 2),
        "tflops": round(4 * (f_self + f_cross) / (total_ms * 1e-3) / 1e12, 1),
        "self_tflops": round(f_self / (self_ms * 1e-3) / 1e12, 1),
        "cross_tflops": round(f_cross / (cross_ms * 1e-3) / 1e12, 1),
        "frac_of_f16_mfma_peak": round(4 * (f_self + f_cross) / (total_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"],
                                       4),
        "note": "time includes the key-rotation pass and the key-split combine; flops count attention only",
    }
    if cpu:
        # RopeAttn's core on the reference's CPU path (f32 rotation, then sdpa as matmul, softmax, matmul;
        # sam3/video.rs:106-145, sam3/nn.rs:26-34) for one layer's self and cross attention
        q0, ks0, vs0, kc0, vc0, _ = layers[0]
        c0, s0 = host(cos), host(sin)
        qh, ksh, vsh, kch, vch = (host(t[0, :, 0]) for t in (q0, ks0, vs0, kc0, vc0))
        ts = best_of(lambda: orc.rope_attention(qh, ksh, vsh, c0, s0, 0, nthreads=cores), 1)
        tc = best_of(lambda: orc.rope_attention(qh, kch, vch, c0, s0, nptr, nthreads=cores), 1)
        res["sam2_memory_attention_f16"]["cpu_baseline"] = cpu_leg(
            ts + tc, 4, 1e3, "ms (4 layers)",
            f"one layer's self ({ts:.3f} s) and cross ({tc:.3f} s) attention in f32 (the reference's CPU sdpa), "
            "scaled by 4 layers")
    del layers, ws

    # SAM 3 ViT image-encoder attention (sam3/vision.rs:96-121) at a 1008 x 1008 input, batch 1, f16: 72 x 72
    # tokens, 16 heads x 64, 32 layers of which 4 global (5184 tokens) and 28 windowed (9 windows of 24 x
    # 24 = 576 tokens); the flash attention the reference reaches through candle_flash_attn, each layer
    # on its own operands (q, k, v as the [nw, n, H, D] slices of the packed qkv_rope output).
    s3 = []
    for i in range(32):
        glob_layer = i in (7, 15, 23, 31)
        nw, n = (1, 5184) if glob_layer else (9, 576)
        qkv = torch.randn(3, nw, n, 16, 64, device=dev, generator=g).half()
        s3.append((nw, n, qkv, torch.empty(nw, n, 16, 64, device=dev, dtype=torch.float16)))
    s3ws = max(lib.sam_hip_flash_attn_workspace_size(1, nw_, n_, n_, 16, 64, 0) for nw_, n_, _, _ in s3[6:8])
    s3buf = torch.empty(max(s3ws, 1), dtype=torch.uint8, device=dev)

    def s3_call(L):
        nw, n, qkv, out = L
        check(lib, lib.sam_hip_flash_attn(qkv[0].data_ptr(), qkv[1].data_ptr(), qkv[2].data_ptr(), out.data_ptr(), 1,
                                          nw, n, n, 16, 64, None, None, None, None, 0.125, None, None, 0, 0, 0,
                                          vp(s3buf.data_ptr()), s3buf.numel(), sp))

    s3_ms = timer.avg_ms(lambda: [s3_call(L) for L in s3], 10, warm_s=0.1)
    s3w_ms = timer.avg_ms(lambda: [s3_call(L) for L in s3 if L[0] == 9], 10)
    s3g_ms = (s3_ms - s3w_ms) / 4
    f_w, f_g = 4.0 * 9 * 16 * 576 * 576 * 64, 4.0 * 16 * 5184 * 5184 * 64
    s3_fl = 28 * f_w + 4 * f_g
    res["sam3_vit_attention_f16"] = {
        "workload": "SAM 3 ViT image-encoder attention, 1008x1008 input, batch 1: 28 windowed layers (9 x 576 tokens) "
                    "+ 4 global layers (5184 tokens), 16 heads x 64, f16 flash attention",
        "ms_per_image": round(s3_ms, 4), "window_layer_us": round(s3w_ms / 28 * 1e3, 2),
        "global_layer_us": round(s3g_ms * 1e3, 2),
        "tflops": round(s3_fl / (s3_ms * 1e-3) / 1e12, 1),
        "frac_of_f16_mfma_peak": round(s3_fl / (s3_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"], 4),
        "global_frac_of_f16_mfma_peak": round(f_g / (s3g_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"], 4),
    }
    if cpu and orc.bf16_available():
        # the reference's CPU flash attention (cpu_gemm.rs:361-417, bf16 on AVX-512 BF16 hosts): one window
        # (16 heads) of a windowed layer and 2 of the 16 heads of a global layer, scaled to the image
        _, _, qkv_w, _ = s3[0]
        _, _, qkv_g, _ = s3[7]
        qw_, kw_, vw_ = (host(qkv_w[j, :1]) for j in range(3))
        qg_, kg_, vg_ = (host(qkv_g[j][:, :, :2]).copy() for j in range(3))
        tw_ = best_of(lambda: orc.bf16_flash_attention(qw_, kw_, vw_, nthreads=cores), 1)
        tg_ = best_of(lambda: orc.bf16_flash_attention(qg_, kg_, vg_, nthreads=cores), 1)
        res["sam3_vit_attention_f16"]["cpu_baseline"] = cpu_leg(
            tw_ * 9 * 28 + tg_ * 8 * 4, 1, 1e3, "ms/image",
            f"bf16 branch of the reference's CPU flash attention: one window of a windowed layer ({tw_:.3f} s, "
            f"x 9 windows x 28 layers) and 2 of 16 heads of a global layer ({tg_:.3f} s, x 8 x 4 layers)")
    del s3, s3buf

    # The ViT-H attention layers of the headline in bf16 (batch 1): the global layer (16 heads x 64x64) on
    # the bf16 MFMA, and a windowed layer (400 units x 14x14), each on fresh operand sets so that every
    # call reads its inputs from HBM, as the headline's layers do.
    for name, (bh, side) in (("global", (HEADS, 64)), ("window", (WINDOWS * HEADS, 14))):
        n = side * side
        qb = torch.randn(bh, n, HD, device=dev, generator=g).bfloat16()
        ktb = torch.randn(bh, HD, n, device=dev, generator=g).bfloat16()
        vb = torch.randn(bh, n, HD, device=dev, generator=g).bfloat16()
        tb = (0.02 * torch.randn(4 * side - 2, HD, device=dev, generator=g)).bfloat16()
        ob = torch.empty_like(qb)
        nbytes = window_bytes(bh, n)
        run = Cycle(cold_sets(nbytes, qb, ktb, vb, ob),
                    lambda q_, k_, v_, o_: check(lib, lib.sam_hip_attn_relpos(
                        q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), tb.data_ptr(), o_.data_ptr(), 2, bh, side, side,
                        HD, HD ** -0.5, sp)))
        ms = timer.avg_ms(run, 40 if name == "global" else 200, warm_s=0.1)
        del run
        f = flops(bh, n)
        leg = {"workload": f"SAM ViT-H {name} attention layer, bf16, batch 1: {bh} x {side}x{side}, hd {HD}",
               "us": round(ms * 1e3, 2), "tflops": round(f / (ms * 1e-3) / 1e12, 1)}
        if name == "global":
            leg["frac_of_bf16_mfma_peak"] = round(f / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["bf16"], 4)
        else:
            leg["gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            leg["frac_of_hbm_peak"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        res[f"vit_h_{name}_layer_bf16"] = leg
        del qb, ktb, vb, ob

    # A global layer past the 64 x 64 grid: ViT-H at a 1536 x 1536 input (96 x 96 tokens, 16 heads x 80),
    # f16. The reference's own GPU sequence stops at 8192 keys (its relpos_softmax limit); the fused
    # kernel walks the 96 columns in two 64-column passes.
    side = 96
    n = side * side
    qw = torch.randn(HEADS, n, HD, device=dev, generator=g).half()
    ktw = torch.randn(HEADS, HD, n, device=dev, generator=g).half()
    vw = torch.randn(HEADS, n, HD, device=dev, generator=g).half()
    tw = (0.02 * torch.randn(4 * side - 2, HD, device=dev, generator=g)).half()
    ow = torch.empty_like(qw)
    ms = timer.avg_ms(lambda: check(lib, lib.sam_hip_attn_relpos(qw.data_ptr(), ktw.data_ptr(), vw.data_ptr(),
                                                                  tw.data_ptr(), ow.data_ptr(), 1, HEADS, side, side,
                                                                  HD, HD ** -0.5, sp)), 10)
    f = flops(HEADS, n)
    res["vit_h_global_layer_96x96_f16"] = {
        "workload": f"SAM ViT-H global attention layer at a 1536x1536 input, f16: {HEADS} x {side}x{side}, hd {HD} "
                    "(past the reference GPU path's 8192-key limit)",
        "us": round(ms * 1e3, 2), "tflops": round(f / (ms * 1e-3) / 1e12, 1),
        "frac_of_f16_mfma_peak": round(f / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"], 4)}
    del qw, ktw, vw, ow

    # Platform references for the MFMA roofline, on this GPU in this run: torch's own flash attention
    # (scaled_dot_product_attention, no bias) at the ViT-H global layer's shape, and a plain hipBLASLt f16
    # GEMM through torch. Neither is part of the path; they show what the platform's own kernels reach
    # against the same 2516.6 TFLOP/s peak.
    import torch.nn.functional as F

    qs, ks, vs = (torch.randn(1, HEADS, 4096, HD, device=dev, generator=g).half() for _ in range(3))
    try:
        with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.FLASH_ATTENTION):
            ms = timer.avg_ms(lambda: F.scaled_dot_product_attention(qs, ks, vs), 30, warm_s=0.1)
        f = flops(HEADS, 4096)
        res["reference_torch_flash_sdpa_vit_h_global_f16"] = {
            "workload": f"torch scaled_dot_product_attention (flash backend, no rel-pos bias), [1, {HEADS}, 4096, {HD}] f16",
            "us": round(ms * 1e3, 2), "tflops": round(f / (ms * 1e-3) / 1e12, 1),
            "frac_of_f16_mfma_peak": round(f / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"], 4)}
    except RuntimeError as e:  # no flash backend in this torch build
        res["reference_torch_flash_sdpa_vit_h_global_f16"] = {"error": str(e)[:120]}
    del qs, ks, vs
    ga = torch.randn(8192, 8192, device=dev, generator=g).half()
    gb = torch.randn(8192, 8192, device=dev, generator=g).half()
    ms = timer.avg_ms(lambda: torch.matmul(ga, gb), 20, warm_s=0.1)
    res["reference_hipblaslt_gemm_f16_8192"] = {
        "workload": "torch.matmul f16 8192 x 8192 x 8192 (hipBLASLt)",
        "us": round(ms * 1e3, 2), "tflops": round(2 * 8192 ** 3 / (ms * 1e-3) / 1e12, 1),
        "frac_of_f16_mfma_peak": round(2 * 8192 ** 3 / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"], 4)}
    del ga, gb

    # Grounding DINO-tiny deformable attention, f32: 4 levels of an 800x1333 input, 8 heads x 32, 4 points.
    shapes = [(100, 167), (50, 84), (25, 42), (13, 21)]
    s = sum(a * b for a, b in shapes)
    hh, dd, ll, pp = 8, 32, 4, 4
    # The gather's own ceiling: 16-byte pieces of random 128-byte rows from one head's value rows (an
    # L2-resident 2.85 MB region), 16 loads in flight per lane, as the deform gather reads its corner rows
    # (measurement kernel in libsam_probe.so). Bytes delivered to registers / time.
    probe = ctypes.CDLL(os.path.join(ROOT, "sam-rs_amd", "libsam_probe.so"))
    probe.sam_probe_gather.argtypes = [vp, ctypes.c_uint, ctypes.c_int, ctypes.c_int, vp, vp]
    region = torch.randn(s * dd, device=dev, generator=g)  # s rows of 128 bytes
    pblocks, psteps = 1024, 256
    pout = torch.empty(pblocks * 256, device=dev)
    def run_probe():
        if probe.sam_probe_gather(region.data_ptr(), s, psteps, pblocks, pout.data_ptr(), sp) != 0:
            raise RuntimeError("gather probe launch failed")

    pms = timer.avg_ms(run_probe, 20)
    gather_ceiling_gbs = pblocks * 256 * psteps * 16 / (pms * 1e-3) / 1e9
    res["gather_ceiling_16b_rows_l2"] = {
        "workload": "16-byte loads of random 128-byte rows of a 2.85 MB region (one DINO-tiny head's value rows), "
                    "8 lanes per row, 16 loads in flight per lane, 1024 x 256 lanes",
        "us": round(pms * 1e3, 2), "gbs": round(gather_ceiling_gbs, 1)}
    del region, pout
    value = torch.randn(1, s, hh, dd, device=dev, generator=g)
    flat = (ctypes.c_int * 8)(*[x for hw in shapes for x in hw])
    for name, q in (("encoder", s), ("decoder", 900)):
        ref = torch.rand(1, q, 1, 1, 1, 2, device=dev, generator=g)
        wh = torch.tensor([[w_, h_] for h_, w_ in shapes], device=dev, dtype=torch.float32).view(1, 1, 1, ll, 1, 2)
        off = 2.0 * torch.randn(1, q, hh, ll, pp, 2, device=dev, generator=g)
        loc = (ref + off / wh).contiguous()
        attn_w = torch.softmax(torch.randn(1, q, hh, ll * pp, device=dev, generator=g), -1).view(1, q, hh, ll, pp)
        attn_w = attn_w.contiguous()
        out = torch.empty(1, q, hh * dd, device=dev)
        nbytes = 4.0 * (s * hh * dd + 3 * q * hh * ll * pp + q * hh * dd)
        run = Cycle(cold_sets(nbytes, value, loc, attn_w, out),
                    lambda va, lo, aw, o: check(lib, lib.sam_hip_deform_attn(va.data_ptr(), lo.data_ptr(), aw.data_ptr(),
                                                                             o.data_ptr(), 0, 1, s, q, hh, dd, ll, pp,
                                                                             flat, sp)))
        ms = timer.avg_ms(run, 50)
        del run
        gathered = 4.0 * q * hh * ll * pp * 4 * dd
        res[f"dino_deform_{name}_f32"] = {
            "workload": f"Grounding DINO-tiny deformable attention, {q} queries over {s} values, 8 heads x 32, "
                        "4 levels x 4 points",
            "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            # the corner rows the gather delivers to registers (4 per point, D f32 each)
            "gathered_bytes": gathered, "gathered_gbs": round(gathered / (ms * 1e-3) / 1e9, 1),
            "frac_of_gather_ceiling": round(gathered / (ms * 1e-3) / 1e9 / gather_ceiling_gbs, 4),
        }
        if cpu:
            vh, lh, ah = host(value), host(loc), host(attn_w)
            tcpu = best_of(lambda: orc.deform_attn(vh, lh, ah, shapes, nthreads=cores), 3)
            res[f"dino_deform_{name}_f32"]["cpu_baseline"] = cpu_leg(
                tcpu, 1, 1e6, "us", f"the whole layer on cpu::DeformAttn (kernels.rs:776-818), best of 3")

        # the same layer through Deform::forward's fused core: offsets, logits and reference points in
        # place of loc and attn (softmax and sampling locations formed in the kernel)
        refs = (ref.view(1, q, 1, 2).expand(1, q, ll, 2) if name == "encoder" else
                torch.cat([ref.view(1, q, 1, 2), 0.05 + 0.5 * torch.rand(1, q, 1, 2, device=dev, generator=g)],
                          -1).expand(1, q, ll, 4)).contiguous()
        logits = torch.randn(1, q, hh, ll, pp, device=dev, generator=g)

        nbytes = 4.0 * (s * hh * dd + 3 * q * hh * ll * pp + q * ll * refs.shape[3] + q * hh * dd)
        nref = refs.shape[3]
        run_core = Cycle(cold_sets(nbytes, value, off, logits, refs, out),
                         lambda va, of, lg, rf, o: check(lib, lib.sam_hip_deform_core(
                             va.data_ptr(), of.data_ptr(), lg.data_ptr(), rf.data_ptr(), o.data_ptr(), 0, 1, s, q, hh,
                             dd, ll, pp, nref, flat, sp)))
        ms = timer.avg_ms(run_core, 50)
        del run_core
        res[f"dino_deform_core_{name}_f32"] = {
            "workload": f"Grounding DINO-tiny Deform::forward core (logit softmax + {refs.shape[3]}-coordinate "
                        f"sampling locations + gather), {q} queries over {s} values, 8 heads x 32, 4 levels x 4 points",
            "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "gathered_bytes": gathered, "gathered_gbs": round(gathered / (ms * 1e-3) / 1e9, 1),
            "frac_of_gather_ceiling": round(gathered / (ms * 1e-3) / 1e9 / gather_ceiling_gbs, 4),
        }
        if cpu:
            oh, gh, rh = host(off), host(logits), host(refs)
            tcpu = best_of(lambda: orc.deform_forward_core(vh, oh, gh, rh, shapes, nthreads=cores), 3)
            res[f"dino_deform_core_{name}_f32"]["cpu_baseline"] = cpu_leg(
                tcpu, 1, 1e6, "us", "the whole layer: softmax and sampling locations (dino/mod.rs:166-178), then "
                                    "cpu::DeformAttn, best of 3")

    # relpos_softmax (the reference's GPU step between its two bmm calls) over materialised f16 scores:
    # a ViT-H global layer (16 heads x 4096 rows of 4096) and a windowed layer (400 units x 196 rows of
    # 196). Compulsory bytes: the scores read once and the probabilities written once (q and the table
    # add under 1%).
    for name, (bh, side) in (("global", (16, 64)), ("window", (400, 14))):
        n = side * side
        sc = torch.randn(bh, n, n, device=dev, generator=g).half()
        qq = torch.randn(bh, n, HD, device=dev, generator=g).half()
        tb = (0.02 * torch.randn(4 * side - 2, HD, device=dev, generator=g)).half()
        pr = torch.empty_like(sc)
        nbytes = 2.0 * bh * n * n * 2 + bh * n * HD * 2
        run = Cycle(cold_sets(nbytes, sc, qq, pr),
                    lambda sc_, qq_, pr_: check(lib, lib.sam_hip_relpos_softmax(
                        sc_.data_ptr(), qq_.data_ptr(), tb.data_ptr(), pr_.data_ptr(), 1, bh * n, side, side, HD,
                        HD ** -0.5, sp)))
        ms = timer.avg_ms(run, 20)
        del run
        res[f"vit_h_relpos_softmax_{name}_f16"] = {
            "workload": f"SAM ViT-H relpos_softmax over materialised scores, {bh} x {n} rows of {n}, hd {HD}, f16",
            "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        if cpu:
            part = 1 if name == "global" else 40  # one head of the global layer, 40 of the 400 window units
            sh_, qh_, th_ = host(sc[:part]), host(qq[:part]), host(tb)
            tcpu = best_of(lambda: orc.relpos_softmax(sh_, qh_, th_, side, side, HD ** -0.5, nthreads=cores), 2)
            res[f"vit_h_relpos_softmax_{name}_f16"]["cpu_baseline"] = cpu_leg(
                tcpu, bh / part, 1e6, "us", f"{part} of the {bh} units on cpu::RelposSoftmax (kernels.rs:62-105, "
                                            f"f32), best of 2, scaled by {bh // part}")
        del sc, pr

    # SAM image preprocessing (image_proc::prepare): a u8 RGB image resized so its longest side is 1024,
    # normalised and zero padded into [1, 3, 1024, 1024], for a 1920x1080 frame and a 4000x3000 photo.
    for name, (ih, iw) in (("1080p", (1080, 1920)), ("12mp", (3000, 4000))):
        img = torch.randint(0, 256, (ih, iw, 3), dtype=torch.uint8, device=dev, generator=g)
        nh, nw, _ = sam_hip.resized_hw(ih, iw, 1024)
        for dname, odt in (("f16", torch.float16), ("f32", torch.float32)):
            out = torch.empty((1, 3, 1024, 1024), dtype=odt, device=dev)
            mean = (ctypes.c_float * 3)(*sam_hip.SAM_MEAN)
            std = (ctypes.c_float * 3)(*sam_hip.SAM_STD)
            code = CODE[dname]
            nbytes = float(ih * iw * 3 + 3 * 1024 * 1024 * out.element_size())
            run = Cycle(cold_sets(nbytes, img, out),
                        lambda im, o: check(lib, lib.sam_hip_preprocess(im.data_ptr(), o.data_ptr(), code, ih, iw, nh,
                                                                        nw, 1024, mean, std, sp)))
            ms = timer.avg_ms(run, 50)
            del run
            res[f"preprocess_{name}_{dname}"] = {
                "workload": f"SAM image preprocessing: u8 {iw}x{ih} RGB -> resize to {nw}x{nh} (antialiased), "
                            f"normalise, pad to 3x1024x1024 {dname}",
                "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
                "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            }
            if cpu:
                ih_ = img.cpu().numpy()
                tcpu = best_of(lambda: orc.preprocess(ih_, nh, nw, 1024, nthreads=cores), 3)
                res[f"preprocess_{name}_{dname}"]["cpu_baseline"] = cpu_leg(
                    tcpu, 1, 1e6, "us", "the whole image on image_proc::resize_normalize (image_proc.rs:57-96, f32), "
                                        "best of 3")

    # The encoder attention sweep (ViT-B / ViT-L / ViT-H, f16, batch 1, 4 and 8): every attention layer of
    # the encoder, each layer on its own q/kT/v, back to back, in ms per image. Windowed layers are
    # batch x 25 windows x heads units of 14x14; global layers batch x heads 64x64 grids.
    for mname, (depth, heads, hd, glob) in (("vit_b", (12, 12, 64, (2, 5, 8, 11))),
                                            ("vit_l", (24, 16, 64, (5, 11, 17, 23))),
                                            ("vit_h", (32, 16, 80, (7, 15, 23, 31)))):
        for batch in (1, 4, 8):
            kinds = {}
            for i in range(depth):
                key = (batch * heads, 64) if i in glob else (batch * WINDOWS * heads, 14)
                kinds[key] = kinds.get(key, 0) + 1
            layer_us = {}
            for (bh, side), count in kinds.items():
                n = side * side
                q = torch.randn(bh, n, hd, device=dev, generator=g).half()
                kt = torch.randn(bh, hd, n, device=dev, generator=g).half()
                v = torch.randn(bh, n, hd, device=dev, generator=g).half()
                table = (0.02 * torch.randn(4 * side - 2, hd, device=dev, generator=g)).half()
                out = torch.empty_like(q)
                # one input set per layer, as in the encoder: a repeated set would stay in the 256 MB
                # last-level cache (a ViT-H windowed layer at batch 1 reads 50 MB)
                sets = [(q, kt, v, out)] + [(q.clone(), kt.clone(), v.clone(), torch.empty_like(q))
                                            for _ in range(count - 1)]

                def run():
                    for qq, kk, vv, oo in sets:
                        check(lib, lib.sam_hip_attn_relpos(qq.data_ptr(), kk.data_ptr(), vv.data_ptr(),
                                                           table.data_ptr(), oo.data_ptr(), 1, bh, side, side, hd,
                                                           hd ** -0.5, sp))

                layer_us[side] = (timer.avg_ms(run, 10 if batch > 1 else 30) * 1e3 / len(sets), count, bh, n)
                del q, kt, v, out, sets
            total_ms = sum(us * c for us, c, _, _ in layer_us.values()) / 1e3
            gf = sum(flops(bh, n, hd) * c for _, c, bh, n in layer_us.values()) / 1e9
            res[f"sweep_{mname}_attention_b{batch}_f16"] = {
                "workload": f"SAM {mname.replace('_', '-').upper()} encoder attention, {depth} layers, {heads} heads x "
                            f"{hd}, batch {batch}, f16",
                "ms_per_image": round(total_ms / batch, 4),
                "window_layer_us": round(layer_us[14][0], 2), "global_layer_us": round(layer_us[64][0], 2),
                "tflops": round(gf / total_ms, 1),
            }
        if cpu:
            # the reference's default CPU attention (bf16 branch on AVX-512 BF16 hosts, else exact f32) per
            # image: one whole windowed layer (25 windows x heads) and one whole global layer, scaled by the
            # encoder's layer counts (the CPU cost is linear in layers and in batch)
            fn = orc.bf16_attention_relpos if orc.bf16_available() else orc.attention_relpos
            rr = np.random.default_rng(3)

            def units(bh, side):
                n = side * side
                return (rr.standard_normal((bh, n, hd), dtype=np.float32),
                        rr.standard_normal((bh, hd, n), dtype=np.float32),
                        rr.standard_normal((bh, n, hd), dtype=np.float32),
                        (0.02 * rr.standard_normal((4 * side - 2, hd))).astype(np.float32))

            wu, gu = units(WINDOWS * heads, 14), units(heads, 64)
            tw = best_of(lambda: fn(*wu, 14, 14, hd ** -0.5, nthreads=cores), 2)
            tg = best_of(lambda: fn(*gu, 64, 64, hd ** -0.5, nthreads=cores), 2)
            ng_ = len(glob)
            leg = cpu_leg(1.0, 1.0, 1e3 * ((depth - ng_) * tw + ng_ * tg), "ms/image",
                          f"{'bf16' if orc.bf16_available() else 'exact f32'} branch of the reference's CPU attention: "
                          f"one whole windowed layer, {WINDOWS} windows x {heads} heads ({tw:.3f} s), and one whole "
                          f"global layer, {heads} heads ({tg:.3f} s), best of 2, times {depth - ng_} windowed and "
                          f"{ng_} global layers")
            for batch in (1, 4, 8):
                res[f"sweep_{mname}_attention_b{batch}_f16"]["cpu_baseline"] = leg

    # Encoder-level timing: the whole SAM image encoder (patch embedding, all blocks with their qkv / proj
    # / MLP linears on hipBLASLt through torch, LayerNorms, the neck) on this library's attention,
    # qkv_split, bias_residual and bias_gelu, f16, one 1024x1024 image; random-init weights N(0, 0.02).
    # The reference's README gives 38 / 74 / 96 ms for these encoders on an RTX 4090 (f16, CUDA).
    import sam_encoder

    img = torch.randn(1, 3, 1024, 1024, device=dev, generator=g).half()
    for name, cfg, readme_ms in (("vit_b", sam_encoder.VIT_B, 38.0), ("vit_l", sam_encoder.VIT_L, 74.0),
                                 ("vit_h", sam_encoder.VIT_H, 96.0)):
        wts = sam_encoder.random_weights(cfg, dtype=torch.float16, device=dev, seed=11)
        with torch.no_grad():
            ms = timer.avg_ms(lambda: sam_encoder.encoder_forward(img, wts), 10)
        res[f"sam_{name}_encoder_f16"] = {
            "workload": f"SAM {name.replace('_', '-').upper()} image encoder forward, 1024x1024, batch 1, f16 "
                        f"({cfg.depth} blocks, dim {cfg.embed_dim}, {cfg.heads} heads)",
            "ms": round(ms, 3), "readme_rtx4090_ms": readme_ms,
            "note": "linears on torch/hipBLASLt, attention and elementwise steps on libsam_hip; synthetic weights",
        }
        del wts

    # qkv_split of a ViT-H block (f16): the qkv projection's output [T, 3 x 1280] plus bias into q, kT, v
    # for the 25 windows x 196 tokens of a windowed block (the grid padded to 70x70) and the 4096 tokens
    # of a global block.
    for name, (tok, n) in (("window", (4900, 196)), ("global", (4096, 4096))):
        y = torch.randn(tok, 3 * 1280, device=dev, generator=g).half()
        bq = torch.randn(3 * 1280, device=dev, generator=g).half()
        packed = torch.empty(3, tok * 1280, device=dev, dtype=torch.float16)
        nbytes = 2.0 * tok * 3 * 1280 * 2
        run = Cycle(cold_sets(nbytes, y, packed),
                    lambda y_, pk: check(lib, lib.sam_hip_qkv_split(y_.data_ptr(), bq.data_ptr(), pk.data_ptr(), 1, tok,
                                                                    n, 16, 80, sp)))
        ms = timer.avg_ms(run, 50)
        del run
        res[f"vit_h_qkv_split_{name}_f16"] = {
            "workload": f"SAM ViT-H qkv_split, {tok} tokens ({n} per window) x 16 heads x 80, f16",
            "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        if cpu:
            yh, bh_ = host(y), host(bq)
            tcpu = best_of(lambda: orc.qkv_split(yh, bh_, n, 16, 80, nthreads=cores), 3)
            res[f"vit_h_qkv_split_{name}_f16"]["cpu_baseline"] = cpu_leg(
                tcpu, 1, 1e6, "us", "the whole block on cpu::QkvSplit (kernels.rs:239-263, f32), best of 3")

    # qkv_rope of a SAM 3 ViT block (f16): the fused qkv projection's output [5184, 3 x 1024] plus bias,
    # 2-D RoPE on q and k, packed [3, T, 16, 64]; windowed blocks use 24x24-token tables (9 windows of a
    # 72x72 grid), global blocks one 72x72 table.
    for name, n in (("window", 576), ("global", 5184)):
        tok, c3 = 5184, 3 * 1024
        y = torch.randn(tok, c3, device=dev, generator=g).half()
        bq = torch.randn(c3, device=dev, generator=g).half()
        cs = torch.rand(n, 64, device=dev, generator=g)
        sn = torch.rand(n, 64, device=dev, generator=g)
        packed = torch.empty(3, tok, 16, 64, device=dev, dtype=torch.float16)
        nbytes = 2.0 * tok * c3 * 2 + 2 * n * 64 * 4
        run = Cycle(cold_sets(nbytes, y, packed),
                    lambda y_, pk: check(lib, lib.sam_hip_qkv_rope(y_.data_ptr(), bq.data_ptr(), cs.data_ptr(),
                                                                   sn.data_ptr(), pk.data_ptr(), 1, tok, n, 16, 64,
                                                                   sp)))
        ms = timer.avg_ms(run, 50)
        del run
        res[f"sam3_qkv_rope_{name}_f16"] = {
            "workload": f"SAM 3 ViT qkv_rope, {tok} tokens (tables of {n} rows) x 16 heads x 64, f16",
            "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        if cpu:
            yh, bh_, ch, sh = host(y), host(bq), host(cs), host(sn)
            tcpu = best_of(lambda: orc.qkv_rope(yh, bh_, ch, sh, n, 16, 64, nthreads=cores), 3)
            res[f"sam3_qkv_rope_{name}_f16"]["cpu_baseline"] = cpu_leg(
                tcpu, 1, 1e6, "us", "the whole block on cpu::QkvRope (kernels.rs:321-362, f32), best of 3")

    # The elementwise steps beside attention in a ViT-H block, f16: the projection output plus bias plus
    # the residual (4096 tokens x 1280), and the MLP's bias + exact GELU (4096 x 5120).
    for name, (rows, cols) in (("bias_residual", (4096, 1280)), ("bias_gelu", (4096, 5120))):
        y = torch.randn(rows, cols, device=dev, generator=g).half()
        resid = torch.randn(rows, cols, device=dev, generator=g).half()
        bvec = torch.randn(cols, device=dev, generator=g).half()
        out = torch.empty_like(y)
        if name == "bias_residual":
            nbytes = 3.0 * rows * cols * 2
            run = Cycle(cold_sets(nbytes, resid, y, out),
                        lambda r_, y_, o: check(lib, lib.sam_hip_bias_residual(r_.data_ptr(), y_.data_ptr(),
                                                                               bvec.data_ptr(), o.data_ptr(), 1,
                                                                               rows * cols, cols, sp)))
        else:
            nbytes = 2.0 * rows * cols * 2
            run = Cycle(cold_sets(nbytes, y, out),
                        lambda y_, o: check(lib, lib.sam_hip_bias_gelu(y_.data_ptr(), bvec.data_ptr(), o.data_ptr(), 1,
                                                                       rows * cols, cols, sp)))
        ms = timer.avg_ms(run, 50)
        del run
        res[f"vit_h_{name}_f16"] = {
            "workload": f"SAM ViT-H {name} over {rows} tokens x {cols} channels, f16",
            "us": round(ms * 1e3, 2), "compulsory_bytes": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        if cpu:
            yh, rh_, bh_ = host(y), host(resid), host(bvec)
            f = (lambda: orc.bias_residual(rh_, yh, bh_)) if name == "bias_residual" else (lambda: orc.bias_gelu(yh, bh_))
            tcpu = best_of(f, 2)
            res[f"vit_h_{name}_f16"]["cpu_baseline"] = cpu_leg(
                tcpu, 1, 1e6, "us", f"the whole tensor on cpu::{'BiasResidual' if name == 'bias_residual' else 'BiasGelu'} "
                                    "(kernels.rs:618-663, f32, one thread), best of 2", kind="port")
            res[f"vit_h_{name}_f16"]["cpu_baseline"]["cores"] = 1

    # SAM ViT-B encoder attention layers, f32 (12 heads x 64): window 300 x 14x14, global 12 x 64x64.
    for name, bh, hw in (("window", 300, 14), ("global", 12, 64)):
        n = hw * hw
        q = torch.randn(bh, n, 64, device=dev, generator=g)
        kt = torch.randn(bh, 64, n, device=dev, generator=g)
        v = torch.randn(bh, n, 64, device=dev, generator=g)
        table = 0.02 * torch.randn(2 * (2 * hw - 1), 64, device=dev, generator=g)
        out = torch.empty_like(q)

        def run():
            check(lib, lib.sam_hip_attn_relpos(q.data_ptr(), kt.data_ptr(), v.data_ptr(), table.data_ptr(),
                                               out.data_ptr(), 0, bh, hw, hw, 64, 0.125, sp))

        ms = timer.avg_ms(run, 20)
        f = flops(bh, n, 64)
        res[f"vit_b_{name}_f32"] = {
            "workload": f"SAM ViT-B {name} attention layer, f32, {bh} x {hw}x{hw}, hd 64",
            "us": round(ms * 1e3, 2), "tflops": round(f / (ms * 1e-3) / 1e12, 2),
            "frac_of_f32_peak": round(f / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f32"], 4),
        }
        if cpu:
            arr = [host(t) for t in (q, kt, v, table)]
            tcpu = best_of(lambda: orc.attention_relpos(*arr, hw, hw, 0.125, nthreads=cores), 2)
            res[f"vit_b_{name}_f32"]["cpu_baseline"] = cpu_leg(
                tcpu, 1, 1e6, "us", "the whole layer on the reference's exact-f32 TiledAttention branch "
                                    "(kernels.rs:181-220), best of 2")
    late = [k for k in ("reference_hipblaslt_gemm_f16_8192", "reference_torch_flash_sdpa_vit_h_global_f16",
                        "dino_deform_core_decoder_f32", "dino_deform_decoder_f32", "dino_deform_core_encoder_f32",
                        "dino_deform_encoder_f32", "sam2_memory_attention_f16", "vit_h_window_layer_bf16",
                        "vit_h_global_layer_bf16") if k in res]
    return {**{k: v for k, v in res.items() if k not in late}, **{k: res[k] for k in late}}


def copy_probe(torch):
    """A device-to-device copy of 256 MiB, five times: reads and writes 256 MiB per launch, the known
    byte count that scales the FETCH_SIZE / WRITE_SIZE counters."""
    dev = torch.device("cuda:0")
    a = torch.ones(64 << 20, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": a.numel() * 4, "launches": 5}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the attention path shards over "
              "(batch, window, head) with no exchange, so N GPUs run N independent copies of this line.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if args.copy_probe:
        copy_probe(torch)
        return

    import sam_hip

    lib = sam_hip.load()
    dev = torch.device("cuda:0")
    dt = {"f16": torch.float16, "bf16": torch.bfloat16}[args.dtype]
    g = torch.Generator(device=dev).manual_seed(0)
    layers = []
    for bh, h, w in layer_shapes(args.batch):
        n = h * w
        q = torch.randn(bh, n, HD, device=dev, generator=g, dtype=torch.float32).to(dt)
        kt = torch.randn(bh, HD, n, device=dev, generator=g, dtype=torch.float32).to(dt)
        v = torch.randn(bh, n, HD, device=dev, generator=g, dtype=torch.float32).to(dt)
        table = (0.02 * torch.randn(2 * h - 1 + 2 * w - 1, HD, device=dev, generator=g)).to(dt)
        out = torch.empty_like(q)
        layers.append((bh, h, w, q, kt, v, table, out))
    scale = HD ** -0.5
    code = CODE[args.dtype]
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)

    def launch(L):
        bh, h, w, q, kt, v, table, out = L
        check(lib, lib.sam_hip_attn_relpos(q.data_ptr(), kt.data_ptr(), v.data_ptr(), table.data_ptr(),
                                           out.data_ptr(), code, bh, h, w, HD, scale, sp))

    keep = {"all": lambda i: True, "global": lambda i: i in GLOBAL_LAYERS,
            "window": lambda i: i not in GLOBAL_LAYERS}[args.layers]

    def step():
        for i, L in enumerate(layers):
            if keep(i):
                launch(L)

    # Warmup: the given number of steps, then more until at least WARM_MS of GPU time has passed since
    # the first. The chip reaches its steady clock only after tens of milliseconds of load, so a fixed
    # small step count would time part of the clock ramp.
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0.record(stream)
    warm_steps = 0
    for _ in range(args.warmup):
        step()
        warm_steps += 1
    w1.record(stream)
    torch.cuda.synchronize()
    warm_ms = w0.elapsed_time(w1)
    while warm_ms < WARM_MS:
        per_step = warm_ms / max(warm_steps, 1)
        for _ in range(1 + int((WARM_MS - warm_ms) / max(per_step, 1e-3))):
            step()
            warm_steps += 1
        w1.record(stream)
        torch.cuda.synchronize()
        warm_ms = w0.elapsed_time(w1)
    # The timed region: plain steps, bracketed by events on the launch stream. Events between the layers
    # would put host calls and queue markers between the kernels and lengthen the step by about a
    # quarter, so the per-kernel durations come from a second region right after it.
    t0e, t1e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0e.record(stream)
    for _ in range(args.steps):
        step()
    t1e.record(stream)
    torch.cuda.synchronize()
    ms_total = t0e.elapsed_time(t1e)
    ms_step = ms_total / args.steps
    # Per-kernel durations. An event pair around every launch adds its marker overhead (a few
    # microseconds) to each kernel, so: the window layers' launches of args.steps steps back to back
    # between one pair of events on the launch stream give the window kernel's duration, and the global
    # kernel's is its share of the timed step, (step - window layers) / global layers. Run alone back to
    # back, the global layers would find their inputs in the last-level cache that the window layers'
    # traffic flushes within a step, and run about 3% faster than they do in it.
    def region(sel):
        idx = [i for i in range(len(layers)) if keep(i) and sel(i)]
        if not idx:
            return 0.0, 0
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(args.steps):
            for i in idx:
                launch(layers[i])
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (args.steps * len(idx)), len(idx)

    win_ms, n_win = region(lambda i: i not in GLOBAL_LAYERS)
    n_glob = sum(1 for i in range(len(layers)) if keep(i) and i in GLOBAL_LAYERS)
    glob_ms = (ms_step - win_ms * n_win) / n_glob if n_glob else 0.0
    if args.layers != "all":
        print(json.dumps({"layers": args.layers, "ms_per_step": ms_step, "global_layer_us": glob_ms * 1e3,
                          "window_layer_us": win_ms * 1e3}), flush=True)
        return

    gbh, wbh = args.batch * HEADS, args.batch * WINDOWS * HEADS
    g_flops = flops(gbh, 4096)
    w_flops = flops(wbh, 196)
    achieved = g_flops / (glob_ms * 1e-3) / 1e12
    peak = MFMA_PEAK_TFLOPS[args.dtype]
    win_gbs = window_bytes(wbh, 196) / (win_ms * 1e-3) / 1e9
    total_flops = len(GLOBAL_LAYERS) * g_flops + (DEPTH - len(GLOBAL_LAYERS)) * w_flops

    line = {
        "metric": "ViT-H encoder attention ms/image (f16) + achieved TFLOP/s vs MFMA peak",
        "value": round(ms_step / args.batch, 4),
        "unit": "ms/image",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "warmup_ms": round(warm_ms, 1),
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic",
        "config": {
            "workload": f"SAM ViT-H encoder attention (fused q.kT + decomposed rel-pos + softmax + .v), "
                        f"1024x1024 images, batch {args.batch}: 28 windowed layers ({wbh} x 14x14, hd 80) + "
                        f"4 global layers ({gbh} x 64x64, hd 80)",
            "batch": args.batch,
            "layers": DEPTH,
            "global_layers": list(GLOBAL_LAYERS),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "attn_relpos_glob_kernel (global 64x64 layer)",
            "achieved": round(achieved, 1),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic_from_profiles() if args.batch == 1 else None,
        },
        "global_layer_us": round(glob_ms * 1e3, 2),
        "window_layer_us": round(win_ms * 1e3, 2),
        "window_layer_gbs": round(win_gbs, 1),
        "window_layer_hbm_frac": round(win_gbs / HBM_PEAK_GBS, 4),
        "encoder_tflops": round(total_flops / (ms_step * 1e-3) / 1e12, 1),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    if not args.no_secondary:
        # last on the line, with the legs of the path's other kernels at its very end, so that a reader of
        # the line's tail sees them
        line["secondary"] = secondary(torch, sam_hip, lib, dev, sp, Timer(torch, stream), cpu=not args.no_cpu_baseline)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
