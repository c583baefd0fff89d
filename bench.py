"""Benchmark: SAM ViT-H image-encoder attention on one MI355X.

One step = the attention core of every encoder layer of ViT-H for one batch of 1024x1024 images:
28 windowed layers (25 windows x 16 heads per image, 14x14 tokens, hd 80, (27, 80) rel-pos tables) and
4 global layers (16 heads per image, 64x64 tokens, hd 80, (127, 80) tables), each one launch of the
fused rel-pos attention kernel on inputs already resident in HBM (fresh q/kT/v per layer).

Prints one JSON line: ms per image, the global-layer kernel's achieved TFLOP/s against the f16 MFMA
peak (timed live with HIP events on the launch stream), and the CPU oracle timed on this host.

    python bench.py [--steps K] [--warmup W] [--batch B] [--dtype f16|bf16] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--dtype", default="f16", choices=["f16", "bf16"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layers", default="all", choices=["all", "global", "window"],
                    help="restrict the step to one layer kind (for profiling one kernel)")
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


def flops(bh, n):
    return 4.0 * bh * n * n * HD


def window_bytes(bh, n, elem=2):
    return float(bh) * n * HD * elem * 4  # q, kT, v read once, out written once


def cpu_baseline():
    """The oracle (C restatement of the reference's exact-f32 CPU attention, OpenMP on every host core)
    on one image's windowed layer and one image's global layer; ms/image = 28 x window + 4 x global."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import sam_oracle

    cores = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    r = np.random.default_rng(1)

    def time_layer(bh, h, w):
        n = h * w
        q = r.standard_normal((bh, n, HD), dtype=np.float32)
        kt = r.standard_normal((bh, HD, n), dtype=np.float32)
        v = r.standard_normal((bh, n, HD), dtype=np.float32)
        table = (0.02 * r.standard_normal((2 * h - 1 + 2 * w - 1, HD))).astype(np.float32)
        t0 = time.perf_counter()
        sam_oracle.attention_relpos(q, kt, v, table, h, w, HD ** -0.5, nthreads=cores)
        return time.perf_counter() - t0

    t_win = time_layer(WINDOWS * HEADS, 14, 14)
    t_glob = time_layer(HEADS, 64, 64)
    ms = 1e3 * ((DEPTH - len(GLOBAL_LAYERS)) * t_win + len(GLOBAL_LAYERS) * t_glob)
    return {
        "value": round(ms, 1), "unit": "ms/image", "cores": cores, "kind": "port",
        "sample": "one windowed layer (400 x 14x14) and one global layer (16 x 64x64) of one image, f32, "
                  f"timed once each ({t_win:.2f} s, {t_glob:.2f} s) and scaled by 28 and 4 layers",
    }


def traffic_from_profiles():
    p = os.path.join(ROOT, "profiles", "attn_relpos_vit_h_global_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the attention path shards over "
              "(batch, window, head) with no exchange, so N GPUs run N independent copies of this line.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import sam_hip

    sam_hip.load()
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
    lib = sam_hip.load()
    code = {"f16": 1, "bf16": 2}[args.dtype]
    stream = torch.cuda.current_stream(dev)
    sp = sam_hip._vp(stream.cuda_stream)

    def launch(L):
        bh, h, w, q, kt, v, table, out = L
        rc = lib.sam_hip_attn_relpos(q.data_ptr(), kt.data_ptr(), v.data_ptr(), table.data_ptr(), out.data_ptr(),
                                     code, bh, h, w, HD, scale, sp)
        if rc:
            raise sam_hip.SamHipError(lib.sam_hip_last_error().decode())

    keep = {"all": lambda i: True, "global": lambda i: i in GLOBAL_LAYERS,
            "window": lambda i: i not in GLOBAL_LAYERS}[args.layers]

    def step(ev=None):
        for i, L in enumerate(layers):
            if not keep(i):
                continue
            if ev is not None and i in GLOBAL_LAYERS:
                ev[0].append(torch.cuda.Event(enable_timing=True))
                ev[1].append(torch.cuda.Event(enable_timing=True))
                ev[0][-1].record(stream)
                launch(L)
                ev[1][-1].record(stream)
            elif ev is not None:
                ev[2].append(torch.cuda.Event(enable_timing=True))
                ev[3].append(torch.cuda.Event(enable_timing=True))
                ev[2][-1].record(stream)
                launch(L)
                ev[3][-1].record(stream)
            else:
                launch(L)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0e, t1e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    evs = ([], [], [], [])
    t0e.record(stream)
    for _ in range(args.steps):
        step(evs)
    t1e.record(stream)
    torch.cuda.synchronize()
    ms_total = t0e.elapsed_time(t1e)
    ms_step = ms_total / args.steps
    glob_ms = sum(a.elapsed_time(b) for a, b in zip(evs[0], evs[1])) / max(len(evs[0]), 1)
    win_ms = sum(a.elapsed_time(b) for a, b in zip(evs[2], evs[3])) / max(len(evs[2]), 1)
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
            "kernel": "attn_relpos_kernel (global 64x64 layer)",
            "achieved": round(achieved, 1),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic_from_profiles(),
        },
        "global_layer_us": round(glob_ms * 1e3, 2),
        "window_layer_us": round(win_ms * 1e3, 2),
        "window_layer_gbs": round(win_gbs, 1),
        "window_layer_hbm_frac": round(win_gbs / HBM_PEAK_GBS, 4),
        "encoder_tflops": round(total_flops / (ms_step * 1e-3) / 1e12, 1),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
