"""Builds libsam_hip.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

    python sam-rs_amd/build_lib.py          # compile every source, link the libraries

Each source compiles to its own object in parallel (the attention kernels have many template
instantiations), then everything links into sam-rs_amd/libsam_hip.so. The measurement kernel that
bench.py uses for the gather ceiling (gather_probe.hip) links into sam-rs_amd/libsam_probe.so, apart
from the product library.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsam_hip.so")
PROBE_LIB = os.path.join(HERE, "libsam_probe.so")
PROBE_SOURCES = ["gather_probe.hip"]

SOURCES = [
    "attn_relpos.hip",
    "attn_relpos_win.hip", "attn_relpos_glob.hip", "attn_relpos_wide.hip",
    "attn_relpos_f32.hip",
    "deform_attn.hip",
    "preprocess.hip",
    "bias_ops.hip",
    "relpos_softmax.hip",
    "qkv_split.hip",
    "flash_attn.hip", "flash_attn_d256.hip", "flash_attn_f32.hip", "flash_noalloc.hip",
    "rope.hip", "qkv_rope.hip",
    "sam_hip_abi.cpp",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "--offload-arch=gfx950"
# Packed-FP32 instructions stay disabled for every device compilation on this target.
FLAGS = [ARCH, "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{errs}")
    if errs.strip():
        sys.stderr.write(errs + "\n")
    return obj


def _link(objs, lib: str) -> None:
    tmp = lib + ".tmp"
    subprocess.run([HIPCC, ARCH, "-shared", "-fPIC", "-o", tmp, *objs], check=True)
    shutil.move(tmp, lib)


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    jobs = jobs or min(len(srcs), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs[:len(SOURCES)], LIB)
    _link(objs[len(SOURCES):], PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build())
