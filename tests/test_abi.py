"""The C ABI library loads, exports every entry point include/sam_hip.h declares, and rejects bad
arguments before touching a GPU (CPU only: no kernel is launched here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sam_hip.h")
LIB = os.path.join(ROOT, "sam-rs_amd", "libsam_hip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sam_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("libsam_hip.so is not built")
    return ctypes.CDLL(LIB)


def test_header_declares_the_entry_points():
    names = declared_functions()
    for want in ("sam_hip_attn_relpos", "sam_hip_relpos_softmax", "sam_hip_qkv_split", "sam_hip_deform_attn",
                 "sam_hip_flash_attn", "sam_hip_flash_attn_workspace_size", "sam_hip_flash_attn_noalloc", "sam_hip_rope", "sam_hip_last_error",
                 "sam_hip_abi_version", "sam_hip_qkv_split_grid", "sam_hip_window_merge"):
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_null_pointers_and_bad_sizes_fail_without_a_launch(lib):
    lib.sam_hip_last_error.restype = ctypes.c_char_p
    vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    lib.sam_hip_attn_relpos.argtypes = [vp] * 5 + [i] * 5 + [f, vp]
    assert lib.sam_hip_attn_relpos(None, None, None, None, None, 1, 1, 2, 3, 8, 0.3, None) == 1
    assert b"null" in lib.sam_hip_last_error()
    fake = vp(0x1000)  # never dereferenced: the checks below fail first
    assert lib.sam_hip_attn_relpos(fake, fake, fake, fake, fake, 7, 1, 2, 3, 8, 0.3, None) == 2
    assert b"dtype" in lib.sam_hip_last_error()
    assert lib.sam_hip_attn_relpos(fake, fake, fake, fake, fake, 1, 1, 65, 3, 8, 0.3, None) == 3
    assert lib.sam_hip_attn_relpos(fake, fake, fake, fake, fake, 1, 1, 2, 3, 12, 0.3, None) == 3
    lib.sam_hip_deform_attn.argtypes = [vp] * 4 + [i] * 8 + [ctypes.POINTER(ctypes.c_int), vp]
    shapes = (ctypes.c_int * 10)(*([2, 3] * 5))
    assert lib.sam_hip_deform_attn(fake, fake, fake, fake, 0, 1, 30, 3, 2, 8, 5, 2, shapes, None) == 3
    assert b"at most 4 levels, got 5" in lib.sam_hip_last_error()
    assert lib.sam_hip_deform_attn(fake, fake, fake, fake, 0, 1, 31, 3, 2, 8, 2, 2, shapes, None) == 1
    lib.sam_hip_qkv_split.argtypes = [vp] * 3 + [i, ctypes.c_long, i, i, i, vp]
    assert lib.sam_hip_qkv_split(fake, fake, fake, 1, 100, 7, 2, 8, None) == 1  # 100 % 7 != 0
    lib.sam_hip_qkv_split_grid.argtypes = [vp] * 3 + [i] * 7 + [vp]
    assert lib.sam_hip_qkv_split_grid(None, fake, fake, 1, 1, 64, 64, 14, 16, 80, None) == 1
    assert lib.sam_hip_qkv_split_grid(fake, fake, fake, 1, 1, 64, 0, 14, 16, 80, None) == 1
    assert lib.sam_hip_qkv_split_grid(fake, fake, fake, 1, 1, 64, 64, 14, 16, 264, None) == 3
    assert lib.sam_hip_qkv_split_grid(fake, fake, fake, 5, 1, 64, 64, 14, 16, 80, None) == 2
    lib.sam_hip_window_merge.argtypes = [vp] * 2 + [i] * 7 + [vp]
    assert lib.sam_hip_window_merge(fake, None, 1, 1, 64, 64, 14, 16, 80, None) == 1
    assert lib.sam_hip_window_merge(fake, fake, 1, 1, 64, 64, 0, 16, 80, None) == 1
    assert lib.sam_hip_window_merge(fake, fake, 1, 1, 64, 64, 300, 16, 80, None) == 3
    assert lib.sam_hip_window_merge(vp(0x1004), fake, 1, 1, 64, 64, 14, 16, 80, None) == 3  # misaligned


def test_flash_and_rope_argument_checks(lib):
    lib.sam_hip_last_error.restype = ctypes.c_char_p
    vp, i, f, lp = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.POINTER(ctypes.c_long)
    lib.sam_hip_flash_attn.argtypes = [vp] * 4 + [i] * 6 + [lp] * 4 + [f, vp, vp, i, i, i, vp, ctypes.c_long, vp]
    lib.sam_hip_flash_attn_workspace_size.argtypes = [i] * 7
    lib.sam_hip_flash_attn_workspace_size.restype = ctypes.c_long
    fake = vp(0x1000)
    args = lambda dt, d, scale=0.1: (fake, fake, fake, fake, dt, 1, 8, 8, 1, d, None, None, None, None, scale, None,
                                     None, 0, 0, 0, None, 0, None)
    assert lib.sam_hip_flash_attn(None, None, None, None, 1, 1, 8, 8, 1, 64, None, None, None, None, 0.1, None,
                                  None, 0, 0, 0, None, 0, None) == 1
    assert lib.sam_hip_flash_attn(*args(3, 64)) == 2  # dtypes are 0, 1, 2
    assert lib.sam_hip_flash_attn(*args(0, 20)) == 3  # f32 keeps the head-dim limits
    assert lib.sam_hip_flash_attn(*args(1, 20)) == 3
    assert lib.sam_hip_flash_attn(*args(1, 264)) == 3
    assert lib.sam_hip_flash_attn(*args(1, 64, -1.0)) == 1
    assert lib.sam_hip_flash_attn_workspace_size(1, 1, 8, 8, 1, 20, 0) == -1
    # RoPE asked for without tables
    assert lib.sam_hip_flash_attn(fake, fake, fake, fake, 1, 1, 8, 8, 1, 64, None, None, None, None, 0.1, None, None,
                                  0, 8, 0, None, 0, None) == 1
    # the masked sdpa: a null mask, missing or negative mask strides, a mask off its element alignment
    lib.sam_hip_sdpa_mask.argtypes = [vp] * 5 + [i] * 6 + [lp] * 5 + [f, vp, ctypes.c_long, vp]
    margs = lambda dt, mask, sm: (fake, fake, fake, mask, fake, dt, 1, 8, 8, 1, 64, None, None, None, sm, None, 0.1,
                                  None, 0, None)
    good = (ctypes.c_long * 4)(0, 0, 8, 1)
    assert lib.sam_hip_sdpa_mask(*margs(1, None, good)) == 1
    assert lib.sam_hip_sdpa_mask(*margs(1, fake, None)) == 1
    assert lib.sam_hip_sdpa_mask(*margs(1, fake, (ctypes.c_long * 4)(0, 0, -8, 1))) == 3
    assert lib.sam_hip_sdpa_mask(*margs(0, vp(0x1002), good)) == 3
    lib.sam_hip_rope.argtypes = [vp] * 4 + [i] * 5 + [lp] * 2 + [i, i, vp]
    assert lib.sam_hip_rope(fake, fake, fake, fake, 1, 1, 8, 1, 12, None, None, 8, 8, None) == 3
    assert lib.sam_hip_rope(fake, fake, fake, fake, 1, 1, 8, 1, 16, None, None, 8, 9, None) == 1


def test_abi_version(lib):
    lib.sam_hip_abi_version.restype = ctypes.c_int
    assert lib.sam_hip_abi_version() >= 1
