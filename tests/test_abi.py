"""The C ABI library loads, exports every entry point include/sam_hip.h declares, and rejects bad
arguments before touching a GPU (CPU only: no kernel is launched here)."""
import ctypes
import os
import re

import pytest
import torch

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
    assert lib.sam_hip_attn_relpos(fake, fake, fake, fake, fake, 1, 1, 129, 3, 8, 0.3, None) == 3
    assert lib.sam_hip_attn_relpos(fake, fake, fake, fake, fake, 0, 1, 65, 3, 8, 0.3, None) == 3  # f32 past 64
    assert lib.sam_hip_attn_relpos(fake, fake, fake, fake, fake, 1, 1 << 20, 64, 64, 8, 0.3, None) == 3
    assert b"beyond 2^31" in lib.sam_hip_last_error()
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


def test_column_counts_beyond_int_are_refused(lib):
    """qkv_split, qkv_split_grid and window_merge index rows of nh*hd (or 3*nh*hd) columns in 32-bit
    arithmetic: a head count that overflows it is refused, even where the total element count passes."""
    lib.sam_hip_last_error.restype = ctypes.c_char_p
    vp, i = ctypes.c_void_p, ctypes.c_int
    fake = vp(0x1000)
    lib.sam_hip_qkv_split.argtypes = [vp] * 3 + [i, ctypes.c_long, i, i, i, vp]
    lib.sam_hip_qkv_split_grid.argtypes = [vp] * 3 + [i] * 7 + [vp]
    lib.sam_hip_window_merge.argtypes = [vp] * 2 + [i] * 7 + [vp]
    nh = (1 << 31) // (3 * 8) + 1  # 3 * nh * 8 just past 2^31; one token, one 1x1 window
    assert lib.sam_hip_qkv_split(fake, fake, fake, 1, 1, 1, nh, 8, None) == 3
    assert b"3*nh*hd" in lib.sam_hip_last_error()
    assert lib.sam_hip_qkv_split_grid(fake, fake, fake, 1, 1, 1, 1, 1, nh, 8, None) == 3
    assert b"3*nh*hd" in lib.sam_hip_last_error()
    nh2 = (1 << 31) // 8 + 1  # nh * 8 just past 2^31, 2^31 + 8 elements in total
    assert lib.sam_hip_window_merge(fake, fake, 1, 1, 1, 1, 1, nh2, 8, None) == 3


def test_qkv_rope_argument_checks(lib):
    """sam_hip_qkv_rope rejects null pointers, non-positive sizes, an odd head dim (RoPE rotates pairs),
    column counts beyond 2^31, too many vectors and misaligned pointers, before any launch."""
    lib.sam_hip_last_error.restype = ctypes.c_char_p
    vp, i, lg = ctypes.c_void_p, ctypes.c_int, ctypes.c_long
    fn = lib.sam_hip_qkv_rope
    fn.argtypes, fn.restype = [vp] * 5 + [i, lg, i, i, i, vp], i
    fake = vp(0x1000)
    assert fn(fake, fake, None, fake, fake, 1, 5184, 576, 16, 64, None) == 1
    assert fn(fake, fake, fake, fake, fake, 3, 5184, 576, 16, 64, None) == 2
    assert fn(fake, fake, fake, fake, fake, 1, 0, 576, 16, 64, None) == 1
    assert fn(fake, fake, fake, fake, fake, 1, 5184, 0, 16, 64, None) == 1
    assert fn(fake, fake, fake, fake, fake, 1, 5184, 576, 16, 63, None) == 1
    assert b"even" in lib.sam_hip_last_error()
    assert fn(fake, fake, fake, fake, fake, 1, 1, 1, 1 << 22, 256, None) == 3
    assert b"beyond 2^31" in lib.sam_hip_last_error()
    assert fn(fake, fake, fake, fake, fake, 1, 1 << 31, 576, 16, 64, None) == 3  # 2^31 * 384 vectors
    assert b"too many tokens" in lib.sam_hip_last_error()
    assert fn(fake, vp(0x1008), fake, fake, fake, 1, 5184, 576, 16, 64, None) == 3
    assert b"aligned" in lib.sam_hip_last_error()


def test_the_switch_turns_every_entry_point_off_and_on(lib):
    """sam_hip_set_enabled mirrors cpu_gemm::set_enabled (cpu_gemm.rs:25-32): while it is off, every
    compute entry point returns SAM_HIP_EDISABLED (5) before reading its arguments (null pointers and
    impossible sizes included, so nothing reaches a device); once it is on again, the ordinary argument
    checks answer."""
    lib.sam_hip_last_error.restype = ctypes.c_char_p
    lib.sam_hip_enabled.restype = ctypes.c_int
    lib.sam_hip_set_enabled.argtypes = [ctypes.c_int]
    vp, i, f, lp = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.POINTER(ctypes.c_long)
    sigs = {
        "sam_hip_attn_relpos": [vp] * 5 + [i] * 5 + [f, vp],
        "sam_hip_relpos_softmax": [vp] * 4 + [i, ctypes.c_long, i, i, i, f, vp],
        "sam_hip_qkv_split": [vp] * 3 + [i, ctypes.c_long, i, i, i, vp],
        "sam_hip_qkv_split_grid": [vp] * 3 + [i] * 7 + [vp],
        "sam_hip_window_merge": [vp] * 2 + [i] * 7 + [vp],
        "sam_hip_deform_attn": [vp] * 4 + [i] * 8 + [vp, vp],
        "sam_hip_deform_core": [vp] * 5 + [i] * 9 + [vp, vp],
        "sam_hip_preprocess": [vp, vp] + [i] * 6 + [vp, vp, vp],
        "sam_hip_bias_residual": [vp] * 4 + [i, ctypes.c_long, i, vp],
        "sam_hip_bias_gelu": [vp] * 3 + [i, ctypes.c_long, i, vp],
        "sam_hip_bias_residual_ln": [vp] * 7 + [i, ctypes.c_long, i, f, vp],
        "sam_hip_flash_attn": [vp] * 4 + [i] * 6 + [lp] * 4 + [f, vp, vp, i, i, i, vp, ctypes.c_long, vp],
        "sam_hip_flash_attn_noalloc": [vp] * 4 + [i] * 6 + [lp] * 4 + [f, vp, vp, i, i, i, vp],
        "sam_hip_sdpa_mask": [vp] * 5 + [i] * 6 + [lp] * 5 + [f, vp, ctypes.c_long, vp],
        "sam_hip_rope": [vp] * 4 + [i] * 5 + [lp] * 2 + [i, i, vp],
        "sam_hip_qkv_rope": [vp] * 5 + [i, ctypes.c_long, i, i, i, vp],
    }
    # every declared compute entry point is covered
    queries = {"sam_hip_flash_attn_workspace_size", "sam_hip_last_error", "sam_hip_abi_version",
               "sam_hip_set_enabled", "sam_hip_enabled"}
    assert set(declared_functions()) - queries == set(sigs)

    def zeros(argtypes):  # null pointers and zero sizes: every call is invalid as an ordinary call
        return [None if t in (vp, lp) else (0.0 if t is f else 0) for t in argtypes]

    assert lib.sam_hip_enabled() == 1
    try:
        lib.sam_hip_set_enabled(0)
        assert lib.sam_hip_enabled() == 0
        for name, argtypes in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = argtypes, ctypes.c_int
            assert fn(*zeros(argtypes)) == 5, name
            assert b"switched off" in lib.sam_hip_last_error(), name
    finally:
        lib.sam_hip_set_enabled(1)
    assert lib.sam_hip_enabled() == 1
    for name, argtypes in sigs.items():
        rc = getattr(lib, name)(*zeros(argtypes))
        assert rc in (1, 2, 3), (name, rc)  # EINVAL, EDTYPE or EUNSUPPORTED: argument checks, no launch


def test_the_switch_reads_sam_hip_disable_at_load_time():
    """SAM_HIP_DISABLE=1 in the environment starts the library switched off (a fresh process, so that
    this process's library state is untouched)."""
    if not os.path.exists(LIB):
        pytest.skip("libsam_hip.so is not built")
    import subprocess
    import sys

    code = ("import ctypes, sys; L = ctypes.CDLL(sys.argv[1]); L.sam_hip_enabled.restype = ctypes.c_int; "
            "print(L.sam_hip_enabled())")
    for env_value, want in (("1", "0"), ("0", "1"), ("", "1")):
        env = dict(os.environ, SAM_HIP_DISABLE=env_value)
        out = subprocess.run([sys.executable, "-c", code, LIB], env=env, capture_output=True, text=True, check=True)
        assert out.stdout.strip() == want, (env_value, out.stdout, out.stderr)


def test_python_flash_refuses_a_mismatched_out():
    """flash_attn writes q.shape elements of q's dtype through `out`: a smaller, narrower or
    differently placed `out` is refused before any library call (CPU tensors suffice)."""
    import sam_hip

    q = torch.zeros(1, 8, 2, 16, dtype=torch.float16)
    for bad in (torch.zeros(1, 4, 2, 16, dtype=torch.float16), torch.zeros(1, 8, 2, 16, dtype=torch.float32),
                torch.zeros(1, 8, 2, 16, dtype=torch.float16, device="meta")):
        with pytest.raises(sam_hip.SamHipError, match="out must match q"):
            sam_hip.flash_attn(q, q, q, out=bad)


def test_abi_version(lib):
    lib.sam_hip_abi_version.restype = ctypes.c_int
    assert lib.sam_hip_abi_version() >= 1
