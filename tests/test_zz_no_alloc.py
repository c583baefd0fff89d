"""sam_hip_flash_attn_noalloc, the flash-attention entry point that allocates nothing: its output
equals sam_hip_flash_attn's (caller workspace) bit for bit, through the C ABI, on two calls in a row
whose second is smaller, so the library's shared workspace array is reused with stale contents from the
first call. Both entry points run the same kernels on the same inputs, so the bar is equality, which
is within every parity bar.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def memory_case(side, frames, n_ptr, d, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    n = side * side
    m = frames * n + n_ptr
    q = torch.randn(1, n, d, device="cuda", generator=g).half()
    k = torch.randn(1, m, d, device="cuda", generator=g).half()
    v = torch.randn(1, m, d, device="cuda", generator=g).half()
    cos, sin = oracle.rope_tables(side, 1.0, d, 10000.0)
    return q, k, v, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), n_ptr


def test_noalloc_matches_workspace_entry_point(hip):
    """SAM 2.1 memory attention: cross-attention (4096 queries, 28736 keys with 64 unrotated pointer
    tokens; key splits and rotated keys in the workspace), then the smaller self-attention (4096 keys),
    then a plain mask-free flash call with few query blocks (key splits, no rotation)."""
    cases = [("cross", memory_case(64, 7, 64, 256, 41)), ("self", memory_case(64, 1, 0, 256, 42))]
    for name, (q, k, v, cos, sin, n_ptr) in cases:
        print(f"noalloc memory attention {name}", flush=True)
        want = hip.rope_attention(q, k, v, cos, sin, n_ptr)
        got = hip.rope_attention(q, k, v, cos, sin, n_ptr, noalloc=True)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), f"{name}: max diff {(got.float() - want.float()).abs().max().item()}"
    g = torch.Generator(device="cuda").manual_seed(43)
    for lq, lk, h, d in [(300, 3000, 2, 128), (100, 700, 1, 64)]:
        print(f"noalloc flash lq={lq} lk={lk} h={h} d={d}", flush=True)
        q, k, v = (torch.randn(1, n, h, d, device="cuda", generator=g).bfloat16() for n in (lq, lk, lk))
        want = hip.flash_attn(q, k, v)
        out = torch.empty_like(q)
        got = hip.flash_attn(q, k, v, out=out, noalloc=True)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert torch.equal(got, want)


def test_noalloc_rejects_calls_beyond_its_array(hip):
    """A call whose workspace exceeds the fixed array fails with a clear error before any launch."""
    L = hip.load()
    need = L.sam_hip_flash_attn_workspace_size(1, 1, 64, 150000, 1, 256, 150000)
    assert need > (64 << 20)
    q = torch.zeros(1, 64, 1, 256, device="cuda", dtype=torch.float16)
    k = torch.zeros(1, 150000, 1, 256, device="cuda", dtype=torch.float16)
    cos = torch.zeros(64, 256, device="cuda")
    with pytest.raises(hip.SamHipError, match="fixed .*-byte array"):
        hip._flash(q, k, k, torch.empty_like(q), "blhd", 0.0625, cos, cos, 0, 150000, noalloc=True)
