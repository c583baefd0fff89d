"""Every compute entry point is deterministic on an MI355X: the same call on the same inputs, repeated
with other launches in between, returns the same bits.

The reference's CPU path is deterministic, and none of these kernels uses atomics or an order that
depends on timing, so any difference would show a race (a read of LDS or of the workspace before the
write it needs, a buffer reused too early). Each case runs at shapes that exercise the kernel's
multi-workgroup paths (key splits, several waves per unit, partial tiles); the calls in between are
the other cases, so stale LDS and workspace contents differ from one repetition to the next.
"""
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


def rnd(g, shape, dtype, std=1.0):
    return (std * torch.randn(shape, device="cuda", generator=g)).to(dtype)


def cases(hip):
    g = torch.Generator(device="cuda").manual_seed(99)
    f16, bf16, f32 = torch.float16, torch.bfloat16, torch.float32
    out = []

    def relpos(h, w, bh, hd, dt):
        q, kt, v = rnd(g, (bh, h * w, hd), dt), rnd(g, (bh, hd, h * w), dt), rnd(g, (bh, h * w, hd), dt)
        t = rnd(g, (2 * h - 1 + 2 * w - 1, hd), dt, 0.02)
        return f"attention_relpos {h}x{w} hd{hd} {dt}", lambda: hip.attention_relpos(q, kt, v, t, h, w, hd ** -0.5)

    for args in [(14, 14, 400, 80, f16), (14, 14, 300, 64, bf16), (64, 64, 4, 80, f16), (64, 64, 2, 64, bf16),
                 (7, 11, 6, 80, f16), (65, 64, 2, 64, f16), (14, 14, 50, 64, f32), (64, 64, 2, 64, f32)]:
        out.append(relpos(*args))

    def softmax(h, w, bh, hd, dt):
        s, q = rnd(g, (bh, h * w, h * w), dt), rnd(g, (bh, h * w, hd), dt)
        t = rnd(g, (2 * h - 1 + 2 * w - 1, hd), dt)
        return f"relpos_softmax {h}x{w} {dt}", lambda: hip.relpos_softmax(s, q, t, h, w, 0.125)

    for args in [(14, 14, 8, 80, f16), (64, 64, 1, 80, bf16), (5, 9, 4, 64, f32)]:
        out.append(softmax(*args))

    def flash(b, lq, lk, h, d, dt):
        q, k, v = rnd(g, (b, lq, h, d), dt), rnd(g, (b, lk, h, d), dt), rnd(g, (b, lk, h, d), dt)
        return f"flash_attn {b}x{lq}x{lk}x{h}x{d} {dt}", lambda: hip.flash_attn(q, k, v)

    for args in [(1, 300, 3000, 2, 64, f16), (9, 576, 576, 4, 64, bf16), (1, 130, 517, 3, 96, f16),
                 (1, 1000, 4096, 1, 256, f16), (1, 70, 1000, 2, 128, f32)]:
        out.append(flash(*args))

    qm, km, vm = rnd(g, (2, 3, 200, 64), f16), rnd(g, (2, 3, 1500, 64), f16), rnd(g, (2, 3, 1500, 64), f16)
    mask = rnd(g, (1, 3, 200, 1500), f16)
    out.append(("sdpa with a mask", lambda: hip.sdpa(qm, km, vm, mask)))

    qr, kr, vr = rnd(g, (1, 4096, 256), f16), rnd(g, (1, 4096 * 2 + 64, 256), f16), rnd(g, (1, 4096 * 2 + 64, 256), f16)
    cos, sin = (torch.from_numpy(x).cuda() for x in oracle.rope_tables(64, 1.0, 256, 10000.0))
    out.append(("rope_attention cross", lambda: hip.rope_attention(qr, kr, vr, cos, sin, 64)))

    shapes = [(100, 167), (50, 84), (25, 42), (13, 21)]
    s = sum(a * b for a, b in shapes)
    value = rnd(g, (1, s, 8, 32), f32)
    loc = torch.rand((1, 5000, 8, 4, 4, 2), device="cuda", generator=g)
    attn = torch.softmax(rnd(g, (1, 5000, 8, 16), f32), -1).reshape(1, 5000, 8, 4, 4)
    out.append(("deform_attn", lambda: hip.deform_attn(value, loc, attn, shapes)))
    offs, logits = rnd(g, (1, 5000, 8, 4, 4, 2), f32, 2.0), rnd(g, (1, 5000, 8, 4, 4), f32)
    refs = torch.rand((1, 5000, 4, 2), device="cuda", generator=g)
    out.append(("deform_core", lambda: hip.deform_core(value, offs, logits, refs, shapes)))

    y, bias = rnd(g, (25 * 196, 3 * 1280), f16), rnd(g, (3 * 1280,), f16)
    out.append(("qkv_split", lambda: hip.qkv_split(y, bias, 196, 16, 80)))
    yr, br = rnd(g, (5184, 3 * 1024), bf16), rnd(g, (3 * 1024,), bf16)
    c3, s3 = (torch.from_numpy(x).cuda() for x in oracle.rope_tables(72, 1.0, 64, 10000.0))
    out.append(("qkv_rope", lambda: hip.qkv_rope(yr, br, c3, s3, 5184, 16, 64)))
    res, yb, bb = rnd(g, (4096, 1280), f16), rnd(g, (4096, 1280), f16), rnd(g, (1280,), f16)
    lw, lb = rnd(g, (1280,), f16), rnd(g, (1280,), f16)
    out.append(("bias_residual_ln", lambda: hip.bias_residual_ln(res, yb, bb, lw, lb)))
    out.append(("bias_gelu", lambda: hip.bias_gelu(yb, bb)))
    img = torch.randint(0, 256, (480, 640, 3), dtype=torch.uint8, device="cuda", generator=g)
    out.append(("preprocess", lambda: hip.prepare(img)[0]))
    return out


def flat(x):
    return [t for t in (x if isinstance(x, (tuple, list)) else (x,))]


def test_every_entry_point_is_deterministic(hip):
    cs = cases(hip)
    first = [[t.clone() for t in flat(fn())] for _, fn in cs]
    torch.cuda.synchronize()
    for rep in range(2):
        for (name, fn), ref in zip(reversed(cs), reversed(first)):
            print(f"determinism: {name}, repetition {rep + 1}", flush=True)
            got = flat(fn())
            torch.cuda.synchronize()
            for a, b in zip(got, ref):
                assert torch.equal(a, b), f"{name}: repetition {rep + 1} differs"


def test_concurrent_streams_match_sequential_calls(hip):
    """Entry points launched on two streams at once (both at the default priority) give the results of
    the same calls made one after the other: no kernel keeps state outside its own call's buffers (the
    no-allocation entry point's shared array is the documented exception and is not used here)."""
    g = torch.Generator(device="cuda").manual_seed(5)
    f16 = torch.float16
    wq, wk, wv = rnd(g, (400, 196, 80), f16), rnd(g, (400, 80, 196), f16), rnd(g, (400, 196, 80), f16)
    wt = rnd(g, (54, 80), f16, 0.02)
    gq, gk, gv = rnd(g, (16, 4096, 80), f16), rnd(g, (16, 80, 4096), f16), rnd(g, (16, 4096, 80), f16)
    gt = rnd(g, (254, 80), f16, 0.02)
    fq, fk, fv = rnd(g, (1, 1000, 2, 64), f16), rnd(g, (1, 8000, 2, 64), f16), rnd(g, (1, 8000, 2, 64), f16)
    a = [lambda: hip.attention_relpos(wq, wk, wv, wt, 14, 14, 80 ** -0.5), lambda: hip.flash_attn(fq, fk, fv)]
    b = [lambda: hip.attention_relpos(gq, gk, gv, gt, 64, 64, 80 ** -0.5), lambda: hip.flash_attn(fq, fk, fv)]
    want = [[f() for f in a], [f() for f in b]]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for rep in range(3):
        print(f"concurrent streams, repetition {rep + 1}", flush=True)
        with torch.cuda.stream(s1):
            got_a = [f() for f in a]
        with torch.cuda.stream(s2):
            got_b = [f() for f in b]
        torch.cuda.synchronize()
        for got, ref in zip(got_a + got_b, want[0] + want[1]):
            assert torch.equal(got, ref)
