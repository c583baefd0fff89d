"""Pins the CPU oracle before anything is checked against it (CPU only).

Each oracle function is compared with an independent float64 formulation (tests/refimpl.py), with
closed forms and special cases, and with brute force on tiny inputs. The `*_mutants_are_caught` tests
plant plausible mistakes (a flipped index sign, swapped tables, a dropped bias term, a transposed
operand, ...) in a copy of the formula, on the CPU, and check that the comparison used here would
reject each of them.
"""
import numpy as np
import pytest

import refimpl

RELPOS_GEOMS = [(2, 3, 1, 8), (7, 11, 2, 80), (14, 14, 2, 64), (1, 5, 2, 16), (64, 64, 1, 80)]


def _rng(seed):
    return np.random.default_rng(seed)


def _relpos_inputs(h, w, bh, hd, seed, table_std=0.5):
    r = _rng(seed)
    n = h * w
    q = r.standard_normal((bh, n, hd)).astype(np.float32)
    kt = r.standard_normal((bh, hd, n)).astype(np.float32)
    v = r.standard_normal((bh, n, hd)).astype(np.float32)
    table = (table_std * r.standard_normal((2 * h - 1 + 2 * w - 1, hd))).astype(np.float32)
    return q, kt, v, table


@pytest.mark.parametrize("h,w,bh,hd", RELPOS_GEOMS)
def test_textbook_and_fallback_index_forms_agree(h, w, bh, hd):
    q, kt, _, table = _relpos_inputs(h, w, bh, hd, 1)
    s = q.astype(np.float64) @ kt
    a = refimpl.relpos_logits64(s, q, table, h, w, 0.3)
    b = refimpl.relpos_logits_fallback_index64(s, q, table, h, w, 0.3)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)


@pytest.mark.parametrize("h,w,bh,hd", RELPOS_GEOMS[:4])
def test_relpos_softmax_matches_textbook(oracle_lib, h, w, bh, hd):
    q, kt, _, table = _relpos_inputs(h, w, bh, hd, 2)
    s = (q @ kt).astype(np.float32)
    scale = hd ** -0.5
    got = oracle_lib.relpos_softmax(s, q, table, h, w, scale)
    want = refimpl.relpos_softmax64(s, q, table, h, w, scale)
    assert np.abs(got - want).max() < 2e-6
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("h,w,bh,hd", RELPOS_GEOMS)
def test_attention_relpos_matches_textbook(oracle_lib, h, w, bh, hd):
    q, kt, v, table = _relpos_inputs(h, w, bh, hd, 3)
    scale = hd ** -0.5
    got = oracle_lib.attention_relpos(q, kt, v, table, h, w, scale)
    want = refimpl.attention_relpos64(q, kt, v, table, h, w, scale)
    err = np.abs(got - want).max() / np.abs(want).max()
    # f32 rounding of the 4096-key logits and sums alone is ~6e-6 of max|out| at 64x64
    assert err < (2e-6 if h * w <= 256 else 1e-5), err


def test_attention_relpos_zero_table_is_plain_attention(oracle_lib):
    q, kt, v, table = _relpos_inputs(7, 11, 2, 80, 4)
    table[:] = 0
    scale = 0.125
    got = oracle_lib.attention_relpos(q, kt, v, table, 7, 11, scale)
    want = refimpl.sdpa64(q, np.swapaxes(kt, 1, 2), v, scale=scale)
    assert np.abs(got - want).max() < 2e-6


def test_attention_relpos_uniform_when_scale_and_table_are_zero(oracle_lib):
    q, kt, v, table = _relpos_inputs(14, 14, 2, 64, 5)
    table[:] = 0
    got = oracle_lib.attention_relpos(q, kt, v, table, 14, 14, 0.0)
    want = np.broadcast_to(v.astype(np.float64).mean(axis=1, keepdims=True), v.shape)
    assert np.abs(got - want).max() < 1e-6


def test_attention_relpos_one_hot_values_recover_probabilities(oracle_lib):
    h, w = 2, 3
    n = h * w
    q, kt, _, table = _relpos_inputs(h, w, 2, n, 6)
    v = np.broadcast_to(np.eye(n, dtype=np.float32), (2, n, n)).copy()
    got = oracle_lib.attention_relpos(q, kt, v, table, h, w, 0.4)
    probs = oracle_lib.relpos_softmax((q @ kt).astype(np.float32), q, table, h, w, 0.4)
    assert np.abs(got - probs).max() < 1e-6


def test_attention_relpos_bias_depends_only_on_offsets():
    """A table whose rows are one-hot in a channel that q selects gives bias = table value at the
    relative offset: check one hand-computed logit of the textbook form."""
    h, w, hd = 3, 4, 2
    table = np.zeros((2 * h - 1 + 2 * w - 1, hd))
    table[: 2 * h - 1, 0] = np.arange(2 * h - 1) * 10.0  # rel_pos_h values 0, 10, ..., in channel 0
    table[2 * h - 1:, 1] = np.arange(2 * w - 1) * 1.0  # rel_pos_w values 0, 1, ..., in channel 1
    q = np.ones((1, h * w, hd))
    s = np.zeros((1, h * w, h * w))
    logits = refimpl.relpos_logits64(s, q, table, h, w, 1.0)
    # query (i=2, j=1) vs key (kh=0, kw=3): rel_pos_h[i-kh+h-1] = rel_pos_h[4] = 40, rel_pos_w[j-kw+w-1] = [1] = 1
    assert logits[0, 2 * w + 1, 0 * w + 3] == 41.0


def _mutants():
    def flip_sign(s, q, table, h, w, scale):  # kh - i instead of i - kh
        t = table.copy()
        t[: 2 * h - 1] = t[: 2 * h - 1][::-1]
        t[2 * h - 1:] = t[2 * h - 1:][::-1]
        return refimpl.relpos_logits64(s, q, t, h, w, scale)

    def swap_tables(s, q, table, h, w, scale):  # table split in the wrong order (rel_pos_w rows first)
        t = np.concatenate([table[2 * h - 1:], table[: 2 * h - 1]])
        return refimpl.relpos_logits64(s, q, t, h, w, scale)

    def drop_rw(s, q, table, h, w, scale):
        t = table.copy()
        t[2 * h - 1:] = 0
        return refimpl.relpos_logits64(s, q, t, h, w, scale)

    def drop_rh(s, q, table, h, w, scale):
        t = table.copy()
        t[: 2 * h - 1] = 0
        return refimpl.relpos_logits64(s, q, t, h, w, scale)

    def scale_bias_too(s, q, table, h, w, scale):  # scale applied to the bias as well
        return refimpl.relpos_logits64(s, q, table * scale, h, w, scale)

    def transposed_keys(s, q, table, h, w, scale):
        return refimpl.relpos_logits64(np.swapaxes(s, 1, 2), q, table, h, w, scale)

    return [flip_sign, swap_tables, drop_rw, drop_rh, scale_bias_too, transposed_keys]


@pytest.mark.parametrize("mutant", _mutants(), ids=lambda f: f.__name__)
def test_relpos_mutants_are_caught(oracle_lib, mutant):
    h, w, bh, hd = 7, 11, 1, 80
    q, kt, _, table = _relpos_inputs(h, w, bh, hd, 7)
    s = (q @ kt).astype(np.float32)
    got = oracle_lib.relpos_softmax(s, q, table, h, w, 0.125)
    bad = refimpl.softmax64(mutant(s.astype(np.float64), q, table, h, w, 0.125))
    assert np.abs(got - bad).max() > 1e-3  # far above the 2e-6 the real comparison allows


# ----------------------------------------------------------------------------------------- qkv split

def test_qkv_split_is_the_reference_permutation(oracle_lib):
    n, nh, hd, win = 196, 3, 16, 2
    r = _rng(8)
    y = r.standard_normal((win * n, 3 * nh * hd)).astype(np.float32)
    b = r.standard_normal(3 * nh * hd).astype(np.float32)
    q, kt, v = oracle_lib.qkv_split(y, b, n, nh, hd)
    qkv = (y + b).reshape(win, n, 3, nh, hd).transpose(2, 0, 3, 1, 4).reshape(3, win * nh, n, hd)
    assert np.array_equal(q, qkv[0])
    assert np.array_equal(kt, qkv[1].transpose(0, 2, 1))
    assert np.array_equal(v, qkv[2])


# ----------------------------------------------------------------------------------------- deform

def _deform_inputs(shapes, b, q, h, d, p, seed, spread=0.5, softmax=True):
    r = _rng(seed)
    s = sum(hh * ww for hh, ww in shapes)
    l = len(shapes)
    value = r.standard_normal((b, s, h, d)).astype(np.float32)
    loc = (r.standard_normal((b, q, h, l, p, 2)) * spread + 0.5).astype(np.float32)
    logits = r.standard_normal((b, q, h, l * p))
    attn = (refimpl.softmax64(logits) if softmax else logits).reshape(b, q, h, l, p).astype(np.float32)
    return value, loc, attn


DEFORM_CASES = [
    ([(7, 9), (4, 5), (2, 3)], 1, 13, 4, 8, 3),  # tests/dino.rs:46-63
    ([(9, 12), (5, 6), (3, 3), (2, 2)], 1, 37, 8, 32, 4),  # tests/kernels.rs:65-83
    ([(5, 4), (3, 2)], 2, 6, 2, 4, 2),
]


@pytest.mark.parametrize("shapes,b,q,h,d,p", DEFORM_CASES)
def test_deform_matches_scalar_spec_and_grid_sample(oracle_lib, shapes, b, q, h, d, p):
    value, loc, attn = _deform_inputs(shapes, b, q, h, d, p, 9)
    got = oracle_lib.deform_attn(value, loc, attn, shapes)
    naive = refimpl.deform_naive64(value, loc, attn, shapes)
    gs = refimpl.deform_grid_sample64(value, loc, attn, shapes)
    assert np.abs(naive - gs).max() < 1e-12
    assert np.abs(got - naive).max() < 1e-5


def test_deform_degenerate_locations_follow_the_reference_cast(oracle_lib):
    """The reference takes a corner index as `x.floor() as i64` (kernels.rs:799-800), Rust's saturating
    cast: NaN gives 0, so a NaN coordinate reads corner 0 of that axis with a NaN weight and the output
    is NaN; +-1e10 and +-inf saturate far outside the level and add nothing; the edges 0 and 1 give the
    half-weighted border pixel (x = -0.5 and W - 0.5). A C cast of NaN is undefined (x86 gives INT_MIN,
    which would skip the corner), so the oracle spells the Rust cast out."""
    shapes = [(4, 5)]
    value = np.arange(20, dtype=np.float32).reshape(1, 20, 1, 1) + 1.0  # pixel k holds k + 1
    pts = [(0.5, np.nan), (np.nan, 0.5), (1e10, 0.5), (-np.inf, 0.5), (0.0, 0.5), (1.0, 0.5), (0.5, 0.5)]
    loc = np.array(pts, np.float32).reshape(1, len(pts), 1, 1, 1, 2)
    attn = np.ones((1, len(pts), 1, 1, 1), np.float32)
    got = oracle_lib.deform_attn(value, loc, attn, shapes)[0, :, 0]
    assert np.isnan(got[0]) and np.isnan(got[1])
    assert got[2] == 0.0 and got[3] == 0.0
    # x = 0: x = -0.5, corners at columns -1 (outside) and 0 with weight 0.5 each; y = 0.5 * 4 - 0.5 =
    # 1.5, rows 1 and 2 with weight 0.5: 0.25 * (pixel 5 + pixel 10) = 0.25 * (6 + 11)
    assert got[4] == np.float32(0.25 * (6 + 11))
    # x = 1: x = 4.5, columns 4 and 5 (outside): 0.25 * (pixel 9 + pixel 14) = 0.25 * (10 + 15)
    assert got[5] == np.float32(0.25 * (10 + 15))
    # the centre: x = 2, y = 1.5: columns 2 and 3 with weights 1 and 0, rows 1 and 2 with 0.5 each
    assert got[6] == np.float32(0.5 * (8 + 13))


def _prep_inputs(shapes, b, q, h, p, nc, seed):
    r = _rng(seed)
    l = len(shapes)
    off = (2.0 * r.standard_normal((b, q, h, l, p, 2))).astype(np.float32)  # ~N(0,2) pixels
    logits = r.standard_normal((b, q, h, l, p)).astype(np.float32)
    if nc == 2:
        refs = r.uniform(0, 1, (b, q, l, 2)).astype(np.float32)
    else:
        refs = np.concatenate([r.uniform(0.1, 0.9, (b, q, l, 2)), r.uniform(0.05, 0.5, (b, q, l, 2))], -1)
        refs = refs.astype(np.float32)
    return off, logits, refs


# Non-square levels (a swapped (W, H) normaliser would show), the DINO point count and an odd one.
PREP_CASES = [([(7, 9), (4, 5), (2, 3)], 1, 13, 4, 3), ([(9, 12), (5, 6), (3, 3), (2, 2)], 1, 37, 8, 4),
              ([(5, 4), (3, 2)], 2, 6, 2, 2)]


@pytest.mark.parametrize("nc", [2, 4])
@pytest.mark.parametrize("shapes,b,q,h,p", PREP_CASES)
def test_deform_prep_matches_float64_module(oracle_lib, shapes, b, q, h, p, nc):
    """dino/mod.rs:166-178 against the Deformable-DETR formulation in float64, then the whole core
    (prep + gather) against torch's grid_sample."""
    off, logits, refs = _prep_inputs(shapes, b, q, h, p, nc, 40 + q + nc)
    loc, attn = oracle_lib.deform_prep(off, logits, refs, shapes)
    loc64, attn64 = refimpl.deform_prep64(off, logits, refs, shapes)
    assert np.abs(loc - loc64).max() < 2e-6
    assert np.abs(attn - attn64).max() < 1e-6
    np.testing.assert_allclose(attn.sum(-1).sum(-1), 1.0, atol=2e-6)
    value = _rng(7).standard_normal((b, sum(hh * ww for hh, ww in shapes), h, 8)).astype(np.float32)
    got = oracle_lib.deform_forward_core(value, off, logits, refs, shapes)
    want = refimpl.deform_grid_sample64(value, loc64, attn64, shapes)
    assert np.abs(got - want).max() < 2e-5


def test_deform_prep_closed_forms(oracle_lib):
    """Zero offsets sample at the reference point; an offset of one level size moves the encoder form
    by exactly 1; an offset of 2P moves the decoder form by exactly the box size; equal logits give
    equal weights 1 / (L*P)."""
    shapes = [(6, 10), (3, 5)]
    b, q, h, p = 1, 5, 2, 4
    l = len(shapes)
    off, logits, refs2 = _prep_inputs(shapes, b, q, h, p, 2, 3)
    _, _, refs4 = _prep_inputs(shapes, b, q, h, p, 4, 4)
    zero = np.zeros_like(off)
    loc, attn = oracle_lib.deform_prep(zero, np.zeros_like(logits), refs2, shapes)
    assert np.array_equal(loc, np.broadcast_to(refs2[:, :, None, :, None, :], loc.shape))
    assert np.array_equal(attn, np.full_like(attn, np.float32(1.0 / (l * p))))
    loc, _ = oracle_lib.deform_prep(zero, logits, refs4, shapes)
    assert np.array_equal(loc, np.broadcast_to(refs4[:, :, None, :, None, :2], loc.shape))
    one = np.empty_like(off)
    for li, (hh, ww) in enumerate(shapes):
        one[:, :, :, li, :, 0] = ww
        one[:, :, :, li, :, 1] = hh
    loc, _ = oracle_lib.deform_prep(one, logits, refs2, shapes)
    assert np.array_equal(loc, np.broadcast_to(refs2[:, :, None, :, None, :] + np.float32(1), loc.shape))
    loc, _ = oracle_lib.deform_prep(np.full_like(off, 2.0 * p), logits, refs4, shapes)
    xy, wh = refs4[:, :, None, :, None, :2], refs4[:, :, None, :, None, 2:]
    assert np.array_equal(loc, np.broadcast_to(xy + wh, loc.shape))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("nc", [2, 4])
def test_deform_prep_rounds_each_step_to_the_dtype(oracle_lib, dtype, nc):
    """With a 16-bit query, each candle op of dino/mod.rs:166-178 returns that dtype. The oracle's
    rounded restatement equals the same steps run as torch CPU tensor ops in that dtype (each
    elementwise op computed in f32 and rounded once; the softmax in f32, rounded at the end): the
    locations bit for bit, the weights to one unit in the last place (the two softmaxes sum in
    different orders). At DINO's 167-wide level the rounding moves sampling points far beyond the
    2e-3 bar, so a restatement that skipped it would not pass as the reference."""
    import torch

    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    shapes = [(100, 167), (50, 84), (25, 42), (13, 21)]
    b, q, h, p = 1, 50, 8, 4
    off, logits, refs = (oracle_lib.round_to(x, dtype) for x in _prep_inputs(shapes, b, q, h, p, nc, 77 + nc))
    off[..., 0] *= 2.0  # offsets of a few pixels at the larger levels
    off = oracle_lib.round_to(off, dtype)
    loc, attn = oracle_lib.deform_prep(off, logits, refs, shapes, dtype=dtype)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(tdt)
    o, r = t(off), t(refs)
    if nc == 2:
        norm = t(np.array([[ww, hh] for hh, ww in shapes], np.float32)).reshape(1, 1, 1, len(shapes), 1, 2)
        want = r[:, :, None, :, None, :] + o / norm
    else:
        rr = r[:, :, None, :, None, :]
        want = rr[..., :2] + ((o * (1.0 / p)) * rr[..., 2:]) * 0.5
    assert want.dtype == tdt
    assert np.array_equal(loc, want.float().numpy())
    aw = torch.softmax(t(logits).float().reshape(b, q, h, -1), -1).to(tdt).float().numpy().reshape(attn.shape)
    ulp = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7}[dtype] * np.maximum(np.abs(aw), 2.0 ** -14)
    assert (np.abs(attn - aw) <= ulp).all()
    # the rounding matters: the f32 restatement of the same rounded inputs lies far from it
    loc32, _ = oracle_lib.deform_prep(off, logits, refs, shapes)
    px = np.abs(loc - loc32)[:, :, :, 0, :, 0].max() * 167  # in pixels of the 167-wide level
    assert px > 2e-3


def test_deform_prep_rejects_a_swapped_normaliser(oracle_lib):
    """A planted mistake, (H, W) in place of (W, H), is caught by the float64 module on non-square
    levels."""
    shapes = [(7, 9), (4, 5)]
    off, logits, refs = _prep_inputs(shapes, 1, 9, 2, 4, 2, 5)
    loc, _ = oracle_lib.deform_prep(off, logits, refs, shapes)
    swapped, _ = oracle_lib.deform_prep(off, logits, refs, [(w, h) for h, w in shapes])
    loc64, _ = refimpl.deform_prep64(off, logits, refs, shapes)
    assert np.abs(loc - loc64).max() < 2e-6
    assert np.abs(swapped[..., 0] - loc64[..., 0]).max() > 1e-3


def test_deform_pixel_centres_are_a_pure_gather(oracle_lib):
    shapes = [(6, 8), (3, 4)]
    b, q, h, d, p = 1, 5, 2, 4, 2
    value, _, _ = _deform_inputs(shapes, b, q, h, d, p, 10)
    r = _rng(11)
    l = len(shapes)
    loc = np.empty((b, q, h, l, p, 2), np.float32)
    picks = np.empty((b, q, h, l, p, 2), np.int64)
    for li, (hh, ww) in enumerate(shapes):
        xs = r.integers(0, ww, size=(b, q, h, p))
        ys = r.integers(0, hh, size=(b, q, h, p))
        loc[:, :, :, li, :, 0] = (xs + 0.5) / ww
        loc[:, :, :, li, :, 1] = (ys + 0.5) / hh
        picks[:, :, :, li, :, 0] = xs
        picks[:, :, :, li, :, 1] = ys
    attn = np.zeros((b, q, h, l, p), np.float32)
    attn[..., 1, 0] = 1.0  # one-hot on (level 1, point 0)
    got = oracle_lib.deform_attn(value, loc, attn, shapes).reshape(b, q, h, d)
    start = shapes[0][0] * shapes[0][1]
    for qi in range(q):
        for hi in range(h):
            x, y = picks[0, qi, hi, 1, 0]
            want = value[0, start + y * shapes[1][1] + x, hi]
            np.testing.assert_allclose(got[0, qi, hi], want, rtol=1e-6, atol=1e-6)


def test_deform_is_zero_beyond_one_pixel_outside(oracle_lib):
    shapes = [(4, 4)]
    value, loc, attn = _deform_inputs(shapes, 1, 3, 1, 4, 2, 12)
    loc[..., 0] = -1.0 / 4  # x = -1.5 px: both corner columns are outside
    got = oracle_lib.deform_attn(value, loc, attn, shapes)
    assert np.all(got == 0)


# ----------------------------------------------------------------------------------------- sdpa / flash

@pytest.mark.parametrize("b,h,lq,lk,d", [(1, 1, 5, 7, 16), (2, 3, 33, 65, 64), (1, 1, 40, 100, 256)])
def test_sdpa_matches_torch_float64(oracle_lib, b, h, lq, lk, d):
    r = _rng(13)
    q, k, v = (r.standard_normal((b, h, x, d)).astype(np.float32) for x in (lq, lk, lk))
    got = oracle_lib.sdpa(q, k, v)
    want = refimpl.sdpa64(q, k, v)
    assert np.abs(got - want).max() < 2e-6


def test_sdpa_closed_forms(oracle_lib):
    r = _rng(14)
    q = r.standard_normal((1, 1, 9, 32)).astype(np.float32)
    v1 = r.standard_normal((1, 1, 1, 32)).astype(np.float32)
    k1 = r.standard_normal((1, 1, 1, 32)).astype(np.float32)
    np.testing.assert_allclose(oracle_lib.sdpa(q, k1, v1), np.broadcast_to(v1, q.shape), rtol=1e-6)
    k = np.broadcast_to(k1, (1, 1, 20, 32)).copy()
    v = r.standard_normal((1, 1, 20, 32)).astype(np.float32)
    np.testing.assert_allclose(oracle_lib.sdpa(q, k, v), np.broadcast_to(v.mean(2, keepdims=True), q.shape),
                               atol=1e-6)
    k = r.standard_normal((1, 1, 20, 32)).astype(np.float32)
    perm = r.permutation(20)
    a = oracle_lib.sdpa(q, k, v)
    b = oracle_lib.sdpa(q, k[:, :, perm], v[:, :, perm])
    assert np.abs(a - b).max() < 1e-6


@pytest.mark.parametrize("mshape", ["bias", "padding", "query_rows"])
def test_sdpa_mask_matches_torch_float64(oracle_lib, mshape):
    """sdpa's additive mask (sam3/nn.rs:29-32) against torch's float64 SDPA with attn_mask, which adds the
    mask to the scaled scores: TinyViT's per-head biases [1, H, N, N], DETR's key-padding mask
    [B, 1, 1, Lk] of 0 / -inf, and a per-query [Lq, 1] column."""
    r = _rng(16)
    b, h, lq, lk, d = 2, 3, 19, 23, 32
    q, k, v = (r.standard_normal((b, h, x, d)).astype(np.float32) for x in (lq, lk, lk))
    if mshape == "bias":
        mask = r.standard_normal((1, h, lq, lk)).astype(np.float32)
    elif mshape == "padding":
        mask = np.zeros((b, 1, 1, lk), np.float32)
        mask[0, ..., 17:] = -np.inf
        mask[1, ..., 3:9] = -np.inf
    else:
        mask = (2.0 * r.standard_normal((lq, 1))).astype(np.float32)
    got = oracle_lib.sdpa(q, k, v, mask)
    want = refimpl.sdpa64(q, k, v, attn_mask=np.broadcast_to(mask, (b, h, lq, lk)))
    assert np.abs(got - want).max() < 2e-6


def test_sdpa_mask_closed_forms(oracle_lib):
    """A zero mask is no mask (bit for bit); a constant mask changes nothing (softmax is shift
    invariant); -inf on a key set is the same as dropping those keys; a row with every key at -inf is
    NaN, as candle's softmax gives, and leaves the other rows alone. A mask applied before the scale,
    (s + m) * scale, a plausible slip that -inf masks cannot show, is far outside the float64
    comparison's tolerance on a finite bias mask (checked here on the same inputs)."""
    r = _rng(17)
    b, h, lq, lk, d = 1, 2, 11, 13, 32
    q, k, v = (r.standard_normal((b, h, x, d)).astype(np.float32) for x in (lq, lk, lk))
    base = oracle_lib.sdpa(q, k, v)
    assert np.array_equal(oracle_lib.sdpa(q, k, v, np.zeros((1, 1, 1, lk), np.float32)), base)
    np.testing.assert_allclose(oracle_lib.sdpa(q, k, v, np.full((1, 1, 1, 1), 3.5, np.float32)), base, atol=2e-6)
    keep = np.ones(lk, bool)
    keep[[1, 4, 12]] = False
    mask = np.where(keep, 0.0, -np.inf).astype(np.float32)[None, None, None, :]
    np.testing.assert_allclose(oracle_lib.sdpa(q, k, v, mask), oracle_lib.sdpa(q, k[:, :, keep], v[:, :, keep]),
                               atol=2e-6)
    m = np.zeros((1, 1, lq, lk), np.float32)
    m[0, 0, 5, :] = -np.inf
    got = oracle_lib.sdpa(q, k, v, m)
    assert np.isnan(got[:, :, 5]).all()
    rows = [i for i in range(lq) if i != 5]
    assert np.array_equal(got[:, :, rows], base[:, :, rows])
    bias = r.standard_normal((1, h, lq, lk))
    want = refimpl.sdpa64(q, k, v, attn_mask=bias)
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64))
    slip = (s + bias) * d ** -0.5
    slip = np.exp(slip - slip.max(-1, keepdims=True))
    slip = np.einsum("bhqk,bhkd->bhqd", slip / slip.sum(-1, keepdims=True), v.astype(np.float64))
    assert np.abs(slip - want).max() > 1e-2
    assert np.abs(oracle_lib.sdpa(q, k, v, bias.astype(np.float32)) - want).max() < 2e-6


@pytest.mark.parametrize("b,lq,lk,h,d", [(1, 5, 7, 2, 16), (2, 17, 9, 3, 64)])
def test_mha_blhd_matches_torch(oracle_lib, b, lq, lk, h, d):
    r = _rng(15)
    q = r.standard_normal((b, lq, h, d)).astype(np.float32)
    k = r.standard_normal((b, lk, h, d)).astype(np.float32)
    v = r.standard_normal((b, lk, h, d)).astype(np.float32)
    got = oracle_lib.mha_blhd(q, k, v)
    want = refimpl.sdpa64(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3))
    assert np.abs(got - want.transpose(0, 2, 1, 3)).max() < 2e-6


# ----------------------------------------------------------------------------------------- rope

@pytest.mark.parametrize("side,hd", [(4, 16), (64, 256), (9, 64)])
def test_rope_tables_match_complex_form(oracle_lib, side, hd):
    cos, sin = oracle_lib.rope_tables(side, 1.0, hd, 10000.0)
    cis = refimpl.axial_rope_cis64(side, hd, 10000.0)
    np.testing.assert_allclose(cos[:, 0::2], cis.real, atol=2e-5)
    np.testing.assert_allclose(sin[:, 0::2], cis.imag, atol=2e-5)
    assert np.array_equal(cos[:, 0::2], cos[:, 1::2]) and np.array_equal(sin[:, 0::2], sin[:, 1::2])
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)  # angle zero at grid (0, 0)


def test_rope_matches_complex_rotation_and_keeps_norms(oracle_lib):
    side, hd = 8, 32
    cos, sin = oracle_lib.rope_tables(side, 1.0, hd, 10000.0)
    x = _rng(16).standard_normal((side * side, hd)).astype(np.float32)
    got = oracle_lib.rope(x, cos, sin)
    want = refimpl.rope_complex64(x, refimpl.axial_rope_cis64(side, hd, 10000.0))
    assert np.abs(got - want).max() < 2e-5
    n_in = x[:, 0::2] ** 2 + x[:, 1::2] ** 2
    n_out = got[:, 0::2].astype(np.float64) ** 2 + got[:, 1::2] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=2e-5, atol=1e-6)


def test_rope_scores_depend_only_on_position_difference(oracle_lib):
    side, hd = 8, 16
    cos, sin = oracle_lib.rope_tables(side, 1.0, hd, 100.0)
    r = _rng(17)
    a, b = r.standard_normal(hd).astype(np.float32), r.standard_normal(hd).astype(np.float32)

    def score(pa, pb):
        ra = oracle_lib.rope(np.tile(a, (side * side, 1)), cos, sin)[pa]
        rb = oracle_lib.rope(np.tile(b, (side * side, 1)), cos, sin)[pb]
        return float(ra.astype(np.float64) @ rb)

    # (row, col) (1,2)->(3,5) and (4,0)->(6,3): same offset (2, 3)
    s1 = score(1 * side + 2, 3 * side + 5)
    s2 = score(4 * side + 0, 6 * side + 3)
    assert abs(s1 - s2) < 1e-4
    assert abs(score(0, 1) - score(0, 2)) > 1e-3


def test_rope_attention_matches_composed_float64(oracle_lib):
    side, d, frames, n_excl = 4, 32, 3, 4
    cos, sin = oracle_lib.rope_tables(side, 1.0, d, 10000.0)
    lq, mk = side * side, frames * side * side + n_excl
    r = _rng(18)
    q = r.standard_normal((lq, d)).astype(np.float32)
    k = r.standard_normal((mk, d)).astype(np.float32)
    v = r.standard_normal((mk, d)).astype(np.float32)
    got = oracle_lib.rope_attention(q, k, v, cos, sin, n_excl)
    cis = refimpl.axial_rope_cis64(side, d, 10000.0)
    qr = refimpl.rope_complex64(q, cis)
    kr = np.concatenate([refimpl.rope_complex64(k[: mk - n_excl], np.tile(cis, (frames, 1))),
                         k[mk - n_excl:].astype(np.float64)])
    want = refimpl.sdpa64(qr, kr, v)
    assert np.abs(got - want).max() < 5e-5


# ----------------------------------------------------------------------------------------- qkv_rope
# Pins of oracle.qkv_rope (kernels.rs:321-362): the identity and quarter-turn tables fix the formula's
# terms and signs exactly, the q/k planes agree bit for bit with the separately pinned rope (the same
# rounding of each product and the sum), tables with NaN odd columns show only the even column is read,
# and period-n rows show the t % n row rule. _qkv_rope_checks runs all of them on an implementation;
# the mutant test plants one plausible mistake per copy and checks that some pin rejects it.

def _qkv_rope_inputs(t, n, nh, hd, seed):
    r = _rng(seed)
    y = r.standard_normal((t, 3 * nh * hd)).astype(np.float32)
    b = r.standard_normal(3 * nh * hd).astype(np.float32)
    return y, b


def _qkv_rope_checks(oracle_lib, impl):
    """Returns the names of the pins that `impl(y, b, cos, sin, n, nh, hd) -> [3, T, nh, hd]` fails."""
    failed = []
    t, n, nh, hd = 11, 4, 3, 8
    y, b = _qkv_rope_inputs(t, n, nh, hd, 31)
    x = (y + b).reshape(t, 3, nh, hd).transpose(1, 0, 2, 3)
    ones, zeros = np.ones((n, hd), np.float32), np.zeros((n, hd), np.float32)
    if not np.array_equal(impl(y, b, ones, zeros, n, nh, hd), x):
        failed.append("identity")
    quarter = x.copy()
    quarter[:2, ..., 0::2], quarter[:2, ..., 1::2] = -x[:2, ..., 1::2], x[:2, ..., 0::2]
    if not np.array_equal(impl(y, b, zeros, ones, n, nh, hd), quarter):
        failed.append("quarter turn")
    side = 2  # n = 4 tokens per window, the rope_tables_hd tables
    cos, sin = oracle_lib.rope_tables(side, 1.0, hd, 100.0)
    got = impl(y, b, cos, sin, n, nh, hd)
    rows = np.arange(t) % n
    for which in range(2):
        for h in range(nh):
            want = oracle_lib.rope(x[which, :, h], cos[rows], sin[rows])
            if not np.array_equal(got[which, :, h], want):
                failed.append("rope")
    if not np.array_equal(got[2], x[2]):
        failed.append("v plane")
    r = _rng(32)
    cr, sr = r.standard_normal((n, hd)).astype(np.float32), r.standard_normal((n, hd)).astype(np.float32)
    cr[:, 1::2] = np.nan
    sr[:, 1::2] = np.nan
    yp = np.tile(y[:n], (3, 1))[:t]  # rows t and t + n equal
    gp = impl(yp, b, cr, sr, n, nh, hd)
    if not np.all(np.isfinite(gp)):
        failed.append("even column")
    if not np.array_equal(gp[:, n:], gp[:, :t - n]):
        failed.append("period n")
    return failed


def test_qkv_rope_passes_every_pin(oracle_lib):
    assert _qkv_rope_checks(oracle_lib, oracle_lib.qkv_rope) == []


def test_qkv_rope_matches_float64_rotation(oracle_lib):
    t, n, nh, hd = 40, 16, 2, 32
    cos, sin = oracle_lib.rope_tables(4, 1.0, hd, 10000.0)
    y, b = _qkv_rope_inputs(t, n, nh, hd, 33)
    got = oracle_lib.qkv_rope(y, b, cos, sin, n, nh, hd)
    x = (y.astype(np.float64) + b).reshape(t, 3, nh, hd)
    cis = refimpl.axial_rope_cis64(4, hd, 10000.0)[np.arange(t) % n]
    for which in range(2):
        for h in range(nh):
            want = refimpl.rope_complex64(x[:, which, h], cis)
            assert np.abs(got[which, :, h] - want).max() < 4e-6 * (1 + np.abs(want).max())
    np.testing.assert_allclose(got[2], x[:, 2], rtol=1e-7, atol=1e-6)


def test_qkv_rope_output_rounding_is_round_to_nearest_even(oracle_lib):
    t, n, nh, hd = 6, 3, 2, 8
    cos, sin = oracle_lib.rope_tables(2, 1.0, hd, 100.0)
    y, b = _qkv_rope_inputs(t, n, nh, hd, 34)
    y, b = oracle_lib.round_to(y, "bf16"), oracle_lib.round_to(b, "bf16")
    f32 = oracle_lib.qkv_rope(y, b, cos[:n], sin[:n], n, nh, hd)
    assert np.array_equal(oracle_lib.qkv_rope(y, b, cos[:n], sin[:n], n, nh, hd, dtype="bf16"),
                          oracle_lib.round_to(f32, "bf16"))


def _qkv_rope_mutants():
    def base(y, b, cos, sin, n, nh, hd, odd=False, row=lambda t, n: t % n, sign=1.0, rot_v=False, fma=False,
             pre_round=False):
        t = y.shape[0]
        x = (y + b).reshape(t, 3, nh * hd).transpose(1, 0, 2).copy()
        if pre_round:  # the bias sum rounded to bf16 first (the CPU tensor fallback's order)
            x = (x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1) & 0xFFFF0000).view(np.float32)
        out = x.copy()
        for tt in range(t):
            rr = row(tt, n)
            c = np.tile(cos[rr, 1::2] if odd else cos[rr, 0::2], nh)
            s = sign * np.tile(sin[rr, 0::2], nh)
            for which in range(3 if rot_v else 2):
                x0, x1 = x[which, tt, 0::2], x[which, tt, 1::2]
                if fma:
                    out[which, tt, 0::2] = (x0.astype(np.float64) * c - (x1 * s)).astype(np.float32)
                else:
                    out[which, tt, 0::2] = x0 * c - x1 * s
                out[which, tt, 1::2] = x1 * c + x0 * s
        return out.reshape(3, t, nh, hd)

    def odd_column(*a):
        return base(*a, odd=True)

    def row_not_modulo(*a):
        return base(*a, row=lambda t, n: min(t, n - 1))

    def sin_sign_flipped(*a):
        return base(*a, sign=-1.0)

    def v_rotated(*a):
        return base(*a, rot_v=True)

    def fused_first_product(*a):
        return base(*a, fma=True)

    def bias_sum_rounded(*a):
        return base(*a, pre_round=True)

    return [odd_column, row_not_modulo, sin_sign_flipped, v_rotated, fused_first_product, bias_sum_rounded]


@pytest.mark.parametrize("mutant", _qkv_rope_mutants(), ids=lambda f: f.__name__)
def test_qkv_rope_mutants_are_caught(oracle_lib, mutant):
    assert _qkv_rope_checks(oracle_lib, mutant) != []


# ----------------------------------------------------------------------------------------- helpers

def test_rounding_helpers_are_round_to_nearest_even(oracle_lib):
    import torch

    x = np.concatenate([_rng(19).standard_normal(10000).astype(np.float32) * 100,
                        np.array([65504, 65519, 65520, 1e-8, -3e-5, 0.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11],
                                 np.float32)])
    assert np.array_equal(oracle_lib.round_to(x, "f16"), x.astype(np.float16).astype(np.float32))
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(oracle_lib.round_to(x, "bf16"), want)


def test_randn_is_seeded_and_normal(oracle_lib):
    a = oracle_lib.randn(7, (100000,))
    b = oracle_lib.randn(7, (100000,))
    c = oracle_lib.randn(8, (100000,))
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02


# ---- image preprocessing (image_proc.rs:57-96)

PREP_CASES = [(1080, 1920, 1024), (480, 640, 1024), (37, 53, 64), (300, 200, 96), (1000, 9, 128), (5, 7, 16)]


def _image(h, w, seed):
    return _rng(seed).integers(0, 256, (h, w, 3), dtype=np.uint8)


def _pil_preprocess(img, nh, nw, size, mean, std):
    """PIL's own antialiased bilinear resize of each channel as a 32-bit float image (double
    accumulation, normalised weights per pass), then (x - mean) / std and zero padding."""
    from PIL import Image

    out = np.zeros((3, size, size), np.float64)
    for c in range(3):
        ch = Image.fromarray(img[:, :, c].astype(np.float32), mode="F")
        res = np.asarray(ch.resize((nw, nh), Image.BILINEAR), dtype=np.float64)
        out[c, :nh, :nw] = (res - mean[c]) / std[c]
    return out


@pytest.mark.parametrize("h,w,size", PREP_CASES)
def test_preprocess_matches_pil_float_resize(oracle_lib, h, w, size):
    img = _image(h, w, h * 31 + w)
    nh, nw = oracle_lib.resized_hw(h, w, size)
    got = oracle_lib.preprocess(img, nh, nw, size)
    want = _pil_preprocess(img, nh, nw, size, oracle_lib.SAM_MEAN, oracle_lib.SAM_STD)
    assert np.abs(got - want).max() < 2e-5
    # a transposed image, or swapped output axes, is far off
    assert np.abs(oracle_lib.preprocess(img[::-1], nh, nw, size) - want).max() > 0.1


def test_preprocess_resized_hw_is_the_longest_side_rule(oracle_lib):
    assert oracle_lib.resized_hw(1080, 1920, 1024) == (576, 1024)
    assert oracle_lib.resized_hw(480, 640, 1024) == (768, 1024)
    assert oracle_lib.resized_hw(1365, 2048, 1024) == (683, 1024)  # 682.5 rounds half up
    assert oracle_lib.resized_hw(2048, 1365, 1024) == (1024, 683)


def test_preprocess_same_size_is_an_exact_normalisation(oracle_lib):
    """nh = h and nw = w: each output pixel's filter is one tap of weight 1, so the result is exactly
    (px - mean) / std in f32."""
    img = _image(23, 41, 5)
    got = oracle_lib.preprocess(img, 23, 41, 48)
    m = np.array(oracle_lib.SAM_MEAN, np.float32)[:, None, None]
    s = np.array(oracle_lib.SAM_STD, np.float32)[:, None, None]
    want = (img.transpose(2, 0, 1).astype(np.float32) - m) / s
    assert np.array_equal(got[:, :23, :41], want)
    assert not got[:, 23:, :].any() and not got[:, :, 41:].any()


def test_preprocess_constant_image_and_padding(oracle_lib):
    img = np.full((90, 70, 3), 200, np.uint8)
    img[..., 1] = 17
    nh, nw = oracle_lib.resized_hw(90, 70, 32)
    got = oracle_lib.preprocess(img, nh, nw, 32, mean=(1.0, 2.0, 3.0), std=(2.0, 4.0, 8.0))
    for c, (v, m, s) in enumerate(zip((200, 17, 200), (1.0, 2.0, 3.0), (2.0, 4.0, 8.0))):
        assert np.allclose(got[c, :nh, :nw], (v - m) / s, rtol=1e-6, atol=1e-6)
        assert not got[c, nh:, :].any() and not got[c, :, nw:].any()


# ---- bias_residual and bias_gelu (kernels.rs:618-663)

def test_bias_residual_is_the_left_to_right_f32_sum(oracle_lib):
    r = _rng(3)
    res, y = r.standard_normal((2, 7, 12)).astype(np.float32), r.standard_normal((2, 7, 12)).astype(np.float32)
    b = r.standard_normal(12).astype(np.float32)
    assert np.array_equal(oracle_lib.bias_residual(res, y, b), (res + y) + b)
    assert not np.array_equal(oracle_lib.bias_residual(res, y, b), res + y + b[::-1])  # bias per column


def test_bias_gelu_matches_float64_erf_and_its_limits(oracle_lib):
    import math

    r = _rng(4)
    y = (3.0 * r.standard_normal((5, 40))).astype(np.float32)
    b = r.standard_normal(40).astype(np.float32)
    got = oracle_lib.bias_gelu(y, b)
    x = (y + b).astype(np.float64)
    want = 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))
    assert np.allclose(got, want, rtol=2e-6, atol=1e-7)
    big = np.array([[0.0, 12.0, -12.0, 1e-30]], np.float32)
    out = oracle_lib.bias_gelu(big, np.zeros(4, np.float32))
    assert out[0, 0] == 0.0 and out[0, 1] == 12.0 and out[0, 2] == 0.0 and out[0, 3] == np.float32(5e-31)


# ------------------------------------------------------------------ bf16 CPU path (cpu_gemm.rs)

bf16_cpu = pytest.mark.skipif("not __import__('sam_oracle').bf16_available()",
                              reason="the reference's bf16 CPU path needs AVX-512 BF16 (cpu_gemm.rs:14-24)")


def test_bf16_bits_round_to_nearest_even(oracle_lib):
    """cpu_gemm.rs:38-45 against torch's f32 -> bfloat16 conversion (round to nearest even), including
    exact halfway cases in both directions."""
    import torch

    r = _rng(61)
    x = np.concatenate([r.standard_normal(5000), r.standard_normal(1000) * 1e30, r.standard_normal(1000) * 1e-30])
    halves = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x3F80C000, 0x7F7F8000], np.uint32).view(np.float32)
    x = np.concatenate([x.astype(np.float32), halves, np.float32([0.0, -0.0, np.inf, -np.inf])])
    got = oracle_lib.bf16_bits(x)
    want = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def _vdpbf16_emulation(a, w):
    """a [m, k] @ w [k, n] as the bf16 microkernel computes it, in numpy float32 from the instruction's
    definition: operands rounded to bf16; per output, for each k pair (2q, 2q+1) in order,
    acc = (acc + a[2q+1] w[2q+1]) + a[2q] w[2q], each product exact in f32, each sum rounded."""
    import torch

    ab = torch.from_numpy(a).bfloat16().float().numpy()
    wb = torch.from_numpy(w).bfloat16().float().numpy()
    m, k = a.shape
    n = w.shape[1]
    if k % 2:
        ab = np.concatenate([ab, np.zeros((m, 1), np.float32)], 1)
        wb = np.concatenate([wb, np.zeros((1, n), np.float32)], 0)
    acc = np.zeros((m, n), np.float32)
    for q in range(ab.shape[1] // 2):
        acc = (acc + np.outer(ab[:, 2 * q + 1], wb[2 * q + 1]).astype(np.float32)).astype(np.float32)
        acc = (acc + np.outer(ab[:, 2 * q], wb[2 * q]).astype(np.float32)).astype(np.float32)
    return acc


@bf16_cpu
@pytest.mark.parametrize("m,k,n", [(11, 27, 45), (70, 80, 33), (8, 16, 32), (1, 1, 1), (130, 33, 70)])
def test_bf16_matmul_is_the_vdpbf16ps_sequence(oracle_lib, m, k, n):
    """The packed bf16 GEMM (odd sizes: partial panels, odd K, partial row blocks) equals, bit for bit,
    an emulation of the instruction sequence written from its definition."""
    r = _rng(62 + m + k + n)
    a = r.standard_normal((m, k)).astype(np.float32)
    w = r.standard_normal((k, n)).astype(np.float32)
    assert np.array_equal(oracle_lib.bf16_matmul(a, w), _vdpbf16_emulation(a, w))


@bf16_cpu
def test_bf16_matmul_reference_bar(oracle_lib):
    """tests/cpu_gemm.rs:11-27: |bf16 matmul - f32 matmul| < 4e-3 of |x| |w| (Frobenius)."""
    r = _rng(63)
    x = r.standard_normal((37, 300)).astype(np.float32)
    w = r.standard_normal((300, 51)).astype(np.float32)
    err = np.abs(oracle_lib.bf16_matmul(x, w) - x.astype(np.float64) @ w).max()
    assert err < 4e-3 * np.linalg.norm(x) * np.linalg.norm(w) / np.sqrt(x.shape[0] * w.shape[1])


@bf16_cpu
def test_bf16_exp_accuracy_and_clamp(oracle_lib):
    """cpu_gemm.rs:272-286: relative error about 1e-7 near 0, plus the f32 rounding of t = x log2(e): the
    product's rounding (at most |t| 2^-24) and the constant's (|t| 2^-25), times ln 2, so at most
    1.04 |t| 2^-24 (checked point by point against float64 exp: below 2e-7 + 1.1 |t| 2^-24); exp(0) = 1
    exactly; below -126 ln 2 the argument clamps to 2^-126."""
    x = np.concatenate([np.linspace(-87.0, 0.0, 200001), -np.logspace(-8, 1.9, 1000)]).astype(np.float32)
    y = oracle_lib.bf16_exp(x)
    rel = np.abs(y.astype(np.float64) / np.exp(x.astype(np.float64)) - 1.0)
    t = np.abs(x.astype(np.float64)) * np.log2(np.e)
    assert (rel <= 2e-7 + 1.1 * t * 2.0 ** -24).all()
    assert oracle_lib.bf16_exp(np.float32([0.0]))[0] == 1.0
    assert oracle_lib.bf16_exp(np.float32([-200.0, -1000.0]))[0] == np.float32(2.0 ** -126)


@bf16_cpu
@pytest.mark.parametrize("h,w,bh,hd", [(14, 14, 6, 64), (64, 64, 2, 64), (7, 11, 3, 80)])
def test_bf16_attention_relpos_reference_bar(oracle_lib, h, w, bh, hd):
    """tests/cpu_gemm.rs:30-50: attention_relpos_cpu with bf16 on vs off over the reference test's three
    geometries, mean relative error < 1.5e-2 (N(0,1) inputs, scale 0.125)."""
    r = _rng(64 + h * w)
    n = h * w
    q = r.standard_normal((bh, n, hd)).astype(np.float32)
    kt = r.standard_normal((bh, hd, n)).astype(np.float32)
    v = r.standard_normal((bh, n, hd)).astype(np.float32)
    t = r.standard_normal((2 * h - 1 + 2 * w - 1, hd)).astype(np.float32)
    got = oracle_lib.bf16_attention_relpos(q, kt, v, t, h, w, 0.125)
    want = oracle_lib.attention_relpos(q, kt, v, t, h, w, 0.125)
    rel = np.abs(got - want).mean() / np.abs(want).mean()
    assert rel < 1.5e-2


@bf16_cpu
def test_bf16_attention_relpos_rounding_points(oracle_lib):
    """The bf16 branch rounds q, kT (for the score GEMM) and P, v (for the output GEMM) to bf16, and keeps
    the rel-pos dot products, the softmax and the accumulations in f32: a float64 model with exactly
    those roundings is within 1e-3, a model that skips the rounding of P is not."""
    import torch

    h, w, bh, hd = 7, 11, 2, 80
    r = _rng(65)
    n = h * w
    q = r.standard_normal((bh, n, hd)).astype(np.float32)
    kt = r.standard_normal((bh, hd, n)).astype(np.float32)
    v = r.standard_normal((bh, n, hd)).astype(np.float32)
    t = (0.5 * r.standard_normal((2 * h - 1 + 2 * w - 1, hd))).astype(np.float32)
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().double().numpy()
    got = oracle_lib.bf16_attention_relpos(q, kt, v, t, h, w, 0.125)
    s = bf(q) @ bf(kt)
    bias = refimpl.relpos_logits64(np.zeros_like(s), q, t, h, w, 0.125)
    p = refimpl.softmax64(0.125 * s + bias)
    with_round = bf(p) @ bf(v)
    without = p @ bf(v)
    e1, e2 = np.abs(got - with_round).max(), np.abs(got - without).max()
    assert e1 < 1e-3 < e2, (e1, e2)


@bf16_cpu
def test_bf16_flash_attention(oracle_lib):
    """cpu_gemm.rs:361-417: against the exact attention (the reference's bf16-vs-f32 bar, mean relative
    < 1.5e-2), and with a single key every query returns that key's value rounded to bf16."""
    import torch

    r = _rng(66)
    b, lq, lk, h, d = 2, 45, 70, 3, 64
    q = r.standard_normal((b, lq, h, d)).astype(np.float32)
    k = r.standard_normal((b, lk, h, d)).astype(np.float32)
    v = r.standard_normal((b, lk, h, d)).astype(np.float32)
    got = oracle_lib.bf16_flash_attention(q, k, v)
    want = oracle_lib.mha_blhd(q, k, v)
    assert np.abs(got - want).mean() / np.abs(want).mean() < 1.5e-2
    one = oracle_lib.bf16_flash_attention(q, k[:, :1], v[:, :1])
    vb = torch.from_numpy(v[:, :1]).bfloat16().float().numpy()
    assert np.array_equal(one, np.broadcast_to(vb, one.shape))
