"""Parity of SAM image preprocessing (libsam_hip.so) with the CPU oracle, on an MI355X.

The oracle restates the reference's CPU path (image_proc.rs:57-96) in f32 with no FMA contraction, and
the kernel does the same operations in the same order, so f32 output must be bit-identical; f16 and
bf16 output must equal the oracle's value rounded to nearest even. Cases: SAM's longest-side rule
(image_proc.rs:21-36) for landscape, portrait and small images, upscaling (no antialiasing), strong
shrinking, squashing to a square (prepare_square, image_proc.rs:43-53), odd sizes, and the reference's
GPU argument errors.
"""
import numpy as np
import pytest
import torch

import sam_oracle as oracle

pytestmark = pytest.mark.gpu
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module")
def hip():
    import sam_hip

    sam_hip.load()
    assert torch.cuda.is_available(), "no GPU visible"
    return sam_hip


def image(h, w, seed):
    return np.random.default_rng(seed).integers(0, 256, (h, w, 3), dtype=np.uint8)


def run(hip, img, nh, nw, size, dtype, mean=None, std=None):
    src = torch.from_numpy(img).cuda()
    kw = {} if mean is None else {"mean": mean, "std": std}
    out = hip.preprocess(src, (nh, nw), size, dtype=TORCH_DT[dtype], **kw)
    torch.cuda.synchronize()
    assert out.shape == (1, 3, size, size) and out.dtype == TORCH_DT[dtype]
    return out[0].float().cpu().numpy()


LONGEST_SIDE = [(1080, 1920, 1024), (1920, 1080, 1024), (480, 640, 1024), (1365, 2048, 1024), (37, 53, 64),
                (1000, 9, 128), (3000, 4000, 1024), (2900, 1900, 96), (1, 1, 64), (2, 1, 1024), (1, 3, 1024)]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("h,w,size", LONGEST_SIDE, ids=[f"{h}x{w}-{s}" for h, w, s in LONGEST_SIDE])
def test_prepare_matches_oracle(hip, h, w, size, dtype):
    print(f"preprocess {h}x{w} -> {size} {dtype}", flush=True)
    img = image(h, w, h + 7 * w)
    nh, nw = oracle.resized_hw(h, w, size)
    assert hip.resized_hw(h, w, size)[:2] == (nh, nw)
    want = oracle.round_to(oracle.preprocess(img, nh, nw, size), dtype)
    got = run(hip, img, nh, nw, size, dtype)
    assert np.array_equal(got, want), f"max abs diff {np.abs(got - want).max():.3g}"


@pytest.mark.parametrize("h,w,size", [(720, 1280, 1008), (64, 48, 1008), (1008, 1008, 1008), (5, 3, 11)])
def test_prepare_square_matches_oracle(hip, h, w, size):
    """SAM 3 squashes the image to size x size (image_proc.rs:43-53), stretching one axis."""
    print(f"prepare_square {h}x{w} -> {size}", flush=True)
    img = image(h, w, 3 * h + w)
    want = oracle.preprocess(img, size, size, size, mean=(127.5,) * 3, std=(127.5,) * 3)
    src = torch.from_numpy(img).cuda()
    got = hip.prepare_square(src, size, mean=(127.5,) * 3, std=(127.5,) * 3)[0].cpu().numpy()
    assert np.array_equal(got, want)


def test_prepare_returns_the_geometry(hip):
    img = image(300, 500, 1)
    t, orig, resized, scale = hip.prepare(torch.from_numpy(img).cuda(), 256)
    assert orig == (300, 500) and resized == (154, 256) and abs(scale - 256 / 500) < 1e-7
    want = oracle.preprocess(img, 154, 256, 256)
    assert np.array_equal(t[0].cpu().numpy(), want)


def test_odd_sizes_and_custom_normalisation(hip):
    img = image(29, 17, 9)
    mean, std = (10.0, 20.0, 30.0), (0.5, 3.0, 7.0)
    for nh, nw, size in [(29, 17, 31), (13, 8, 13), (40, 33, 40), (1, 1, 3)]:
        want = oracle.preprocess(img, nh, nw, size, mean=mean, std=std)
        assert np.array_equal(run(hip, img, nh, nw, size, "f32", mean, std), want), (nh, nw, size)


def test_preprocess_errors(hip):
    src = torch.zeros(8, 8, 3, dtype=torch.uint8, device="cuda")
    with pytest.raises(hip.SamHipError, match="does not fit"):
        hip.preprocess(src, (9, 4), 8)
    with pytest.raises(hip.SamHipError, match="std"):
        hip.preprocess(src, (4, 4), 8, std=(1.0, 0.0, 1.0))
    with pytest.raises(hip.SamHipError, match="u8"):
        hip.preprocess(src.float(), (4, 4), 8)
    wide = torch.zeros(2, 4000, 3, dtype=torch.uint8, device="cuda")
    with pytest.raises(hip.SamHipError, match="columns to 40 needs more than 64 filter taps"):
        hip.preprocess(wide, (1, 40), 64)
    tall = torch.zeros(4000, 2, 3, dtype=torch.uint8, device="cuda")
    with pytest.raises(hip.SamHipError, match="rows to 40 needs more than 64 filter taps"):
        hip.preprocess(tall, (40, 1), 64)


def test_unaligned_image_and_strong_shrink(hip):
    """An image that starts one byte into its allocation (the kernel gathers single bytes, so any
    alignment works) and an 8000-row image shrunk 7.8x (31 taps per column)."""
    h, w, size = 333, 517, 256
    img = image(h, w, 12)
    nh, nw = oracle.resized_hw(h, w, size)
    buf = torch.zeros(h * w * 3 + 1, dtype=torch.uint8, device="cuda")
    buf[1:] = torch.from_numpy(img.reshape(-1)).cuda()
    src = buf[1:].view(h, w, 3)
    assert src.data_ptr() % 4 != 0
    got = hip.preprocess(src, (nh, nw), size)[0].cpu().numpy()
    assert np.array_equal(got, oracle.preprocess(img, nh, nw, size))
    big = image(8000, 600, 13)
    nh, nw = oracle.resized_hw(8000, 600, 1024)
    got = hip.preprocess(torch.from_numpy(big).cuda(), (nh, nw), 1024)[0].cpu().numpy()
    assert np.array_equal(got, oracle.preprocess(big, nh, nw, 1024))
