"""The CPU oracle against the committed golden fixtures (float64 brute force on inputs exact in every
dtype; see tests/golden/make_golden.py). CPU only."""
import numpy as np
import pytest

import golden_io

REL = 1e-5  # the f32 parity bar, max|diff| / max|expected|


def rel_err(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


def test_every_kind_has_fixtures():
    for kind in ("relpos", "deform", "flash", "rope"):
        assert golden_io.names(kind), kind


@pytest.mark.parametrize("name", golden_io.names("relpos"))
def test_oracle_attention_relpos_golden(oracle_lib, name):
    g = golden_io.load("relpos", name)
    h, w, bh, hd = (int(x) for x in g["geom"])
    out = oracle_lib.attention_relpos(g["q"], g["kt"], g["v"], g["table"], h, w, float(g["scale"][0]))
    assert rel_err(out, g["out"]) <= REL


@pytest.mark.parametrize("name", [n for n in golden_io.names("relpos") if golden_io.load("relpos", n)["s"].size])
def test_oracle_relpos_softmax_golden(oracle_lib, name):
    g = golden_io.load("relpos", name)
    h, w, bh, hd = (int(x) for x in g["geom"])
    p = oracle_lib.relpos_softmax(g["s"].astype(np.float32), g["q"], g["table"], h, w, float(g["scale"][0]))
    assert np.abs(p - g["probs"]).max() <= 1e-6


@pytest.mark.parametrize("name", golden_io.names("deform"))
def test_oracle_deform_golden(oracle_lib, name):
    g = golden_io.load("deform", name)
    out = oracle_lib.deform_attn(g["value"], g["loc"], g["attn"], [tuple(x) for x in g["shapes"].tolist()])
    assert rel_err(out, g["out"]) <= REL


@pytest.mark.parametrize("name", golden_io.names("flash"))
def test_oracle_flash_golden(oracle_lib, name):
    g = golden_io.load("flash", name)
    assert rel_err(oracle_lib.mha_blhd(g["q"], g["k"], g["v"]), g["out"]) <= REL
    t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))
    assert rel_err(oracle_lib.sdpa(t(g["q"]), t(g["k"]), t(g["v"])), t(g["out"])) <= REL


@pytest.mark.parametrize("name", golden_io.names("rope"))
def test_oracle_rope_golden(oracle_lib, name):
    g = golden_io.load("rope", name)
    side = int(g["side"][0])
    x = g["x"]
    cos, sin = oracle_lib.rope_tables(side, 1.0, x.shape[1], 10000.0)
    reps = x.shape[0] // (side * side)
    out = oracle_lib.rope(x, np.concatenate([cos] * reps), np.concatenate([sin] * reps))
    # f32 tables: the angle pos * theta^(-k) is rounded to f32 before cos/sin
    assert np.abs(out - g["out"]).max() <= 1e-5
