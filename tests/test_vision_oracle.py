"""Pins the oracle's image tower (ora_vision_*, oracle/ge_oracle.c) before it checks the GPU.

BASELINE config 5's tower has no counterpart in the reference (whose gemma4v tower differs in
width, head size, norms and MLP), so there are no reference fixtures for it. Each function is
pinned by closed forms and invariants, and the whole forward by the independent float64 numpy
statement in tests/npref.py (its own GGUF reader, einsum attention, pooling as a reshape).
"""
import numpy as np
import pytest

import gemma_embed as ge
import ge_oracle as ora
import npref

RNG = np.random.default_rng(77)


def test_layernorm_closed_form_and_invariants():
    x = RNG.normal(size=(9, 1152)).astype(np.float32) * 3 + 2
    w = np.ones(1152, np.float32)
    b = np.zeros(1152, np.float32)
    y = ora.layernorm(x, 1152, w, b, 1e-6).reshape(9, 1152).astype(np.float64)
    assert np.abs(y.mean(axis=1)).max() < 1e-5
    assert np.abs(y.var(axis=1) - 1).max() < 1e-4
    # shift and positive scale of the input do not change the output
    y2 = ora.layernorm(x * 4 + 7, 1152, w, b, 0.0).reshape(9, 1152)
    y3 = ora.layernorm(x, 1152, w, b, 0.0).reshape(9, 1152)
    assert np.abs(y2 - y3).max() < 1e-4
    # weight and bias against float64
    w = RNG.normal(size=1152).astype(np.float32)
    b = RNG.normal(size=1152).astype(np.float32)
    got = ora.layernorm(x, 1152, w, b, 1e-6).reshape(9, 1152)
    want = npref.layernorm(x.astype(np.float64), w, b, 1e-6)
    assert np.abs(got - want).max() < 1e-4 * np.abs(want).max()


@pytest.mark.parametrize("gx,gy,merge", [(6, 9, 3), (3, 3, 3), (4, 2, 2), (5, 7, 1)])
def test_pool_closed_form(gx, gy, merge):
    d = 8
    x = RNG.normal(size=(gx * gy, d)).astype(np.float32)
    got = ora.pool(x, gx, gy, merge, d)
    want = np.zeros_like(got, dtype=np.float64)
    for oy in range(gy // merge):
        for ox in range(gx // merge):
            rows = [(merge * oy + dy) * gx + merge * ox + dx for dy in range(merge) for dx in range(merge)]
            want[oy * (gx // merge) + ox] = x[rows].astype(np.float64).mean(axis=0)
    assert np.abs(got - want).max() < 1e-6
    if merge == 1:
        assert np.array_equal(got, x)
    c = np.full((gx * gy, d), 0.375, np.float32)
    assert np.array_equal(ora.pool(c, gx, gy, merge, d), np.full_like(got, 0.375))


def test_synthetic_vision_file_layout(tiny_vision_gguf):
    g = npref.Gguf(tiny_vision_gguf)
    s = ge.TINY_VISION
    d, ff = s["hidden"], s["feed_forward"]
    assert g.meta["general.architecture"] == "clip"
    assert g.meta["clip.vision.projector_type"] == "gemma3"
    assert g.meta["clip.vision.block_count"] == s["layers"]
    assert g.meta["clip.vision.projector.scale_factor"] == s["merge"]
    assert g.tensors["v.patch_embd.weight"][0] == [3 * s["patch_size"] ** 2, d]
    assert g.tensors["v.position_embd.weight"][0] == [d, s["positions"], 2]
    assert g.tensors["v.blk.0.ffn_up.weight"][0] == [d, ff]
    assert g.tensors["v.blk.0.ffn_down.weight"][0] == [ff, d]
    assert g.tensors["v.blk.0.ffn_down.weight"][1] == 1  # F16: 4304 is not a multiple of 32
    assert g.tensors["mm.input_projection.weight"][0] == [d, s["proj_dims"]]
    # value rules: Q8_0 rows keep their input's scale (rms of a row ~ 1.15 / sqrt(K) * sqrt(K))
    w = g.tensor("v.blk.0.attn_q.weight")
    assert 0.7 < np.sqrt((w ** 2).sum(axis=1)).mean() < 1.6
    ln = g.tensor("v.blk.1.ln2.weight")
    assert abs(ln.mean() - 1) < 0.02 and abs(ln.std() - 0.1) < 0.02
    down = g.tensor("v.blk.0.ffn_down.weight")
    assert abs(down.std() * np.sqrt(ff) - 1) < 0.05


KEEP = [(n, l) for n in ("layer_inp_normed", "Qcur", "Kcur", "Vcur", "kqv_out", "attn_out", "ffn_inp",
                         "ffn_inp_normed", "ffn_gelu", "ffn_out", "layer_out") for l in range(2)] + \
       [(n, -1) for n in ("inp", "pos_embd", "pooled", "pooled_normed", "projected")]


@pytest.mark.parametrize("gx,gy", [(6, 9), (3, 3), (12, 6)])
def test_vision_forward_tiny_vs_float64(tiny_vision_gguf, gx, gy):
    g = npref.Gguf(tiny_vision_gguf)
    with ora.VisionOracle(tiny_vision_gguf) as v:
        patches = ge.image_patches(gx * 100 + gy, [(gx, gy)], v.area)
        out, tr = v.forward(patches, gx, gy, keep=KEEP)
    want, wtr = npref.vision_forward(g, patches.astype(np.float64), gx, gy, keep=tuple(KEEP))
    assert out.shape == want.shape
    for key in KEEP:
        a, b = tr[key], wtr[key]
        assert a.shape == b.shape, key
        assert np.abs(a - b).max() < 2e-4 * np.abs(b).max(), key


def test_vision_forward_rejects_bad_grids(tiny_vision_gguf):
    with ora.VisionOracle(tiny_vision_gguf) as v:
        p = np.zeros((4 * 6, v.area), np.float32)
        with pytest.raises(ValueError):
            v.forward(p, 4, 6)  # 4 is not a multiple of the merge size 3
        p = np.zeros((15 * 3, v.area), np.float32)
        with pytest.raises(ValueError):
            v.forward(p, 15, 3)  # past the 12 position rows


def test_vision_open_rejects_text_model(tiny_gguf):
    with pytest.raises(ValueError, match="clip"):
        ora.VisionOracle(tiny_gguf)
