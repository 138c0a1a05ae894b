"""The image tower on the GPU against the CPU oracle, through the C-ABI.

Bars as for the text path: every traced tensor within max|d| / max|ref| <= 1e-2 of the oracle,
the projected vectors at cosine >= 0.99999 per token. Bitwise invariants as the reference checks
them for text packing (MetalForwardTests.swift:54-120): an image's vectors do not depend on the
other images of its batch, nor on the batch size that selects the GEMM tiles."""
import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge

pytestmark = pytest.mark.gpu

TOL = 1e-2
COSINE_BAR = 0.99999
NAMES = ["layer_inp_normed", "Qcur", "Kcur", "Vcur", "kqv_out", "attn_out", "ffn_inp", "ffn_inp_normed", "ffn_gelu",
         "ffn_out", "layer_out"]
GLOBAL = ["inp", "pos_embd", "pooled", "pooled_normed", "projected"]


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def split_rows(a, counts):
    out, r = [], 0
    for n in counts:
        out.append(a[r:r + n])
        r += n
    return out


@pytest.fixture(scope="module")
def ctx():
    c = ge.Context.create(0)
    print("device:", c.device_name, flush=True)
    yield c
    c.close()


@pytest.fixture(scope="module")
def tiny_tower(ctx, tiny_vision_gguf):
    ctx.vision_load(tiny_vision_gguf)
    o = ora.VisionOracle(tiny_vision_gguf)
    yield ctx, o
    o.close()


GRIDS = [(6, 9), (12, 3), (3, 3)]


def test_tiny_tower_every_trace_vs_oracle(tiny_tower):
    ctx, o = tiny_tower
    patches = ge.image_patches(21, GRIDS, o.area)
    per_image = split_rows(patches, [gx * gy for gx, gy in GRIDS])
    keep = [(n, l) for n in NAMES for l in range(o.layers)] + [(n, -1) for n in GLOBAL]
    want = [o.forward(p, gx, gy, keep=keep)[1] for p, (gx, gy) in zip(per_image, GRIDS)]
    for name, layer in keep:
        got = ctx.vision_trace(patches, GRIDS, name, layer)
        pooled = name in ("pooled", "pooled_normed", "projected")
        counts = [(gx // 3) * (gy // 3) if pooled else gx * gy for gx, gy in GRIDS]
        width = got.size // sum(counts)
        parts = split_rows(got.reshape(-1, width), counts)
        for i, part in enumerate(parts):
            w = want[i][(name, layer)].reshape(part.shape)
            assert max_rel(part, w) <= TOL, (name, layer, i, max_rel(part, w))


def test_tiny_tower_vectors_vs_oracle(tiny_tower):
    ctx, o = tiny_tower
    patches = ge.image_patches(22, GRIDS, o.area)
    vecs, secs = ctx.vision_encode(patches, GRIDS, o.proj_dims)
    assert secs > 0
    rows = split_rows(vecs, [(gx // 3) * (gy // 3) for gx, gy in GRIDS])
    for i, ((gx, gy), p) in enumerate(zip(GRIDS, split_rows(patches, [gx * gy for gx, gy in GRIDS]))):
        want, _ = o.forward(p, gx, gy)
        assert max_rel(rows[i], want) <= TOL, i
        for t in range(want.shape[0]):
            assert cosine(rows[i][t], want[t]) >= COSINE_BAR, (i, t)


def test_tiny_tower_images_independent_of_batch(tiny_tower):
    """Bitwise: alone, in a batch, and in a batch large enough for other GEMM tiles."""
    ctx, o = tiny_tower
    grids = [(12, 12)] * 6 + [(6, 9)]  # 918 patches: the tiled GEMMs, not the short-batch kernel
    patches = ge.image_patches(23, grids, o.area)
    batch, _ = ctx.vision_encode(patches, grids, o.proj_dims)
    rows = split_rows(batch, [(gx // 3) * (gy // 3) for gx, gy in grids])
    pats = split_rows(patches, [gx * gy for gx, gy in grids])
    for i in (0, 6):
        alone, _ = ctx.vision_encode(pats[i], [grids[i]], o.proj_dims)
        assert np.array_equal(alone, rows[i]), i
    again, _ = ctx.vision_encode(patches, grids, o.proj_dims)
    assert np.array_equal(again, batch)


def test_tiny_tower_staged_run_matches_encode(tiny_tower):
    ctx, o = tiny_tower
    patches = ge.image_patches(24, GRIDS, o.area)
    want, _ = ctx.vision_encode(patches, GRIDS, o.proj_dims)
    ctx.vision_stage(patches, GRIDS)
    ctx.vision_run()
    ctx.vision_run()
    assert np.array_equal(ctx.vision_read(o.proj_dims), want)


def test_tiny_tower_rejects_bad_batches(tiny_tower):
    ctx, o = tiny_tower
    p = np.zeros((4 * 6, o.area), np.float32)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.vision_encode(p, [(4, 6)], o.proj_dims)  # not a multiple of the merge size
    assert e.value.code == ge.GE_ERR_INVALID
    p = np.zeros((15 * 3, o.area), np.float32)
    with pytest.raises(ge.GemmaEmbedError):
        ctx.vision_encode(p, [(15, 3)], o.proj_dims)  # past the 12 position rows
    p = np.zeros((10, o.area), np.float32)
    with pytest.raises(ge.GemmaEmbedError):
        ctx.vision_encode(p, [(3, 3)], o.proj_dims)  # 9 patches in the grid, 10 given


def test_vision_needs_an_uploaded_tower():
    c = ge.Context.create(0)
    try:
        with pytest.raises(ge.GemmaEmbedError) as e:
            c.vision_encode(np.zeros((9, 768), np.float32), [(3, 3)], 768)
        assert e.value.code == ge.GE_ERR_STATE
    finally:
        c.close()


@pytest.fixture(scope="module")
def config5(config5_vision_gguf):
    c = ge.Context.create(0)
    c.vision_load(config5_vision_gguf)
    o = ora.VisionOracle(config5_vision_gguf)
    yield c, o
    o.close()
    c.close()


@pytest.mark.timeout(300)
def test_config5_image_vs_oracle(config5):
    """One 768 x 768 image (48 x 48 patches) through all 16 layers."""
    c, o = config5
    patches = ge.image_patches(31, [(48, 48)], o.area)
    vecs, _ = c.vision_encode(patches, [(48, 48)], o.proj_dims)
    want, _ = o.forward(patches, 48, 48)
    assert vecs.shape == (256, 768)
    assert max_rel(vecs, want) <= TOL
    assert min(cosine(vecs[t], want[t]) for t in range(256)) >= COSINE_BAR


def test_config5_batch_of_eight_bitwise(config5):
    """BASELINE config 5's batch: each image's vectors equal its own single-image run."""
    c, o = config5
    grids = [(48, 48)] * 8
    patches = ge.image_patches(32, grids, o.area)
    batch, _ = c.vision_encode(patches, grids, o.proj_dims)
    assert batch.shape == (8 * 256, 768) and np.all(np.isfinite(batch))
    for i in (0, 5):
        alone, _ = c.vision_encode(patches[i * 2304:(i + 1) * 2304], [(48, 48)], o.proj_dims)
        assert np.array_equal(alone, batch[i * 256:(i + 1) * 256]), i


@pytest.mark.parametrize("grids", [
    [(48, 48)] * 2,                # 4608 rows: the MLP-up launch (GELU and bias) ends in half tiles
    [(48, 48)] * 2 + [(24, 24)],   # 5184 rows: the QKV launch (head-padded outputs) ends in half tiles
    [(48, 48)] * 6,                # 13824 rows: the o and down launches end in half tiles, the
                                   # right half of their last column tile past the 1152 outputs
])
def test_config5_half_tile_batches_bitwise(config5, grids):
    """Batches whose 128 x 256 GEMM launches leave a small last partial round of workgroup slots,
    which then runs as 128 x 128 half tiles: each image's vectors must equal its own run alone."""
    c, o = config5
    patches = ge.image_patches(33, grids, o.area)
    batch, _ = c.vision_encode(patches, grids, o.proj_dims)
    rows = split_rows(batch, [(gx // 3) * (gy // 3) for gx, gy in grids])
    pats = split_rows(patches, [gx * gy for gx, gy in grids])
    assert np.all(np.isfinite(batch))
    for i in sorted({0, len(grids) - 1}):
        alone, _ = c.vision_encode(pats[i], [grids[i]], o.proj_dims)
        assert np.array_equal(alone, rows[i]), i


def test_tower_with_128_wide_heads_and_q8_down(tmp_path):
    """The other head path (head dim 128 through the text path's LDS-copy attention, no padding)
    and a Q8_0 ffn_down, on a small tower with a 2 x 2 merge."""
    spec = dict(layers=2, hidden=256, heads=2, feed_forward=1024, patch_size=16, merge=2, proj_dims=128, positions=16,
                eps=1e-6, ffn_down_type=ge.GE_TYPE_Q8_0, seed=13)
    path = ge.synth_write_vision_gguf(str(tmp_path / "small_vision.gguf"), **spec)
    grids = [(8, 6), (4, 4), (16, 2)]
    c = ge.Context.create(0)
    try:
        c.vision_load(path)
        with ora.VisionOracle(path) as o:
            patches = ge.image_patches(41, grids, o.area)
            vecs, _ = c.vision_encode(patches, grids, o.proj_dims, merge=2)
            rows = split_rows(vecs, [(gx // 2) * (gy // 2) for gx, gy in grids])
            pats = split_rows(patches, [gx * gy for gx, gy in grids])
            for i, (gx, gy) in enumerate(grids):
                want, tr = o.forward(pats[i], gx, gy, keep=[("kqv_out", 1), ("layer_out", 1)])
                assert max_rel(rows[i], want) <= TOL, i
                assert min(cosine(rows[i][t], want[t]) for t in range(want.shape[0])) >= COSINE_BAR, i
            for name in ("kqv_out", "layer_out"):
                got = c.vision_trace(patches, grids, name, 1).reshape(patches.shape[0], -1)
                for i, ((gx, gy), part) in enumerate(zip(grids, split_rows(got, [gx * gy for gx, gy in grids]))):
                    _, tr = o.forward(pats[i], gx, gy, keep=[(name, 1)])
                    assert max_rel(part, tr[(name, 1)].reshape(part.shape)) <= TOL, (name, i)
    finally:
        c.close()
