"""Vector rows and the image forward on the GPU against the CPU oracle, through the C-ABI.

A token id -(r + 1) enters row r of the vectors buffer into the residual stream unscaled
(PackedBatch, Metal/MetalForward.swift:6-32; embed_q8, Shaders/Elementwise.metal:25-29;
CPUReference.swift:190-202). The image forward (MetalForward.run(images:), :213-219) runs the tower
and then the text tower over [bos, <|image>, vectors, <image|>, eos] per image (InputRow.swift:52-56).
Bars as for the text path: max |d| / max |ref| <= 1e-2 and cosine >= 0.99999 on the pooled vectors."""
import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge
import npref

pytestmark = pytest.mark.gpu

TOL = 1e-2
COSINE_BAR = 0.99999
MARKERS = [2, 500, 501, 1]  # bos, <|image>, <image|>, eos in the 512-token synthetic vocabulary


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module")
def c2_model(config2_gguf):
    m = ge.EmbeddingModel.load(config2_gguf)
    yield m
    m.close()


@pytest.mark.parametrize("which", ["tiny", "tiny_ple"])
def test_vector_rows_vs_oracle(which, tiny_gguf, tiny_ple_gguf):
    path = tiny_gguf if which == "tiny" else tiny_ple_gguf
    print(f"vector rows: {which}", flush=True)
    m = ge.EmbeddingModel.load(path)
    try:
        ctx = m.context
        d = ctx.out_dims if which == "tiny" else npref.Gguf(path).meta["gemma-embedding2.embedding_length"]
        vec = (np.random.default_rng(8).standard_normal((9, d)) * 2).astype(np.float32)
        ctx.set_vectors(vec)
        seqs = [[2, 500, -1, -2, -3, 501, 1], [2, 17, 33, 1], [2, 500, -4, -5, -6, -7, -8, -9, 501, 1] + [40] * 60]
        pooled, _ = ctx.forward(seqs)
        with ora.OracleModel(path) as o:
            for i, s in enumerate(seqs):
                want, _ = o.forward(np.array(s, np.int32), vectors=vec)
                assert max_rel(pooled[i], want) <= TOL, i
                assert cosine(pooled[i], want) >= COSINE_BAR, i
            # a trace names the rows: inp_scaled holds the vectors themselves
            got = ctx.trace([seqs[0]], "inp_scaled").reshape(len(seqs[0]), d)
            assert np.array_equal(got[2:5], vec[:3])
    finally:
        m.close()


def test_vector_rows_equal_to_token_rows_give_the_same_bits(c2_model, config2_gguf):
    """A vector row holding a token's scaled embedding row is that token, to the bit, in every
    regime: a short pack (32 tokens, without graph replay), and a long one split into parts
    (4800 tokens of 8 sequences) on several streams."""
    ctx = c2_model.context
    g = npref.Gguf(config2_gguf)
    emb = g.raw("token_embd.weight").reshape(-1, 768 // 32 * 34)
    toks = ge.synth_tokens(61, 2, 262144, 4800)

    def scaled(t):
        blk = emb[t].reshape(-1, 34)
        dq = blk[:, :2].copy().view(np.float16).astype(np.float32) * blk[:, 2:].view(np.int8).astype(np.float32)
        return dq.reshape(-1) * np.float32(np.sqrt(np.float32(768)))

    for n_seq, length in ((1, 32), (8, 600)):
        seqs = [list(toks[i * length:(i + 1) * length]) for i in range(n_seq)]
        pick = [(i, j) for i in range(n_seq) for j in (3, 7, length - 2)]
        ctx.set_vectors(np.stack([scaled(seqs[i][j]) for i, j in pick]))
        mixed = [list(s) for s in seqs]
        for r, (i, j) in enumerate(pick):
            mixed[i][j] = -(r + 1)
        want, _ = ctx.forward(seqs)
        got, _ = ctx.forward(mixed)
        assert np.array_equal(got, want), (n_seq, length)
        again, _ = ctx.forward(seqs)  # a short pack without vectors still replays its graph
        assert np.array_equal(again, want)
    ctx.set_vectors(np.zeros((0, 768), np.float32))


def test_vector_rows_are_checked(c2_model):
    ctx = c2_model.context
    ctx.set_vectors(np.zeros((3, 768), np.float32))
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.forward([[2, -4, 1]])  # a fourth row
    assert e.value.code == ge.GE_ERR_INVALID
    ctx.set_vectors(np.zeros((3, 512), np.float32))  # not the residual stream's width: no rows
    with pytest.raises(ge.GemmaEmbedError):
        ctx.forward([[2, -1, 1]])
    ctx.set_vectors(np.zeros((0, 768), np.float32))
    with pytest.raises(ge.GemmaEmbedError):
        ctx.forward([[2, -1, 1]])


@pytest.fixture(scope="module")
def image_model(tmp_path_factory, tiny_gguf):
    """The tiny 128-wide text model with a tower projecting to 128 (2 x 2 merge, 128-wide heads)."""
    spec = dict(layers=2, hidden=256, heads=2, feed_forward=1024, patch_size=16, merge=2, proj_dims=128,
                positions=16, eps=1e-6, seed=17)
    vpath = ge.synth_write_vision_gguf(str(tmp_path_factory.mktemp("img") / "tower.gguf"), **spec)
    m = ge.EmbeddingModel.load(tiny_gguf)
    m.context.vision_load(vpath)
    yield m, vpath
    m.close()


GRIDS = [(8, 6), (4, 4), (16, 2), (2, 2)]


def test_image_forward_vs_oracle(image_model, tiny_gguf):
    m, vpath = image_model
    ctx = m.context
    with ora.VisionOracle(vpath) as vo, ora.OracleModel(tiny_gguf) as to:
        patches = ge.image_patches(71, GRIDS, vo.area)
        pooled, secs = ctx.image_forward(patches, GRIDS, MARKERS)
        assert secs > 0 and pooled.shape == (len(GRIDS), 128)
        p0 = 0
        for i, (gx, gy) in enumerate(GRIDS):
            vec, _ = vo.forward(patches[p0:p0 + gx * gy], gx, gy)
            p0 += gx * gy
            n = vec.shape[0]
            seq = np.array([MARKERS[0], MARKERS[1]] + [-(r + 1) for r in range(n)] + MARKERS[2:], np.int32)
            want, _ = to.forward(seq, vectors=vec)
            assert max_rel(pooled[i], want) <= TOL, i
            assert cosine(pooled[i], want) >= COSINE_BAR, i


def test_image_forward_matches_host_vector_rows(image_model):
    """The tower's rows read in HBM give the bits of the same rows uploaded from the host."""
    m, _ = image_model
    ctx = m.context
    patches = ge.image_patches(72, GRIDS, 3 * 16 * 16)
    pooled, _ = ctx.image_forward(patches, GRIDS, MARKERS)
    vec, _ = ctx.vision_encode(patches, GRIDS, 128, merge=2)
    ctx.set_vectors(vec)
    seqs, r = [], 0
    for gx, gy in GRIDS:
        n = (gx // 2) * (gy // 2)
        seqs.append([MARKERS[0], MARKERS[1]] + [-(r + k + 1) for k in range(n)] + MARKERS[2:])
        r += n
    host, _ = ctx.forward(seqs)
    assert np.array_equal(host, pooled)
    again, _ = ctx.image_forward(patches, GRIDS, MARKERS)
    assert np.array_equal(again, pooled)
    alone, _ = ctx.image_forward(patches[:48], GRIDS[:1], MARKERS)  # independent of the other images
    assert np.array_equal(alone[0], pooled[0])
    ctx.set_vectors(np.zeros((0, 128), np.float32))


def test_image_forward_needs_matching_widths(c2_model, tmp_path):
    ctx = c2_model.context
    spec = dict(layers=1, hidden=256, heads=2, feed_forward=512, patch_size=16, merge=2, proj_dims=128,
                positions=8, eps=1e-6, seed=3)
    ctx.vision_load(ge.synth_write_vision_gguf(str(tmp_path / "narrow.gguf"), **spec))
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.image_forward(np.zeros((4, 768), np.float32), [(2, 2)], MARKERS)
    assert e.value.code == ge.GE_ERR_INVALID


def test_image_forward_rejects_bad_markers_and_patch_rows(image_model):
    """Markers are vocabulary ids (InputRow.swift SpanMarkers): a negative one would name a vector
    row. Patch rows must be the tower's 3 p^2 floats wide."""
    m, _ = image_model
    ctx = m.context
    patches = ge.image_patches(73, GRIDS[:1], 3 * 16 * 16)
    for bad in ([-1, 500, 501, 1], [2, 500, 501, 512]):
        with pytest.raises(ge.GemmaEmbedError) as e:
            ctx.image_forward(patches, GRIDS[:1], bad)
        assert e.value.code == ge.GE_ERR_INVALID
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.image_forward(patches[:, :700], GRIDS[:1], MARKERS)
    assert e.value.code == ge.GE_ERR_INVALID
    # a call that fails once staging has begun (a grid that is not a multiple of the merge size)
    # leaves no batch staged: nothing stale can run
    ctx.batch_stage([[2, 3, 1]])
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.image_forward(ge.image_patches(75, [(3, 3)], 768), [(3, 3)], MARKERS)
    assert e.value.code == ge.GE_ERR_INVALID
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.batch_run()
    assert e.value.code == ge.GE_ERR_STATE
    ok, _ = ctx.image_forward(patches, GRIDS[:1], MARKERS)
    assert np.all(np.isfinite(ok))


def test_vision_outputs_are_sized_by_capacity(image_model):
    """ge_vision_encode / ge_vision_read take the capacity of the caller's buffer and refuse a
    smaller one instead of writing past it."""
    import ctypes as C
    m, _ = image_model
    ctx = m.context
    info = ctx.vision_info()
    assert (info.patch_area, info.merge, info.proj_dims) == (768, 2, 128)
    patches = np.ascontiguousarray(ge.image_patches(74, GRIDS[:1], info.patch_area), np.float32)
    tokens = (GRIDS[0][0] // 2) * (GRIDS[0][1] // 2)
    out = np.zeros(tokens * 128, np.float32)
    grid = (ge.ge_image_grid * 1)(ge.ge_image_grid(*GRIDS[0]))
    rc = ge.lib.ge_vision_encode(ctx.handle, patches.ctypes.data_as(C.POINTER(C.c_float)), patches.shape[0], grid, 1,
                                 out.ctypes.data_as(C.POINTER(C.c_float)), out.size - 1, None)
    assert rc == ge.GE_ERR_INVALID
    rc = ge.lib.ge_vision_encode(ctx.handle, patches.ctypes.data_as(C.POINTER(C.c_float)), patches.shape[0], grid, 1,
                                 out.ctypes.data_as(C.POINTER(C.c_float)), out.size, None)
    assert rc == ge.GE_OK
    assert ge.lib.ge_vision_read(ctx.handle, out.ctypes.data_as(C.POINTER(C.c_float)), out.size - 128) == ge.GE_ERR_INVALID
    with pytest.raises(ge.GemmaEmbedError):
        ctx.vision_encode(patches, GRIDS[:1], 768)  # not the tower's projection width


def test_replaced_vector_rows_drop_a_staged_batch_that_reads_past_them(c2_model):
    """A staged batch names vector rows; replacing the rows with fewer (or of another width) drops
    it rather than letting it read stale rows."""
    ctx = c2_model.context
    ctx.set_vectors(np.ones((6, 768), np.float32))
    ctx.batch_stage([[2, -6, 1]])
    ctx.set_vectors(np.ones((6, 768), np.float32))  # still covers row 5: the batch stays
    ctx.batch_run()
    ctx.batch_read()
    ctx.set_vectors(np.ones((3, 768), np.float32))  # row 5 is gone
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.batch_run()
    assert e.value.code == ge.GE_ERR_STATE
    ctx.set_vectors(np.ones((6, 768), np.float32))
    ctx.batch_stage([[2, -2, 1]])
    ctx.set_vectors(np.ones((6, 512), np.float32))  # another width
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.batch_run()
    assert e.value.code == ge.GE_ERR_STATE
    ctx.set_vectors(np.zeros((0, 768), np.float32))
