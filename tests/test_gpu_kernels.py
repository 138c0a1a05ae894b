"""The forward's row kernels through their per-op C-ABI entries, against the CPU oracle, mirroring
the reference's kernel tests (Tests/GemmaEmbedTests/KernelTests.swift:363-548): RMSNorm with and
without a weight, with a pre-scale and in place; the residual norm and its fused next norm; QK
norm + RoPE at head dims 256 and 512; the embedding gather with token and vector rows; mean
pooling over sequences of 1, 7, 33 and 100 rows."""
import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge
import npref

pytestmark = pytest.mark.gpu

EPS = 1e-6


def max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module")
def ctx():
    c = ge.Context.create(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def c2(config2_gguf):
    return npref.Gguf(config2_gguf)


class Dev:
    """Device copies of host arrays for one test, freed at the end."""

    def __init__(self, ctx):
        self.ctx, self.ptrs = ctx, []

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = self.ctx.alloc(max(a.nbytes, 16))
        self.ctx.upload(p, a)
        self.ptrs.append(p)
        return p

    def zeros(self, nbytes):
        return self.put(np.zeros(nbytes, np.uint8))

    def close(self):
        for p in self.ptrs:
            self.ctx.free(p)


@pytest.fixture
def dev(ctx):
    d = Dev(ctx)
    yield d
    d.close()


def rng_floats(seed, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


@pytest.mark.parametrize("width,weight,pre_scale", [(768, "blk.0.attn_norm.weight", 1.0), (256, "blk.0.attn_q_norm.weight", 1.0),
                                                    (256, "blk.5.attn_k_norm.weight", 1.0), (768, None, 1.0),
                                                    (768, "output_norm.weight", 1 / np.sqrt(768))])
def test_rmsnorm(ctx, dev, c2, width, weight, pre_scale):
    rows = 37
    x = rng_floats(3, rows * width, 5.0).reshape(rows, width)
    w = c2.tensor(weight).astype(np.float32) if weight else None
    want = ora.rmsnorm(x, width, w, EPS, pre_scale)
    dx, do = dev.put(x), dev.zeros(x.nbytes)
    dw = dev.put(w) if w is not None else None
    ctx.rmsnorm(dx, do, dw, rows, width, EPS, pre_scale)
    assert max_rel(ctx.download(do, x.shape, np.float32), want) < 1e-5
    ctx.rmsnorm(dx, dx, dw, rows, width, EPS, pre_scale)  # in place
    assert max_rel(ctx.download(dx, x.shape, np.float32), want) < 1e-5


@pytest.mark.parametrize("scale", [1.0, 0.8])
def test_rmsnorm_residual_and_fused_next_norm(ctx, dev, c2, scale):
    """x = (x + rmsnorm(t) w) scale, and with the next block's weight also h = rmsnorm(x) w_next:
    the fused x update equals the unfused one bit for bit (KernelTests.swift:385-423)."""
    rows, d = 229, 768
    x = rng_floats(19, rows * d, 3.0).reshape(rows, d)
    t16 = rng_floats(20, rows * d, 5.0).reshape(rows, d).astype(np.float16)
    w = c2.tensor("blk.4.post_ffw_norm.weight").astype(np.float32)
    wn = c2.tensor("blk.5.attn_norm.weight").astype(np.float32)
    want_x = (x + ora.rmsnorm(t16.astype(np.float32), d, w, EPS)) * np.float32(scale)
    want_h = ora.rmsnorm(want_x, d, wn, EPS)
    dx, dt, dw, dwn = dev.put(x), dev.put(t16), dev.put(w), dev.put(wn)
    ctx.rmsnorm_residual(dx, dt, dw, scale, None, None, rows, d, EPS)
    plain = ctx.download(dx, x.shape, np.float32)
    assert max_rel(plain, want_x) < 1e-5
    dx2, dh = dev.put(x), dev.zeros(rows * d * 2)
    ctx.rmsnorm_residual(dx2, dt, dw, scale, dwn, dh, rows, d, EPS)
    assert np.array_equal(ctx.download(dx2, x.shape, np.float32), plain)
    h = ctx.download(dh, x.shape, np.float16).astype(np.float32)
    assert max_rel(h, want_h) < 1e-3  # fp16 output


@pytest.mark.parametrize("hd,heads,kv_heads,base", [(256, 3, 1, 1e4), (512, 4, 1, 1e6), (256, 4, 2, 1e4)])
def test_qk_norm_rope_vs_oracle(ctx, dev, hd, heads, kv_heads, base):
    """Weighted RMSNorm + NeoX RoPE on q and k, unweighted norm on v, at positions i * 13 % 2048
    (KernelTests.swift:449-476)."""
    T = 131
    slots = heads + 2 * kv_heads
    qkv = rng_floats(9, T * slots * hd, 4.0).reshape(T, slots, hd)
    qn = (1 + 0.1 * rng_floats(10, hd)).astype(np.float32)
    kn = (1 + 0.1 * rng_floats(11, hd)).astype(np.float32)
    pos = (np.arange(T) * 13 % 2048).astype(np.int32)
    table = ora.rope_table(hd, base, 2048)
    want_q = ora.rope(ora.rmsnorm(qkv[:, :heads].reshape(-1, hd), hd, qn, EPS), heads, hd, table, pos)
    want_k = ora.rope(ora.rmsnorm(qkv[:, heads:heads + kv_heads].reshape(-1, hd), hd, kn, EPS), kv_heads, hd, table, pos)
    want_v = ora.rmsnorm(qkv[:, heads + kv_heads:].reshape(-1, hd), hd, None, EPS)
    dq, dk, dv = dev.zeros(T * heads * hd * 2), dev.zeros(T * kv_heads * hd * 2), dev.zeros(T * kv_heads * hd * 2)
    ctx.qk_norm_rope(dev.put(qkv), T, heads, kv_heads, hd, dev.put(qn), dev.put(kn), EPS, dev.put(pos), base, dq, dk, dv)
    for d, want, n in ((dq, want_q, heads), (dk, want_k, kv_heads), (dv, want_v, kv_heads)):
        got = ctx.download(d, (T, n * hd), np.float16).astype(np.float32)
        assert max_rel(got, np.asarray(want).reshape(T, n * hd)) < 1e-3  # fp16 outputs


def test_qk_norm_rope_rejects_positions_past_the_table(ctx, dev):
    T, hd = 4, 256
    qkv = np.zeros((T, 3 * hd), np.float32)
    ones = np.ones(hd, np.float32)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.qk_norm_rope(dev.put(qkv), T, 1, 1, hd, dev.put(ones), dev.put(ones), EPS,
                         dev.put(np.array([0, 1, 8192, 3], np.int32)), 1e4, dev.zeros(T * hd * 2), dev.zeros(T * hd * 2),
                         dev.zeros(T * hd * 2))
    assert e.value.code == ge.GE_ERR_INVALID


@pytest.fixture(scope="module")
def table(ctx, c2):
    raw = np.asarray(c2.raw("token_embd.weight"))
    t = ctx.q8_create(raw, 262144, 768)
    yield t
    ctx.q8_destroy(t)


def dequant_rows(c2, ids):
    emb = np.asarray(c2.raw("token_embd.weight")).reshape(262144, 24, 34)
    blk = emb[ids]
    return (blk[:, :, :2].copy().view(np.float16).astype(np.float32) * blk[:, :, 2:].view(np.int8).astype(np.float32)).reshape(len(ids), 768)


def test_embedding(ctx, dev, c2, table):
    """Rows of the Q8_0 table times sqrt(d), ids at both ends of the vocabulary (KernelTests.swift:478-495)."""
    ids = np.array([2, 8071, 236787, 3927, 1354, 1109, 7609, 1, 0, 262143], np.int32)
    scale = float(np.sqrt(np.float32(768)))
    dx = dev.zeros(len(ids) * 768 * 4)
    ctx.embed(table, dev.put(ids), len(ids), scale, None, 0, None, EPS, dx, None)
    got = ctx.download(dx, (len(ids), 768), np.float32)
    want = dequant_rows(c2, ids) * np.float32(scale)
    assert max_rel(got, want) < 1e-6


def test_embedding_with_vector_rows_and_norm(ctx, dev, c2, table):
    """Negative ids copy rows of the vectors buffer exactly and unscaled (KernelTests.swift:497-528);
    the fused first norm gives rmsnorm(x) * w in fp16."""
    vectors = rng_floats(11, 4 * 768, 3.0).reshape(4, 768)
    ids = np.array([2, 255999, -1, -2, -3, -4, 258882, 1, -3, 8071], np.int32)
    scale = float(np.sqrt(np.float32(768)))
    w = c2.tensor("blk.0.attn_norm.weight").astype(np.float32)
    dx, dh = dev.zeros(len(ids) * 768 * 4), dev.zeros(len(ids) * 768 * 2)
    ctx.embed(table, dev.put(ids), len(ids), scale, dev.put(vectors), 4, dev.put(w), EPS, dx, dh)
    got = ctx.download(dx, (len(ids), 768), np.float32)
    for t, i in enumerate(ids):
        if i < 0:
            assert np.array_equal(got[t], vectors[-i - 1]), t
        else:
            assert max_rel(got[t], dequant_rows(c2, [i])[0] * np.float32(scale)) < 1e-6, t
    h = ctx.download(dh, (len(ids), 768), np.float16).astype(np.float32)
    assert max_rel(h, ora.rmsnorm(got, 768, w, EPS)) < 1e-3
    with pytest.raises(ge.GemmaEmbedError) as e:  # a fifth vector row
        ctx.embed(table, dev.put(np.array([2, -5], np.int32)), 2, scale, dev.put(vectors), 4, None, EPS, dx, None)
    assert e.value.code == ge.GE_ERR_INVALID
    with pytest.raises(ge.GemmaEmbedError):  # past the table
        ctx.embed(table, dev.put(np.array([262144], np.int32)), 1, scale, None, 0, None, EPS, dx, None)


def test_mean_pool(ctx, dev):
    """Sequences of 1, 7, 33 and 100 rows of width 768 (KernelTests.swift:530-548)."""
    lengths = [1, 7, 33, 100]
    width, total = 768, sum(lengths)
    x = rng_floats(6, total * width).reshape(total, width)
    seqs, start = [], 0
    for n in lengths:
        seqs.append((start, n))
        start += n
    sq = np.asarray(seqs, np.uint32)
    dp = dev.zeros(len(lengths) * width * 4)
    ctx.mean_pool(dev.put(x), total, width, dev.put(sq), len(lengths), dp)
    got = ctx.download(dp, (len(lengths), width), np.float32)
    for s, (st, n) in enumerate(seqs):
        want = x[st:st + n].astype(np.float64).mean(axis=0)
        assert max_rel(got[s], want) < 1e-5, s
    with pytest.raises(ge.GemmaEmbedError) as e:  # a sequence past the rows
        ctx.mean_pool(dev.put(x), total - 1, width, dev.put(sq), len(lengths), dp)
    assert e.value.code == ge.GE_ERR_INVALID
