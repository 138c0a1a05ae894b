"""Pins the C oracle (oracle/ge_oracle.c) before it is trusted as the GPU path's checker.

The reference's own golden vectors (Tests/GemmaEmbedTests/Fixtures/*.jsonl) need the real
embeddinggemma-2 GGUF, which is not available, so each oracle function is pinned here by what
the mathematics fixes: exact enumerations, known-answer blocks, closed forms, invariants, and
an independent float64 numpy forward (tests/npref.py) on the tiny and the config-2 model.
"""
import math

import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge
import npref

RNG = np.random.default_rng(1234)


# ------------------------------------------------------------------ fp16 (Weights.swift:27,37)

def test_half_to_float_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([ora.half_to_float(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_float_to_half_rounds_to_nearest_even():
    xs = np.concatenate([
        RNG.standard_normal(20000).astype(np.float32) * 10.0 ** RNG.integers(-9, 6, 20000),
        np.float32([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                    6.1e-5, 1 + 2 ** -11, 1 + 3 * 2 ** -11]),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([ora.float_to_half(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ Q8_0 dequant (Weights.swift:33-41)

def _block(scale_bits: int, q) -> bytes:
    return struct_pack_block(scale_bits, q)


def struct_pack_block(scale_bits, q):
    return bytes([scale_bits & 0xFF, scale_bits >> 8]) + np.asarray(q, dtype=np.int8).tobytes()


@pytest.mark.parametrize("scale_bits,scale", [(0x3C00, 1.0), (0x3800, 0.5), (0xBC00, -1.0), (0x0001, 2.0 ** -24),
                                              (0x2E66, 0.0999755859375)])
def test_q8_known_answer_blocks(scale_bits, scale):
    q = np.arange(-127, -127 + 32, dtype=np.int8)
    q2 = np.array([127, -127, 0, 1, -1] + [3] * 27, dtype=np.int8)
    row = _block(scale_bits, q) + _block(scale_bits, q2)
    got = ora.dequant_row(8, row, 64)
    want = np.concatenate([q, q2]).astype(np.float64) * scale
    assert np.array_equal(got.astype(np.float64), want)


def test_f16_bf16_f32_rows():
    v = RNG.standard_normal(96).astype(np.float32)
    assert np.array_equal(ora.dequant_row(0, v.tobytes(), 96), v)
    h = v.astype(np.float16)
    assert np.array_equal(ora.dequant_row(1, h.tobytes(), 96), h.astype(np.float32))
    b = (v.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(ora.dequant_row(30, b.tobytes(), 96), (b.astype(np.uint32) << 16).view(np.float32))


# ------------------------------------------------------------------ matmul (CPUReference.swift:63-74)

@pytest.mark.parametrize("m,k,n", [(1, 8, 1), (5, 37, 3), (64, 768, 96), (33, 1152, 17), (7, 13, 9)])
def test_matmul_vs_float64(m, k, n):
    x = RNG.standard_normal((m, k)).astype(np.float32)
    w = RNG.standard_normal((n, k)).astype(np.float32)
    got = ora.matmul(x, w)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    # fp32 accumulation: error ~ sqrt(k) * eps * |x||w|
    tol = 4 * np.sqrt(k) * 6e-8 * np.abs(x).max() * np.abs(w).max() * np.sqrt(k)
    assert np.abs(got - want).max() <= tol
    # a transposed operand would give a different matrix entirely
    if n == m and n > 1:
        assert np.abs(got - want.T).max() > 10 * tol


def test_matmul_thread_count_invariant():
    x = RNG.standard_normal((70, 200)).astype(np.float32)
    w = RNG.standard_normal((50, 200)).astype(np.float32)
    assert np.array_equal(ora.matmul(x, w, threads=1), ora.matmul(x, w, threads=7))


# ------------------------------------------------------------------ rmsnorm (CPUReference.swift:77-90)

def test_rmsnorm_unit_rms_and_float64():
    x = RNG.standard_normal((9, 768)).astype(np.float32) * 30
    y = ora.rmsnorm(x, 768, None, 1e-6).reshape(9, 768)
    assert np.allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1)), 1.0, atol=1e-6)
    w = (1 + 0.1 * RNG.standard_normal(768)).astype(np.float32)
    got = ora.rmsnorm(x, 768, w, 1e-6).reshape(9, 768)
    want = npref.rmsnorm(x.astype(np.float64), w.astype(np.float64), 1e-6)
    assert np.abs(got - want).max() < 1e-5 * np.abs(want).max()


def test_rmsnorm_scale_invariance_and_eps():
    x = RNG.standard_normal((4, 256)).astype(np.float32)
    a = ora.rmsnorm(x, 256, None, 1e-6)
    b = ora.rmsnorm(x * 1024, 256, None, 1e-6)
    assert np.abs(a - b).max() < 1e-5
    # eps is added to the mean square, not to the RMS: a zero row stays zero, a tiny row is damped
    z = np.zeros((1, 64), np.float32)
    assert np.all(ora.rmsnorm(z, 64, None, 1e-6) == 0)
    t = np.full((1, 64), 1e-3, np.float32)
    assert abs(ora.rmsnorm(t, 64, None, 1e-6).reshape(-1)[0] - 1e-3 / math.sqrt(1e-6 + 1e-6)) < 1e-5


def test_rmsnorm_prescale():
    x = RNG.standard_normal((3, 128)).astype(np.float32)
    w = RNG.standard_normal(128).astype(np.float32)
    got = ora.rmsnorm(x, 128, w, 1e-6, prescale=0.25)
    want = npref.rmsnorm(0.25 * x.astype(np.float64), w.astype(np.float64), 1e-6)
    assert np.abs(got.reshape(3, 128) - want).max() < 1e-5 * np.abs(want).max()


# ------------------------------------------------------------------ gelu_tanh (CPUReference.swift:92-95)

def test_gelu_tanh_identity_and_erf_bound():
    from scipy.special import erf
    xs = np.linspace(-12, 12, 4001)
    g = np.array([ora.gelu_tanh(float(x)) for x in xs])
    gm = np.array([ora.gelu_tanh(float(-x)) for x in xs])
    # gelu(x) - gelu(-x) = x holds for 0.5 x (1 + tanh(u(x))) with u odd
    assert np.abs(g - gm - xs).max() < 1e-5
    exact = 0.5 * xs * (1 + erf(xs / math.sqrt(2)))
    # the tanh form is within 1e-3 of the erf form everywhere; dropping the cubic term is not
    assert np.abs(g - exact).max() < 1e-3
    assert np.abs(0.5 * xs * (1 + np.tanh(math.sqrt(2 / math.pi) * xs)) - exact).max() > 1e-2
    assert ora.gelu_tanh(0.0) == 0.0


# ------------------------------------------------------------------ RoPE (RopeTable.swift, CPUReference.swift:98-113)

def test_rope_table_closed_form():
    t = ora.rope_table(256, 1e4, 8192)
    assert np.all(t[0, :, 0] == 1) and np.all(t[0, :, 1] == 0)
    pos = np.arange(8192, dtype=np.float64)
    # pair 0 turns by exactly one radian per position
    assert np.abs(t[:, 0, 0] - np.cos(pos)).max() < 1e-7
    i = np.arange(128)
    ang = pos[:, None] * 1e4 ** (-2.0 * i / 256)[None, :]
    assert np.abs(t[..., 0] - np.cos(ang)).max() < 1e-7
    assert np.abs(t[..., 1] - np.sin(ang)).max() < 1e-7


def test_rope_matches_complex_rotation():
    T, H, hd = 40, 3, 256
    x = RNG.standard_normal((T, H, hd)).astype(np.float32)
    pos = RNG.integers(0, 8192, T).astype(np.int32)
    pos[0] = 0
    table = ora.rope_table(hd, 1e6, 8192)
    got = ora.rope(x, H, hd, table, pos).reshape(T, H, hd)
    want = npref.rope(x.astype(np.float64), 1e6, pos)
    assert np.abs(got - want).max() < 1e-4
    assert np.array_equal(got[0], x[0])  # position 0 is the identity
    half = hd // 2
    n_in = x[..., :half] ** 2 + x[..., half:] ** 2
    n_out = got[..., :half] ** 2 + got[..., half:] ** 2
    assert np.abs(n_in - n_out).max() < 1e-4 * n_in.max()


# ------------------------------------------------------------------ attention (CPUReference.swift:117-174)

@pytest.mark.parametrize("T,H,KV,hd,window", [(17, 3, 1, 32, 0), (40, 4, 2, 16, 16), (33, 2, 2, 8, 7), (5, 4, 1, 8, 0)])
def test_attention_vs_float64(T, H, KV, hd, window):
    q = RNG.standard_normal((T, H, hd)).astype(np.float32) * 2
    k = RNG.standard_normal((T, KV, hd)).astype(np.float32)
    v = RNG.standard_normal((T, KV, hd)).astype(np.float32)
    got = ora.attention(q, k, v, T, H, KV, hd, 1.0, window)
    want = npref.attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), window)
    assert np.abs(got - want).max() < 2e-5 * max(1.0, np.abs(want).max())


def test_attention_invariants():
    T, H, KV, hd = 30, 4, 2, 16
    q = RNG.standard_normal((T, H, hd)).astype(np.float32)
    k = RNG.standard_normal((T, KV, hd)).astype(np.float32)
    v = np.broadcast_to(RNG.standard_normal((1, KV, hd)).astype(np.float32), (T, KV, hd)).copy()
    out = ora.attention(q, k, v, T, H, KV, hd, 1.0, 0)
    # equal value rows: every output row is that row (softmax weights sum to 1)
    for h in range(H):
        assert np.abs(out[:, h] - v[0, h // (H // KV)]).max() < 1e-5
    # window: keys farther than window // 2 cannot move a query's output
    v = RNG.standard_normal((T, KV, hd)).astype(np.float32)
    a = ora.attention(q, k, v, T, H, KV, hd, 1.0, 8)
    k2, v2 = k.copy(), v.copy()
    k2[20:] += 5
    v2[20:] -= 3
    b = ora.attention(q, k2, v2, T, H, KV, hd, 1.0, 8)
    assert np.array_equal(a[:16], b[:16])  # |i - j| > 4 for i < 16, j >= 20
    assert not np.array_equal(a[16:], b[16:])


# ------------------------------------------------------------------ whole forward (CPUReference.swift:183-283)

def test_forward_tiny_vs_float64(tiny_gguf):
    g = npref.Gguf(tiny_gguf)
    keep = [(n, l) for n in ("l_out", "kqv_out", "Qcur_pos", "ffn_geglu") for l in range(2)] + [("result_embd", -1)]
    with ora.OracleModel(tiny_gguf) as m:
        for seed, T in ((1, 40), (2, 7), (3, 1), (4, 64)):
            import gemma_embed as ge
            toks = ge.synth_tokens(seed, 2, m.vocab, T)
            pooled, tr = m.forward(toks, keep=keep)
            want, wtr = npref.forward(g, toks, keep=tuple(keep))
            assert np.abs(pooled - want).max() < 2e-4 * np.abs(want).max(), seed
            for key in keep:
                a, b = tr[key], wtr[key]
                assert np.abs(a - b).max() < 2e-4 * np.abs(b).max(), (seed, key)


@pytest.mark.timeout(300)
def test_forward_config2_vs_float64(config2_gguf):
    """The 24-layer config-2 model (window active at T > 257) against float64."""
    import gemma_embed as ge
    g = npref.Gguf(config2_gguf)
    keep = [("l_out", l) for l in range(24)]
    toks = ge.synth_tokens(11, 2, 262144, 300)
    with ora.OracleModel(config2_gguf) as m:
        pooled, tr = m.forward(toks, keep=keep)
    want, wtr = npref.forward(g, toks, keep=tuple(keep))
    for key in keep:
        a, b = tr[key], wtr[key]
        assert np.abs(a - b).max() < 1e-3 * np.abs(b).max(), key
    cos = float(np.dot(pooled, want) / np.linalg.norm(pooled) / np.linalg.norm(want))
    assert cos > 0.9999999


def test_forward_per_layer_inputs_vs_float64(tiny_ple_gguf):
    """The per-layer-input branch (CPUReference.swift:206-210, :259-269) against float64."""
    import gemma_embed as ge
    g = npref.Gguf(tiny_ple_gguf)
    keep = [(n, l) for n in ("pe_in", "l_out", "per_layer_embd_out") for l in range(2)] + \
           [("inp_per_layer", -1), ("result_embd", -1)]
    with ora.OracleModel(tiny_ple_gguf) as m:
        for seed, T in ((21, 40), (22, 3), (23, 64)):
            toks = ge.synth_tokens(seed, 2, m.vocab, T)
            pooled, tr = m.forward(toks, keep=keep)
            want, wtr = npref.forward(g, toks, keep=tuple(keep))
            assert np.abs(pooled - want).max() < 2e-4 * np.abs(want).max(), seed
            for key in keep:
                a, b = tr[key], wtr[key]
                assert a.shape == b.shape, key
                assert np.abs(a - b).max() < 2e-4 * np.abs(b).max(), (seed, key)
            # the branch changes the result: without it the layer outputs differ
            assert not np.allclose(tr[("pe_in", 1)], tr[("l_out", 1)])


def test_forward_vector_rows(tiny_gguf, tiny_ple_gguf):
    """Vector rows (CPUReference.swift:190-202): an id -(r + 1) enters row r of the vectors unscaled.
    A vector row equal to a token's scaled embedding row gives that token's bits exactly (a scaled
    vector or a shifted row index does not), and random vector rows agree with float64."""
    import gemma_embed as ge
    for path in (tiny_gguf, tiny_ple_gguf):
        g = npref.Gguf(path)
        with ora.OracleModel(path) as m:
            d = m.hidden
            toks = ge.synth_tokens(31, 2, m.vocab, 12)
            emb = g.tensor("token_embd.weight").astype(np.float32) * np.sqrt(np.float32(d))
            vec = np.stack([emb[toks[5]], emb[toks[3]], emb[toks[9]]]).astype(np.float32)
            mixed = toks.copy()
            mixed[3], mixed[5], mixed[9] = -2, -1, -3
            a, ta = m.forward(toks, keep=[("l_out", 1)])
            b, tb = m.forward(mixed, keep=[("l_out", 1)], vectors=vec)
            assert np.array_equal(a, b) and np.array_equal(ta[("l_out", 1)], tb[("l_out", 1)])
            rnd = np.random.default_rng(5).standard_normal((4, d)).astype(np.float32) * 3
            seq = np.array([2, 7, -1, -2, -3, -4, 9, 1], np.int32)
            pooled, tr = m.forward(seq, keep=[("inp_scaled", -1), ("l_out", 1)], vectors=rnd)
            want, wtr = npref.forward(g, seq, keep=(("inp_scaled", -1), ("l_out", 1)), vectors=rnd)
            assert np.array_equal(tr[("inp_scaled", -1)].reshape(8, d)[2:6], rnd)
            assert np.abs(pooled - want).max() < 2e-4 * np.abs(want).max()
            assert np.abs(tr[("l_out", 1)] - wtr[("l_out", 1)]).max() < 2e-4 * np.abs(wtr[("l_out", 1)]).max()
            with pytest.raises(ValueError):
                m.forward(seq, vectors=rnd[:3])  # -4 names a fourth row
            with pytest.raises(ValueError):
                m.forward(seq)


def test_forward_rejects_bad_tokens(tiny_gguf):
    with ora.OracleModel(tiny_gguf) as m:
        with pytest.raises(ValueError):
            m.forward([1, 2, m.vocab])
        with pytest.raises(ValueError):
            m.forward([])


def test_open_rejects_non_gguf(tmp_path):
    p = tmp_path / "junk.gguf"
    p.write_bytes(b"\x41" * 4096)  # GGUFReaderTests.swift:68-75
    with pytest.raises(ValueError, match="invalid GGUF"):
        ora.OracleModel(str(p))


def test_fp16_emulation_is_the_float64_forward_without_rounding(tmp_path):
    """tests/fp16_emulation.py with rounding off is tests/npref.py's float64 forward (so its rounded
    run differs from the reference's arithmetic only by the fp16 roundings it injects), and its
    rounding is fp16's round-to-nearest-even on values in the normal range."""
    import fp16_emulation as emu
    path = ge.synth_write_gguf(str(tmp_path / "tiny.gguf"), **ge.TINY)
    g = npref.Gguf(path)
    toks = [int(t) for t in ge.synth_tokens(5, 2, 512, 37)]
    keep = [("l_out", 0), ("l_out", 1), ("kqv_out", 1), ("ffn_geglu", 0)]
    pooled, tr = emu.forward(g, toks, False, keep)
    want_pooled, want = npref.forward(g, np.asarray(toks), keep=tuple(keep))
    assert np.allclose(pooled, want_pooled, rtol=1e-12, atol=1e-12)
    for k in keep:
        assert np.allclose(tr[k].reshape(-1), want[k], rtol=1e-10, atol=1e-12), k
    x = np.random.default_rng(3).standard_normal(10000) * 100
    x[0] = 2.0 ** 14 * 1.5  # the largest entry maps to 2^14 exactly: no rescaling error
    assert np.array_equal(emu.f16(x), x.astype(np.float16).astype(np.float64))
    _, rounded = emu.forward(g, toks, True, keep)
    assert 0 < np.abs(rounded[("l_out", 1)] - tr[("l_out", 1)]).max() / np.abs(tr[("l_out", 1)]).max() < 1e-2
