"""Whole-forward parity on the GPU against the CPU oracle, through the C-ABI.

Bars: per-layer max relative error max|d| / max|ref| <= 1e-2 on
every layer's output, final pooled-embedding cosine >= 0.99999. Also the reference's bitwise
invariants (packing independence, determinism; MetalForwardTests.swift:54-120) and the
embed API's options, truncation, batching and progress (EmbeddingModelTests.swift)."""
import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge

pytestmark = pytest.mark.gpu

PER_LAYER_TOL = 1e-2
COSINE_BAR = 0.99999


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module")
def tiny_model(tiny_gguf):
    m = ge.EmbeddingModel.load(tiny_gguf)
    print("device:", m.info.device_name.decode(), flush=True)
    yield m
    m.close()


@pytest.fixture(scope="module")
def c2_model(config2_gguf):
    m = ge.EmbeddingModel.load(config2_gguf, batch_token_budget=8192)
    yield m
    m.close()


@pytest.fixture(scope="module")
def c2_oracle(config2_gguf):
    m = ora.OracleModel(config2_gguf)
    yield m
    m.close()


def test_tiny_forward_vs_oracle(tiny_model, tiny_gguf):
    seqs = [ge.synth_tokens(s, 2, 512, n).tolist() for s, n in ((1, 40), (2, 7), (3, 1), (4, 64), (5, 33))]
    pooled = tiny_model.embed_tokens(seqs)
    with ora.OracleModel(tiny_gguf) as o:
        for i, s in enumerate(seqs):
            want, tr = o.forward(s, keep=[("l_out", 0), ("l_out", 1)])
            assert cosine(pooled[i], want) >= COSINE_BAR, i
    for layer in range(2):
        got = tiny_model.context.trace(seqs, "l_out", layer)
        off = 0
        with ora.OracleModel(tiny_gguf) as o:
            for s in seqs:
                _, tr = o.forward(s, keep=[("l_out", layer)])
                assert max_rel(got[off:off + len(s)], tr[("l_out", layer)].reshape(len(s), -1)) <= PER_LAYER_TOL
                off += len(s)


@pytest.fixture(scope="module")
def config2_batch():
    # 32 texts x 512 tokens, ids uniform in [2, 262144)
    toks = ge.synth_tokens(3, 2, 262144, 32 * 512).reshape(32, 512)
    return [t.tolist() for t in toks]


def normalised(v):
    v = np.asarray(v, np.float64)
    return v / np.linalg.norm(v)


@pytest.mark.timeout(600)
def test_config2_pooled_vs_oracle(c2_model, c2_oracle, config2_batch):
    """All 32 texts of BASELINE config 2 in one pack against the oracle: cosine and the largest
    difference of the normalised vectors (the reference's own GPU-vs-CPU bar is 1e-4,
    MetalForwardTests.swift:213-214)."""
    print("config2 forward 32 x 512 (one pack of 16384)", flush=True)
    pooled, secs = c2_model.context.forward(config2_batch)
    print(f"gpu forward {secs * 1e3:.2f} ms", flush=True)
    assert pooled.shape == (32, 768)
    worst_cos, worst_abs = 1.0, 0.0
    for i in range(32):
        want, _ = c2_oracle.forward(config2_batch[i])
        c = cosine(pooled[i], want)
        d = float(np.abs(normalised(pooled[i]) - normalised(want)).max())
        worst_cos, worst_abs = min(worst_cos, c), max(worst_abs, d)
        print(f"seq {i} cosine {c:.9f} max_abs(normalised) {d:.2e}", flush=True)
        assert c >= COSINE_BAR, i
    print(f"config2: min cosine {worst_cos:.9f}, max abs difference of normalised vectors {worst_abs:.2e}", flush=True)
    assert worst_abs < 1e-4


def test_1500_token_text_vs_oracle(c2_model, c2_oracle, config2_batch):
    """The reference's GPU-vs-oracle check at its size (MetalForwardTests.swift:198-215): one
    1500-token text, cosine > 0.99999 and max |d| < 1e-4 of the normalised vectors, here on the
    config-2 model at default precision (sliding layers clip to their 512-token window)."""
    text = (config2_batch[5] + config2_batch[6] + config2_batch[7])[:1500]
    got = c2_model.embed_tokens([text])[0]
    want, _ = c2_oracle.forward(text)
    d = float(np.abs(normalised(got) - normalised(want)).max())
    print(f"1500 tokens: cosine {cosine(got, want):.9f}, max |d| {d:.3g}", flush=True)
    assert cosine(got, want) > 0.99999 and d < 1e-4


def test_config2_per_layer_vs_oracle(c2_model, c2_oracle, config2_batch):
    names = [("l_out", l) for l in range(24)] + [("Qcur_pos", 0), ("Kcur_pos", 5), ("Vcur_normed", 5),
                                                  ("kqv_out", 0), ("kqv_out", 5), ("ffn_geglu", 3),
                                                  ("attn_out", 11), ("result_embd", -1)]
    batch = config2_batch[:4]
    idx = 2  # check the third sequence of the pack: its rows start at 1024
    _, tr = c2_oracle.forward(batch[idx], keep=names)
    worst = 0.0
    for name, layer in names:
        got = c2_model.context.trace(batch, name, layer)
        rows = got[idx * 512:(idx + 1) * 512]
        want = tr[(name, layer)].reshape(512, -1)
        r = max_rel(rows, want)
        worst = max(worst, r) if name == "l_out" else worst
        print(f"{name}-{layer}: max_rel {r:.3e}", flush=True)
        assert r <= PER_LAYER_TOL, (name, layer)
    print(f"worst l_out max_rel {worst:.3e}", flush=True)


@pytest.mark.parametrize("lengths", [(400, 37, 100), (100, 37, 64), (20, 25, 10)], ids=["tiled", "mid", "short"])
def test_every_trace_tensor_vs_oracle(c2_model, c2_oracle, config2_batch, lengths):
    """Every named intermediate the C-ABI traces (llama.cpp names), at a sliding (0) and a global (5)
    layer, against the oracle on the middle text of a pack: the embedding, the norms, the raw and
    the normed/rotated projections, attention, the GeGLU product, the FFN output, the layer output
    and the final norm and projection. A pack of at most 512 tokens runs its GEMMs on the skinny
    kernel (the mid pack: 201 rows, a partial last row block), one of at most 64 also replays as a
    graph (short)."""
    batch = [config2_batch[2 + 4 * i][:n] for i, n in enumerate(lengths)]
    idx, lo = 1, lengths[0]
    per_layer = ["attn_norm", "Qcur", "Kcur", "Vcur", "Qcur_pos", "Kcur_pos", "Vcur_normed", "kqv_out",
                 "attn_out", "ffn_norm", "ffn_geglu", "ffn_out", "pe_in", "l_out"]
    names = [("inp_scaled", -1), ("result_norm", -1), ("result_embd", -1)] + \
        [(n, l) for l in (0, 5) for n in per_layer]
    _, tr = c2_oracle.forward(batch[idx], keep=names)
    n = len(batch[idx])
    for name, layer in names:
        got = c2_model.context.trace(batch, name, layer)[lo:lo + n]
        want = tr[(name, layer)].reshape(n, -1)
        r = max_rel(got, want)
        print(f"{name}-{layer}: max_rel {r:.3e}", flush=True)
        assert r <= PER_LAYER_TOL, (name, layer)


def test_split_batch_matches_single_stream(c2_model, config2_batch):
    """A pack of >= 4096 tokens runs as two halves of whole sequences on two streams; with
    profiling on, the same pack runs on one stream. Same kernels on the same rows: the vectors
    must be identical."""
    ctx = c2_model.context
    print("config2 pack of 16384: two streams vs one", flush=True)
    split, _ = ctx.forward(config2_batch)
    ctx.profile_enable("")
    try:
        single, _ = ctx.forward(config2_batch)
    finally:
        ctx.profile_disable()
    assert np.array_equal(split, single)
    # an odd number of uneven sequences: the cut lands at a sequence start near the middle
    uneven = [t[: 100 + 61 * i] for i, t in enumerate(config2_batch[:13])]
    split, _ = ctx.forward(uneven)
    ctx.profile_enable("")
    try:
        single, _ = ctx.forward(uneven)
    finally:
        ctx.profile_disable()
    assert np.array_equal(split, single)


@pytest.mark.timeout(300)
def test_split_forward_repeats_bitwise(c2_model, config2_batch):
    """The pack split into parts on several streams, whose layers run unsynchronised on shared
    buffer slices, run 50 times (and three times queued back to back): every run equals the
    single-stream result bit for bit (the reference's concurrent-vs-serial check,
    MetalImageForwardTests.swift:189-224)."""
    ctx = c2_model.context
    ctx.profile_enable("")
    try:
        single, _ = ctx.forward(config2_batch)
    finally:
        ctx.profile_disable()
    ctx.batch_stage(config2_batch)
    for i in range(50):
        ctx.batch_run()
        got = ctx.batch_read()
        assert np.array_equal(got, single), f"run {i} differs from the single-stream forward"
    for _ in range(3):
        ctx.batch_run()
    assert np.array_equal(ctx.batch_read(), single)
    print("50 split forwards equal the single-stream forward", flush=True)


@pytest.fixture(scope="module")
def outlier_gguf(model_dir):
    import os
    return ge.synth_write_gguf(os.path.join(model_dir, "outlier_norms.gguf"), **ge.OUTLIER_NORMS)


@pytest.mark.timeout(300)
def test_outlier_norm_weights_vs_oracle(outlier_gguf):
    """Residual-stream norm weights with entries of 50 to 300 (ge.OUTLIER_NORMS), against the oracle:
    pooled vectors at cosine >= 0.99999, and every traced intermediate within 1e-2 or, where the
    fp16-operand arithmetic itself moves it further, within twice what a float64 emulation of the
    kernels' fp16 rounding points gives (tests/fp16_emulation.py; recorded per text, layer and
    tensor in tests/golden/outlier_fp16_emulation.json). The FFN intermediates stay near 1e-3, so
    the fp16 range scales chosen at load hold with such weights. The attention outputs of the
    global layer do not: its queries' best keys nearly tie (a 0.1% quantile gap of 0.005 between
    the two largest scores), and the 2^-11 roundings of the dequantised weights alone, through the
    five layers before it, move them by up to 13% (emulated: 0.204 with every rounding)."""
    import json
    import os
    import npref
    g = npref.Gguf(outlier_gguf)
    assert np.abs(g.tensor("blk.0.ffn_norm.weight")).max() >= 50  # the outliers are there
    emulated = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                           "outlier_fp16_emulation.json")))
    assert emulated["spec"]["seed"] == ge.OUTLIER_NORMS["seed"]
    m = ge.EmbeddingModel.load(outlier_gguf)
    try:
        seqs = [ge.synth_tokens(t["seed"], 2, 262144, t["length"]).tolist() for t in emulated["texts"]]
        lengths = [len(x) for x in seqs]
        pooled = m.embed_tokens(seqs)
        names = [(n, l) for l in range(6) for n in ("l_out", "kqv_out", "ffn_geglu", "ffn_out")]
        with ora.OracleModel(outlier_gguf) as o:
            want = [o.forward(sq, keep=names) for sq in seqs]
        for i in range(len(seqs)):
            c = cosine(pooled[i], want[i][0])
            print(f"outlier norms: text {i} ({lengths[i]} tokens) cosine {c:.8f}", flush=True)
            assert c >= COSINE_BAR, i
        for name, layer in names:
            got = m.context.trace(seqs, name, layer)
            off = 0
            for i, n in enumerate(lengths):
                err = max_rel(got[off:off + n], want[i][1][(name, layer)].reshape(n, -1))
                off += n
                emu = emulated["texts"][i]["max_rel"][f"{name}/{layer}"]
                print(f"outlier norms: {name} layer {layer} text {i}: max_rel {err:.2e} (fp16 emulation {emu:.2e})",
                      flush=True)
                assert err <= max(PER_LAYER_TOL, 2 * emu), (name, layer, i)
    finally:
        m.close()


def test_attention_item_size_does_not_change_results(c2_model, config2_batch):
    """A pack of 16384 tokens (256 work items of 64 queries) and one of 8192 tokens (fewer than one
    64-query item per CU: 32-query items) give the same texts the same bits."""
    ctx = c2_model.context
    full, _ = ctx.forward(config2_batch)
    half, _ = ctx.forward(config2_batch[:16])
    assert np.array_equal(full[:16], half)
    quarter, _ = ctx.forward(config2_batch[20:24])
    assert np.array_equal(full[20:24], quarter)


def test_pooled_vector_is_the_mean_of_the_token_projections(c2_model, config2_batch):
    """The forward pools the final norm's fp32 rows and projects each sequence's mean once; the
    reference projects every token and averages (CPUReference.swift:274-282). Both are linear, so
    the pooled vector equals the mean of the traced per-token projections (result_embd) up to fp32
    rounding, for texts alone and in a pack, on the skinny (short) and the tiled path."""
    ctx = c2_model.context
    for texts in ([config2_batch[3][:9], config2_batch[7][:50], config2_batch[2][:20]], config2_batch[:2]):
        pooled, _ = ctx.forward(texts)
        per_token = ctx.trace(texts, "result_embd", -1)
        off = 0
        for i, t in enumerate(texts):
            mean = per_token[off:off + len(t)].astype(np.float64).mean(axis=0)
            off += len(t)
            err = np.abs(pooled[i] - mean).max() / np.abs(mean).max()
            print(f"text {i} ({len(t)} tokens): pooled vs mean of projections {err:.2e}", flush=True)
            assert err < 1e-5, i


def test_packing_invariance_and_determinism(c2_model, config2_batch):
    batch = config2_batch[:8]
    a = c2_model.embed_tokens(batch)
    b = c2_model.embed_tokens(batch)
    assert np.array_equal(a, b)  # run to run
    alone = c2_model.embed_tokens([batch[5]])
    assert np.array_equal(alone[0], a[5])  # a text alone vs inside a batch (MetalForwardTests.swift:54-73)
    mixed = c2_model.embed_tokens([batch[5][:100], batch[1], batch[5]])
    assert np.array_equal(mixed[2], a[5])
    assert np.array_equal(mixed[1], a[1])


def test_short_texts_alone_match_larger_packs(c2_model, config2_batch):
    """A pack of at most 512 tokens runs its GEMMs on the skinny kernel and the QKV epilogue as a
    separate row pass (and, up to 64 tokens, replays as a graph); inside a pack of more than 512
    tokens the same text runs on the tiled kernels. The vector must have the same bits either
    way (MetalForwardTests.swift:95-120: counts around the tile boundaries, alone and between a
    19- and a 500-token text)."""
    body = config2_batch[7]
    ctx = c2_model.context
    for count in (1, 2, 13, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 480, 511, 512):
        subject = body[:count]
        packed, _ = ctx.forward([config2_batch[3][:19], subject, config2_batch[4][:500]])
        alone, _ = ctx.forward([subject])
        assert np.array_equal(alone[0], packed[1]), count
    for lengths in ([5, 8], [8, 8], [8, 9], [30, 34], [100, 200, 150]):
        small = [config2_batch[9 + i][:n] for i, n in enumerate(lengths)]
        got, _ = ctx.forward(small)
        want, _ = ctx.forward(small + [config2_batch[20][:500]])
        for i in range(len(lengths)):
            assert np.array_equal(got[i], want[i]), (lengths, i)


def test_short_pack_graph_replays_match_eager(c2_model, config2_batch, c2_oracle):
    """Packs of at most 64 tokens replay their forward as a HIP graph from the second run of a
    shape on. Every replay, with other shapes and eager work queued between replays, must equal
    the shape's first (eager) run bitwise; new ids in a known shape must give their own vectors."""
    ctx = c2_model.context
    a = [config2_batch[11][:9]]
    b = [config2_batch[12][:20], config2_batch[13][:5]]
    first_a, _ = ctx.forward(a)
    first_b, _ = ctx.forward(b)
    for i in range(4):
        got, _ = ctx.forward(a)
        assert np.array_equal(got, first_a), i
        ctx.forward([config2_batch[14 + i][:300]])
        got, _ = ctx.forward(b)
        assert np.array_equal(got, first_b), i
    a2 = [config2_batch[15][:9]]
    replayed, _ = ctx.forward(a2)
    packed, _ = ctx.forward([a2[0], config2_batch[16][:100]])
    assert np.array_equal(replayed[0], packed[0])
    want, _ = c2_oracle.forward(a2[0])
    assert cosine(replayed[0], want) >= COSINE_BAR


def test_short_pack_graph_cache_eviction(config2_gguf, config2_batch):
    """A context keeps the graphs of at most 32 short-pack shapes; a 33rd shape evicts the oldest.
    Here the oldest graph's replay is still queued (ge_batch_run returns before the GPU is done)
    when the new shape evicts it: the eviction waits for the streams, and every result equals
    the shape's eager run bitwise. A fresh model, so that the cache starts empty and the 32 shapes
    below fill it in order."""
    m = ge.EmbeddingModel.load(config2_gguf, batch_token_budget=8192)
    try:
        _graph_cache_eviction(m.context, config2_batch[21])
    finally:
        m.close()


def _graph_cache_eviction(ctx, text):
    lengths = list(range(64, 32, -1))  # 32 shapes, the largest first (the workspace never grows)
    first = {}
    for n in lengths:
        first[n], _ = ctx.forward([text[:n]])  # eager: records the shape
        again, _ = ctx.forward([text[:n]])  # captured, then replayed
        assert np.array_equal(again, first[n]), n
    oldest, new = lengths[0], 32
    ctx.batch_stage([text[:oldest]])
    ctx.batch_run()  # replays the oldest graph; not waited for
    ctx.batch_stage([text[:new]])
    ctx.batch_run()  # a 33rd shape: evicts the oldest graph, then runs eagerly
    got_new = ctx.batch_read()
    want_new, _ = ctx.forward([text[:new]])  # the same shape again: captured and replayed
    assert np.array_equal(got_new, want_new)
    for n in (oldest, oldest, oldest, 40):
        got, _ = ctx.forward([text[:n]])  # the evicted shape is recorded, captured and replayed again
        assert np.array_equal(got, first[n]), n
    print("33 short-pack shapes: eviction of a queued graph, all runs bitwise equal", flush=True)


def test_embed_api_options(c2_model, config2_batch):
    texts = [t[: 20 + 37 * i] for i, t in enumerate(config2_batch[:10])]
    full = c2_model.embed(texts, ge.EmbedOptions(normalise=False))
    raw = c2_model.embed_tokens(texts)
    for i in range(10):
        assert np.allclose(full[i].vector, raw[i], atol=1e-5 * np.abs(raw[i]).max())
        assert full[i].token_count == len(texts[i]) and not full[i].truncated
    for dims in (768, 512, 256, 128):
        e = c2_model.embed(texts[:3], ge.EmbedOptions(dimensions=dims))
        for i in range(3):
            v = raw[i][:dims] / np.linalg.norm(raw[i][:dims])
            assert e[i].vector.shape == (dims,)
            assert abs(np.linalg.norm(e[i].vector) - 1) < 1e-5
            assert np.allclose(e[i].vector, v, atol=1e-5)
    with pytest.raises(ge.GemmaEmbedError) as err:
        c2_model.embed(texts[:1], ge.EmbedOptions(dimensions=100))
    assert err.value.kind == "invalidOptions"


def test_embed_truncation_keeps_eos(c2_model, config2_batch):
    text = config2_batch[0]
    e = c2_model.embed([text], ge.EmbedOptions(max_tokens=16))[0]
    assert e.truncated and e.token_count == 16
    direct = c2_model.embed_tokens([text[:15] + [c2_model.info.eos_id]])[0]
    assert np.allclose(e.vector, direct / np.linalg.norm(direct), atol=1e-5)
    assert not c2_model.embed([text[:10]], ge.EmbedOptions(max_tokens=16))[0].truncated


def test_embed_batching_progress_and_cancel(c2_model, config2_batch):
    texts = [t[: 50 + 300 * (i % 3)] for i, t in enumerate(config2_batch[:20])]
    events = []
    auto = c2_model.embed(texts, progress=lambda p: events.append(p))
    one = c2_model.embed(texts, ge.EmbedOptions(batch_size=1))
    three = c2_model.embed(texts, ge.EmbedOptions(batch_size=3))
    for i in range(20):
        assert np.abs(auto[i].vector - one[i].vector).max() < 1e-5
        assert np.abs(auto[i].vector - three[i].vector).max() < 1e-5
    assert events and events[-1].completed_texts == 20 and events[-1].total_texts == 20
    assert events[-1].completed_tokens == sum(len(t) for t in texts)
    with pytest.raises(ge.GemmaEmbedError) as err:
        c2_model.embed(texts, ge.EmbedOptions(batch_size=1), progress=lambda p: True)
    assert err.value.kind == "cancelled"


def _forwards_run(model, texts, options, progress):
    """Runs embed with the context's kernel profile on and returns how many forwards it launched
    (one embedding-gather launch per forward) and what the call raised, if anything."""
    ctx = model.context
    ctx.profile_enable("")
    ctx.profile_reset()
    raised = None
    try:
        model.embed(texts, options, progress=progress)
    except ge.GemmaEmbedError as e:
        raised = e
    finally:
        ctx.profile_disable()
    stats = ctx.profile_stats()
    return sum(n for name, (n, _) in stats.items() if name.startswith("embed_norm")), raised


def test_embed_one_forward_per_planned_batch_and_cancel(config2_gguf, config2_batch):
    """By default each planned batch is one forward, bounded by the batch budget
    (EmbeddingModel.swift:157-172, EmbedOptions.swift:194), and a cancel returned after the first
    batch stops before the second batch's GPU work (Task.checkCancellation, :162)."""
    texts = [t[:300] for t in config2_batch[:12]]  # 3600 tokens: batches of 1000 at budget 1000
    with ge.EmbeddingModel.load(config2_gguf, batch_token_budget=1000) as m:
        n, raised = _forwards_run(m, texts, ge.EmbedOptions(), None)
        assert raised is None and n == 4, n
        calls = []
        n, raised = _forwards_run(m, texts, ge.EmbedOptions(), lambda p: calls.append(p) or True)
        assert raised is not None and raised.kind == "cancelled"
        assert n == 1 and len(calls) == 1 and calls[0].completed_texts == 3, (n, calls)
        ref = m.embed(texts)
    # merged device packs (pack_tokens above the budget): same vectors, fewer forwards
    with ge.EmbeddingModel.load(config2_gguf, batch_token_budget=1000, pack_tokens=8192) as m:
        n, raised = _forwards_run(m, texts, ge.EmbedOptions(), None)
        assert raised is None and n == 1, n
        got = m.embed(texts)
    for a, b in zip(ref, got):
        assert np.array_equal(a.vector, b.vector)


def config3_texts():
    """BASELINE config 3 as the bench draws it: 256 texts, lengths U[8, 256] (SplitMix64 seed 31),
    ids U[2, 262144) (seed 32)."""
    lengths = ge.synth_tokens(31, 8, 257, 256)
    ids = ge.synth_tokens(32, 2, 262144, int(lengths.sum()))
    texts, off = [], 0
    for n in lengths:
        texts.append(ids[off:off + n].tolist())
        off += n
    return texts


@pytest.fixture(scope="module")
def config3_default(c2_model, c2_oracle):
    """Config 3 through embed at the default load (fp16 scores), Matryoshka 256, and the max |d|
    of the normalised vectors against the oracle on the 32 shortest texts plus texts 0, 77, 255."""
    texts = config3_texts()
    out = c2_model.embed(texts, ge.EmbedOptions(dimensions=256))
    assert len(out) == 256 and all(o.vector.shape == (256,) for o in out)
    pick = sorted(range(256), key=lambda i: len(texts[i]))[:32] + [0, 77, 255]
    worst = (0.0, -1)
    for i in pick:
        want, _ = c2_oracle.forward(texts[i])
        w = want[:256] / np.linalg.norm(want[:256])
        assert cosine(out[i].vector, w) >= COSINE_BAR, i
        worst = max(worst, (float(np.abs(out[i].vector - w).max()), i))
    print(f"config 3 default: max |d| {worst[0]:.3e} (text {worst[1]}, {len(texts[worst[1]])} tokens)", flush=True)
    return worst


# Bound of the fp16-operand design on these texts: the float64 emulation of its roundings
# (tests/fp16_emulation.py) gives a mean max |d| of 6.8e-5 and a worst of 9.1e-5 over 80 of
# config 3's texts; GPU draws of the same distribution reached 1.26e-4 on one text of 44.
FP16_DESIGN_MAX_ABS = 2e-4


def test_config3_ragged_vs_oracle(config3_default):
    """256 texts, lengths U[8, 256], packed by token count, Matryoshka 256:
    cosine >= 0.99999 on every checked text, and max |d| within the fp16 design's bound."""
    assert config3_default[0] < FP16_DESIGN_MAX_ABS, config3_default


@pytest.mark.xfail(reason="fp16 q.k scores: config 3's worst short text reaches 1.0-1.3e-4 against the "
                          "reference's 1e-4 (MetalForwardTests.swift:213-214); the split_scores load "
                          "option meets it (3.2e-5), the default does not", strict=False)
def test_config3_default_meets_the_reference_max_abs(config3_default):
    assert config3_default[0] < 1e-4, config3_default


def test_split_scores_meet_the_reference_bar_on_config3(config2_gguf, c2_oracle):
    """Loaded with split_scores (ge_set_split_scores(ctx, 0)), config 2's 256-wide layers run the
    QKV projection on hi/lo fp16 operand pairs and score on attention_split_kernel<256, 3>. On
    BASELINE config 3's texts (the bench's seeds, Matryoshka 256) the vectors then meet the
    reference's own bars against the oracle, cosine > 0.99999 and max |diff| < 1e-4 of the
    normalised vectors (MetalForwardTests.swift:213-214), which fp16 scores miss on some short
    texts (1.26e-4 in the bench's sample). A text's vector is the same bits alone and in the pack."""
    lengths = [int(n) for n in ge.synth_tokens(31, 8, 257, 256)]
    ids = ge.synth_tokens(32, 2, 262144, sum(lengths))
    texts, off = [], 0
    for n in lengths:
        texts.append(ids[off:off + n].tolist())
        off += n
    sample = list(range(24)) + sorted(range(24, 256), key=lambda i: lengths[i])[:8]
    m = ge.EmbeddingModel.load(config2_gguf, split_scores=True)
    try:
        opts = ge.EmbedOptions(dimensions=256)
        out = m.embed(texts, opts)
        alone = m.embed([texts[sample[-1]]], opts)[0].vector
    finally:
        m.close()
    assert np.array_equal(alone, out[sample[-1]].vector)
    worst = 0.0
    for i in sample:
        want, _ = c2_oracle.forward(texts[i])
        w = want[:256] / np.linalg.norm(want[:256])
        g = np.asarray(out[i].vector, np.float64)
        assert cosine(g, w) > 0.99999, i
        worst = max(worst, float(np.abs(g - w).max()))
    print(f"split scores, config 3 sample of {len(sample)} texts: max |diff| {worst:.3g}")
    assert worst < 1e-4


def test_split_scores_texts_longer_than_the_window(config2_gguf, c2_oracle, config2_batch):
    """split_scores on texts longer than the 512-token window (sliding layers clip their key range
    and mask by it; global layers see every key), packed with a short one: against the oracle at
    the reference's bars, and each text's vector the same bits alone as in the pack."""
    texts = [config2_batch[0] + config2_batch[1][:600], config2_batch[2][:700], config2_batch[3][:40]]
    m = ge.EmbeddingModel.load(config2_gguf, split_scores=True)
    try:
        pooled = m.embed_tokens(texts)
        alone = m.embed_tokens([texts[1]])[0]
    finally:
        m.close()
    assert np.array_equal(alone, pooled[1])
    for i, t in enumerate(texts):
        want, _ = c2_oracle.forward(t)
        d = float(np.abs(normalised(pooled[i]) - normalised(want)).max())
        print(f"split scores, text of {len(t)} tokens: cosine {cosine(pooled[i], want):.9f} max |diff| {d:.3g}", flush=True)
        assert cosine(pooled[i], want) > 0.99999 and d < 1e-4, i


@pytest.fixture(scope="module")
def config4_texts():
    # 4 texts x 8192 tokens, ids uniform in [2, 262144)
    toks = ge.synth_tokens(8, 2, 262144, 4 * 8192).reshape(4, 8192)
    return [t.tolist() for t in toks]


def test_config4_long_context_vs_oracle(config2_gguf, c2_oracle, config4_texts):
    """the 24-layer encoder over 4 texts of 8192 tokens (sliding window 512 on
    local layers, full 8192 x 8192 attention on the global layers 5, 11, 17, 23), as one
    32768-token pack. The last text against the oracle: pooled cosine and per-layer error at a
    global and the last layer; the same text alone must give the same bits."""
    m = ge.EmbeddingModel.load(config2_gguf, batch_token_budget=32768)
    try:
        ctx = m.context
        print("config4 forward 4 x 8192 (one pack of 32768)", flush=True)
        pooled, secs = ctx.forward(config4_texts)
        print(f"gpu forward {secs * 1e3:.2f} ms", flush=True)
        assert pooled.shape == (4, 768) and np.all(np.isfinite(pooled))
        alone, _ = ctx.forward([config4_texts[3]])
        assert np.array_equal(alone[0], pooled[3])
        print("oracle forward of one 8192-token text (about half a minute)", flush=True)
        keep = [("l_out", 5), ("l_out", 23)]
        want, tr = c2_oracle.forward(config4_texts[3], keep=keep)
        c = cosine(pooled[3], want)
        print(f"text 3 cosine {c:.9f} max_rel {max_rel(pooled[3], want):.3e}", flush=True)
        assert c >= COSINE_BAR
        for name, layer in keep:
            got = ctx.trace([config4_texts[3]], name, layer)
            r = max_rel(got, tr[(name, layer)].reshape(8192, -1))
            print(f"{name}-{layer}: max_rel {r:.3e}", flush=True)
            assert r <= PER_LAYER_TOL, (name, layer)
    finally:
        m.close()


def test_growing_batches_in_one_context(config2_gguf, c2_oracle):
    """Batches that grow from one short text (the workspace and the transposed-V buffer grow
    between calls; a grown V^T row length must stay a multiple of 8 columns), each against the
    oracle."""
    m = ge.EmbeddingModel.load(config2_gguf, batch_token_budget=8192)
    try:
        for lengths in ([8], [16], [40], [8, 200], [1000], [3, 5, 7]):
            texts = [ge.synth_tokens(20 + n, 2, 262144, n).tolist() for n in lengths]
            print(f"lengths {lengths}", flush=True)
            pooled, _ = m.context.forward(texts)
            for i, t in enumerate(texts):
                want, _ = c2_oracle.forward(t)
                assert cosine(pooled[i], want) >= COSINE_BAR, (lengths, i)
    finally:
        m.close()


def test_rejects_bad_batches(c2_model):
    ctx = c2_model.context
    with pytest.raises(ge.GemmaEmbedError) as e:
        ctx.forward([[5, 262144]])
    assert e.value.kind == "invalid"
    with pytest.raises(ge.GemmaEmbedError):
        ctx.forward([[]])
    with pytest.raises(ge.GemmaEmbedError):
        ctx.forward([list(range(2, 8200))])  # longer than the 8192-token context


def _split(a, lengths):
    out, r = [], 0
    for n in lengths:
        out.append(a[r:r + n])
        r += n
    return out


def test_per_layer_inputs_every_trace_vs_oracle(tiny_ple_gguf):
    """The per-layer-input branch (CPUReference.swift:206-210, :259-269) on the GPU: the per-layer
    inputs, the residual before and after the branch, and the pooled vectors."""
    m = ge.EmbeddingModel.load(tiny_ple_gguf)
    try:
        seqs = [ge.synth_tokens(s, 2, 512, n).tolist() for s, n in ((31, 40), (32, 7), (33, 64), (34, 100))]
        lengths = [len(x) for x in seqs]
        pooled = m.embed_tokens(seqs)
        names = [("inp_per_layer", -1)] + [(n, l) for l in range(2) for n in ("pe_in", "l_out")] + [("attn_norm", 1)]
        with ora.OracleModel(tiny_ple_gguf) as o:
            want = [o.forward(sq, keep=names) for sq in seqs]
            for i in range(len(seqs)):
                assert cosine(pooled[i], want[i][0]) >= COSINE_BAR, i
            for name, layer in names:
                got = m.context.trace(seqs, name, layer)
                for i, part in enumerate(_split(got, lengths)):
                    assert max_rel(part, want[i][1][(name, layer)].reshape(part.shape)) <= PER_LAYER_TOL, (name, layer, i)
        # a short text alone (the graph-replayed short path) has the bits it has inside the pack
        for _ in range(3):
            alone, _ = m.context.forward([seqs[1]])
            assert np.array_equal(alone[0], pooled[1])
    finally:
        m.close()


@pytest.mark.timeout(300)
def test_reference_real_architecture_vs_oracle(real_shapes_gguf):
    """The reference's real architecture at its real shapes (Model/Architecture.md:7-9): d 512,
    4 query heads, sliding layers with 2 KV heads of 256 and window 1024, global layers with 1 KV
    head of 512, GeGLU 2048, per-layer inputs of 512; synthetic weights."""
    m = ge.EmbeddingModel.load(real_shapes_gguf)
    try:
        seqs = [ge.synth_tokens(s, 2, 262144, n).tolist() for s, n in ((41, 9), (42, 300), (43, 1500))]
        lengths = [len(x) for x in seqs]
        pooled = m.embed_tokens(seqs)
        layers = (0, 5, 11, 23)
        keep = [("l_out", l) for l in layers]
        with ora.OracleModel(real_shapes_gguf) as o:
            want = [o.forward(sq, keep=keep) for sq in seqs]
        for i in range(len(seqs)):
            c = cosine(pooled[i], want[i][0])
            print(f"real shapes: text {i} ({lengths[i]} tokens) cosine {c:.8f}", flush=True)
            assert c >= COSINE_BAR, i
        # the 9-token text alone runs the short-batch kernels (K of 512, 1024 and 2048: 8 or 16
        # k-steps in flight) and must have the bits it has inside the pack
        for _ in range(3):
            alone, _ = m.context.forward([seqs[0]])
            assert np.array_equal(alone[0], pooled[0])
        for l in layers:
            got = m.context.trace(seqs, "l_out", l)
            for i, part in enumerate(_split(got, lengths)):
                assert max_rel(part, want[i][1][("l_out", l)].reshape(part.shape)) <= PER_LAYER_TOL, (l, i)
        # the raw projection of a sliding layer (its fp32 trace path) and the attention of a sliding
        # and a global layer. The global layer (head dim 512) scores dot products of two normed
        # 512-wide vectors at scale 1 (magnitudes of several hundred): its QKV projection and scores
        # run at split precision, without which its attention output reached 1.1e-2.
        keep2 = [("Qcur", 0), ("Vcur_normed", 0), ("Qcur", 5), ("kqv_out", 4), ("kqv_out", 5)]
        with ora.OracleModel(real_shapes_gguf) as o:
            want2 = [o.forward(sq, keep=keep2)[1] for sq in seqs]
        for name, l in keep2:
            got = m.context.trace(seqs, name, l)
            for i, part in enumerate(_split(got, lengths)):
                err = max_rel(part, want2[i][(name, l)].reshape(part.shape))
                print(f"real shapes: {name} layer {l} text {i}: max_rel {err:.2e}", flush=True)
                assert err <= PER_LAYER_TOL, (name, l, i)
    finally:
        m.close()


@pytest.mark.timeout(300)
def test_reference_real_architecture_split_pack_bitwise(real_shapes_gguf):
    """A pack of at least 4096 tokens runs as parts on several streams, through every layer type
    of the real architecture (fused and fp32 QKV, head dims 256 and 512, the per-layer-input
    branch): each text must have the bits it has alone (one stream)."""
    m = ge.EmbeddingModel.load(real_shapes_gguf, batch_token_budget=16384)
    try:
        seqs = [ge.synth_tokens(s, 2, 262144, n).tolist() for s, n in ((51, 1500), (52, 1300), (53, 1200), (54, 700))]
        packed = m.embed_tokens(seqs)
        for i, sq in enumerate(seqs):
            alone, _ = m.context.forward([sq])
            assert np.array_equal(alone[0], packed[i]), i
        with ora.OracleModel(real_shapes_gguf) as o:
            want, _ = o.forward(seqs[3])
        assert cosine(packed[3], want) >= COSINE_BAR
    finally:
        m.close()
