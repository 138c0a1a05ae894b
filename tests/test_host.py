"""Host-side logic that needs no GPU: batch planning, finish, synthetic GGUF writer and the
loader's validation (the reference's EmbeddingModelTests.testBatchPlanning,
GGUFReaderTests.testRejectsNonGGUF and the shape/type checks of ModelWeights.init)."""
import struct

import numpy as np
import pytest

import gemma_embed as ge
import npref


def test_batch_planning_matches_reference_cases():
    # EmbeddingModelTests.swift:101-109
    assert ge.plan_batches([[5], [5], [5], [5]], [10]) == [range(0, 2), range(2, 4)]
    assert ge.plan_batches([[50], [5]], [10]) == [range(0, 1), range(1, 2)]
    assert ge.plan_batches([[1], [1], [1]], [10], batch_size=2) == [range(0, 2), range(2, 3)]
    assert ge.plan_batches([], [10]) == []
    assert ge.plan_batches([[1, 3], [1, 3], [1, 1]], [10, 6]) == [range(0, 2), range(2, 3)]
    assert ge.plan_batches([[6, 0], [6, 0]], [10, 6]) == [range(0, 1), range(1, 2)]


def test_batch_planning_config2_default_budget():
    # 32 texts x 512 tokens at the default 8192-token budget: two packs of 16 texts
    assert ge.plan_batches([[512]] * 32, [8192]) == [range(0, 16), range(16, 32)]
    assert ge.plan_batches([[512]] * 32, [16384]) == [range(0, 32)]


def test_batch_planning_brute_force():
    rng = np.random.default_rng(5)
    for _ in range(200):
        n = int(rng.integers(0, 30))
        costs = rng.integers(1, 40, n).tolist()
        budget = int(rng.integers(1, 100))
        got = ge.plan_batches(costs, [budget])
        # consecutive, covering, non-empty; each cut happens exactly where adding the next
        # item would exceed the budget (or a single oversized item stands alone)
        assert [r.start for r in got] == ([0] + [r.stop for r in got[:-1]] if got else [])
        assert (got[-1].stop if got else 0) == n
        for r in got:
            assert len(r) >= 1
            s = sum(costs[r.start:r.stop])
            assert len(r) == 1 or s <= budget
            if r.stop < n:
                assert s + costs[r.stop] > budget


def test_finish_matryoshka_and_l2():
    v = np.arange(1, 769, dtype=np.float32) / 100
    for dims in (768, 512, 256, 128):
        out = ge.finish(v, dims, True)
        assert out.shape == (dims,)
        assert abs(float(np.linalg.norm(out)) - 1) < 1e-5
        assert np.allclose(out, v[:dims] / np.linalg.norm(v[:dims]), atol=1e-6)
    assert np.array_equal(ge.finish(v, 256, False), v[:256])
    assert np.array_equal(ge.finish(np.zeros(768, np.float32), 128, True), np.zeros(128, np.float32))
    with pytest.raises(ge.GemmaEmbedError):
        ge.finish(v, 1000, True)


def test_synth_tokens_are_seeded_and_in_range():
    a = ge.synth_tokens(3, 2, 262144, 10000)
    b = ge.synth_tokens(3, 2, 262144, 10000)
    assert np.array_equal(a, b)
    assert a.min() >= 2 and a.max() < 262144
    assert not np.array_equal(a, ge.synth_tokens(4, 2, 262144, 10000))
    # roughly uniform
    assert abs(a.mean() - 131073) < 3 * 262142 / np.sqrt(12 * 10000)


def test_splitmix_matches_reference_seeded_random():
    # KernelTests.swift:9-26: state = seed + golden; next: state += golden; mix(state)
    def ref(seed, n):
        m = (1 << 64) - 1
        g = 0x9E3779B97F4A7C15
        s = (seed + g) & m
        out = []
        for _ in range(n):
            s = (s + g) & m
            z = s
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
            out.append(z ^ (z >> 31))
        return out
    words = ref(3, 16)
    want = [2 + (((w >> 32) * (262144 - 2)) >> 32) for w in words]
    assert ge.synth_tokens(3, 2, 262144, 16).tolist() == want


def test_synth_gguf_follows_the_weight_rules(tiny_gguf):
    g = npref.Gguf(tiny_gguf)
    a = "gemma-embedding2."
    assert g.meta["general.architecture"] == "gemma-embedding2"
    assert g.meta[a + "block_count"] == 2 and g.meta[a + "embedding_length"] == 128
    assert g.meta[a + "attention.sliding_window_pattern"] == [True, False]
    assert len(g.meta["tokenizer.ggml.tokens"]) == 512
    shape, typ, _ = g.tensors["blk.0.ffn_gate.weight"]
    assert shape == [128, 256] and typ == 8
    blocks = np.asarray(g.raw("token_embd.weight")).reshape(-1, 34)
    q = blocks[:, 2:].view(np.int8).astype(np.int64)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    assert q.min() >= -127 and q.max() <= 127 and q.min() == -127 and q.max() == 127
    # d = |z| max|q| / 127 with z ~ N(0, 0.02): d * 127 / max|q| is half-normal with sigma 0.02
    z = d * 127 / np.abs(q).max(axis=1)
    assert np.all(z >= 0)
    assert abs(z.mean() - 0.02 * np.sqrt(2 / np.pi)) < 0.002
    w = g.tensor("blk.1.ffn_norm.weight")
    assert abs(w.mean() - 1) < 0.03 and abs(w.std() - 0.1) < 0.03
    assert "per_layer_model_proj.weight" not in g.tensors


def test_synth_gguf_is_deterministic(tmp_path):
    a = ge.synth_write_gguf(str(tmp_path / "a.gguf"), **ge.TINY)
    b = ge.synth_write_gguf(str(tmp_path / "b.gguf"), **ge.TINY)
    assert open(a, "rb").read() == open(b, "rb").read()
    spec = dict(ge.TINY, seed=8)
    c = ge.synth_write_gguf(str(tmp_path / "c.gguf"), **spec)
    assert open(a, "rb").read() != open(c, "rb").read()


def test_load_rejects_non_gguf(tmp_path):
    p = tmp_path / "junk.gguf"
    p.write_bytes(b"\x41" * 4096)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "invalidGGUF" and "bad magic" in e.value.message


def test_load_rejects_truncated_file(tmp_path, tiny_gguf):
    data = open(tiny_gguf, "rb").read()
    p = tmp_path / "cut.gguf"
    p.write_bytes(data[: len(data) // 2])
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "invalidGGUF" and "extends past the end" in e.value.message


def test_load_rejects_missing_file(tmp_path):
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(tmp_path / "nope.gguf"))
    assert e.value.kind == "invalidGGUF"


def _rewrite_meta_key(data: bytes, key: str, new_key: str) -> bytes:
    kb = key.encode()
    i = data.index(struct.pack("<Q", len(kb)) + kb)
    nb = new_key.encode()
    assert len(nb) == len(kb)
    return data[: i + 8] + nb + data[i + 8 + len(kb):]


def test_load_rejects_wrong_architecture(tmp_path, tiny_gguf):
    data = open(tiny_gguf, "rb").read()
    data = data.replace(b"gemma-embedding2", b"gemma-embeddingX", 1)
    p = tmp_path / "arch.gguf"
    p.write_bytes(data)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "model" and "unsupported architecture" in e.value.message


def test_load_rejects_missing_tensor(tmp_path, tiny_gguf):
    data = open(tiny_gguf, "rb").read()
    data = _rewrite_meta_key(data, "blk.1.ffn_up.weight", "blk.1.ffn_uq.weight")
    p = tmp_path / "missing.gguf"
    p.write_bytes(data)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "model" and "lacks tensor blk.1.ffn_up.weight" in e.value.message


def test_load_rejects_missing_metadata(tmp_path, tiny_gguf):
    data = open(tiny_gguf, "rb").read()
    data = _rewrite_meta_key(data, "gemma-embedding2.feed_forward_length", "gemma-embedding2.feed_forward_lengtX")
    p = tmp_path / "meta.gguf"
    p.write_bytes(data)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "model" and "feed_forward_length" in e.value.message


def _gguf_header(kv: bytes, n_kv: int, tensors: bytes = b"", n_tensors: int = 0) -> bytes:
    return b"GGUF" + struct.pack("<IQQ", 3, n_tensors, n_kv) + kv + tensors


def _gguf_key(name: str) -> bytes:
    return struct.pack("<Q", len(name)) + name.encode()


@pytest.mark.parametrize("count", [2 ** 61, 2 ** 62, 2 ** 64 - 1])
def test_load_rejects_array_count_past_the_file(tmp_path, count):
    """A metadata array whose element count times its element size wraps 64 bits: rejected as an
    invalid file, not an uncaught C++ exception that would abort the caller."""
    kv = _gguf_key("general.junk") + struct.pack("<IIQ", 9, 4, count) + b"\0" * 16
    p = tmp_path / "count.gguf"
    p.write_bytes(_gguf_header(kv, 1).ljust(100, b"\0"))
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "invalidGGUF" and "past the end of the header" in e.value.message


@pytest.mark.parametrize("shape,offset,msg", [
    ((2 ** 32, 2 ** 32), 0, "invalid shape"),          # element count past 2^63
    ((2 ** 63 - 1, 2), 0, "invalid shape"),
    ((0, 4), 0, "invalid shape"),
    ((33, 2), 0, "partial blocks"),                     # Q8_0 rows of whole 32-blocks only
    ((32, 2), 2 ** 64 - 32, "extends past the end"),   # offset + bytes wraps 64 bits
])
def test_load_rejects_tensor_extents(tmp_path, shape, offset, msg):
    t = _gguf_key("blk.0.x.weight") + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
    t += struct.pack("<IQ", 8, offset)  # Q8_0
    p = tmp_path / "extent.gguf"
    p.write_bytes(_gguf_header(b"", 0, t, 1).ljust(256, b"\0"))
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.EmbeddingModel.load(str(p))
    assert e.value.kind == "invalidGGUF" and msg in e.value.message, e.value.message
