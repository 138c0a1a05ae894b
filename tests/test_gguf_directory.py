"""The GGUF reader against the reference's real weight file's directory (GGUFReaderTests.swift:8-66).

The real `embeddinggemma-2-Q8_0.gguf` is not available here; its tensor directory and text-path
metadata are, in the reference's fixture (Fixtures/model.json, copied as data into
tests/golden/real_model_directory.json by tests/golden/make_real_directory.py). The synthetic
writer's REAL_SHAPES file has that directory, so reading it with the library's GGUF reader must
give the fixture's 413 tensors (names, ne shapes, types, data offsets in file order), the same
type counts and the text configuration the fixture's metadata implies. Its context_length is the
real file's 262144, which the configuration caps at 8192 (ModelConfig.swift:52, :95)."""
import json
import os

import numpy as np
import pytest

import gemma_embed as ge

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def fixture():
    return json.load(open(os.path.join(HERE, "golden", "real_model_directory.json")))


@pytest.fixture(scope="module")
def real_file(tmp_path_factory, fixture):
    ctx = fixture["metadata"]["gemma-embedding2.context_length"]
    path = str(tmp_path_factory.mktemp("real") / "real_shapes_ctx.gguf")
    return ge.synth_write_gguf(path, **dict(ge.REAL_SHAPES, context_length=ctx))


def test_tensor_directory_matches_fixture(real_file, fixture):
    with ge.GgufFile(real_file) as g:
        assert g.version == fixture["gguf_version"] == 3
        assert g.tensor_count == fixture["tensor_count"] == 413
        got = g.tensors()
        for (name, shape, typ, off), (wn, ws, wt, wo) in zip(got, fixture["tensors"]):
            assert (name, shape, typ, off) == (wn, ws, wt, wo), name
        counts = {}
        for _, _, typ, _ in got:
            counts[typ] = counts.get(typ, 0) + 1
        assert counts == fixture["tensor_type_counts"] == {"Q8_0": 218, "F32": 194, "BF16": 1}
        # 32-byte alignment; the last tensor ends the file (GGUFReaderTests.swift:24-27)
        assert g.data_offset % 32 == 0
        last = max(got, key=lambda t: t[3])
        n = int(np.prod(last[1]))
        nbytes = {"F32": 4 * n, "F16": 2 * n, "BF16": 2 * n, "Q8_0": n // 32 * 34}[last[2]]
        assert g.data_offset + last[3] + nbytes == g.file_size


def test_text_config_matches_fixture_metadata(real_file, fixture):
    meta = fixture["metadata"]
    a = "gemma-embedding2."
    with ge.GgufFile(real_file) as g:
        info = g.text_config()
    assert info.architecture.decode() == meta["general.architecture"]
    assert info.layers == meta[a + "block_count"] == 24
    assert info.hidden == meta[a + "embedding_length"]
    assert info.out_dims == meta[a + "embedding_length_out"]
    assert info.per_layer_input == meta[a + "embedding_length_per_layer_input"]
    assert info.feed_forward == meta[a + "feed_forward_length"]
    assert info.heads == meta[a + "attention.head_count"]
    assert info.sliding_window == meta[a + "attention.sliding_window"]
    assert info.vocab == fixture["vocab_size"] == 262144
    assert info.bos_id == meta["tokenizer.ggml.bos_token_id"] and info.eos_id == meta["tokenizer.ggml.eos_token_id"]
    assert info.eps == pytest.approx(meta[a + "attention.layer_norm_rms_epsilon"], rel=1e-6)
    assert info.quantization.decode() == "Q8_0"
    # the real file says 262144; the reference caps the context at 8192 whatever the file says
    assert meta[a + "context_length"] == 262144
    assert info.max_tokens == 8192


def test_synthetic_metadata_carries_the_fixture_values(real_file, fixture):
    """Every text-path metadata value of the synthetic file equals the real file's (an independent
    GGUF reader, tests/npref.py)."""
    import npref
    g = npref.Gguf(real_file)
    for k, want in fixture["metadata"].items():
        got = g.meta[k]
        if isinstance(want, float):
            assert got == pytest.approx(want, rel=1e-6), k
        else:
            assert got == want, k


def test_reader_rejects_non_gguf(tmp_path):
    p = tmp_path / "junk.gguf"
    p.write_bytes(b"\x41" * 4096)
    with pytest.raises(ge.GemmaEmbedError) as e:
        ge.GgufFile(str(p))
    assert e.value.kind == "invalidGGUF"
