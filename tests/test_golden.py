"""The golden fixtures of tests/golden/ (written by tests/golden/make_golden.py from the oracle on
seeded synthetic models, in the style of the reference's Fixtures/activations.jsonl and
embeddings.jsonl).

CPU: the synthetic-model generator still writes byte-identical files (SHA-256), the oracle still
produces the recorded outputs, and numpy float64 agrees with the recorded config-1 GEMM.
GPU: the HIP forward and GEMM, through the C-ABI, against the recorded outputs at the forward's
tolerances (cosine >= 0.99999 for pooled vectors, max relative error <= 1e-2 per tensor)."""
import hashlib
import json
import os

import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge
import npref

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FORWARD_FIXTURES = ["tiny_forward.json", "config2_forward.json"]


def load(name):
    with open(os.path.join(HERE, name)) as f:
        return json.load(f)


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("golden_models")
    return {name: ge.synth_write_gguf(str(d / f"{name}.gguf"), **getattr(ge, name)) for name in ("TINY", "CONFIG2")}


def check_summary(got, rec, tol):
    got = np.asarray(got, np.float64).reshape(-1)
    scale = max(np.abs(got).max(), 1e-30)
    assert abs(np.abs(got).sum() - rec["abs_sum"]) <= tol * abs(rec["abs_sum"]), rec["name"]
    assert np.abs(got[:len(rec["first"])] - rec["first"]).max() <= tol * scale, rec["name"]
    assert np.abs(got[-len(rec["last"]):] - rec["last"]).max() <= tol * scale, rec["name"]
    assert abs(got.sum() - rec["sum"]) <= tol * np.abs(got).sum(), rec["name"]


@pytest.mark.parametrize("fixture", FORWARD_FIXTURES)
def test_synthetic_model_generator_is_unchanged(models, fixture):
    g = load(fixture)
    assert g["spec"] == getattr(ge, g["model"])
    assert sha256(models[g["model"]]) == g["gguf_sha256"]


@pytest.mark.parametrize("fixture", FORWARD_FIXTURES)
def test_oracle_reproduces_golden_forward(models, fixture):
    g = load(fixture)
    with ora.OracleModel(models[g["model"]]) as m:
        for text in g["texts"]:
            keep = [(t["name"], t["layer"]) for t in text["tensors"]]
            pooled, traces = m.forward(text["tokens"], keep=keep, threads=4)
            assert max_rel(pooled, text["pooled"]) <= 1e-5
            for rec in text["tensors"]:
                check_summary(traces[(rec["name"], rec["layer"])], rec, 1e-5)


def test_config1_gemm_fixture_vs_float64(models):
    """Recorded oracle GEMM against an independent float64 product of the same operands."""
    g = load("config1_gemm.json")
    assert sha256(models["CONFIG2"]) == g["gguf_sha256"]
    x = np.random.default_rng(1).standard_normal((128, 768)).astype(np.float32)
    w = npref.Gguf(models["CONFIG2"]).tensor("blk.0.ffn_gate.weight").astype(np.float64)
    y = x.astype(np.float64) @ w.T
    assert max_rel(y.reshape(-1)[g["sample_index"]], g["sample_value"]) <= 1e-5
    assert max_rel(y.sum(axis=1), g["row_sums"]) <= 1e-5
    y32 = ora.matmul(x, w.astype(np.float32))
    assert max_rel(y32.reshape(-1)[g["sample_index"]], g["sample_value"]) <= 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("fixture", FORWARD_FIXTURES)
def test_gpu_forward_vs_golden(models, fixture):
    g = load(fixture)
    print(f"golden {fixture}: {len(g['texts'])} texts", flush=True)
    texts = [t["tokens"] for t in g["texts"]]
    with ge.EmbeddingModel.load(models[g["model"]]) as m:
        pooled, _ = m.context.forward(texts)
        for i, text in enumerate(g["texts"]):
            assert cosine(pooled[i], text["pooled"]) >= 0.99999, i
            assert max_rel(pooled[i], text["pooled"]) <= 1e-2, i
        # per-layer outputs of the first text, alone in its pack
        first = g["texts"][0]
        for rec in first["tensors"]:
            if rec["name"] != "l_out":
                continue
            got = m.context.trace([first["tokens"]], rec["name"], rec["layer"])
            check_summary(got, rec, 1e-2)


@pytest.mark.gpu
def test_gpu_config1_gemm_vs_golden(models):
    g = load("config1_gemm.json")
    print("golden config-1 GEMM 128 x 1152 x 768", flush=True)
    x16 = np.random.default_rng(1).standard_normal((128, 768)).astype(np.float32).astype(np.float16)
    gg = npref.Gguf(models["CONFIG2"])
    ctx = ge.Context.create(0)
    try:
        w = ctx.q8_create(np.asarray(gg.raw("blk.0.ffn_gate.weight")), 1152, 768)
        dx, dy = ctx.alloc(x16.nbytes), ctx.alloc(128 * 1152 * 4)
        try:
            ctx.upload(dx, x16)
            ctx.gemm_q8(w, dx, 128, dy)
            y = ctx.download(dy, (128, 1152), np.float32)
        finally:
            ctx.free(dx)
            ctx.free(dy)
            ctx.q8_destroy(w)
    finally:
        ctx.close()
    # fp16 rounding of X and of each dequantised weight: relative 2^-12 each
    assert max_rel(y.reshape(-1)[g["sample_index"]], g["sample_value"]) <= 3e-3
    assert max_rel(y.astype(np.float64).sum(axis=1), g["row_sums"]) <= 3e-3
