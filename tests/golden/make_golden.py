#!/usr/bin/env python3
"""Writes the golden fixtures of this directory from the CPU oracle on seeded synthetic models.

    python tests/golden/make_golden.py        (from the repository root, after the build)

The fixtures follow the reference's fixture style (Fixtures/activations.jsonl: per named
tensor, its sum and corner values; Fixtures/embeddings.jsonl: one vector per text), but hold the
outputs of synthetic models, since the reference's fixtures need its real weights. Each file
records the inputs that made it (model spec and seeds, token ids) and a SHA-256 of the synthetic
GGUF, so a change of the model generator shows up as a fixture mismatch, not as a silent drift.
The fixtures pin the oracle against its own past outputs (a regression check) and give the GPU
tests an input/output pair that needs no oracle run; the oracle itself is pinned independently
by tests/test_oracle.py.
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "gemma-embed-swift_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import gemma_embed as ge  # noqa: E402
import ge_oracle as ora  # noqa: E402

CORNER = 4
# (fixture file, model spec name, token seed, sequence lengths, traced tensors)
CASES = [
    ("tiny_forward.json", "TINY", 11, [2, 5, 17, 40],
     ["inp_scaled", "attn_norm", "Qcur_pos", "kqv_out", "attn_out", "ffn_geglu", "ffn_out", "l_out", "result_norm"]),
    ("config2_forward.json", "CONFIG2", 21, [64, 7],
     ["inp_scaled", "kqv_out", "attn_out", "ffn_out", "l_out", "result_norm"]),
]


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def summary(a):
    a = np.asarray(a, np.float32).reshape(-1)
    return {"sum": float(a.astype(np.float64).sum()), "abs_sum": float(np.abs(a.astype(np.float64)).sum()),
            "first": [float(v) for v in a[:CORNER]], "last": [float(v) for v in a[-CORNER:]]}


def make_case(tmp, fname, spec_name, seed, lengths, names):
    spec = getattr(ge, spec_name)
    path = ge.synth_write_gguf(os.path.join(tmp, spec_name + ".gguf"), **spec)
    with ora.OracleModel(path) as m:
        ids = ge.synth_tokens(seed, 2, m.vocab, sum(lengths))
        texts, off = [], 0
        for n in lengths:
            texts.append([int(t) for t in ids[off:off + n]])
            off += n
        layers = list(range(m.layers))
        keep = [(n, -1) for n in names if n in ("inp_scaled", "result_norm")] + \
               [(n, l) for n in names if n not in ("inp_scaled", "result_norm") for l in layers]
        out = {"generator": "tests/golden/make_golden.py", "model": spec_name, "spec": spec,
               "gguf_sha256": sha256(path), "token_seed": seed, "texts": []}
        for toks in texts:
            pooled, traces = m.forward(toks, keep=keep, threads=8)
            tensors = [{"name": n, "layer": l, **summary(traces[(n, l)])} for (n, l) in keep if (n, l) in traces]
            out["texts"].append({"tokens": toks, "pooled": [float(v) for v in pooled], "tensors": tensors})
    with open(os.path.join(HERE, fname), "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {fname}: {len(texts)} texts, {sum(len(t['tensors']) for t in out['texts'])} tensor summaries")


def make_config1(tmp):
    """X fp32 [128 x 768] ~ N(0,1) (numpy default_rng(1)), W Q8_0 [1152 x 768]
    (blk.0.ffn_gate.weight of the config-2 model), Y = X W^T fp32 [128 x 1152]."""
    import npref
    path = ge.synth_write_gguf(os.path.join(tmp, "CONFIG2.gguf"), **ge.CONFIG2)
    g = npref.Gguf(path)
    x = np.random.default_rng(1).standard_normal((128, 768)).astype(np.float32)
    w = g.tensor("blk.0.ffn_gate.weight").astype(np.float32)
    y = ora.matmul(x, w)
    rng = np.random.default_rng(5)
    idx = rng.integers(0, y.size, 64)
    out = {"generator": "tests/golden/make_golden.py", "x": "numpy default_rng(1).standard_normal((128, 768)) as fp32",
           "w": "blk.0.ffn_gate.weight of the CONFIG2 synthetic model", "gguf_sha256": sha256(path),
           "shape": [128, 1152], **summary(y), "row_sums": [float(v) for v in y.astype(np.float64).sum(axis=1)],
           "sample_index": [int(i) for i in idx], "sample_value": [float(y.reshape(-1)[i]) for i in idx]}
    with open(os.path.join(HERE, "config1_gemm.json"), "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote config1_gemm.json")


if __name__ == "__main__":
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    with tempfile.TemporaryDirectory() as tmp:
        for case in CASES:
            make_case(tmp, *case)
        make_config1(tmp)
