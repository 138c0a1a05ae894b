#!/usr/bin/env python3
"""Writes outlier_fp16_emulation.json: for the outlier-norm synthetic model (ge.OUTLIER_NORMS) and
the texts of tests/test_gpu_forward.py::test_outlier_norm_weights_vs_oracle, the max relative
error of every traced intermediate of tests/fp16_emulation.py's forward (the GPU kernels' fp16
rounding points) against the plain float64 forward, and the pooled vectors' cosine.

    python tests/golden/make_fp16_emulation.py      (from the repository root, after the build)
"""
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "gemma-embed-swift_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import gemma_embed as ge  # noqa: E402
import fp16_emulation as emu  # noqa: E402
import npref  # noqa: E402

TEXTS = ((61, 300), (62, 512), (63, 77))  # (token seed, length), ids uniform in [2, 262144)
NAMES = ("l_out", "kqv_out", "ffn_geglu", "ffn_out")


def main():
    with tempfile.TemporaryDirectory() as tmp:
        path = ge.synth_write_gguf(os.path.join(tmp, "outlier.gguf"), **ge.OUTLIER_NORMS)
        g = npref.Gguf(path)
        layers = ge.OUTLIER_NORMS["layers"]
        keep = [(n, l) for l in range(layers) for n in NAMES]
        texts = []
        for seed, n in TEXTS:
            toks = [int(t) for t in ge.synth_tokens(seed, 2, 262144, n)]
            ref_pool, ref = emu.forward(g, toks, False, keep)
            emu_pool, got = emu.forward(g, toks, True, keep)
            errs = {f"{name}/{layer}": float(np.abs(got[(name, layer)] - ref[(name, layer)]).max() /
                                             np.abs(ref[(name, layer)]).max()) for name, layer in keep}
            cos = float(emu_pool @ ref_pool / np.linalg.norm(emu_pool) / np.linalg.norm(ref_pool))
            texts.append({"seed": seed, "length": n, "max_rel": errs, "pooled_cosine": cos})
            print(f"text {seed}/{n}: worst {max(errs.values()):.3e}, pooled cosine {cos:.9f}", file=sys.stderr)
    out = {"generator": "tests/golden/make_fp16_emulation.py", "model": "OUTLIER_NORMS", "spec": ge.OUTLIER_NORMS,
           "texts": texts}
    with open(os.path.join(HERE, "outlier_fp16_emulation.json"), "w") as f:
        json.dump(out, f, indent=0)


if __name__ == "__main__":
    main()
