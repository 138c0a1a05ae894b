"""Writes real_model_directory.json: the tensor directory and text-path metadata of the
reference's real weight file, taken from the reference's own fixture
(Tests/GemmaEmbedTests/Fixtures/model.json, the file GGUFReaderTests.swift:8-66 checks its GGUF
reader against). Data only: tensor names, ne shapes, types and data-section offsets, counts, and
the metadata values the text path reads. Run in a container that holds /root/reference.
"""
import json
import os
import sys

SRC = "/root/reference/Tests/GemmaEmbedTests/Fixtures/model.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "real_model_directory.json")

TEXT_KEYS = [
    "general.architecture", "gemma-embedding2.block_count", "gemma-embedding2.context_length",
    "gemma-embedding2.embedding_length", "gemma-embedding2.embedding_length_out",
    "gemma-embedding2.embedding_length_per_layer_input", "gemma-embedding2.feed_forward_length",
    "gemma-embedding2.attention.head_count", "gemma-embedding2.attention.head_count_kv",
    "gemma-embedding2.attention.sliding_window", "gemma-embedding2.attention.sliding_window_pattern",
    "gemma-embedding2.attention.key_length", "gemma-embedding2.attention.value_length",
    "gemma-embedding2.attention.key_length_swa", "gemma-embedding2.attention.value_length_swa",
    "gemma-embedding2.rope.freq_base", "gemma-embedding2.rope.freq_base_swa",
    "gemma-embedding2.attention.layer_norm_rms_epsilon", "tokenizer.ggml.bos_token_id", "tokenizer.ggml.eos_token_id",
]


def main():
    src = json.load(open(SRC))
    meta = {}
    for k in TEXT_KEYS:
        v = src["metadata"][k]
        meta[k] = v["items"] if "items" in v else v["value"]
    out = {
        "source": "reference Tests/GemmaEmbedTests/Fixtures/model.json (" + src["file"] + ")",
        "gguf_version": src["gguf_version"],
        "kv_count": src["kv_count"],
        "tensor_count": src["tensor_count"],
        "tensor_type_counts": src["tensor_type_counts"],
        "vocab_size": src["metadata"]["tokenizer.ggml.tokens"]["len"],
        "metadata": meta,
        "tensors": [[t["name"], t["shape_ne"], t["type"], t["offset"]] for t in src["tensors"]],
    }
    with open(OUT, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {OUT}: {len(out['tensors'])} tensors", file=sys.stderr)


if __name__ == "__main__":
    main()
