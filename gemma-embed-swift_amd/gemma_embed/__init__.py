"""ctypes binding of libgemmaembed.so, the MI355X GemmaEmbed text-encoder library.

Mirrors the reference's Swift API names (Sources/GemmaEmbed/EmbeddingModel.swift):
``EmbeddingModel.load`` / ``embed`` / ``embed_tokens`` / ``similarity``, ``EmbedOptions``,
``plan_batches`` (EmbeddingModel.batches) and ``finish``. Errors raise ``GemmaEmbedError``
carrying the C status code (Errors.swift:6-24). Compute always runs in the native library: when
``libgemmaembed.so`` is missing, importing this module raises instead of falling back.
"""
from __future__ import annotations

import ctypes as C
import itertools
import os
from dataclasses import dataclass
from typing import Callable, Iterable, List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# GE_LIBRARY names another build of the same library (the sanitizer build the CPU tests load).
LIB_PATH = os.environ.get("GE_LIBRARY") or os.path.join(os.path.dirname(_HERE), "libgemmaembed.so")

GE_OK = 0
ERRORS = {
    1: "invalid",
    2: "invalidGGUF",
    3: "model",
    4: "gpuFailure",
    5: "invalidOptions",
    6: "state",
    7: "cancelled",
    8: "noDevice",
}
(GE_ERR_INVALID, GE_ERR_GGUF, GE_ERR_MODEL, GE_ERR_GPU, GE_ERR_OPTIONS, GE_ERR_STATE, GE_ERR_CANCELLED,
 GE_ERR_NO_DEVICE) = range(1, 9)
GE_TYPE_F32, GE_TYPE_F16, GE_TYPE_Q8_0, GE_TYPE_BF16 = 0, 1, 8, 30


class GemmaEmbedError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{ERRORS.get(code, code)}] {message}")
        self.code = code
        self.kind = ERRORS.get(code, str(code))
        self.message = message


class ge_seq(C.Structure):
    _fields_ = [("start", C.c_uint32), ("length", C.c_uint32)]


class ge_attention_work(C.Structure):
    _fields_ = [("seq_start", C.c_uint32), ("seq_len", C.c_uint32), ("q0", C.c_uint32)]


class ge_load_options(C.Structure):
    _fields_ = [("device", C.c_int32), ("batch_token_budget", C.c_int32), ("warm_up", C.c_int32),
                ("split_scores", C.c_int32), ("pack_tokens", C.c_int32)]


class ge_embed_options(C.Structure):
    _fields_ = [("max_tokens", C.c_int32), ("dimensions", C.c_int32), ("normalise", C.c_int32),
                ("batch_size", C.c_int32)]


class ge_tensor_desc(C.Structure):
    _fields_ = [("name", C.c_char_p), ("offset", C.c_uint64), ("type", C.c_int32), ("ndim", C.c_int32),
                ("shape", C.c_int64 * 4)]


class ge_model_info(C.Structure):
    _fields_ = [("architecture", C.c_char * 64), ("name", C.c_char * 128),
                ("layers", C.c_int32), ("hidden", C.c_int32), ("out_dims", C.c_int32),
                ("feed_forward", C.c_int32), ("per_layer_input", C.c_int32), ("heads", C.c_int32),
                ("vocab", C.c_int32), ("sliding_window", C.c_int32), ("max_tokens", C.c_int32),
                ("eps", C.c_float), ("quantization", C.c_char * 16), ("device_name", C.c_char * 128),
                ("file_size", C.c_int64), ("bos_id", C.c_int32), ("eos_id", C.c_int32)]


class ge_synth_spec(C.Structure):
    _fields_ = [("layers", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32),
                ("feed_forward", C.c_int32), ("out_dims", C.c_int32), ("per_layer_input", C.c_int32),
                ("vocab", C.c_int32), ("sliding_window", C.c_int32), ("head_dim_swa", C.c_int32),
                ("head_dim_global", C.c_int32), ("kv_heads_swa", C.c_int32), ("kv_heads_global", C.c_int32),
                ("eps", C.c_float), ("rope_base", C.c_float), ("rope_base_swa", C.c_float),
                ("pattern", C.POINTER(C.c_uint8)), ("seed", C.c_uint64), ("context_length", C.c_int32),
                ("norm_outliers", C.c_int32), ("norm_outlier", C.c_float)]


class ge_vision_info(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("layers", "hidden", "heads", "patch_size", "patch_area", "merge",
                                          "proj_dims", "positions")]


class ge_synth_vision_spec(C.Structure):
    _fields_ = [("layers", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32),
                ("feed_forward", C.c_int32), ("patch_size", C.c_int32), ("merge", C.c_int32),
                ("proj_dims", C.c_int32), ("positions", C.c_int32), ("eps", C.c_float),
                ("ffn_down_type", C.c_int32), ("seed", C.c_uint64)]


class ge_image_grid(C.Structure):
    _fields_ = [("grid_x", C.c_int32), ("grid_y", C.c_int32)]


PROGRESS_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32, C.c_int32, C.c_int64)

# Every symbol include/gemmaembed.h declares, with its ctypes signature.
_P = C.c_void_p
_I = C.c_int
_PI32 = C.POINTER(C.c_int32)
_PF = C.POINTER(C.c_float)
SIGNATURES = {
    "ge_create": (_I, [C.c_int, C.POINTER(_P)]),
    "ge_destroy": (None, [_P]),
    "ge_last_error": (C.c_char_p, [_P]),
    "ge_create_error": (C.c_char_p, []),
    "ge_device_name": (C.c_char_p, [_P]),
    "ge_upload_model": (_I, [_P, _P, _P, C.c_size_t]),
    "ge_set_split_scores": (_I, [_P, C.c_int32]),
    "ge_forward": (_I, [_P, _PI32, _PI32, C.c_int32, C.POINTER(ge_seq), C.c_int32, _PF, C.POINTER(C.c_double)]),
    "ge_forward_trace": (_I, [_P, _PI32, _PI32, C.c_int32, C.POINTER(ge_seq), C.c_int32, C.c_char_p, C.c_int32,
                              _PF, C.c_size_t, C.POINTER(C.c_size_t)]),
    "ge_batch_stage": (_I, [_P, _PI32, _PI32, C.c_int32, C.POINTER(ge_seq), C.c_int32]),
    "ge_batch_run": (_I, [_P]),
    "ge_batch_read": (_I, [_P, _PF]),
    "ge_sync": (_I, [_P]),
    "ge_profile_enable": (_I, [_P, C.c_char_p]),
    "ge_profile_disable": (_I, [_P]),
    "ge_profile_reset": (_I, [_P]),
    "ge_profile_get": (_I, [_P, C.c_int32, C.POINTER(C.c_char_p), C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
    "ge_dev_alloc": (_P, [_P, C.c_size_t]),
    "ge_dev_free": (_I, [_P, _P]),
    "ge_dev_upload": (_I, [_P, _P, _P, C.c_size_t]),
    "ge_dev_download": (_I, [_P, _P, _P, C.c_size_t]),
    "ge_op_f32_to_f16": (_I, [_P, _P, _P, C.c_size_t]),
    "ge_op_f16_to_f32": (_I, [_P, _P, _P, C.c_size_t]),
    "ge_op_q8_create": (_I, [_P, _P, C.c_int32, C.c_int32, C.POINTER(_P)]),
    "ge_op_q8_destroy": (_I, [_P, _P]),
    "ge_op_gemm_q8": (_I, [_P, _P, _P, C.c_int32, _P, C.c_int32]),
    "ge_op_gemm_q8_geglu": (_I, [_P, _P, _P, _P, C.c_int32, _P]),
    "ge_attention_queries": (C.c_int32, []),
    "ge_op_attention": (_I, [_P, _P, _P, _P, _P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                             C.c_float]),
    "ge_forward_noalloc": (_I, [_P, _PI32, _PI32, C.c_int32, C.POINTER(ge_seq), C.c_int32, _PF,
                                C.POINTER(C.c_double)]),
    "ge_op_rmsnorm": (_I, [_P, _P, _P, _P, C.c_int32, C.c_int32, C.c_float, C.c_float]),
    "ge_op_rmsnorm_residual": (_I, [_P, _P, _P, _P, C.c_float, _P, _P, C.c_int32, C.c_int32, C.c_float]),
    "ge_op_qk_norm_rope": (_I, [_P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _P, _P, C.c_float, _P, C.c_float,
                                _P, _P, _P]),
    "ge_op_embed": (_I, [_P, _P, _P, C.c_int32, C.c_float, _P, C.c_int32, _P, C.c_float, _P, _P]),
    "ge_op_mean_pool": (_I, [_P, _P, C.c_int32, C.c_int32, _P, C.c_int32, _P]),
    "ge_op_attention_split": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                   C.c_int32, C.c_float]),
    "ge_model_load": (_I, [C.c_char_p, C.POINTER(ge_load_options), C.POINTER(_P), C.c_char_p, C.c_size_t]),
    "ge_gguf_open": (_I, [C.c_char_p, C.POINTER(_P), C.c_char_p, C.c_size_t]),
    "ge_gguf_close": (None, [_P]),
    "ge_gguf_counts": (_I, [_P, C.POINTER(C.c_uint32), C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                            C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "ge_gguf_tensor": (_I, [_P, C.c_int64, C.POINTER(ge_tensor_desc)]),
    "ge_gguf_text_config": (_I, [_P, C.POINTER(ge_model_info), C.c_char_p, C.c_size_t]),
    "ge_model_free": (None, [_P]),
    "ge_model_last_error": (C.c_char_p, [_P]),
    "ge_model_get_info": (_I, [_P, C.POINTER(ge_model_info)]),
    "ge_model_context": (_P, [_P]),
    "ge_model_embed": (_I, [_P, _PI32, _PI32, C.c_int32, C.POINTER(ge_embed_options), _PF, _PI32,
                            C.POINTER(C.c_uint8), PROGRESS_FN, _P]),
    "ge_model_embed_tokens": (_I, [_P, _PI32, _PI32, C.c_int32, _PF]),
    "ge_plan_batches": (_I, [_PI32, C.c_int32, _PI32, C.c_int32, C.c_int32, _PI32, _PI32]),
    "ge_finish": (_I, [_PF, C.c_int32, C.c_int32, C.c_int32, _PF]),
    "ge_synth_write_gguf": (_I, [C.c_char_p, C.POINTER(ge_synth_spec), C.c_char_p, C.c_size_t]),
    "ge_synth_tokens": (_I, [C.c_uint64, C.c_int32, C.c_int32, C.c_int32, _PI32]),
    "ge_synth_uniform": (_I, [C.c_uint64, C.c_float, C.c_float, C.c_int64, _PF]),
    "ge_synth_write_vision_gguf": (_I, [C.c_char_p, C.POINTER(ge_synth_vision_spec), C.c_char_p, C.c_size_t]),
    "ge_upload_vision": (_I, [_P, _P, _P, C.c_size_t]),
    "ge_vision_load": (_I, [_P, C.c_char_p, C.c_char_p, C.c_size_t]),
    "ge_vision_encode": (_I, [_P, _PF, C.c_int32, C.POINTER(ge_image_grid), C.c_int32, _PF, C.c_size_t,
                              C.POINTER(C.c_double)]),
    "ge_vision_get_info": (_I, [_P, C.POINTER(ge_vision_info)]),
    "ge_image_forward": (_I, [_P, _PF, C.c_int32, C.POINTER(ge_image_grid), C.c_int32, _PI32, _PF,
                              C.POINTER(C.c_double)]),
    "ge_set_vectors": (_I, [_P, _PF, C.c_int32, C.c_int32]),
    "ge_vision_stage": (_I, [_P, _PF, C.c_int32, C.POINTER(ge_image_grid), C.c_int32]),
    "ge_vision_run": (_I, [_P]),
    "ge_vision_read": (_I, [_P, _PF, C.c_size_t]),
    "ge_vision_tokens": (C.c_int32, [_P]),
    "ge_vision_trace": (_I, [_P, _PF, C.c_int32, C.POINTER(ge_image_grid), C.c_int32, C.c_char_p, C.c_int32, _PF,
                             C.c_size_t, C.POINTER(C.c_size_t)]),
}


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C gemma-embed-swift_amd)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _flat_i32(sequences) -> np.ndarray:
    """The sequences' ids back to back as int32 (out-of-range ids raise OverflowError)."""
    n = sum(len(s) for s in sequences)
    return np.fromiter(itertools.chain.from_iterable(sequences), dtype=np.int32, count=n)


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


# ---------------------------------------------------------------------------- pure host helpers

def plan_batches(costs: Sequence[Sequence[int]] | Sequence[int], budgets: Sequence[int],
                 batch_size: Optional[int] = None) -> List[range]:
    """EmbeddingModel.batches (EmbeddingModel.swift:200-215) through the native implementation."""
    c = np.asarray(costs, dtype=np.int32)
    if c.ndim == 1:
        c = c.reshape(-1, 1)
    n = c.shape[0] if c.size else 0
    b = _i32(budgets)
    if c.size == 0:
        c = np.zeros((0, len(b)), dtype=np.int32)
    c = np.ascontiguousarray(c)
    starts = np.zeros(n + 1, dtype=np.int32)
    nr = C.c_int32(0)
    rc = lib.ge_plan_batches(_ptr(c, C.c_int32), n, _ptr(b, C.c_int32), len(b), int(batch_size or 0),
                             _ptr(starts, C.c_int32), C.byref(nr))
    if rc != GE_OK:
        raise GemmaEmbedError(rc, "ge_plan_batches")
    return [range(int(starts[i]), int(starts[i + 1])) for i in range(nr.value)]


def finish(vector: np.ndarray, dimensions: int, normalise: bool = True) -> np.ndarray:
    """EmbeddingModel.finish (EmbeddingModel.swift:260-267)."""
    v = np.ascontiguousarray(vector, dtype=np.float32)
    out = np.zeros(dimensions, dtype=np.float32)
    rc = lib.ge_finish(_ptr(v, C.c_float), v.size, dimensions, int(normalise), _ptr(out, C.c_float))
    if rc != GE_OK:
        raise GemmaEmbedError(rc, "ge_finish: dimensions out of range")
    return out


def synth_tokens(seed: int, lo: int, hi: int, count: int) -> np.ndarray:
    out = np.zeros(count, dtype=np.int32)
    rc = lib.ge_synth_tokens(seed, lo, hi, count, _ptr(out, C.c_int32))
    if rc != GE_OK:
        raise GemmaEmbedError(rc, "ge_synth_tokens")
    return out


# Synthetic model shapes. CONFIG2 is BASELINE.json's "Gemma-3-style" encoder (configs 2-4):
# 24 layers, d 768, 3 query heads / 1 KV head of 256, GeGLU 1152, window 512, global layers at
# 5, 11, 17, 23 with RoPE base 1e6 (sliding 1e4), vocab 262144, output 768, no per-layer input.
CONFIG2 = dict(layers=24, hidden=768, heads=3, feed_forward=1152, out_dims=768, per_layer_input=0,
               vocab=262144, sliding_window=512, head_dim_swa=256, head_dim_global=256, kv_heads_swa=1,
               kv_heads_global=1, eps=1e-6, rope_base=1e6, rope_base_swa=1e4,
               pattern=[1, 1, 1, 1, 1, 0] * 4, seed=4)
# A two-layer model small enough for brute-force float64 checks.
TINY = dict(layers=2, hidden=128, heads=2, feed_forward=256, out_dims=128, per_layer_input=0, vocab=512,
            sliding_window=16, head_dim_swa=128, head_dim_global=128, kv_heads_swa=1, kv_heads_global=1,
            eps=1e-6, rope_base=1e6, rope_base_swa=1e4, pattern=[1, 0], seed=7)
# The same with the per-layer-input branch (64-wide per-layer inputs).
TINY_PLE = dict(TINY, per_layer_input=64, heads=2, kv_heads_swa=1, kv_heads_global=1, seed=9)
# Config 2's shapes over 6 layers (one global) with norm weights carrying outliers of 50 to 300,
# as trained models' residual-stream norms do: stresses the fp16 range scales chosen at load.
OUTLIER_NORMS = dict(CONFIG2, layers=6, pattern=[1, 1, 1, 1, 1, 0], norm_outliers=4, norm_outlier=300.0, seed=21)
# The reference's real architecture (Model/Architecture.md:7-9, Fixtures/model.json): d 512, 4 query
# heads, sliding layers of 2 KV heads of 256 (window 1024, RoPE 1e4), global layers 5, 11, 17, 23 of
# 1 KV head of 512 (RoPE 1e6), GeGLU 2048, per-layer inputs of 512, output 768; synthetic weights.
REAL_SHAPES = dict(layers=24, hidden=512, heads=4, feed_forward=2048, out_dims=768, per_layer_input=512,
                   vocab=262144, sliding_window=1024, head_dim_swa=256, head_dim_global=512, kv_heads_swa=2,
                   kv_heads_global=1, eps=1e-6, rope_base=1e6, rope_base_swa=1e4,
                   pattern=[1, 1, 1, 1, 1, 0] * 4, seed=12)


def synth_write_gguf(path: str, **spec) -> str:
    """Writes a seeded synthetic gemma-embedding2 GGUF (see ge_synth_write_gguf)."""
    pattern = np.ascontiguousarray(spec["pattern"], dtype=np.uint8)
    s = ge_synth_spec()
    for k in ("layers", "hidden", "heads", "feed_forward", "out_dims", "per_layer_input", "vocab",
              "sliding_window", "head_dim_swa", "head_dim_global", "kv_heads_swa", "kv_heads_global"):
        setattr(s, k, int(spec[k]))
    s.eps, s.rope_base, s.rope_base_swa = spec["eps"], spec["rope_base"], spec["rope_base_swa"]
    s.pattern = _ptr(pattern, C.c_uint8)
    s.seed = int(spec["seed"])
    s.context_length = int(spec.get("context_length", 0))
    s.norm_outliers = int(spec.get("norm_outliers", 0))
    s.norm_outlier = float(spec.get("norm_outlier", 0.0))
    err = C.create_string_buffer(512)
    rc = lib.ge_synth_write_gguf(path.encode(), C.byref(s), err, 512)
    if rc != GE_OK:
        raise GemmaEmbedError(rc, err.value.decode())
    return path


# BASELINE config 5's image tower, and a two-layer version of it with small grids for tests.
CONFIG5_VISION = dict(layers=16, hidden=1152, heads=16, feed_forward=4304, patch_size=16, merge=3, proj_dims=768,
                      positions=48, eps=1e-6, ffn_down_type=0, seed=5)
TINY_VISION = dict(CONFIG5_VISION, layers=2, positions=12, seed=11)


def synth_write_vision_gguf(path: str, **spec) -> str:
    """Writes a seeded synthetic image-encoder GGUF (see ge_synth_write_vision_gguf)."""
    s = ge_synth_vision_spec()
    for k in ("layers", "hidden", "heads", "feed_forward", "patch_size", "merge", "proj_dims", "positions",
              "ffn_down_type"):
        setattr(s, k, int(spec.get(k, 0)))
    s.eps = float(spec["eps"])
    s.seed = int(spec["seed"])
    err = C.create_string_buffer(512)
    rc = lib.ge_synth_write_vision_gguf(path.encode(), C.byref(s), err, 512)
    if rc != GE_OK:
        raise GemmaEmbedError(rc, err.value.decode())
    return path


def synth_uniform(seed: int, lo: float, hi: float, count: int) -> np.ndarray:
    out = np.zeros(count, dtype=np.float32)
    rc = lib.ge_synth_uniform(seed, lo, hi, count, _ptr(out, C.c_float))
    if rc != GE_OK:
        raise GemmaEmbedError(rc, "ge_synth_uniform")
    return out


def image_patches(seed: int, grids: Sequence[Tuple[int, int]], area: int) -> np.ndarray:
    """Synthetic pixels uniform in [-1, 1) as patch rows [sum(gx * gy), area]."""
    n = sum(gx * gy for gx, gy in grids)
    return synth_uniform(seed, -1.0, 1.0, n * area).reshape(n, area)


def _grid_array(grids) -> C.Array:
    arr = (ge_image_grid * max(len(grids), 1))()
    for i, (gx, gy) in enumerate(grids):
        arr[i].grid_x, arr[i].grid_y = int(gx), int(gy)
    return arr


# ---------------------------------------------------------------------------- device context

def pack(sequences: Sequence[Sequence[int]]):
    """PackedBatch.append (Metal/MetalForward.swift:17-21): ids back to back, positions from 0."""
    lengths = [len(s) for s in sequences]
    seqs, start = [], 0
    for n in lengths:
        seqs.append((start, n))
        start += n
    pos = np.concatenate([np.arange(n, dtype=np.int32) for n in lengths]) if lengths else np.zeros(0, np.int32)
    return _flat_i32(sequences), pos, seqs


def _seq_array(seqs) -> C.Array:
    arr = (ge_seq * max(len(seqs), 1))()
    for i, (st, ln) in enumerate(seqs):
        arr[i].start, arr[i].length = st, ln
    return arr


class Context:
    """A device context (ge_ctx). Owned contexts are destroyed on close(); borrowed ones
    (a loaded model's) are not."""

    def __init__(self, handle: int, owned: bool, out_dims: int = 0):
        self.handle = C.c_void_p(handle)
        self.owned = owned
        self.out_dims = out_dims

    @classmethod
    def create(cls, device: int = 0) -> "Context":
        h = C.c_void_p()
        rc = lib.ge_create(device, C.byref(h))
        if rc != GE_OK:
            raise GemmaEmbedError(rc, lib.ge_create_error().decode())
        return cls(h.value, True)

    def close(self):
        if self.owned and self.handle:
            lib.ge_destroy(self.handle)
        self.handle = C.c_void_p()

    def _check(self, rc: int, what: str):
        if rc != GE_OK:
            raise GemmaEmbedError(rc, f"{what}: {lib.ge_last_error(self.handle).decode()}")

    @property
    def device_name(self) -> str:
        return lib.ge_device_name(self.handle).decode()

    def forward_noalloc(self, sequences: Sequence[Sequence[int]]):
        """ge_forward_noalloc: as forward(), with no device allocation (the library's scratch array)."""
        toks, pos, seqs = pack(sequences)
        out = np.zeros((len(seqs), self.out_dims), dtype=np.float32)
        secs = C.c_double(0)
        self._check(lib.ge_forward_noalloc(self.handle, _ptr(toks, C.c_int32), _ptr(pos, C.c_int32), len(toks),
                                           _seq_array(seqs), len(seqs), _ptr(out, C.c_float), C.byref(secs)),
                    "ge_forward_noalloc")
        return out, secs.value

    def forward(self, sequences: Sequence[Sequence[int]]):
        """One packed batch -> (pooled [n_seqs, out_dims], gpu_seconds)."""
        toks, pos, seqs = pack(sequences)
        out = np.zeros((len(seqs), self.out_dims), dtype=np.float32)
        secs = C.c_double(0)
        self._check(lib.ge_forward(self.handle, _ptr(toks, C.c_int32), _ptr(pos, C.c_int32), len(toks),
                                   _seq_array(seqs), len(seqs), _ptr(out, C.c_float), C.byref(secs)), "ge_forward")
        return out, secs.value

    def trace(self, sequences: Sequence[Sequence[int]], name: str, layer: int = -1) -> np.ndarray:
        """The named intermediate (llama.cpp names) over the packed tokens, fp32 [T, width]."""
        toks, pos, seqs = pack(sequences)
        need = C.c_size_t(0)
        sa = _seq_array(seqs)
        self._check(lib.ge_forward_trace(self.handle, _ptr(toks, C.c_int32), _ptr(pos, C.c_int32), len(toks), sa,
                                         len(seqs), name.encode(), layer, None, 0, C.byref(need)), "ge_forward_trace")
        out = np.zeros(need.value, dtype=np.float32)
        self._check(lib.ge_forward_trace(self.handle, _ptr(toks, C.c_int32), _ptr(pos, C.c_int32), len(toks), sa,
                                         len(seqs), name.encode(), layer, _ptr(out, C.c_float), out.size,
                                         C.byref(need)), "ge_forward_trace")
        return out.reshape(len(toks), -1)

    # ---- image tower
    def vision_load(self, path: str):
        err = C.create_string_buffer(512)
        rc = lib.ge_vision_load(self.handle, path.encode(), err, 512)
        if rc != GE_OK:
            raise GemmaEmbedError(rc, err.value.decode())

    def vision_info(self) -> "ge_vision_info":
        """The uploaded tower's shapes (patch area, merge size, projection width, ...)."""
        info = ge_vision_info()
        self._check(lib.ge_vision_get_info(self.handle, C.byref(info)), "ge_vision_get_info")
        return info

    def _patches(self, patches: np.ndarray) -> Tuple[np.ndarray, "ge_vision_info"]:
        info = self.vision_info()
        p = np.ascontiguousarray(patches, dtype=np.float32)
        if p.ndim != 2 or p.shape[1] != info.patch_area:
            raise GemmaEmbedError(GE_ERR_INVALID, f"patches of shape {p.shape}: the tower takes rows of "
                                                  f"{info.patch_area} floats")
        return p, info

    def vision_encode(self, patches: np.ndarray, grids: Sequence[Tuple[int, int]], proj_dims: Optional[int] = None,
                      merge: Optional[int] = None):
        """Patches [P, area] of images with the given grids -> (vectors [tokens, proj_dims], gpu_seconds).
        The output is sized from the loaded tower; proj_dims and merge, when given, must match it."""
        p, info = self._patches(patches)
        if (proj_dims is not None and proj_dims != info.proj_dims) or (merge is not None and merge != info.merge):
            raise GemmaEmbedError(GE_ERR_INVALID, f"the tower has merge {info.merge} and {info.proj_dims}-wide vectors")
        tokens = sum((gx // info.merge) * (gy // info.merge) for gx, gy in grids)
        out = np.zeros((tokens, info.proj_dims), dtype=np.float32)
        secs = C.c_double(0)
        self._check(lib.ge_vision_encode(self.handle, _ptr(p, C.c_float), p.shape[0], _grid_array(grids), len(grids),
                                         _ptr(out, C.c_float), out.size, C.byref(secs)), "ge_vision_encode")
        return out, secs.value

    def image_forward(self, patches: np.ndarray, grids: Sequence[Tuple[int, int]], markers: Sequence[int]):
        """Image tower, then the text tower over [bos, begin, vectors, end, eos] per image ->
        (pooled [images, out_dims] unnormalised, gpu_seconds of both towers)."""
        p, _ = self._patches(patches)
        mk = np.ascontiguousarray(markers, dtype=np.int32)
        if mk.size != 4:
            raise GemmaEmbedError(GE_ERR_INVALID, "four marker ids: bos, image begin, image end, eos")
        out = np.zeros((len(grids), self.out_dims), dtype=np.float32)
        secs = C.c_double(0)
        self._check(lib.ge_image_forward(self.handle, _ptr(p, C.c_float), p.shape[0], _grid_array(grids), len(grids),
                                         _ptr(mk, C.c_int32), _ptr(out, C.c_float), C.byref(secs)), "ge_image_forward")
        return out, secs.value

    def set_vectors(self, rows: np.ndarray):
        """Vector rows [n, hidden] fp32 for the negative ids of later batches (-(r + 1) is row r)."""
        v = np.ascontiguousarray(rows, dtype=np.float32)
        v2 = v.reshape(v.shape[0], -1) if v.size else v.reshape(0, 0)
        self._check(lib.ge_set_vectors(self.handle, _ptr(v2, C.c_float) if v2.size else None, v2.shape[0],
                                       v2.shape[1] if v2.ndim == 2 else 0), "ge_set_vectors")

    def vision_trace(self, patches: np.ndarray, grids: Sequence[Tuple[int, int]], name: str, layer: int = -1):
        p, _ = self._patches(patches)
        ga = _grid_array(grids)
        need = C.c_size_t(0)
        self._check(lib.ge_vision_trace(self.handle, _ptr(p, C.c_float), p.shape[0], ga, len(grids), name.encode(),
                                        layer, None, 0, C.byref(need)), "ge_vision_trace")
        out = np.zeros(need.value, dtype=np.float32)
        self._check(lib.ge_vision_trace(self.handle, _ptr(p, C.c_float), p.shape[0], ga, len(grids), name.encode(),
                                        layer, _ptr(out, C.c_float), out.size, C.byref(need)), "ge_vision_trace")
        return out

    def vision_stage(self, patches: np.ndarray, grids: Sequence[Tuple[int, int]]):
        p, _ = self._patches(patches)
        self._check(lib.ge_vision_stage(self.handle, _ptr(p, C.c_float), p.shape[0], _grid_array(grids), len(grids)),
                    "ge_vision_stage")

    def vision_run(self):
        self._check(lib.ge_vision_run(self.handle), "ge_vision_run")

    def vision_read(self, proj_dims: Optional[int] = None) -> np.ndarray:
        info = self.vision_info()
        if proj_dims is not None and proj_dims != info.proj_dims:
            raise GemmaEmbedError(GE_ERR_INVALID, f"the tower's vectors are {info.proj_dims} wide")
        n = lib.ge_vision_tokens(self.handle)
        out = np.zeros((max(n, 0), info.proj_dims), dtype=np.float32)
        self._check(lib.ge_vision_read(self.handle, _ptr(out, C.c_float), out.size), "ge_vision_read")
        return out

    def batch_stage(self, sequences: Sequence[Sequence[int]]):
        toks, pos, seqs = pack(sequences)
        self._check(lib.ge_batch_stage(self.handle, _ptr(toks, C.c_int32), _ptr(pos, C.c_int32), len(toks),
                                       _seq_array(seqs), len(seqs)), "ge_batch_stage")
        self._staged = len(seqs)

    def batch_run(self):
        self._check(lib.ge_batch_run(self.handle), "ge_batch_run")

    def batch_read(self) -> np.ndarray:
        out = np.zeros((self._staged, self.out_dims), dtype=np.float32)
        self._check(lib.ge_batch_read(self.handle, _ptr(out, C.c_float)), "ge_batch_read")
        return out

    def sync(self):
        self._check(lib.ge_sync(self.handle), "ge_sync")

    def profile_enable(self, prefix: str = ""):
        self._check(lib.ge_profile_enable(self.handle, prefix.encode()), "ge_profile_enable")

    def profile_disable(self):
        self._check(lib.ge_profile_disable(self.handle), "ge_profile_disable")

    def profile_reset(self):
        self._check(lib.ge_profile_reset(self.handle), "ge_profile_reset")

    def profile_stats(self) -> dict:
        stats, i = {}, 0
        while True:
            name, n, ms = C.c_char_p(), C.c_int64(), C.c_double()
            if lib.ge_profile_get(self.handle, i, C.byref(name), C.byref(n), C.byref(ms)) != GE_OK:
                break
            stats[name.value.decode()] = (n.value, ms.value)
            i += 1
        return stats

    # -- device memory and per-op entry points
    def alloc(self, nbytes: int) -> int:
        p = lib.ge_dev_alloc(self.handle, nbytes)
        if not p:
            raise GemmaEmbedError(4, f"ge_dev_alloc: {lib.ge_last_error(self.handle).decode()}")
        return p

    def free(self, p: int):
        self._check(lib.ge_dev_free(self.handle, C.c_void_p(p)), "ge_dev_free")

    def upload(self, p: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self._check(lib.ge_dev_upload(self.handle, C.c_void_p(p), a.ctypes.data_as(C.c_void_p), a.nbytes),
                    "ge_dev_upload")

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.zeros(shape, dtype=dtype)
        self._check(lib.ge_dev_download(self.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(p), out.nbytes),
                    "ge_dev_download")
        return out

    def f32_to_f16(self, src: int, dst: int, n: int):
        self._check(lib.ge_op_f32_to_f16(self.handle, C.c_void_p(src), C.c_void_p(dst), n), "ge_op_f32_to_f16")

    def f16_to_f32(self, src: int, dst: int, n: int):
        self._check(lib.ge_op_f16_to_f32(self.handle, C.c_void_p(src), C.c_void_p(dst), n), "ge_op_f16_to_f32")

    def q8_create(self, rows_q8: np.ndarray, rows: int, cols: int) -> int:
        h = C.c_void_p()
        b = np.ascontiguousarray(rows_q8, dtype=np.uint8)
        self._check(lib.ge_op_q8_create(self.handle, b.ctypes.data_as(C.c_void_p), rows, cols, C.byref(h)),
                    "ge_op_q8_create")
        return h.value

    def q8_destroy(self, h: int):
        self._check(lib.ge_op_q8_destroy(self.handle, C.c_void_p(h)), "ge_op_q8_destroy")

    def gemm_q8(self, w: int, x: int, m: int, y: int, y_f16: bool = False):
        self._check(lib.ge_op_gemm_q8(self.handle, C.c_void_p(w), C.c_void_p(x), m, C.c_void_p(y), int(y_f16)),
                    "ge_op_gemm_q8")

    def gemm_q8_geglu(self, gate: int, up: int, x: int, m: int, act: int):
        self._check(lib.ge_op_gemm_q8_geglu(self.handle, C.c_void_p(gate), C.c_void_p(up), C.c_void_p(x), m,
                                            C.c_void_p(act)), "ge_op_gemm_q8_geglu")

    def attention(self, q: int, k: int, v: int, out: int, work: int, n_work: int, heads: int, kv_heads: int,
                  head_dim: int, half_window: int, scale: float = 1.0):
        self._check(lib.ge_op_attention(self.handle, C.c_void_p(q), C.c_void_p(k), C.c_void_p(v), C.c_void_p(out),
                                        C.c_void_p(work), n_work, heads, kv_heads, head_dim, half_window, scale),
                    "ge_op_attention")

    # ---- the forward's row kernels on device memory (pointers from alloc)
    def rmsnorm(self, x: int, out: int, w: Optional[int], rows: int, width: int, eps: float, pre_scale: float = 1.0):
        self._check(lib.ge_op_rmsnorm(self.handle, C.c_void_p(x), C.c_void_p(out), C.c_void_p(w) if w else None, rows,
                                      width, eps, pre_scale), "ge_op_rmsnorm")

    def rmsnorm_residual(self, x: int, t16: int, w: int, scale: float, next_w: Optional[int], h16: Optional[int],
                         rows: int, width: int, eps: float):
        self._check(lib.ge_op_rmsnorm_residual(self.handle, C.c_void_p(x), C.c_void_p(t16), C.c_void_p(w), scale,
                                               C.c_void_p(next_w) if next_w else None,
                                               C.c_void_p(h16) if h16 else None, rows, width, eps),
                    "ge_op_rmsnorm_residual")

    def qk_norm_rope(self, qkv: int, tokens: int, heads: int, kv_heads: int, head_dim: int, q_norm: int, k_norm: int,
                     eps: float, positions: int, rope_base: float, q: int, k: int, v: int):
        self._check(lib.ge_op_qk_norm_rope(self.handle, C.c_void_p(qkv), tokens, heads, kv_heads, head_dim,
                                           C.c_void_p(q_norm), C.c_void_p(k_norm), eps, C.c_void_p(positions), rope_base,
                                           C.c_void_p(q), C.c_void_p(k), C.c_void_p(v)), "ge_op_qk_norm_rope")

    def embed(self, table, tokens: int, n_tokens: int, scale: float, vectors: Optional[int], n_vectors: int,
              norm_w: Optional[int], eps: float, x: int, h16: Optional[int]):
        self._check(lib.ge_op_embed(self.handle, table, C.c_void_p(tokens), n_tokens, scale,
                                    C.c_void_p(vectors) if vectors else None, n_vectors,
                                    C.c_void_p(norm_w) if norm_w else None, eps, C.c_void_p(x),
                                    C.c_void_p(h16) if h16 else None), "ge_op_embed")

    def mean_pool(self, x: int, rows: int, width: int, seqs: int, n_seqs: int, pooled: int):
        self._check(lib.ge_op_mean_pool(self.handle, C.c_void_p(x), rows, width, C.c_void_p(seqs), n_seqs,
                                        C.c_void_p(pooled)), "ge_op_mean_pool")

    def attention_split(self, q: int, q_lo: int, k: int, k_lo: int, v: int, out: int, work: int, n_work: int,
                        heads: int, kv_heads: int, head_dim: int, half_window: int, scale: float = 1.0):
        """Split-precision scores: q and k as fp16 (hi, lo) pairs in device memory."""
        self._check(lib.ge_op_attention_split(self.handle, C.c_void_p(q), C.c_void_p(q_lo), C.c_void_p(k),
                                              C.c_void_p(k_lo), C.c_void_p(v), C.c_void_p(out), C.c_void_p(work),
                                              n_work, heads, kv_heads, head_dim, half_window, scale),
                    "ge_op_attention_split")


def attention_work(sequences_ranges, queries: Optional[int] = None) -> np.ndarray:
    """AttentionWork.items (Metal/MetalForward.swift:47-57) as a (n, 3) uint32 array."""
    q = queries or lib.ge_attention_queries()
    items = []
    for start, length in sequences_ranges:
        for q0 in range(0, length, q):
            items.append((start, length, q0))
    return np.asarray(items, dtype=np.uint32).reshape(-1, 3)


# ---------------------------------------------------------------------------- GGUF reader (host only)

class GgufFile:
    """The library's GGUF reader on its own (GGUFFile(url:), GGUF/GGUFFile.swift:21-67): counts, the
    tensor directory in file order, and the text configuration ModelConfig.init derives. No GPU."""

    TYPE_NAMES = {GE_TYPE_F32: "F32", GE_TYPE_F16: "F16", GE_TYPE_Q8_0: "Q8_0", GE_TYPE_BF16: "BF16"}

    def __init__(self, path: str):
        h = _P()
        err = C.create_string_buffer(512)
        rc = lib.ge_gguf_open(path.encode(), C.byref(h), err, 512)
        if rc != GE_OK:
            raise GemmaEmbedError(rc, err.value.decode())
        self.handle = h
        v, kv, nt, do, fs = C.c_uint32(), C.c_int64(), C.c_int64(), C.c_uint64(), C.c_uint64()
        lib.ge_gguf_counts(h, C.byref(v), C.byref(kv), C.byref(nt), C.byref(do), C.byref(fs))
        self.version, self.kv_count, self.tensor_count = v.value, kv.value, nt.value
        self.data_offset, self.file_size = do.value, fs.value

    def tensors(self) -> List[Tuple[str, List[int], str, int]]:
        """(name, ne shape, type name, offset in the data section) in file order."""
        out = []
        d = ge_tensor_desc()
        for i in range(self.tensor_count):
            rc = lib.ge_gguf_tensor(self.handle, i, C.byref(d))
            if rc != GE_OK:
                raise GemmaEmbedError(rc, f"tensor {i}")
            out.append((d.name.decode(), [int(d.shape[k]) for k in range(d.ndim)],
                        self.TYPE_NAMES.get(d.type, str(d.type)), int(d.offset)))
        return out

    def text_config(self) -> "ge_model_info":
        info = ge_model_info()
        err = C.create_string_buffer(512)
        rc = lib.ge_gguf_text_config(self.handle, C.byref(info), err, 512)
        if rc != GE_OK:
            raise GemmaEmbedError(rc, err.value.decode())
        return info

    def close(self):
        if self.handle:
            lib.ge_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


# ---------------------------------------------------------------------------- host API mirror

@dataclass
class EmbedOptions:
    """EmbedOptions (EmbedOptions.swift:35-56) minus the task prefix (applied before tokenizing)."""
    max_tokens: int = 2048
    dimensions: int = 768
    normalise: bool = True
    batch_size: Optional[int] = None

    allowed_dimensions = (768, 512, 256, 128)


@dataclass
class Embedding:
    """Embedding (EmbedOptions.swift:148-161)."""
    vector: np.ndarray
    token_count: int
    truncated: bool


@dataclass
class EmbeddingProgress:
    completed_texts: int
    total_texts: int
    completed_tokens: int


class EmbeddingModel:
    """EmbeddingModel (EmbeddingModel.swift:24-290) over pre-tokenized texts."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)
        info = ge_model_info()
        if lib.ge_model_get_info(self._h, C.byref(info)) != GE_OK:
            raise GemmaEmbedError(1, "ge_model_get_info")
        self.info = info
        self.context = Context(lib.ge_model_context(self._h), owned=False, out_dims=info.out_dims)

    @classmethod
    def load(cls, path: str, device: int = 0, batch_token_budget: int = 8192, warm_up: bool = True,
             split_scores: bool = False, pack_tokens: int = 0):
        """split_scores: hi/lo fp16 q and k (near-fp32 scores) on every layer whose query grouping
        allows it, not only the head-dim-512 ones (ge_set_split_scores). pack_tokens: largest
        device pack of embed(); 0 = the batch budget (one forward per planned batch)."""
        opt = ge_load_options(device, batch_token_budget, int(warm_up), int(split_scores), int(pack_tokens))
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        rc = lib.ge_model_load(path.encode(), C.byref(opt), C.byref(h), err, 1024)
        if rc != GE_OK:
            raise GemmaEmbedError(rc, err.value.decode())
        return cls(h.value)

    def close(self):
        if self._h:
            lib.ge_model_free(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _err(self, rc: int):
        raise GemmaEmbedError(rc, lib.ge_model_last_error(self._h).decode())

    def embed(self, texts: Sequence[Sequence[int]], options: EmbedOptions = EmbedOptions(),
              progress: Optional[Callable[[EmbeddingProgress], Optional[bool]]] = None) -> List[Embedding]:
        """embed(_:options:progress:) (EmbeddingModel.swift:145-175) over token id lists. A
        progress callback returning True cancels before the next batch."""
        lengths = _i32([len(t) for t in texts])
        flat = _flat_i32(texts)
        n = len(texts)
        out = np.zeros((max(n, 1), options.dimensions), dtype=np.float32)
        counts = np.zeros(max(n, 1), dtype=np.int32)
        cut = np.zeros(max(n, 1), dtype=np.uint8)
        opt = ge_embed_options(options.max_tokens, options.dimensions, int(options.normalise),
                               int(options.batch_size or 0))

        def cb(_user, done, total, tokens):
            if progress is None:
                return 0
            return 1 if progress(EmbeddingProgress(done, total, tokens)) else 0

        fn = PROGRESS_FN(cb)
        rc = lib.ge_model_embed(self._h, _ptr(flat, C.c_int32), _ptr(lengths, C.c_int32), n, C.byref(opt),
                                _ptr(out, C.c_float), _ptr(counts, C.c_int32), _ptr(cut, C.c_uint8), fn, None)
        if rc != GE_OK:
            self._err(rc)
        return [Embedding(out[i].copy(), int(counts[i]), bool(cut[i])) for i in range(n)]

    def embed_tokens(self, sequences: Sequence[Sequence[int]]) -> np.ndarray:
        """embedTokens (EmbeddingModel.swift:285-289): unnormalised pooled vectors, one batch."""
        lengths = _i32([len(t) for t in sequences])
        flat = _flat_i32(sequences)
        out = np.zeros((len(sequences), self.info.out_dims), dtype=np.float32)
        rc = lib.ge_model_embed_tokens(self._h, _ptr(flat, C.c_int32), _ptr(lengths, C.c_int32), len(sequences),
                                       _ptr(out, C.c_float))
        if rc != GE_OK:
            self._err(rc)
        return out

    @staticmethod
    def similarity(a: Embedding, b: Embedding) -> float:
        """Dot product over the shorter length (EmbeddingModel.swift:178-182)."""
        n = min(a.vector.size, b.vector.size)
        return float(np.dot(a.vector[:n].astype(np.float32), b.vector[:n].astype(np.float32)))
