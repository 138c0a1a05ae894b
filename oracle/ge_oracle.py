"""ctypes wrapper of the CPU oracle (oracle/libgeoracle.so).

TEST INFRASTRUCTURE ONLY: the checker of the HIP path and the timed CPU baseline. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it. It restates the
reference's Model/CPUReference.swift in C; see ge_oracle.c for the per-function citations.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Dict, Iterable, Optional, Tuple

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgeoracle.so")
TRACE_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_char_p, C.c_int, C.POINTER(C.c_float), C.c_size_t)

_F = C.POINTER(C.c_float)
_SIG = {
    "ora_open": (C.c_void_p, [C.c_char_p, C.c_char_p, C.c_int]),
    "ora_close": (None, [C.c_void_p]),
    "ora_hidden": (C.c_int, [C.c_void_p]),
    "ora_output_dims": (C.c_int, [C.c_void_p]),
    "ora_layers": (C.c_int, [C.c_void_p]),
    "ora_vocab": (C.c_int, [C.c_void_p]),
    "ora_forward": (C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int, _F, TRACE_FN, C.c_void_p, C.c_int]),
    "ora_forward_rows": (C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int, _F, C.c_int, _F, TRACE_FN, C.c_void_p,
                                   C.c_int]),
    "ora_dequant_row": (None, [C.c_int, C.c_void_p, C.c_int, _F]),
    "ora_half_to_float": (C.c_float, [C.c_uint16]),
    "ora_float_to_half": (C.c_uint16, [C.c_float]),
    "ora_matmul": (None, [_F, C.c_int, C.c_int, _F, C.c_int, _F, C.c_int]),
    "ora_rmsnorm": (None, [_F, C.c_int, C.c_int, _F, C.c_float, C.c_float, _F]),
    "ora_gelu_tanh": (C.c_float, [C.c_float]),
    "ora_rope_table": (None, [C.c_int, C.c_float, C.c_int, _F]),
    "ora_rope": (None, [_F, C.c_int, C.c_int, C.c_int, _F, C.POINTER(C.c_int32)]),
    "ora_attention": (None, [_F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, _F, C.c_int]),
    "ora_vision_open": (C.c_void_p, [C.c_char_p, C.c_char_p, C.c_int]),
    "ora_vision_close": (None, [C.c_void_p]),
    "ora_vision_hidden": (C.c_int, [C.c_void_p]),
    "ora_vision_proj_dims": (C.c_int, [C.c_void_p]),
    "ora_vision_merge": (C.c_int, [C.c_void_p]),
    "ora_vision_patch_area": (C.c_int, [C.c_void_p]),
    "ora_vision_layers": (C.c_int, [C.c_void_p]),
    "ora_vision_forward": (C.c_int, [C.c_void_p, _F, C.c_int, C.c_int, _F, TRACE_FN, C.c_void_p, C.c_int]),
    "ora_layernorm": (None, [_F, C.c_int, C.c_int, _F, _F, C.c_float, _F]),
    "ora_pool": (None, [_F, C.c_int, C.c_int, C.c_int, C.c_int, _F]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run make -C oracle")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIG.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def _f(a: np.ndarray):
    return a.ctypes.data_as(_F)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleModel:
    """A GGUF opened by the oracle (ModelConfig / ModelWeights / CPUReference)."""

    def __init__(self, path: str):
        err = C.create_string_buffer(512)
        h = lib.ora_open(path.encode(), err, 512)
        if not h:
            raise ValueError(err.value.decode())
        self.h = C.c_void_p(h)
        self.hidden = lib.ora_hidden(self.h)
        self.out_dims = lib.ora_output_dims(self.h)
        self.layers = lib.ora_layers(self.h)
        self.vocab = lib.ora_vocab(self.h)

    def close(self):
        if self.h:
            lib.ora_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def forward(self, tokens, keep: Optional[Iterable[Tuple[str, int]]] = None, threads: int = 0,
                vectors: Optional[np.ndarray] = None):
        """CPUReference.forward for one sequence -> (pooled, {(name, layer): array}). With `vectors`
        ([rows, hidden] fp32), a token id -(r + 1) is row r of it, entered unscaled."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        vec = None if vectors is None else np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1, self.hidden)
        pooled = np.zeros(self.out_dims, dtype=np.float32)
        want = set(keep or [])
        traces: Dict[Tuple[str, int], np.ndarray] = {}

        def cb(_u, name, layer, data, count):
            key = (name.decode(), int(layer))
            if key in want:
                traces[key] = np.ctypeslib.as_array(data, shape=(count,)).copy()

        fn = TRACE_FN(cb)
        rc = lib.ora_forward_rows(self.h, t.ctypes.data_as(C.POINTER(C.c_int32)), t.size,
                                  _f(vec) if vec is not None else None, 0 if vec is None else vec.shape[0], _f(pooled),
                                  fn if want else TRACE_FN(), None, threads)
        if rc != 0:
            raise ValueError(f"ora_forward failed ({rc})")
        return pooled, traces


class VisionOracle:
    """An image-encoder GGUF opened by the oracle (the config-5 tower, ora_vision_*)."""

    def __init__(self, path: str):
        err = C.create_string_buffer(512)
        h = lib.ora_vision_open(path.encode(), err, 512)
        if not h:
            raise ValueError(err.value.decode())
        self.h = C.c_void_p(h)
        self.hidden = lib.ora_vision_hidden(self.h)
        self.proj_dims = lib.ora_vision_proj_dims(self.h)
        self.merge = lib.ora_vision_merge(self.h)
        self.area = lib.ora_vision_patch_area(self.h)
        self.layers = lib.ora_vision_layers(self.h)

    def close(self):
        if self.h:
            lib.ora_vision_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def forward(self, patches, grid_x: int, grid_y: int, keep: Optional[Iterable[Tuple[str, int]]] = None,
                threads: int = 0):
        """One image -> (vectors [tokens, proj_dims], {(name, layer): array})."""
        p = f32(patches)
        tokens = (grid_x // self.merge) * (grid_y // self.merge)
        out = np.zeros((tokens, self.proj_dims), dtype=np.float32)
        want = set(keep or [])
        traces: Dict[Tuple[str, int], np.ndarray] = {}

        def cb(_u, name, layer, data, count):
            key = (name.decode(), int(layer))
            if key in want:
                traces[key] = np.ctypeslib.as_array(data, shape=(count,)).copy()

        fn = TRACE_FN(cb)
        rc = lib.ora_vision_forward(self.h, _f(p), grid_x, grid_y, _f(out), fn if want else TRACE_FN(), None, threads)
        if rc != 0:
            raise ValueError(f"ora_vision_forward failed ({rc})")
        return out, traces


def layernorm(x: np.ndarray, width: int, weight: np.ndarray, bias: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x, w, b = f32(x), f32(weight), f32(bias)
    out = np.zeros_like(x)
    lib.ora_layernorm(_f(x), x.size // width, width, _f(w), _f(b), eps, _f(out))
    return out


def pool(x: np.ndarray, grid_x: int, grid_y: int, merge: int, width: int) -> np.ndarray:
    x = f32(x)
    out = np.zeros(((grid_x // merge) * (grid_y // merge), width), dtype=np.float32)
    lib.ora_pool(_f(x), grid_x, grid_y, merge, width, _f(out))
    return out


def dequant_row(type_: int, row: bytes, cols: int) -> np.ndarray:
    out = np.zeros(cols, dtype=np.float32)
    buf = C.create_string_buffer(bytes(row), len(row))
    lib.ora_dequant_row(type_, buf, cols, _f(out))
    return out


def half_to_float(h: int) -> float:
    return float(lib.ora_half_to_float(h))


def float_to_half(x: float) -> int:
    return int(lib.ora_float_to_half(x))


def matmul(x: np.ndarray, w: np.ndarray, threads: int = 0) -> np.ndarray:
    """y = x @ w.T with x [M, K], w [N, K]."""
    x, w = f32(x), f32(w)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    lib.ora_matmul(_f(x), m, k, _f(w), n, _f(y), threads)
    return y


def rmsnorm(x: np.ndarray, width: int, weight: Optional[np.ndarray] = None, eps: float = 1e-6,
            prescale: float = 1.0) -> np.ndarray:
    x = f32(x)
    out = np.zeros_like(x)
    wp = _f(f32(weight)) if weight is not None else None
    keep = f32(weight) if weight is not None else None
    if keep is not None:
        wp = _f(keep)
    lib.ora_rmsnorm(_f(x), x.size // width, width, wp, eps, prescale, _f(out))
    return out


def gelu_tanh(x: float) -> float:
    return float(lib.ora_gelu_tanh(x))


def rope_table(head_dim: int, base: float, positions: int) -> np.ndarray:
    out = np.zeros(positions * head_dim, dtype=np.float32)
    lib.ora_rope_table(head_dim, base, positions, _f(out))
    return out.reshape(positions, head_dim // 2, 2)


def rope(x: np.ndarray, heads: int, head_dim: int, table: np.ndarray, positions) -> np.ndarray:
    y = f32(x).copy()
    p = np.ascontiguousarray(positions, dtype=np.int32)
    t = f32(table)
    lib.ora_rope(_f(y), p.size, heads, head_dim, _f(t), p.ctypes.data_as(C.POINTER(C.c_int32)))
    return y


def attention(q, k, v, tokens: int, heads: int, kv_heads: int, head_dim: int, scale: float = 1.0,
              window: int = 0, threads: int = 0) -> np.ndarray:
    q, k, v = f32(q), f32(k), f32(v)
    out = np.zeros(tokens * heads * head_dim, dtype=np.float32)
    lib.ora_attention(_f(q), _f(k), _f(v), tokens, heads, kv_heads, head_dim, scale, window, _f(out), threads)
    return out.reshape(tokens, heads, head_dim)
