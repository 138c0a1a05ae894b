"""Independent float64 numpy statement of the text forward, for pinning the C oracle.

Written from the reference's written spec (Sources/GemmaEmbed/Model/Architecture.md:1-45) and
the GGUF layout (GGUF/GGUFFile.swift:21-67), with its own GGUF reader. It shares no code with
oracle/ge_oracle.c: attention is a masked softmax over an einsum score matrix, RoPE is complex
multiplication, and every product is float64, so a transposed operand, a wrong index, a dropped
term or a wrong mask in the oracle shows up as a difference far above float32 rounding.
"""
from __future__ import annotations

import struct
from typing import Dict, List, Optional, Tuple

import numpy as np

SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class Gguf:
    def __init__(self, path: str):
        self.buf = np.memmap(path, dtype=np.uint8, mode="r")
        b = self.buf
        self.pos = 0
        magic, version = struct.unpack_from("<II", b, 0)
        assert magic == 0x46554747 and version in (2, 3)
        self.pos = 8
        nt, nkv = struct.unpack_from("<QQ", b, self.pos)
        self.pos += 16
        self.meta = {}
        for _ in range(nkv):
            key = self._str()
            t = self._u32()
            self.meta[key] = self._val(t)
        self.tensors = {}
        for _ in range(nt):
            name = self._str()
            nd = self._u32()
            shape = list(struct.unpack_from("<" + "Q" * nd, b, self.pos))
            self.pos += 8 * nd
            typ = self._u32()
            off = struct.unpack_from("<Q", b, self.pos)[0]
            self.pos += 8
            self.tensors[name] = (shape, typ, off)
        align = self.meta.get("general.alignment", 32)
        self.data = (self.pos + align - 1) // align * align

    def _u32(self):
        v = struct.unpack_from("<I", self.buf, self.pos)[0]
        self.pos += 4
        return v

    def _str(self):
        n = struct.unpack_from("<Q", self.buf, self.pos)[0]
        self.pos += 8
        s = bytes(self.buf[self.pos:self.pos + n]).decode()
        self.pos += n
        return s

    def _val(self, t):
        if t == 8:
            return self._str()
        if t == 9:
            et = self._u32()
            n = struct.unpack_from("<Q", self.buf, self.pos)[0]
            self.pos += 8
            if et == 8:
                return [self._str() for _ in range(n)]
            return [self._val(et) for _ in range(n)]
        fmt = SCALAR[t]
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def raw(self, name: str) -> np.ndarray:
        shape, typ, off = self.tensors[name]
        n = int(np.prod(shape))
        nbytes = {0: n * 4, 1: n * 2, 30: n * 2, 8: n // 32 * 34}[typ]
        return self.buf[self.data + off:self.data + off + nbytes]

    def tensor(self, name: str) -> np.ndarray:
        """Dequantised float64 [rows][cols] (ne order reversed)."""
        shape, typ, _ = self.tensors[name]
        raw = self.raw(name)
        cols = shape[0]
        if typ == 0:
            v = raw.view(np.float32).astype(np.float64)
        elif typ == 1:
            v = raw.view(np.float16).astype(np.float64)
        elif typ == 30:
            v = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        elif typ == 8:
            blocks = raw.reshape(-1, 34)
            d = blocks[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
            q = blocks[:, 2:].view(np.int8).astype(np.float64)
            v = (d * q).reshape(-1)
        else:
            raise ValueError(typ)
        return v.reshape(-1, cols) if len(shape) > 1 else v


def rmsnorm(x: np.ndarray, w: Optional[np.ndarray], eps: float) -> np.ndarray:
    r = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return r * w if w is not None else r


def gelu_tanh(x):
    return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))


def rope(x: np.ndarray, base: float, positions: np.ndarray) -> np.ndarray:
    """NeoX rotation as complex multiplication: (x_i + j x_{i+hd/2}) * exp(j pos base^(-2i/hd))."""
    hd = x.shape[-1]
    half = hd // 2
    inv = base ** (-2.0 * np.arange(half) / hd)
    ang = positions[:, None].astype(np.float64) * inv[None, :]
    z = (x[..., :half] + 1j * x[..., half:]) * np.exp(1j * ang)[:, None, :]
    return np.concatenate([z.real, z.imag], axis=-1)


def attention(q, k, v, window: int) -> np.ndarray:
    """q [T, H, hd], k/v [T, KV, hd]; softmax(q k^T) v with |i - j| > window // 2 masked."""
    T, H, hd = q.shape
    KV = k.shape[1]
    kk = np.repeat(k, H // KV, axis=1)
    vv = np.repeat(v, H // KV, axis=1)
    s = np.einsum("ihd,jhd->hij", q, kk)
    if window:
        i = np.arange(T)
        mask = np.abs(i[:, None] - i[None, :]) > window // 2
        s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hij,jhd->ihd", p, vv)


def forward(g: Gguf, tokens: np.ndarray, keep: Tuple = (), vectors=None) -> Tuple[np.ndarray, Dict]:
    """Mean-pooled, unnormalised output for one sequence, float64; keep = (name, layer) traces.
    A token id -(r + 1) is row r of `vectors`, entered unscaled (CPUReference.swift:197-199)."""
    a = "gemma-embedding2."
    m = g.meta
    L, d, H = m[a + "block_count"], m[a + "embedding_length"], m[a + "attention.head_count"]
    eps = m[a + "attention.layer_norm_rms_epsilon"]
    window = m[a + "attention.sliding_window"]
    kvh = m[a + "attention.head_count_kv"]
    pattern = m[a + "attention.sliding_window_pattern"]
    hd_g, hd_s = m[a + "attention.key_length"], m[a + "attention.key_length_swa"]
    rb_g = m[a + "rope.freq_base"]
    rb_s = m.get(a + "rope.freq_base_swa", rb_g)
    ple = "per_layer_model_proj.weight" in g.tensors
    T = len(tokens)
    pos = np.arange(T)
    traces = {}

    def tr(name, layer, val):
        if (name, layer) in keep:
            traces[(name, layer)] = np.array(val, dtype=np.float64).reshape(-1)

    emb = g.raw("token_embd.weight").reshape(-1, d // 32 * 34)
    rows = []
    for t in tokens:
        if t < 0:
            rows.append(None)
            continue
        blk = emb[t].reshape(-1, 34)
        dd = blk[:, :2].copy().view(np.float16).astype(np.float64)
        rows.append((dd * blk[:, 2:].view(np.int8)).reshape(-1) * np.sqrt(np.float32(d)).astype(np.float64))
    x = np.stack([np.asarray(vectors, np.float64).reshape(-1, d)[-t - 1] if r is None else r
                  for t, r in zip(tokens, rows)])
    tr("inp_scaled", -1, x)
    if ple:
        pl = m[a + "embedding_length_per_layer_input"]
        per = x @ g.tensor("per_layer_model_proj.weight").T / np.sqrt(d)
        per = rmsnorm(per.reshape(T, L, pl), g.tensor("per_layer_proj_norm.weight"), eps)
        tr("inp_per_layer", -1, per)
    for l in range(L):
        b = f"blk.{l}."
        sw = bool(pattern[l])
        hd = hd_s if sw else hd_g
        KV = kvh[l]
        h = rmsnorm(x, g.tensor(b + "attn_norm.weight"), eps)
        q = (h @ g.tensor(b + "attn_q.weight").T).reshape(T, H, hd)
        k = (h @ g.tensor(b + "attn_k.weight").T).reshape(T, KV, hd)
        v = (h @ g.tensor(b + "attn_v.weight").T).reshape(T, KV, hd)
        tr("Qcur", l, q)
        q = rmsnorm(q, g.tensor(b + "attn_q_norm.weight"), eps)
        k = rmsnorm(k, g.tensor(b + "attn_k_norm.weight"), eps)
        v = rmsnorm(v, None, eps)
        base = rb_s if sw else rb_g
        q, k = rope(q, base, pos), rope(k, base, pos)
        tr("Qcur_pos", l, q)
        tr("Kcur_pos", l, k)
        tr("Vcur_normed", l, v)
        att = attention(q, k, v, window if sw else 0).reshape(T, H * hd)
        tr("kqv_out", l, att)
        x = x + rmsnorm(att @ g.tensor(b + "attn_output.weight").T, g.tensor(b + "post_attention_norm.weight"), eps)
        tr("attn_out", l, x)
        f = rmsnorm(x, g.tensor(b + "ffn_norm.weight"), eps)
        act = gelu_tanh(f @ g.tensor(b + "ffn_gate.weight").T) * (f @ g.tensor(b + "ffn_up.weight").T)
        tr("ffn_geglu", l, act)
        x = x + rmsnorm(act @ g.tensor(b + "ffn_down.weight").T, g.tensor(b + "post_ffw_norm.weight"), eps)
        tr("pe_in", l, x)
        scale = float(g.tensor(b + "layer_output_scale.weight")[0]) if b + "layer_output_scale.weight" in g.tensors else 1.0
        if ple:
            gg = gelu_tanh(x @ g.tensor(b + "inp_gate.weight").T) * per[:, l, :]
            p = rmsnorm(gg @ g.tensor(b + "proj.weight").T, g.tensor(b + "post_norm.weight"), eps)
            tr("per_layer_embd_out", l, p)
            x = (x + p) * scale
        else:
            x = x * scale
        tr("l_out", l, x)
    y = rmsnorm(x, g.tensor("output_norm.weight"), eps) @ g.tensor("output.weight").T
    tr("result_embd", -1, y)
    return y.mean(axis=0), traces


# ---------------------------------------------------------------------------- image tower

def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def vision_forward(g: Gguf, patches: np.ndarray, gx: int, gy: int, keep: Tuple = ()) -> Tuple[np.ndarray, Dict]:
    """BASELINE config 5's tower for one image, float64: pre-LayerNorm blocks with biased
    projections, softmax(q k^T / sqrt(hd)) attention over all patches, gelu_tanh MLP, final
    LayerNorm, merge x merge mean pooling (as a reshape), weighted RMSNorm and projection."""
    a = "clip.vision."
    m = g.meta
    L, d, H = m[a + "block_count"], m[a + "embedding_length"], m[a + "attention.head_count"]
    eps, merge = m[a + "attention.layer_norm_epsilon"], m[a + "projector.scale_factor"]
    hd = d // H
    P = gx * gy
    traces = {}

    def tr(name, layer, val):
        if (name, layer) in keep:
            traces[(name, layer)] = np.array(val, dtype=np.float64).reshape(-1)

    def lin(x, name):
        return x @ g.tensor(name + ".weight").T

    x = np.asarray(patches, dtype=np.float64) @ g.tensor("v.patch_embd.weight").T
    tr("inp", -1, x)
    shape, _, _ = g.tensors["v.position_embd.weight"]
    npos = shape[1]
    table = g.tensor("v.position_embd.weight")  # [2 npos, d]
    col, row = np.arange(P) % gx, np.arange(P) // gx
    x = x + g.tensor("v.patch_embd.bias") + table[col] + table[npos + row]
    tr("pos_embd", -1, x)
    for l in range(L):
        b = f"v.blk.{l}."
        h = layernorm(x, g.tensor(b + "ln1.weight"), g.tensor(b + "ln1.bias"), eps)
        tr("layer_inp_normed", l, h)
        q = lin(h, b + "attn_q") + g.tensor(b + "attn_q.bias")
        k = lin(h, b + "attn_k") + g.tensor(b + "attn_k.bias")
        v = lin(h, b + "attn_v") + g.tensor(b + "attn_v.bias")
        tr("Qcur", l, q)
        tr("Kcur", l, k)
        tr("Vcur", l, v)
        s = np.einsum("ihd,jhd->hij", q.reshape(P, H, hd), k.reshape(P, H, hd)) / np.sqrt(hd)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        att = np.einsum("hij,jhd->ihd", p, v.reshape(P, H, hd)).reshape(P, d)
        tr("kqv_out", l, att)
        o = lin(att, b + "attn_out")
        tr("attn_out", l, o)
        x = x + o + g.tensor(b + "attn_out.bias")
        tr("ffn_inp", l, x)
        f = layernorm(x, g.tensor(b + "ln2.weight"), g.tensor(b + "ln2.bias"), eps)
        tr("ffn_inp_normed", l, f)
        u = gelu_tanh(lin(f, b + "ffn_up") + g.tensor(b + "ffn_up.bias"))
        tr("ffn_gelu", l, u)
        o = lin(u, b + "ffn_down")
        tr("ffn_out", l, o)
        x = x + o + g.tensor(b + "ffn_down.bias")
        tr("layer_out", l, x)
    y = layernorm(x, g.tensor("v.post_ln.weight"), g.tensor("v.post_ln.bias"), eps)
    pooled = y.reshape(gy // merge, merge, gx // merge, merge, d).mean(axis=(1, 3)).reshape(-1, d)
    tr("pooled", -1, pooled)
    pn = rmsnorm(pooled, g.tensor("mm.soft_emb_norm.weight"), eps)
    tr("pooled_normed", -1, pn)
    out = pn @ g.tensor("mm.input_projection.weight").T
    tr("projected", -1, out)
    return out, traces
