"""The text forward in float64 with the GPU kernels' fp16 rounding points, for bounding what the
fp16-operand design can match (test infrastructure, built on tests/npref.py).

The GPU path rounds to fp16, each time to the nearest representable value (relative 2^-11):
  - the dequantised weights (fp16(q d), once at upload);
  - every GEMM input: the normed rows h, the attention output, the GeGLU product;
  - the projections that feed a norm (QKV, attention output, FFN down), stored as fp16 times a
    power of two;
  - q, k and v after their norms and RoPE; the softmax weights P before the P.V product.
The final norm's rows stay fp32: their mean per sequence goes through the output projection in
fp32 on the exact Q8_0 weights (projecting the mean equals the mean of the projections).
Sums are fp32 on the GPU and float64 here. Powers of two do not change a relative rounding, so
each rounded tensor is scaled into fp16's normal range here before rounding, as the kernels' range
scales do. Comparing this with the float64 forward (no rounding) shows how far the design itself
moves each intermediate from the reference's arithmetic."""
from __future__ import annotations

import numpy as np

from npref import gelu_tanh, rmsnorm, rope


def f16(a):
    """fp16 rounding of a tensor, after scaling it by a power of two so its largest entry sits at
    2^14 (no overflow, no subnormals for the entries that matter)."""
    a = np.asarray(a, np.float64)
    fin = np.isfinite(a)
    m = float(np.abs(a[fin]).max()) if fin.any() else 1.0
    e = 2.0 ** (np.floor(np.log2(max(m, 1e-300))) - 14)
    return (a / e).astype(np.float16).astype(np.float64) * e


def _attention(q, k, v, window, round_p):
    T, H, hd = q.shape
    KV = k.shape[1]
    kk, vv = np.repeat(k, H // KV, axis=1), np.repeat(v, H // KV, axis=1)
    s = np.einsum("ihd,jhd->hij", q, kk)
    if window:
        i = np.arange(T)
        s = np.where((np.abs(i[:, None] - i[None, :]) > window // 2)[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    l = p.sum(axis=-1, keepdims=True)
    if round_p:
        p = f16(p)
    return np.einsum("hij,jhd->ihd", p, vv) / l.transpose(1, 0, 2)


def forward(g, tokens, rounded: bool, keep=()):
    """Traces (name, layer) of the forward of a model without per-layer inputs; rounded=False is
    the plain float64 forward."""
    a = "gemma-embedding2."
    m = g.meta
    L, d, H = m[a + "block_count"], m[a + "embedding_length"], m[a + "attention.head_count"]
    eps, window = m[a + "attention.layer_norm_rms_epsilon"], m[a + "attention.sliding_window"]
    kvh, pattern = m[a + "attention.head_count_kv"], m[a + "attention.sliding_window_pattern"]
    hd_g, hd_s = m[a + "attention.key_length"], m[a + "attention.key_length_swa"]
    rb_g = m[a + "rope.freq_base"]
    rb_s = m.get(a + "rope.freq_base_swa", rb_g)
    assert "per_layer_model_proj.weight" not in g.tensors
    r = f16 if rounded else (lambda z: z)
    cache = {}

    def W(name):
        if name not in cache:
            cache[name] = r(g.tensor(name))
        return cache[name]

    T = len(tokens)
    pos = np.arange(T)
    emb = g.raw("token_embd.weight").reshape(-1, d // 32 * 34)
    x = np.stack([(emb[t].reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float64) *
                   emb[t].reshape(-1, 34)[:, 2:].view(np.int8)).reshape(-1) for t in tokens])
    x = x * np.sqrt(np.float32(d)).astype(np.float64)
    out = {}
    for l in range(L):
        b = f"blk.{l}."
        sw = bool(pattern[l])
        hd, KV = (hd_s if sw else hd_g), kvh[l]
        h = r(rmsnorm(x, g.tensor(b + "attn_norm.weight"), eps))
        q = r((h @ W(b + "attn_q.weight").T).reshape(T, H, hd))
        k = r((h @ W(b + "attn_k.weight").T).reshape(T, KV, hd))
        v = r((h @ W(b + "attn_v.weight").T).reshape(T, KV, hd))
        q = rmsnorm(q, g.tensor(b + "attn_q_norm.weight"), eps)
        k = rmsnorm(k, g.tensor(b + "attn_k_norm.weight"), eps)
        v = r(rmsnorm(v, None, eps))
        base = rb_s if sw else rb_g
        q, k = r(rope(q, base, pos)), r(rope(k, base, pos))
        att = r(_attention(q, k, v, window if sw else 0, rounded).reshape(T, H * hd))
        out[("kqv_out", l)] = att
        x = x + rmsnorm(r(att @ W(b + "attn_output.weight").T), g.tensor(b + "post_attention_norm.weight"), eps)
        f = r(rmsnorm(x, g.tensor(b + "ffn_norm.weight"), eps))
        act = r(gelu_tanh(f @ W(b + "ffn_gate.weight").T) * (f @ W(b + "ffn_up.weight").T))
        out[("ffn_geglu", l)] = act
        down = r(act @ W(b + "ffn_down.weight").T)
        out[("ffn_out", l)] = down
        x = x + rmsnorm(down, g.tensor(b + "post_ffw_norm.weight"), eps)
        out[("l_out", l)] = x
    pooled = rmsnorm(x, g.tensor("output_norm.weight"), eps).mean(axis=0) @ g.tensor("output.weight").T
    return pooled, {k: v for k, v in out.items() if k in keep}
