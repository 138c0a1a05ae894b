"""Per-kernel parity on the GPU through the C-ABI, against the CPU oracle on the same inputs
(the reference's KernelTests.swift style: max |got - want| / max |want|, TestSupport.swift:100-110).

Inputs the GPU takes in fp16 are rounded to fp16 first and the oracle gets the same rounded
values, so the remaining difference is the kernel's own arithmetic: fp16 rounding of each
dequantised weight (relative 2^-12) and fp32 accumulation order."""
import numpy as np
import pytest

import ge_oracle as ora
import gemma_embed as ge
import npref

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(77)


def max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module")
def ctx():
    c = ge.Context.create(0)
    print("device:", c.device_name, flush=True)
    yield c
    c.close()


@pytest.fixture(scope="module")
def c2(config2_gguf):
    return npref.Gguf(config2_gguf)


def f16_round(a):
    return np.asarray(a, np.float32).astype(np.float16)


def run_gemm(ctx, raw_q8, rows, cols, x16, y_f16=False):
    M = x16.shape[0]
    w = ctx.q8_create(raw_q8, rows, cols)
    dx = ctx.alloc(x16.nbytes)
    dy = ctx.alloc(M * rows * (2 if y_f16 else 4))
    try:
        ctx.upload(dx, x16)
        ctx.gemm_q8(w, dx, M, dy, y_f16)
        y = ctx.download(dy, (M, rows), np.float16 if y_f16 else np.float32)
    finally:
        ctx.free(dx)
        ctx.free(dy)
        ctx.q8_destroy(w)
    return y.astype(np.float32)


GEMM_SHAPES = [  # (tensor, M): every config-2 projection plus ragged row counts, on the skinny
    # kernel (M <= 512) and on the tiled one
    ("blk.0.attn_q.weight", 200), ("blk.0.attn_k.weight", 129), ("blk.0.attn_v.weight", 1),
    ("blk.0.attn_output.weight", 300), ("blk.0.ffn_gate.weight", 128), ("blk.0.ffn_up.weight", 513),
    ("blk.0.ffn_down.weight", 257), ("output.weight", 64), ("blk.0.attn_q.weight", 700),
    ("blk.0.attn_output.weight", 600), ("blk.0.ffn_down.weight", 1100),
]


@pytest.mark.parametrize("name,M", GEMM_SHAPES)
def test_gemm_q8_vs_oracle(ctx, c2, name, M):
    shape, _, _ = c2.tensors[name]
    cols, rows = shape
    print(f"gemm {name} M={M} N={rows} K={cols}", flush=True)
    x16 = f16_round(RNG.standard_normal((M, cols)))
    y = run_gemm(ctx, np.asarray(c2.raw(name)), rows, cols, x16)
    want = ora.matmul(x16.astype(np.float32), c2.tensor(name).astype(np.float32))
    assert max_rel(y, want) < 2e-3


def test_gemm_config1(ctx, c2):
    """X fp32 [128 x 768] ~ N(0, 1), W Q8_0 [1152 x 768] (blk.0.ffn_gate of the
    config-2 model, drawn by the same Q8_0 rule), Y fp32 [128 x 1152]."""
    x = np.random.default_rng(1).standard_normal((128, 768)).astype(np.float32)
    name = "blk.0.ffn_gate.weight"
    y = run_gemm(ctx, np.asarray(c2.raw(name)), 1152, 768, f16_round(x))
    want = ora.matmul(x, c2.tensor(name).astype(np.float32))
    # the input's own fp16 rounding (2^-12 relative) is inside this bound
    assert max_rel(y, want) < 3e-3


def test_gemm_f16_output_and_row_independence(ctx, c2):
    name = "blk.3.attn_output.weight"
    x16 = f16_round(RNG.standard_normal((600, 768)))
    raw = np.asarray(c2.raw(name))
    y = run_gemm(ctx, raw, 768, 768, x16, y_f16=True)
    want = ora.matmul(x16.astype(np.float32), c2.tensor(name).astype(np.float32))
    assert max_rel(y, want) < 3e-3
    # a row's result does not depend on the other rows or on M (no split-K, fixed K order)
    y32 = run_gemm(ctx, raw, 768, 768, x16)
    y_part = run_gemm(ctx, raw, 768, 768, x16[131:140].copy())
    assert np.array_equal(y32[131:140], y_part)


@pytest.mark.parametrize("name", ["blk.2.attn_output.weight", "blk.2.ffn_down.weight"])
def test_gemm_row_boundaries_bitwise(ctx, c2, name):
    """The reference's batch-register GEMM check (BatchRegisterGemmTests.swift:81-137): a row's
    result is the same bits at every batch size. The 768-wide projections change kernel and tile
    with the row count (skinny up to 512, 128 x 128 below 6144, 128 x 256 below 12288, 256 x 192
    from there); each batch below is compared with the same rows of a 16384-row launch."""
    shape, _, _ = c2.tensors[name]
    cols, rows = shape
    raw = np.asarray(c2.raw(name))
    x16 = f16_round(RNG.standard_normal((16384, cols)))
    full = run_gemm(ctx, raw, rows, cols, x16, y_f16=True)
    for M in (1, 63, 64, 65, 511, 512, 513, 2047, 2048, 2049, 6143, 6144, 8192, 12287, 12288, 12289):
        lo = min(777, 16384 - M)
        print(f"{name}: rows [{lo}, {lo + M}) against the 16384-row launch", flush=True)
        part = run_gemm(ctx, raw, rows, cols, x16[lo:lo + M].copy(), y_f16=True)
        assert np.array_equal(full[lo:lo + M], part), M


@pytest.mark.parametrize("name,y_f16", [("blk.1.attn_q.weight", False), ("blk.1.ffn_down.weight", True),
                                         ("output.weight", False)])
def test_gemm_short_batches_match_tiled_rows(ctx, c2, name, y_f16):
    """Up to 512 rows run on the skinny kernel; the same rows inside a 600-row batch run on the
    tiled kernel. Same MFMA, operand order and k order: the same bits."""
    shape, _, _ = c2.tensors[name]
    cols, rows = shape
    raw = np.asarray(c2.raw(name))
    x16 = f16_round(RNG.standard_normal((600, cols)))
    full = run_gemm(ctx, raw, rows, cols, x16, y_f16)
    for lo, n in ((0, 1), (5, 7), (100, 32), (200, 33), (236, 64), (88, 300), (50, 512)):
        part = run_gemm(ctx, raw, rows, cols, x16[lo:lo + n].copy(), y_f16)
        assert np.array_equal(full[lo:lo + n], part), (lo, n)


def q8_raw(rows, cols, rng):
    """Q8_0 rows as the GGUF stores them: per 32 values an fp16 scale, then 32 int8."""
    nb = rows * cols // 32
    blocks = np.zeros((nb, 34), np.uint8)
    d = (np.abs(rng.standard_normal(nb)) * 0.02 / 127 + 1e-4).astype(np.float16)
    blocks[:, :2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    return blocks.reshape(-1)


def q8_dequant(raw, rows, cols):
    b = raw.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(rows, cols)


@pytest.mark.parametrize("cols", [640, 1024, 1152])
def test_gemm_short_batch_every_pipeline_depth(ctx, cols):
    """K / 16 = 40, 64 and 72 reach each depth of the skinny kernel's load pipeline (8, 16 and 24
    k-steps in flight for the plain GEMM; 4, 16 and 12 for the GeGLU pairs). Batches of up to 512
    rows match the same rows of a 600-row batch on the tiled kernel bit for bit, and the oracle
    within the fp16 rounding of the dequantised weights."""
    rng = np.random.default_rng(cols)
    rows = 256
    raw = q8_raw(rows, cols, rng)
    x16 = f16_round(rng.standard_normal((600, cols)))
    full = run_gemm(ctx, raw, rows, cols, x16)
    want = ora.matmul(x16[:64].astype(np.float32), q8_dequant(raw, rows, cols))
    assert max_rel(full[:64], want) < 3e-3
    for lo, n in ((0, 1), (40, 64), (250, 33), (80, 512)):
        assert np.array_equal(full[lo:lo + n], run_gemm(ctx, raw, rows, cols, x16[lo:lo + n].copy())), (lo, n)
    g = ctx.q8_create(q8_raw(rows, cols, rng), rows, cols)
    u = ctx.q8_create(q8_raw(rows, cols, rng), rows, cols)

    def geglu(x):
        dx, da = ctx.alloc(x.nbytes), ctx.alloc(x.shape[0] * rows * 2)
        try:
            ctx.upload(dx, x)
            ctx.gemm_q8_geglu(g, u, dx, x.shape[0], da)
            return ctx.download(da, (x.shape[0], rows), np.float16)
        finally:
            ctx.free(dx)
            ctx.free(da)
    try:
        xs = f16_round(rng.standard_normal((600, cols)) * 0.05)
        gfull = geglu(xs)
        assert np.all(np.isfinite(gfull.astype(np.float32)))
        for lo, n in ((0, 3), (40, 64), (250, 50), (70, 512)):
            assert np.array_equal(gfull[lo:lo + n], geglu(xs[lo:lo + n].copy())), (lo, n)
    finally:
        ctx.q8_destroy(g)
        ctx.q8_destroy(u)


def test_gemm_geglu_short_batch_matches_tiled_rows(ctx, c2):
    M = 600
    x16 = f16_round(RNG.standard_normal((M, 768)) * 0.05)
    g = ctx.q8_create(np.asarray(c2.raw("blk.4.ffn_gate.weight")), 1152, 768)
    u = ctx.q8_create(np.asarray(c2.raw("blk.4.ffn_up.weight")), 1152, 768)

    def geglu(x):
        dx, da = ctx.alloc(x.nbytes), ctx.alloc(x.shape[0] * 1152 * 2)
        try:
            ctx.upload(dx, x)
            ctx.gemm_q8_geglu(g, u, dx, x.shape[0], da)
            return ctx.download(da, (x.shape[0], 1152), np.float16)
        finally:
            ctx.free(dx)
            ctx.free(da)
    try:
        full = geglu(x16)
        for lo, n in ((0, 3), (40, 64), (250, 50), (60, 512)):
            assert np.array_equal(full[lo:lo + n], geglu(x16[lo:lo + n].copy())), (lo, n)
    finally:
        ctx.q8_destroy(g)
        ctx.q8_destroy(u)


def test_gemm_geglu_row_boundaries_bitwise(ctx, c2):
    """Gate/up rows at every batch size against a 20000-row launch. Launches whose 128 x 256 tiles
    leave a last partial round of at most a quarter of the workgroup slots run those tiles as
    128 x 128 halves (16384 rows: 1024 whole tiles and 256 halves; 8192: 512 and 128; 20000 rows,
    0.76 of a round, whole tiles only); a row's bits must not depend on which."""
    x16 = f16_round(RNG.standard_normal((20000, 768)) * 0.05)
    g = ctx.q8_create(np.asarray(c2.raw("blk.3.ffn_gate.weight")), 1152, 768)
    u = ctx.q8_create(np.asarray(c2.raw("blk.3.ffn_up.weight")), 1152, 768)

    def geglu(x):
        dx, da = ctx.alloc(x.nbytes), ctx.alloc(x.shape[0] * 1152 * 2)
        try:
            ctx.upload(dx, x)
            ctx.gemm_q8_geglu(g, u, dx, x.shape[0], da)
            return ctx.download(da, (x.shape[0], 1152), np.float16)
        finally:
            ctx.free(dx)
            ctx.free(da)
    try:
        full = geglu(x16)
        for M, lo in ((16384, 3616), (16383, 1), (8192, 8187), (9000, 7000), (4096, 12288), (600, 19400), (64, 16320)):
            print(f"gate/up rows [{lo}, {lo + M}) against the 20000-row launch", flush=True)
            assert np.array_equal(full[lo:lo + M], geglu(x16[lo:lo + M].copy())), (M, lo)
    finally:
        ctx.q8_destroy(g)
        ctx.q8_destroy(u)


def test_gemm_geglu_vs_oracle(ctx, c2):
    M = 333
    x16 = f16_round(RNG.standard_normal((M, 768)) * 0.05)
    g = ctx.q8_create(np.asarray(c2.raw("blk.2.ffn_gate.weight")), 1152, 768)
    u = ctx.q8_create(np.asarray(c2.raw("blk.2.ffn_up.weight")), 1152, 768)
    dx, da = ctx.alloc(x16.nbytes), ctx.alloc(M * 1152 * 2)
    try:
        ctx.upload(dx, x16)
        ctx.gemm_q8_geglu(g, u, dx, M, da)
        act = ctx.download(da, (M, 1152), np.float16).astype(np.float32)
    finally:
        ctx.free(dx)
        ctx.free(da)
        ctx.q8_destroy(g)
        ctx.q8_destroy(u)
    xf = x16.astype(np.float32)
    gate = ora.matmul(xf, c2.tensor("blk.2.ffn_gate.weight").astype(np.float32))
    up = ora.matmul(xf, c2.tensor("blk.2.ffn_up.weight").astype(np.float32))
    want = np.vectorize(ora.gelu_tanh)(gate) * up
    assert max_rel(act, want) < 3e-3


ATTN_CASES = [  # (lengths, H, KV, hd, half_window): the reference's packed-length mixes (KernelTests.swift:552-559)
    ([1, 7, 64], 3, 1, 256, 0),
    ([100, 33, 5], 3, 1, 256, 16),
    ([1024, 5], 3, 1, 256, 256),
    ([600], 3, 1, 256, 0),
    ([70, 1, 129], 4, 2, 256, 64),
    ([300, 31], 4, 1, 512, 0),
    ([96, 40], 2, 1, 128, 8),
    ([257], 4, 4, 128, 0),
    ([130, 64], 4, 1, 128, 32),  # four query heads per KV head: the 32-query-wave kernel
    # the reference's long mixes at both head dims and both GQA ratios, with and without a window
    ([2048], 3, 1, 256, 0),
    ([2048, 3, 1024, 7], 4, 2, 256, 256),
    ([2048, 3, 1024, 7], 4, 1, 512, 0),
    ([2048, 3, 1024, 7], 4, 2, 512, 256),
    ([1024, 5], 4, 1, 512, 256),
]


@pytest.mark.parametrize("lengths,H,KV,hd,hw", ATTN_CASES)
def test_attention_vs_oracle(ctx, lengths, H, KV, hd, hw):
    print(f"attention lengths={lengths} H={H} KV={KV} hd={hd} hw={hw}", flush=True)
    T = sum(lengths)
    slack = 64
    q = f16_round(RNG.standard_normal((T, H, hd)) * 1.5)
    k = f16_round(RNG.standard_normal((T, KV, hd)))
    v = f16_round(RNG.standard_normal((T, KV, hd)))
    ranges, s = [], 0
    for n in lengths:
        ranges.append((s, n))
        s += n
    work = ge.attention_work(ranges)
    pad = lambda a: np.concatenate([a, np.zeros((slack,) + a.shape[1:], a.dtype)])
    dq, dk, dv = ctx.alloc(pad(q).nbytes), ctx.alloc(pad(k).nbytes), ctx.alloc(pad(v).nbytes)
    do, dw = ctx.alloc(pad(q).nbytes), ctx.alloc(work.nbytes)
    try:
        ctx.upload(dq, pad(q))
        ctx.upload(dk, pad(k))
        ctx.upload(dv, pad(v))
        ctx.upload(dw, work)
        ctx.attention(dq, dk, dv, do, dw, len(work), H, KV, hd, hw, 1.0)
        out = ctx.download(do, (T, H, hd), np.float16).astype(np.float32)
    finally:
        for p in (dq, dk, dv, do, dw):
            ctx.free(p)
    for st, n in ranges:
        want = ora.attention(q[st:st + n].astype(np.float32), k[st:st + n].astype(np.float32),
                             v[st:st + n].astype(np.float32), n, H, KV, hd, 1.0, 2 * hw)
        assert max_rel(out[st:st + n], want) < 5e-3, (st, n)


def split_f16(a):
    """fp16 (hi, lo) with hi + lo = a to about 2^-22 relative (hi = fp16(a), lo = fp16(a - hi))."""
    a = np.asarray(a, np.float32)
    hi = a.astype(np.float16)
    lo = (a - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


def rms_normed(x, w):
    """RMSNorm over the last axis times w (the reference's QK norm, CPUReference.swift:77-90)."""
    return (x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w).astype(np.float32)


SPLIT_CASES = [  # (lengths, H, KV, half_window, correlation of the rows with one shared direction, head dim)
    ([1024, 300], 4, 1, 0, 0.0, 512),
    ([2048, 7, 129], 4, 1, 0, 0.95, 512),
    ([700, 1], 8, 2, 256, 0.5, 512),
    # head dim 256 with 3 query heads per KV head (attention_split_kernel<256, 3>, config 2's layers
    # under split_scores), sequences longer than the window so that the window's key range and its
    # mask act, and empty-neighbour edge cases
    ([1024, 300], 3, 1, 256, 0.5, 256),
    ([700, 1], 3, 1, 256, 0.0, 256),
    ([2048, 7, 129], 3, 1, 256, 0.95, 256),
    ([2048, 7, 129], 6, 2, 0, 0.5, 256),
]


@pytest.mark.parametrize("lengths,H,KV,hw,corr,hd", SPLIT_CASES)
def test_attention_split_normed_vs_oracle(ctx, lengths, H, KV, hw, corr, hd):
    """RMS-normed, weighted q and k at attention scale 1 (the reference's global layers of width
    512, Model/Architecture.md:8-9, CPUReference.swift:225-233; config 2's width 256 when split
    scores are loaded): scores of several hundred. The oracle gets the fp32 q and k; the GPU gets
    them as split fp16 pairs. fp16 operands alone put such cases at 6-8e-3 of max |want| (a
    near-tie between keys moves with a 0.02 score shift); the split scores leave the fp16 rounding
    of V and P (~4e-4)."""
    print(f"split attention lengths={lengths} H={H} KV={KV} hw={hw} corr={corr} hd={hd}", flush=True)
    T, slack = sum(lengths), 64
    rng = np.random.default_rng(1000 + T)
    base = rng.standard_normal(hd)
    mix = lambda shape: corr * base + np.sqrt(1 - corr * corr) * rng.standard_normal(shape)
    wq, wk = 1 + 0.1 * rng.standard_normal(hd), 1 + 0.1 * rng.standard_normal(hd)
    q, k = rms_normed(mix((T, H, hd)), wq), rms_normed(mix((T, KV, hd)), wk)
    v = f16_round(rms_normed(rng.standard_normal((T, KV, hd)), 1.0))
    qh, ql = split_f16(q)
    kh, kl = split_f16(k)
    ranges, s = [], 0
    for n in lengths:
        ranges.append((s, n))
        s += n
    work = ge.attention_work(ranges)
    pad = lambda a: np.concatenate([a, np.zeros((slack,) + a.shape[1:], a.dtype)])
    bufs = [ctx.alloc(pad(a).nbytes) for a in (qh, ql, kh, kl, v, qh)] + [ctx.alloc(work.nbytes)]
    try:
        for b, a in zip(bufs, (qh, ql, kh, kl, v)):
            ctx.upload(b, pad(a))
        ctx.upload(bufs[6], work)
        ctx.attention_split(bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], bufs[5], bufs[6], len(work), H, KV, hd, hw, 1.0)
        out = ctx.download(bufs[5], (T, H, hd), np.float16).astype(np.float32)
    finally:
        for b in bufs:
            ctx.free(b)
    for st, n in ranges:
        want = ora.attention(q[st:st + n], k[st:st + n], v[st:st + n].astype(np.float32), n, H, KV, hd, 1.0, 2 * hw)
        err = max_rel(out[st:st + n], want)
        print(f"  sequence [{st}, +{n}): max_rel {err:.2e}", flush=True)
        assert err < 2e-3, (st, n)


def test_attention_split_rejects_unsupported(ctx):
    d = ctx.alloc(1024)
    try:
        with pytest.raises(ge.GemmaEmbedError):
            ctx.attention_split(d, d, d, d, d, d, d, 1, 3, 1, 512, 0, 1.0)  # 3 query heads per KV head
        with pytest.raises(ge.GemmaEmbedError):
            ctx.attention_split(d, d, d, d, d, d, d, 1, 4, 1, 256, 0, 1.0)  # head dim 256
    finally:
        ctx.free(d)
