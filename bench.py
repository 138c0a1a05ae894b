#!/usr/bin/env python3
"""Benchmark of the MI355X GemmaEmbed text-encoder forward.

One step = one forward pass of the 24-layer Q8_0 encoder over 32 texts x 512 tokens, packed as
one 16384-token batch whose token ids, positions, sequence ranges and attention work list are
already resident in HBM (staged once before the timed region). The timed region is bracketed by
device synchronisation; `value` is embedded tokens per second over the K timed steps.

Also reported on the same JSON line:
  roofline      the dominant kernel (the fused gate/up GeGLU GEMM): algorithmic FLOPs per launch
                divided by its mean launch time from HIP events on the library's stream during
                the timed steps, against MI355X's dense fp16 MFMA peak (2.5 PFLOP/s);
  gemm_all      the same for all Q8_0 GEMM launches together;
  variants      two device packs of 8192 tokens per step (the reference's default budget),
                restaged each time; the full host API path at the reference's default options
                (token ids in host memory -> normalised vectors, PCIe included); BASELINE
                config 4 (4 texts x 8192 tokens, one resident pack); and BASELINE config 5 (the
                16-layer image tower over 8 resident 768 x 768 images); and the reference's own
                architecture at its real shapes on the shapes of its published benchmarks, through
                the host API, beside the reference's published M3 Max times (context only: a
                different chip and real weights);
  cpu_baseline  the CPU oracle (a C restatement of the reference's CPUReference.swift) on a
                bounded sample of the same workload, on this host's cores;
  parity        the timed pack's pooled vectors against the oracle's on the texts cpu_baseline
                ran: min cosine and max abs difference of the L2-normalised vectors;
  config3 / config1 variants  BASELINE configs 3 (256 ragged texts, Matryoshka 256) and 1 (one
                Q8_0 GEMM) on the GPU and, on a sample, on the CPU oracle.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gemma-embed-swift_amd"))

METRIC = "embedded tokens/sec, 24L Q8_0 encoder 32×512 @1 GPU; Q8 GEMM % MFMA peak"
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
HBM_PEAK_GBS = 8000.0
TEXTS, TOKENS = 32, 512
D, FF, OUT, HD, H, KV, LAYERS = 768, 1152, 768, 256, 3, 1, 24


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemm_flops(m: int):
    """Algorithmic FLOPs (2 M N K, M = real tokens) of one launch of each GEMM class; they launch
    once per layer."""
    qkv = 2 * m * (H + 2 * KV) * HD * D
    o = 2 * m * D * H * HD
    gu = 2 * m * 2 * FF * D
    down = 2 * m * D * FF
    return {"gemm_qkv": qkv, "gemm_o": o, "gemm_gate_up": gu, "gemm_down": down}


def projection_flops(seqs: int):
    """The output projection runs once per sequence, on its pooled final-norm row (fp32)."""
    return 2 * seqs * OUT * D


def gemm_bytes(m: int):
    """Algorithmic HBM bytes of one launch: fp16 activations in, fp16 dequantised weights, output
    (fp32, or fp16 for the GeGLU product)."""
    b = {}
    for name, n, k, out_bytes in (("gemm_qkv", (H + 2 * KV) * HD, D, 4), ("gemm_o", D, H * HD, 4),
                                  ("gemm_gate_up", 2 * FF, D, 2), ("gemm_down", D, FF, 4)):
        n_out = n // 2 if name == "gemm_gate_up" else n
        b[name] = 2 * m * k + 2 * n * k + out_bytes * m * n_out
    return b


def attention_flops(lengths, window=512, pattern=(1, 1, 1, 1, 1, 0) * 4):
    """4 * hd * H * visible (query, key) pairs, summed over layers."""
    total = 0
    hw = window // 2
    for sliding in pattern:
        for n in lengths:
            if sliding:
                # pairs with |i - j| <= hw inside a sequence of n
                pairs = sum(min(n - 1, i + hw) - max(0, i - hw) + 1 for i in range(n))
            else:
                pairs = n * n
            total += 4 * HD * H * pairs
    return total


VIT = dict(images=8, grid=48, area=768, d=1152, ff=4304, heads=16, hd=72, layers=16, proj=768, merge=3)


def vision_flops():
    """Algorithmic FLOPs of one config-5 batch at the tower's true widths (the padding of the
    heads to 96 and of the MLP to 4352 columns is not counted): 2 M N K per GEMM and
    4 hd H P^2 per image and layer for the attention."""
    v = VIT
    P = v["images"] * v["grid"] ** 2
    d, ff = v["d"], v["ff"]
    gemm = 2 * P * v["area"] * d + v["layers"] * 2 * P * d * (3 * d + d + 2 * ff) \
        + 2 * (P // v["merge"] ** 2) * d * v["proj"]
    attn = v["layers"] * v["images"] * 4 * v["hd"] * v["heads"] * (v["grid"] ** 2) ** 2
    return gemm, attn


def vision_variant(tmp: str, reps: int):
    """8 synthetic 768 x 768 images (48 x 48 patches of 16 x 16 x 3 fp32 pixels
    uniform in [-1, 1]) through the 16-layer tower, pooled 3 x 3 to 256 tokens each and projected
    to 768: patches resident in HBM, one batch per step."""
    import numpy as np
    import gemma_embed as ge
    path = os.path.join(tmp, "config5_vision.gguf")
    ge.synth_write_vision_gguf(path, **ge.CONFIG5_VISION)
    v = VIT
    grids = [(v["grid"], v["grid"])] * v["images"]
    patches = ge.image_patches(51, grids, v["area"])
    ctx = ge.Context.create(0)
    try:
        ctx.vision_load(path)
        ctx.vision_stage(patches, grids)
        for _ in range(2):
            ctx.vision_run()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            ctx.vision_run()
        ctx.sync()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        out = ctx.vision_read(v["proj"])
        if out.shape != (v["images"] * 256, v["proj"]) or not np.all(np.isfinite(out)):
            raise SystemExit("bad config-5 output")
        ctx.profile_reset()
        ctx.profile_enable("")
        ctx.vision_run()
        ctx.sync()
        stats = ctx.profile_stats()
        ctx.profile_disable()
    finally:
        ctx.close()
    gemm, attn = vision_flops()
    kernels = {k: {"launches": n, "avg_us": round(t / max(n, 1) * 1e3, 2), "ms": round(t, 4)} for k, (n, t) in stats.items()}
    gemm_ms = sum(t for k, (n, t) in stats.items() if k.startswith("vit_gemm"))
    attn_ms = stats.get("vit_attention", (0, 0.0))[1]
    return {"workload": "config5: 16-layer ViT (width 1152, 16 heads of 72, MLP 4304, Q8_0), 8 images x 2304 patches, "
                        "3x3 pooled to 256 tokens each, projected to 768",
            "images_per_s": round(v["images"] / (ms * 1e-3), 2), "ms_per_batch": round(ms, 3),
            "patches_per_s": round(v["images"] * v["grid"] ** 2 / (ms * 1e-3), 1),
            "tflops": round((gemm + attn) / (ms * 1e-3) / 1e12, 1),
            "frac": round((gemm + attn) / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
            "gemm_tflops": round(gemm / (gemm_ms * 1e-3) / 1e12, 1) if gemm_ms else None,
            "attention_tflops": round(attn / (attn_ms * 1e-3) / 1e12, 1) if attn_ms else None,
            "algorithmic_flops": gemm + attn, "kernels": kernels}


def image_embed_variant(tmp: str, text_path: str, reps: int):
    """The whole image embedding (MetalForward.run(images:)): config 5's 8 images through the tower,
    then each image's [bos, <|image>, 256 vectors, <image|>, eos] (260 rows) through the 24-layer
    config-2 text tower, whose width is the tower's projection width. GPU time of both towers per
    batch (median), patches already in HBM when it starts (the patch upload precedes it)."""
    import numpy as np
    import gemma_embed as ge
    v = VIT
    grids = [(v["grid"], v["grid"])] * v["images"]
    patches = ge.image_patches(52, grids, v["area"])
    markers = [2, 255998, 255999, 1]
    model = ge.EmbeddingModel.load(text_path)
    try:
        ctx = model.context
        ctx.vision_load(os.path.join(tmp, "config5_vision.gguf"))
        for _ in range(2):
            ctx.image_forward(patches, grids, markers)
        secs = sorted(ctx.image_forward(patches, grids, markers)[1] for _ in range(reps))
        pooled, _ = ctx.image_forward(patches, grids, markers)
        if pooled.shape != (v["images"], 768) or not np.all(np.isfinite(pooled)):
            raise SystemExit("bad image-embedding output")
    finally:
        model.close()
    ms = secs[len(secs) // 2] * 1e3
    return {"workload": "config5 tower + config-2 text tower over 8 x 260 rows (vector rows from the tower in HBM)",
            "images_per_s": round(v["images"] / (ms * 1e-3), 2), "ms_per_batch": round(ms, 3)}


def reference_shapes_variant(tmp: str, reps: int):
    """The reference's own architecture at its real shapes (d 512, per-layer inputs; synthetic
    weights) on the shapes of its published benchmarks (benchmarks/hillclimb-2026-10-27.json, Apple M3
    Max with the real model, first run's medians: an 8 x 1024-token pack in 0.4078 s, 32 x 64 in 0.0604 s, 8 x 256
    in 0.0686 s, a 1 x 64-token call in 6.18 ms, 12 queries of 171 tokens in all as 12 separate
    calls in 52.2 ms), through the host API: token ids in host memory -> normalised vectors, the
    reference's own boundary (COMPARISON.md:57-60)."""
    import numpy as np
    import gemma_embed as ge
    path = os.path.join(tmp, "real_shapes.gguf")
    ge.synth_write_gguf(path, **ge.REAL_SHAPES)
    model = ge.EmbeddingModel.load(path)
    try:
        opts = ge.EmbedOptions()

        def pack_of(seed, n, length):
            return [r.tolist() for r in ge.synth_tokens(seed, 2, 262144, n * length).reshape(n, length)]

        def timed(fn, n):
            fn()
            fn()
            t0 = time.perf_counter()
            for _ in range(n):
                r = fn()
            return (time.perf_counter() - t0) / n, r

        pack = pack_of(81, 8, 1024)
        one = [ge.synth_tokens(82, 2, 262144, 64).tolist()]
        p32x64, p8x256 = pack_of(83, 32, 64), pack_of(84, 8, 256)
        queries = [ge.synth_tokens(85 + i, 2, 262144, 15 if i < 3 else 14).tolist() for i in range(12)]  # 171 tokens
        pack_s, out = timed(lambda: model.embed(pack, opts), reps)
        one_s, _ = timed(lambda: model.embed(one, opts), reps * 4)
        s32x64, _ = timed(lambda: model.embed(p32x64, opts), reps)
        s8x256, _ = timed(lambda: model.embed(p8x256, opts), reps)
        queries_s, _ = timed(lambda: [model.embed([q], opts) for q in queries], reps)
        if not all(np.all(np.isfinite(e.vector)) for e in out):
            raise SystemExit("non-finite output (reference shapes)")
    finally:
        model.close()
    return {"model": "reference architecture at its real shapes: d 512, 4 heads, KV 2x256 sliding / 1x512 global, "
                     "GeGLU 2048, per-layer inputs 512, 24 layers; synthetic Q8_0 weights",
            "pack_8x1024_s": round(pack_s, 5), "pack_8x1024_tokens_per_s": round(8 * 1024 / pack_s, 1),
            "reference_m3max_pack_8x1024_s": 0.4078,
            "pack_32x64_s": round(s32x64, 5), "reference_m3max_pack_32x64_s": 0.0604,
            "pack_8x256_s": round(s8x256, 5), "reference_m3max_pack_8x256_s": 0.0686,
            "call_1x64_ms": round(one_s * 1e3, 3), "reference_m3max_call_1x64_ms": 6.18,
            "queries_12_separate_calls_ms": round(queries_s * 1e3, 3), "reference_m3max_queries_12_ms": 52.2}


def measured_traffic(label: str):
    """HBM bytes per launch of `label` at this workload, from the committed rocprofv3 summary of
    counter runs of the standalone probe `gemma-embed-swift_amd/ge_probe` over the same kernel at
    the same shape (FETCH_SIZE, then WRITE_SIZE, each scaled by what the same counter reads for a
    conversion kernel of known size). Returns (bytes, kernel) or (None, None)."""
    import re
    path = os.path.join(ROOT, "profiles", f"{label}_config2_traffic.md")
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None, None
    m = re.search(rf"traffic_bytes_per_launch {label} (.+) grid (\d+): (\d+)", text)
    return (int(m.group(3)), m.group(1)) if m else (None, None)


def library_gemm_comparison(reps: int = 30):
    """This library's Q8_0 GEMM (`ge_op_gemm_q8`, fp16 activations in, fp16 out) against hipBLASLt
    (through torch.matmul: the same activations times a dense fp16 weight, fp16 out) on the
    forward's four projection shapes at config 2's M = 16384. The library's time per launch is
    the mean of its dispatch events over `reps` synchronous calls; hipBLASLt is timed the same
    way (events around each call, a synchronisation after it) and also back to back."""
    import numpy as np
    import torch
    import gemma_embed as ge

    m = TEXTS * TOKENS
    shapes = (("qkv", (H + 2 * KV) * HD, D), ("o", D, H * HD), ("gate_up", 2 * FF, D), ("down", D, FF))
    rng = np.random.default_rng(5)
    ctx = ge.Context.create(0)
    rows = []
    try:
        for name, n, k in shapes:
            raw = rng.integers(0, 256, size=(n, k // 32, 34), dtype=np.uint8)
            raw[:, :, 0:2] = np.frombuffer(np.full(n * (k // 32), 0.001, np.float16).tobytes(),
                                           np.uint8).reshape(n, k // 32, 2)
            x = (rng.standard_normal((m, k)) * 0.5).astype(np.float16)
            w = ctx.q8_create(raw, n, k)
            dx, dy = ctx.alloc(x.nbytes), ctx.alloc(m * n * 2)
            try:
                ctx.upload(dx, x)
                ctx.gemm_q8(w, dx, m, dy, True)
                ctx.profile_reset()
                ctx.profile_enable("gemm")
                for _ in range(reps):
                    ctx.gemm_q8(w, dx, m, dy, True)
                launches, total_ms = ctx.profile_stats()["gemm"]
                ctx.profile_disable()
            finally:
                ctx.free(dx)
                ctx.free(dy)
                ctx.q8_destroy(w)
            ours_us = total_ms * 1e3 / launches
            tx = torch.from_numpy(x).cuda()
            tw = torch.randn(n, k, device="cuda", dtype=torch.float16) * 0.01
            for _ in range(3):
                torch.matmul(tx, tw.t())
            torch.cuda.synchronize()
            # one call at a time with a synchronisation after each, as ge_op_gemm_q8 does
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            lib_ms = 0.0
            for _ in range(reps):
                e0.record()
                torch.matmul(tx, tw.t())
                e1.record()
                torch.cuda.synchronize()
                lib_ms += e0.elapsed_time(e1)
            lib_us = lib_ms * 1e3 / reps
            # and back to back
            e0.record()
            for _ in range(reps):
                torch.matmul(tx, tw.t())
            e1.record()
            torch.cuda.synchronize()
            lib_b2b_us = e0.elapsed_time(e1) * 1e3 / reps
            flops = 2.0 * m * n * k
            rows.append({"gemm": name, "M": m, "N": n, "K": k,
                         "q8_us": round(ours_us, 2), "q8_frac": round(flops / ours_us * 1e-6 / PEAK_FP16_TFLOPS, 4),
                         "hipblaslt_fp16_us": round(lib_us, 2), "hipblaslt_fp16_back_to_back_us": round(lib_b2b_us, 2),
                         "hipblaslt_frac": round(flops / lib_us * 1e-6 / PEAK_FP16_TFLOPS, 4)})
            log(f"{name}: q8 {ours_us:.2f} us, hipBLASLt fp16 {lib_us:.2f} us ({lib_b2b_us:.2f} back to back)")
            del tx, tw
    finally:
        ctx.close()
    return rows


def cpu_threads() -> int:
    threads = len(os.sched_getaffinity(0))
    env_threads = os.environ.get("OMP_NUM_THREADS")
    if env_threads and env_threads.isdigit():
        threads = min(threads, int(env_threads))
    return threads


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def oracle_sample(model_path: str, texts, budget_s: float, label: str):
    """The oracle forward on this host's cores over whole texts until about budget_s seconds of CPU
    work: (pooled vectors of the texts done, tokens, seconds, threads)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ge_oracle as ora

    threads = cpu_threads()
    vectors, done_tokens, t_total = [], 0, 0.0
    with ora.OracleModel(model_path) as m:
        for seq in texts:
            t0 = time.perf_counter()
            pooled, _ = m.forward(seq, threads=threads)
            t_total += time.perf_counter() - t0
            vectors.append(pooled)
            done_tokens += len(seq)
            log(f"cpu oracle ({label}): {len(vectors)} texts, {t_total:.1f} s")
            if t_total >= budget_s:
                break
    return vectors, done_tokens, t_total, threads


def cpu_baseline(model_path: str, batch, budget_s: float = 12.0):
    """The oracle forward on this host's cores over whole texts of the workload until about
    budget_s seconds of CPU work, scaled to tokens/s; also returns the oracle's pooled vectors."""
    vectors, done_tokens, t_total, threads = oracle_sample(model_path, batch, budget_s, "config 2")
    n = len(vectors)
    return {"value": done_tokens / t_total, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{n} of the {len(batch)} config-2 texts ({done_tokens} tokens), oracle forward "
                      f"(ge_oracle.c, OpenMP {threads} threads), {t_total:.2f} s"}, vectors


def parity(gpu_vectors, oracle_vectors, dims=None):
    """Cosine and the largest difference of the L2-normalised vectors (Matryoshka-truncated to
    `dims` first when given), GPU against oracle, over the texts both computed (the reference's
    bars: cosine > 0.99999 and max abs difference < 1e-4, MetalForwardTests.swift:213-214)."""
    import numpy as np
    cos, mabs = 1.0, 0.0
    for g, o in zip(gpu_vectors, oracle_vectors):
        g, o = np.asarray(g, np.float64), np.asarray(o, np.float64)
        if dims:
            g, o = g[:dims], o[:dims]
        g, o = g / np.linalg.norm(g), o / np.linalg.norm(o)
        cos = min(cos, float(g @ o))
        mabs = max(mabs, float(np.abs(g - o).max()))
    return {"texts": min(len(gpu_vectors), len(oracle_vectors)), "min_cosine": round(cos, 9),
            "max_abs_normalised": float(f"{mabs:.3e}"), "bar_cosine": 0.99999, "bar_max_abs": 1e-4}


def config3_texts():
    """256 texts of lengths uniform in [8, 256] (SplitMix64 seed 31), ids uniform in
    [2, 262144) (seed 32)."""
    import gemma_embed as ge
    lengths = [int(n) for n in ge.synth_tokens(31, 8, 257, 256)]
    ids = ge.synth_tokens(32, 2, 262144, sum(lengths))
    texts, off = [], 0
    for n in lengths:
        texts.append([int(t) for t in ids[off:off + n]])
        off += n
    return texts


def config3_variant(model_path: str, reps: int, with_cpu: bool):
    """BASELINE config 3 through the host API at the reference's default options with Matryoshka 256:
    the 256 ragged texts are planned by token count (budget 8192), run, truncated to 256 dims and
    L2-normalised. Reports the host API's rate (ids in host memory -> normalised vectors, PCIe
    included), the GPU time of the device forwards of the same planned batches (each batch staged
    and run; its GPU seconds from events on the library's stream), and the oracle on a sample of
    the same texts on this host's cores, with the parity of those texts' vectors."""
    import numpy as np
    import gemma_embed as ge
    texts = config3_texts()
    tokens = sum(len(t) for t in texts)
    model = ge.EmbeddingModel.load(model_path)
    try:
        opts = ge.EmbedOptions(dimensions=256)
        out = model.embed(texts, opts)
        t0 = time.perf_counter()
        for _ in range(reps):
            out = model.embed(texts, opts)
        api_s = (time.perf_counter() - t0) / reps
        vecs = np.stack([e.vector for e in out])
        if vecs.shape != (256, 256) or not np.all(np.isfinite(vecs)):
            raise SystemExit("bad config-3 output")
        ranges = ge.plan_batches([len(t) for t in texts], [8192])
        ctx = model.context
        gpu_s = []
        for _ in range(reps):
            total = 0.0
            for r in ranges:
                total += ctx.forward(texts[r.start:r.stop])[1]
            gpu_s.append(total)
        gpu_s = sorted(gpu_s)[len(gpu_s) // 2]
    finally:
        model.close()
    # the same texts with split-precision scores on every layer (ge_load_options.split_scores)
    split = ge.EmbeddingModel.load(model_path, split_scores=True)
    try:
        svecs = np.stack([e.vector for e in split.embed(texts, opts)])
        sctx = split.context
        split_s = sorted(sum(sctx.forward(texts[r.start:r.stop])[1] for r in ranges) for _ in range(reps))
        split_s = split_s[len(split_s) // 2]
    finally:
        split.close()
    res = {"workload": "config3: 256 texts, lengths U[8, 256], planned by token count (budget 8192), "
                       "Matryoshka 256 + L2", "tokens": tokens, "planned_batches": len(ranges),
           "host_api_pcie_inclusive_tokens_per_s": round(tokens / api_s, 1),
           "gpu_forward_tokens_per_s": round(tokens / gpu_s, 1), "gpu_forward_ms": round(gpu_s * 1e3, 3),
           "split_scores": {"gpu_forward_tokens_per_s": round(tokens / split_s, 1),
                            "gpu_forward_ms": round(split_s * 1e3, 3)}}
    if with_cpu:
        oracle_vecs, done, secs, threads = oracle_sample(model_path, texts, 6.0, "config 3")
        res["cpu_oracle"] = {"tokens_per_s": round(done / secs, 1), "cores": threads, "kind": "port",
                             "sample": f"{len(oracle_vecs)} of the 256 texts ({done} tokens), {secs:.2f} s"}
        res["parity"] = parity(vecs, oracle_vecs, dims=256)
        res["split_scores"]["parity"] = parity(svecs, oracle_vecs, dims=256)
    return res


def config1_variant(model_path: str, with_cpu: bool):
    """one Q8_0 GEMM, X fp32 [128 x 768] ~ N(0, 1), W Q8_0 [1152 x 768]
    (blk.0.ffn_gate.weight of the synthetic config-2 model), Y fp32 [128 x 1152]: the oracle's
    sgemm on the dequantised weight (the reference caches the dequantised matrix,
    CPUReference.swift:31-38), median of 5 on this host's cores, and the GPU kernel
    (ge_op_gemm_q8 on fp16 X), median launch time."""
    import numpy as np
    import gemma_embed as ge
    with ge.GgufFile(model_path) as g:
        name, shape, typ, off = next(t for t in g.tensors() if t[0] == "blk.0.ffn_gate.weight")
        assert shape == [768, 1152] and typ == "Q8_0"
        raw = np.fromfile(model_path, dtype=np.uint8, count=1152 * 24 * 34, offset=g.data_offset + off)
    x = np.random.default_rng(1).standard_normal((128, 768)).astype(np.float32)
    flops = 2 * 128 * 1152 * 768
    res = {"workload": "config1: Y[128 x 1152] = X[128 x 768] W^T, W Q8_0", "flops": flops}
    ctx = ge.Context.create(0)
    try:
        w = ctx.q8_create(raw, 1152, 768)
        x16 = x.astype(np.float16)
        dx, dy = ctx.alloc(x16.nbytes), ctx.alloc(128 * 1152 * 4)
        try:
            ctx.upload(dx, x16)
            for _ in range(3):
                ctx.gemm_q8(w, dx, 128, dy, False)
            times = []
            for _ in range(20):
                ctx.profile_reset()
                ctx.profile_enable("gemm")
                ctx.gemm_q8(w, dx, 128, dy, False)
                times.append(ctx.profile_stats()["gemm"][1])
                ctx.profile_disable()
            y = ctx.download(dy, (128, 1152), np.float32)
        finally:
            ctx.free(dx)
            ctx.free(dy)
            ctx.q8_destroy(w)
    finally:
        ctx.close()
    gpu_ms = sorted(times)[len(times) // 2]
    res["gpu_ms"] = round(gpu_ms, 5)
    res["gpu_gflops"] = round(flops / (gpu_ms * 1e-3) / 1e9, 1)
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import ge_oracle as ora
        blocks = raw.reshape(-1, 34)  # Q8_0: fp16 scale, 32 int8 quants (Model/Weights.swift:33-41)
        wf = (blocks[:, :2].copy().view(np.float16).astype(np.float32) *
              blocks[:, 2:].view(np.int8).astype(np.float32)).reshape(1152, 768)
        threads = cpu_threads()
        cpu_times, want = [], None
        for _ in range(5):
            t0 = time.perf_counter()
            want = ora.matmul(x, wf, threads=threads)
            cpu_times.append(time.perf_counter() - t0)
        cpu_s = sorted(cpu_times)[2]
        res["cpu_oracle"] = {"ms": round(cpu_s * 1e3, 4), "gflops": round(flops / cpu_s / 1e9, 2), "cores": threads,
                             "kind": "port", "runs": 5, "statistic": "median"}
        res["max_rel_vs_oracle"] = float(f"{np.abs(y - want).max() / np.abs(want).max():.3e}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--model", default=None, help="existing config-2 GGUF (default: generate one)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="only compare the Q8_0 GEMM with hipBLASLt (torch.matmul) on the forward's projection "
                         "shapes and print that as one JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported "
                                   "(the forward shards as pure data parallelism, one context per GPU)"}))
        sys.exit(2)
    if args.library_gemm:
        print(json.dumps({"library_gemm": library_gemm_comparison(), "peak_tflops": PEAK_FP16_TFLOPS}))
        return

    import numpy as np
    import gemma_embed as ge

    tmp = tempfile.mkdtemp(prefix="ge_bench_")
    path = args.model or os.path.join(tmp, "config2.gguf")
    if not args.model:
        t0 = time.perf_counter()
        ge.synth_write_gguf(path, **ge.CONFIG2)
        log(f"wrote synthetic config-2 model in {time.perf_counter() - t0:.1f} s")
    ids = ge.synth_tokens(3, 2, 262144, TEXTS * TOKENS).reshape(TEXTS, TOKENS)
    batch = [r.tolist() for r in ids]
    n_tokens = TEXTS * TOKENS

    model = ge.EmbeddingModel.load(path, batch_token_budget=16384)
    ctx = model.context
    log(f"loaded on {model.info.device_name.decode()}")

    # ---- main measurement: one resident 16384-token pack per step
    ctx.batch_stage(batch)
    for _ in range(args.warmup):
        ctx.batch_run()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.batch_run()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    # The same K steps again with the GEMM launches stamped by their own dispatches
    # (hipExtLaunchKernelGGL start/stop events on the library's stream).
    ctx.profile_reset()
    ctx.profile_enable("gemm")
    t1 = time.perf_counter()
    for _ in range(args.steps):
        ctx.batch_run()
    ctx.sync()
    profiled_ms = (time.perf_counter() - t1) * 1e3 / args.steps
    stats = ctx.profile_stats()
    ctx.profile_disable()
    pooled = ctx.batch_read()
    if not np.all(np.isfinite(pooled)):
        raise SystemExit("non-finite pooled output")
    ms_per_step = elapsed * 1e3 / args.steps
    value = n_tokens / (elapsed / args.steps)
    log(f"resident pack: {ms_per_step:.3f} ms/step, {value:,.0f} tokens/s")

    flops = gemm_flops(n_tokens)
    step_gemm_flops = LAYERS * (flops["gemm_qkv"] + flops["gemm_o"] + flops["gemm_gate_up"] + flops["gemm_down"])
    dom = "gemm_gate_up"
    launches, total_ms = stats.get(dom, (0, 0.0))
    avg_ms = total_ms / max(launches, 1)
    achieved = flops[dom] / (avg_ms * 1e-3) / 1e12 if launches else 0.0
    gemm_ms = sum(v[1] for k, v in stats.items() if k in flops) / args.steps
    gemm_all = step_gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0

    # ---- per-kernel breakdown: a separate pass with every launch bracketed by events
    ctx.profile_reset()
    ctx.profile_enable("")
    for _ in range(3):
        ctx.batch_run()
    ctx.sync()
    all_stats = ctx.profile_stats()
    ctx.profile_disable()
    per_kernel = {k: {"launches_per_step": v[0] // 3, "avg_us": round(v[1] / max(v[0], 1) * 1e3, 2),
                      "ms_per_step": round(v[1] / 3, 4)} for k, v in all_stats.items()}

    # ---- variant: two device packs of 8192 tokens (the reference's default budget), restaged each step
    halves = [batch[:16], batch[16:]]
    for _ in range(2):
        for h in halves:
            ctx.forward(h)
    t0 = time.perf_counter()
    reps = max(3, args.steps // 2)
    for _ in range(reps):
        for h in halves:
            ctx.forward(h)
    default_budget = n_tokens * reps / (time.perf_counter() - t0)
    # ---- variant: the host API end to end at the reference's default options (ids in host memory
    # -> normalised 768-d vectors; batch token budget 8192, one forward per planned batch), and the
    # same with consecutive planned batches merged into device packs of up to 32768 tokens
    opts = ge.EmbedOptions()
    api_rates = {}
    for label, pack in (("default", 0), ("packs_32768", 32768)):
        api_model = ge.EmbeddingModel.load(path, pack_tokens=pack)
        try:
            api_model.embed(batch, opts)
            t0 = time.perf_counter()
            for _ in range(reps):
                api_model.embed(batch, opts)
            api_rates[label] = n_tokens * reps / (time.perf_counter() - t0)
        finally:
            api_model.close()
    api_rate = api_rates["default"]
    log(f"packs of 8192: {default_budget:,.0f} tok/s; embed API at default options {api_rate:,.0f} tok/s, "
        f"with device packs of up to 32768 tokens {api_rates['packs_32768']:,.0f} tok/s")
    # ---- variant: BASELINE config 4, 4 texts x 8192 tokens as one resident 32768-token pack
    long_texts, long_len = 4, 8192
    long_batch = [r.tolist() for r in ge.synth_tokens(8, 2, 262144, long_texts * long_len).reshape(long_texts, long_len)]
    ctx.batch_stage(long_batch)
    ctx.batch_run()
    ctx.sync()
    long_reps = 3
    t0 = time.perf_counter()
    for _ in range(long_reps):
        ctx.batch_run()
    ctx.sync()
    long_ms = (time.perf_counter() - t0) * 1e3 / long_reps
    long_rate = long_texts * long_len / (long_ms * 1e-3)
    if not np.all(np.isfinite(ctx.batch_read())):
        raise SystemExit("non-finite pooled output (config 4)")
    long_flops = LAYERS * sum(gemm_flops(long_texts * long_len)[k] for k in ("gemm_qkv", "gemm_o", "gemm_gate_up", "gemm_down")) \
        + projection_flops(long_texts) + attention_flops([long_len] * long_texts)
    log(f"config 4 (4 x 8192): {long_ms:.2f} ms/step, {long_rate:,.0f} tok/s")

    vision = vision_variant(tmp, max(3, args.steps // 2))
    image_embed = None
    if not args.model:  # the synthetic config-2 text tower is 768 wide, the tower's projection width
        image_embed = image_embed_variant(tmp, path, max(3, args.steps // 2))
        log(f"image embedding (tower + text tower, 8 images): {image_embed['ms_per_batch']:.2f} ms/batch, "
            f"{image_embed['images_per_s']:.1f} images/s")
    ref_shapes = reference_shapes_variant(tmp, max(3, args.steps // 4))
    log(f"reference shapes: 8 x 1024 in {ref_shapes['pack_8x1024_s'] * 1e3:.2f} ms "
        f"({ref_shapes['pack_8x1024_tokens_per_s']:,.0f} tok/s), 32 x 64 in {ref_shapes['pack_32x64_s'] * 1e3:.2f} ms, "
        f"8 x 256 in {ref_shapes['pack_8x256_s'] * 1e3:.2f} ms, 1 x 64 call {ref_shapes['call_1x64_ms']:.2f} ms, "
        f"12 queries as separate calls {ref_shapes['queries_12_separate_calls_ms']:.2f} ms")
    log(f"config 5 (8 images): {vision['ms_per_batch']:.2f} ms/batch, {vision['images_per_s']:.1f} images/s, "
        f"{vision['tflops']} TFLOP/s")

    total_flops = step_gemm_flops + attention_flops([TOKENS] * TEXTS) + projection_flops(TEXTS)
    traffic, traffic_kernel = measured_traffic(dom)
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "config2: 24-layer Q8_0 encoder, 32 texts x 512 tokens as one resident 16384-token pack",
                   "texts": TEXTS, "tokens_per_text": TOKENS, "batch_token_budget": 16384,
                   "model": "synthetic gemma-embedding2 d768 3q/1kv hd256 ff1152 vocab262144, window 512, 5:1 pattern"},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": f"profiles/{dom}_config2_traffic.md ({traffic_kernel})" if traffic else None,
                     "algorithmic_bytes": gemm_bytes(n_tokens)[dom],
                     "avg_launch_us": round(avg_ms * 1e3, 2), "flops_per_launch": flops[dom],
                     "profiled_ms_per_step": round(profiled_ms, 4)},
        "gemm_all": {"achieved": round(gemm_all, 2), "unit": "TFLOP/s", "frac": round(gemm_all / PEAK_FP16_TFLOPS, 4),
                     "ms_per_step": round(gemm_ms, 4)},
        "end_to_end_roofline_frac": round(total_flops / (ms_per_step * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
        "kernels": per_kernel,
        "variants": {"packs_of_8192_tokens_per_s": round(default_budget, 1),
                     "embed_api_default_options_pcie_inclusive_tokens_per_s": round(api_rate, 1),
                     "embed_api_packs_32768_pcie_inclusive_tokens_per_s": round(api_rates["packs_32768"], 1),
                     "config4_4x8192": {"tokens_per_s": round(long_rate, 1), "ms_per_step": round(long_ms, 3),
                                        "tflops": round(long_flops / (long_ms * 1e-3) / 1e12, 1)},
                     "config5_vision_8_images": vision,
                     "image_embedding_8_images": image_embed,
                     "reference_shapes_host_api": ref_shapes},
    }
    model.close()
    config3 = config3_variant(path, 3, not args.no_cpu)
    log(f"config 3 (256 ragged texts): GPU forwards {config3['gpu_forward_tokens_per_s']:,.0f} tok/s, host API "
        f"{config3['host_api_pcie_inclusive_tokens_per_s']:,.0f} tok/s")
    config1 = config1_variant(path, not args.no_cpu)
    log(f"config 1 (one Q8_0 GEMM 128 x 1152 x 768): GPU {config1['gpu_ms'] * 1e3:.1f} us")
    result["variants"]["config3_ragged_256"] = config3
    result["variants"]["config1_gemm"] = config1
    if not args.no_cpu:
        result["cpu_baseline"], oracle_vectors = cpu_baseline(path, batch)
        # the timed pack's own vectors (pooled, in text order) against the oracle's on the same texts
        result["parity"] = parity(pooled, oracle_vectors)
        log(f"parity over {result['parity']['texts']} texts: min cosine {result['parity']['min_cosine']}, "
            f"max abs {result['parity']['max_abs_normalised']}")
    print(json.dumps(result))


if __name__ == "__main__":
    main()
