// ge_probe: a small standalone program for profilers (rocprofv3 kernel traces and counters).
//
// It runs one kernel of the forward at its config-2 shape through the C-ABI, with no Python and
// no model file, so a profiler sees a short program with few dispatches:
//
//   ge_probe gate_up [reps]   the gate/up GEMM with the GeGLU epilogue (ge_op_gemm_q8_geglu:
//                             M = 16384 tokens, K = 768, F = 1152 gate and 1152 up rows), the
//                             forward's dominant kernel (Kernels.gemm with the geglu epilogue,
//                             Metal/MetalForward.swift:524-557; Shaders/GEMM.metal:41-67)
//   ge_probe attention [reps] the attention of a sliding-window layer (ge_op_attention: 32
//                             sequences of 512 tokens, 3 query heads, 1 KV head, head dim 256,
//                             half window 256; Kernels.attention, Metal/MetalForward.swift:669-694)
//   ge_probe embed [reps]     the host API end to end on config 2 (a synthetic 24-layer model
//                             written to a temporary GGUF; 32 texts x 512 ids): the time per
//                             call of ge_model_embed at the 8192- and 16384-token budgets, and
//                             of the resident pack (ge_batch_run) for comparison
//   ge_probe vision [reps]    BASELINE config 5: the synthetic 16-layer image tower (written to a
//                             temporary GGUF) over 8 resident images of 48 x 48 patches
//                             (ge_vision_run), the time per batch
//   ge_probe reference_shapes [reps]
//                             the reference's own architecture at its real shapes (d 512, 4 query
//                             heads, KV 2 x 256 sliding / 1 x 512 global, GeGLU 2048, per-layer
//                             inputs 512, 24 layers; synthetic weights): a resident 8 x 1024-token
//                             pack and a 1 x 64-token pack (ge_batch_run), the time per forward
//   ge_probe forward [reps] [parts]
//                             the whole config-2 forward (synthetic 24-layer model, a resident pack of
//                             32 x 512 tokens): every kernel class of the text path at its config-2
//                             shape. By default on one stream with every launch timed by HIP events
//                             (ge_profile_enable), so each kernel runs at M = 16384 and the probe
//                             prints a per-kernel table; with "parts" the pack runs as the timed
//                             forward does (four parts on four streams, no events)
//   ge_probe reference_forward [reps]
//                             the same for the reference's real architecture (8 x 1024 tokens)
//   ge_probe calibrate        fp16 -> fp32 conversion of 2^28 values (reads 512 MiB, writes 1 GiB):
//                             the known-size kernel that scales the HBM byte counters
//
// Inputs are synthetic: Q8_0 rows with random int8 quants and fp16 scales, activations uniform
// in [-0.5, 0.5). Each call of the GeGLU entry point also interleaves the two matrices and builds
// their fragment-order copy; a profile reads the GEMM kernel's own rows.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gemmaembed.h"
#include "halfconv.hpp"
#include "prng.hpp"

namespace {

int fail(ge_ctx* c, const char* what) {
    std::fprintf(stderr, "ge_probe: %s: %s\n", what, c ? ge_last_error(c) : ge_create_error());
    if (c) ge_destroy(c);
    return 1;
}

// Q8_0 rows: per 32 values an fp16 scale then 32 int8 quants (34 bytes).
std::vector<uint8_t> synth_q8(uint64_t seed, int rows, int cols) {
    ge::SeededRandom rng(seed);
    std::vector<uint8_t> raw((size_t)rows * (cols / 32) * 34);
    for (size_t b = 0; b < raw.size() / 34; b++) {
        uint8_t* blk = raw.data() + b * 34;
        const uint16_t s = ge::float_to_half(float(0.0005 + 0.001 * rng.unit()));
        std::memcpy(blk, &s, 2);
        for (int i = 0; i < 32; i++) blk[2 + i] = uint8_t(int8_t(int(rng.next() % 255) - 127));
    }
    return raw;
}

int probe_gate_up(ge_ctx* c, int reps) {
    const int M = 16384, K = 768, F = 1152;
    ge_q8_matrix *gate = nullptr, *up = nullptr;
    const std::vector<uint8_t> g = synth_q8(11, F, K), u = synth_q8(12, F, K);
    if (ge_op_q8_create(c, g.data(), F, K, &gate) != 0) return fail(c, "q8_create");
    if (ge_op_q8_create(c, u.data(), F, K, &up) != 0) return fail(c, "q8_create");
    std::vector<uint16_t> x((size_t)M * K);
    ge::SeededRandom rng(13);
    for (auto& v : x) v = ge::float_to_half(float(rng.unit() - 0.5));
    void* dx = ge_dev_alloc(c, x.size() * 2);
    void* da = ge_dev_alloc(c, (size_t)M * F * 2);
    if (!dx || !da) return fail(c, "dev_alloc");
    if (ge_dev_upload(c, dx, x.data(), x.size() * 2) != 0) return fail(c, "dev_upload");
    for (int r = 0; r < reps; r++)
        if (ge_op_gemm_q8_geglu(c, gate, up, dx, M, da) != 0) return fail(c, "gemm_q8_geglu");
    std::printf("ge_probe gate_up: %d launches of M=%d K=%d F=%d done\n", reps, M, K, F);
    std::fflush(stdout);
    ge_dev_free(c, dx);
    ge_dev_free(c, da);
    ge_op_q8_destroy(c, gate);
    ge_op_q8_destroy(c, up);
    return 0;
}

int probe_attention(ge_ctx* c, int reps) {
    const int S = 32, L = 512, T = S * L, H = 3, KV = 1, HD = 256, slack = 64;
    ge::SeededRandom rng(14);
    auto rand_f16 = [&](size_t n, double amp) {
        std::vector<uint16_t> v(n);
        for (auto& x : v) x = ge::float_to_half(float(amp * (rng.unit() - 0.5)));
        return v;
    };
    const std::vector<uint16_t> q = rand_f16((size_t)(T + slack) * H * HD, 3.0);
    const std::vector<uint16_t> k = rand_f16((size_t)(T + slack) * KV * HD, 2.0);
    const std::vector<uint16_t> v = rand_f16((size_t)(T + slack) * KV * HD, 2.0);
    std::vector<ge_attention_work> work;
    const int qpw = ge_attention_queries();
    for (int s = 0; s < S; s++)
        for (int q0 = 0; q0 < L; q0 += qpw) work.push_back(ge_attention_work{uint32_t(s * L), uint32_t(L), uint32_t(q0)});
    void* dq = ge_dev_alloc(c, q.size() * 2);
    void* dk = ge_dev_alloc(c, k.size() * 2);
    void* dv = ge_dev_alloc(c, v.size() * 2);
    void* dout = ge_dev_alloc(c, q.size() * 2);
    void* dw = ge_dev_alloc(c, work.size() * sizeof(ge_attention_work));
    if (!dq || !dk || !dv || !dout || !dw) return fail(c, "dev_alloc");
    if (ge_dev_upload(c, dq, q.data(), q.size() * 2) != 0 || ge_dev_upload(c, dk, k.data(), k.size() * 2) != 0 ||
        ge_dev_upload(c, dv, v.data(), v.size() * 2) != 0 ||
        ge_dev_upload(c, dw, work.data(), work.size() * sizeof(ge_attention_work)) != 0)
        return fail(c, "dev_upload");
    for (int r = 0; r < reps; r++)
        if (ge_op_attention(c, dq, dk, dv, dout, dw, int32_t(work.size()), H, KV, HD, 256, 1.0f) != 0)
            return fail(c, "attention");
    std::printf("ge_probe attention: %d launches of %d x %d tokens, H=%d KV=%d hd=%d, half window 256 done\n", reps, S,
                L, H, KV, HD);
    std::fflush(stdout);
    for (void* p : {dq, dk, dv, dout, dw}) ge_dev_free(c, p);
    return 0;
}

int probe_embed(int reps) {
    // BASELINE config 2's model shape (the Python package's CONFIG2)
    uint8_t pattern[24];
    for (int l = 0; l < 24; l++) pattern[l] = (l % 6 == 5) ? 0 : 1;
    ge_synth_spec spec{};
    spec.layers = 24, spec.hidden = 768, spec.heads = 3, spec.feed_forward = 1152, spec.out_dims = 768;
    spec.per_layer_input = 0, spec.vocab = 262144, spec.sliding_window = 512;
    spec.head_dim_swa = 256, spec.head_dim_global = 256, spec.kv_heads_swa = 1, spec.kv_heads_global = 1;
    spec.eps = 1e-6f, spec.rope_base = 1e6f, spec.rope_base_swa = 1e4f, spec.pattern = pattern, spec.seed = 4;
    char err[512] = {0};
    const char* path = "/tmp/ge_probe_config2.gguf";
    if (ge_synth_write_gguf(path, &spec, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: synth: %s\n", err);
        return 1;
    }
    const int texts = 32, len = 512;
    std::vector<int32_t> ids(size_t(texts) * len), lengths(texts, len);
    ge_synth_tokens(3, 2, 262144, texts * len, ids.data());
    std::vector<float> out(size_t(texts) * 768);
    for (int budget : {8192, 16384}) {
        ge_load_options lo{0, budget, 1};
        ge_model* m = nullptr;
        if (ge_model_load(path, &lo, &m, err, sizeof err) != 0) {
            std::fprintf(stderr, "ge_probe: load: %s\n", err);
            return 1;
        }
        ge_embed_options eo{2048, 768, 1, 0};
        auto call = [&] {
            return ge_model_embed(m, ids.data(), lengths.data(), texts, &eo, out.data(), nullptr, nullptr, nullptr, nullptr);
        };
        for (int r = 0; r < 2; r++)
            if (call() != 0) return std::fprintf(stderr, "ge_probe: embed: %s\n", ge_model_last_error(m)), 1;
        const auto t0 = std::chrono::steady_clock::now();
        for (int r = 0; r < reps; r++)
            if (call() != 0) return std::fprintf(stderr, "ge_probe: embed: %s\n", ge_model_last_error(m)), 1;
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / reps;
        std::printf("ge_model_embed, budget %d: %.3f ms per call of %d x %d ids, %.0f tokens/s\n", budget, ms, texts, len,
                    texts * len / (ms * 1e-3));
        if (budget == 16384) {
            ge_ctx* c = ge_model_context(m);
            std::vector<int32_t> pos(ids.size());
            std::vector<ge_seq> seqs(texts);
            for (int t = 0; t < texts; t++) {
                seqs[t] = ge_seq{uint32_t(t * len), uint32_t(len)};
                for (int i = 0; i < len; i++) pos[size_t(t) * len + i] = i;
            }
            if (ge_batch_stage(c, ids.data(), pos.data(), int32_t(ids.size()), seqs.data(), texts) != 0) return fail(c, "stage");
            for (int r = 0; r < 2; r++) ge_batch_run(c);
            ge_sync(c);
            const auto t1 = std::chrono::steady_clock::now();
            for (int r = 0; r < reps; r++) ge_batch_run(c);
            ge_sync(c);
            const double rms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t1).count() / reps;
            const auto t2 = std::chrono::steady_clock::now();
            for (int r = 0; r < reps; r++) {
                ge_batch_stage(c, ids.data(), pos.data(), int32_t(ids.size()), seqs.data(), texts);
                ge_batch_run(c);
                ge_batch_read(c, out.data());
            }
            const double sms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t2).count() / reps;
            std::printf("resident pack: %.3f ms per forward; stage + run + read: %.3f ms\n", rms, sms);
        }
        std::fflush(stdout);
        ge_model_free(m);
    }
    std::remove(path);
    return 0;
}

int probe_vision(ge_ctx* c, int reps) {
    ge_synth_vision_spec spec{};
    spec.layers = 16, spec.hidden = 1152, spec.heads = 16, spec.feed_forward = 4304, spec.patch_size = 16;
    spec.merge = 3, spec.proj_dims = 768, spec.positions = 48, spec.eps = 1e-6f, spec.ffn_down_type = 0, spec.seed = 5;
    char err[512] = {0};
    const char* path = "/tmp/ge_probe_config5_vision.gguf";
    if (ge_synth_write_vision_gguf(path, &spec, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: synth: %s\n", err);
        return 1;
    }
    if (ge_vision_load(c, path, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: vision load: %s\n", err);
        return 1;
    }
    std::remove(path);
    const int images = 8, grid = 48, area = 768;
    std::vector<float> patches(size_t(images) * grid * grid * area);
    ge_synth_uniform(51, -1.0f, 1.0f, int64_t(patches.size()), patches.data());
    std::vector<ge_image_grid> grids(images, ge_image_grid{grid, grid});
    if (ge_vision_stage(c, patches.data(), images * grid * grid, grids.data(), images) != 0) return fail(c, "vision stage");
    for (int r = 0; r < 2; r++)
        if (ge_vision_run(c) != 0) return fail(c, "vision run");
    ge_sync(c);
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; r++)
        if (ge_vision_run(c) != 0) return fail(c, "vision run");
    ge_sync(c);
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / reps;
    std::vector<float> out(size_t(images) * 256 * 768);
    if (ge_vision_read(c, out.data(), out.size()) != 0) return fail(c, "vision read");
    std::printf("config 5 image tower: %.3f ms per batch of %d images, %.1f images/s\n", ms, images, images / (ms * 1e-3));
    std::fflush(stdout);
    return 0;
}

int probe_reference_shapes(int reps) {
    uint8_t pattern[24];
    for (int i = 0; i < 24; i++) pattern[i] = (i % 6 == 5) ? 0 : 1;
    ge_synth_spec spec{};
    spec.layers = 24, spec.hidden = 512, spec.heads = 4, spec.feed_forward = 2048, spec.out_dims = 768;
    spec.per_layer_input = 512, spec.vocab = 262144, spec.sliding_window = 1024;
    spec.head_dim_swa = 256, spec.head_dim_global = 512, spec.kv_heads_swa = 2, spec.kv_heads_global = 1;
    spec.eps = 1e-6f, spec.rope_base = 1e6f, spec.rope_base_swa = 1e4f, spec.pattern = pattern, spec.seed = 12;
    char err[512] = {0};
    const char* path = "/tmp/ge_probe_reference_shapes.gguf";
    if (ge_synth_write_gguf(path, &spec, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: synth: %s\n", err);
        return 1;
    }
    ge_load_options lo{0, 8192, 1};
    ge_model* m = nullptr;
    if (ge_model_load(path, &lo, &m, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: load: %s\n", err);
        return 1;
    }
    std::remove(path);
    ge_ctx* c = ge_model_context(m);
    const int shapes[2][2] = {{8, 1024}, {1, 64}};
    for (const auto& shape : shapes) {
        const int texts = shape[0], len = shape[1];
        std::vector<int32_t> ids(size_t(texts) * len), pos(ids.size());
        std::vector<ge_seq> seqs(static_cast<size_t>(texts));
        ge_synth_tokens(3, 2, 262144, int32_t(ids.size()), ids.data());
        for (int t = 0; t < texts; t++) {
            seqs[size_t(t)] = ge_seq{uint32_t(t * len), uint32_t(len)};
            for (int i = 0; i < len; i++) pos[size_t(t) * len + i] = i;
        }
        if (ge_batch_stage(c, ids.data(), pos.data(), int32_t(ids.size()), seqs.data(), texts) != 0) return fail(c, "stage");
        for (int r = 0; r < 3; r++) ge_batch_run(c);
        ge_sync(c);
        const auto t0 = std::chrono::steady_clock::now();
        for (int r = 0; r < reps; r++) ge_batch_run(c);
        ge_sync(c);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / reps;
        std::printf("reference shapes, %d x %d tokens: %.3f ms per resident forward, %.0f tokens/s\n", texts, len, ms,
                    texts * len / (ms * 1e-3));
        std::fflush(stdout);
    }
    ge_model_free(m);
    return 0;
}

// The whole image embedding: config 5's 8 images through the tower, then each image's 260 framed
// rows through the 24-layer config-2 text tower (ge_image_forward), GPU time of both towers.
int probe_image_embed(int reps) {
    uint8_t pattern[24];
    for (int i = 0; i < 24; i++) pattern[i] = (i % 6 == 5) ? 0 : 1;
    ge_synth_spec spec{};
    spec.layers = 24, spec.hidden = 768, spec.heads = 3, spec.feed_forward = 1152, spec.out_dims = 768;
    spec.per_layer_input = 0, spec.vocab = 262144, spec.sliding_window = 512;
    spec.head_dim_swa = 256, spec.head_dim_global = 256, spec.kv_heads_swa = 1, spec.kv_heads_global = 1;
    spec.eps = 1e-6f, spec.rope_base = 1e6f, spec.rope_base_swa = 1e4f, spec.pattern = pattern, spec.seed = 4;
    char err[512] = {0};
    const char* path = "/tmp/ge_probe_config2.gguf";
    if (ge_synth_write_gguf(path, &spec, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: synth: %s\n", err);
        return 1;
    }
    ge_load_options lo{0, 8192, 1};
    ge_model* m = nullptr;
    if (ge_model_load(path, &lo, &m, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: load: %s\n", err);
        return 1;
    }
    std::remove(path);
    ge_ctx* c = ge_model_context(m);
    ge_synth_vision_spec vs{};
    vs.layers = 16, vs.hidden = 1152, vs.heads = 16, vs.feed_forward = 4304, vs.patch_size = 16;
    vs.merge = 3, vs.proj_dims = 768, vs.positions = 48, vs.eps = 1e-6f, vs.ffn_down_type = 0, vs.seed = 5;
    const char* vpath = "/tmp/ge_probe_config5_vision.gguf";
    if (ge_synth_write_vision_gguf(vpath, &vs, err, sizeof err) != 0 || ge_vision_load(c, vpath, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: vision: %s\n", err);
        return 1;
    }
    std::remove(vpath);
    const int images = 8, grid = 48, area = 768;
    std::vector<float> patches(size_t(images) * grid * grid * area), pooled(size_t(images) * 768);
    ge_synth_uniform(52, -1.0f, 1.0f, int64_t(patches.size()), patches.data());
    std::vector<ge_image_grid> grids(images, ge_image_grid{grid, grid});
    const int32_t markers[4] = {2, 255998, 255999, 1};
    std::vector<double> secs;
    for (int r = 0; r < reps + 2; r++) {
        double s = 0;
        if (ge_image_forward(c, patches.data(), images * grid * grid, grids.data(), images, markers, pooled.data(), &s) != 0)
            return fail(c, "image forward");
        if (r >= 2) secs.push_back(s);
    }
    std::sort(secs.begin(), secs.end());
    const double ms = secs[secs.size() / 2] * 1e3;
    std::printf("image embedding (config 5 tower + config-2 text tower): %.3f ms per batch of %d images, %.1f images/s\n",
                ms, images, images / (ms * 1e-3));
    std::fflush(stdout);
    ge_model_free(m);
    return 0;
}

// A synthetic model written to a temporary GGUF and loaded (config 2, or the reference's real
// shapes), the file removed once loaded.
ge_model* load_synthetic(bool real_shapes) {
    static uint8_t pattern[24];
    for (int l = 0; l < 24; l++) pattern[l] = (l % 6 == 5) ? 0 : 1;
    ge_synth_spec spec{};
    spec.layers = 24, spec.heads = real_shapes ? 4 : 3, spec.out_dims = 768, spec.vocab = 262144;
    spec.hidden = real_shapes ? 512 : 768, spec.feed_forward = real_shapes ? 2048 : 1152;
    spec.per_layer_input = real_shapes ? 512 : 0, spec.sliding_window = real_shapes ? 1024 : 512;
    spec.head_dim_swa = 256, spec.head_dim_global = real_shapes ? 512 : 256;
    spec.kv_heads_swa = real_shapes ? 2 : 1, spec.kv_heads_global = 1;
    spec.eps = 1e-6f, spec.rope_base = 1e6f, spec.rope_base_swa = 1e4f, spec.pattern = pattern;
    spec.seed = real_shapes ? 12 : 4;
    char err[512] = {0};
    const char* path = real_shapes ? "/tmp/ge_probe_reference_shapes.gguf" : "/tmp/ge_probe_config2.gguf";
    if (ge_synth_write_gguf(path, &spec, err, sizeof err) != 0) {
        std::fprintf(stderr, "ge_probe: synth: %s\n", err);
        return nullptr;
    }
    ge_load_options lo{0, 16384, 1};
    ge_model* m = nullptr;
    if (ge_model_load(path, &lo, &m, err, sizeof err) != 0) std::fprintf(stderr, "ge_probe: load: %s\n", err);
    std::remove(path);
    return m;
}

// The whole forward over a resident pack (config 2: 32 x 512; real shapes: 8 x 1024), per-kernel
// HIP-event times unless `parts`.
int probe_forward(int reps, bool real_shapes, bool parts) {
    ge_model* m = load_synthetic(real_shapes);
    if (!m) return 1;
    ge_ctx* c = ge_model_context(m);
    const int texts = real_shapes ? 8 : 32, len = real_shapes ? 1024 : 512;
    std::vector<int32_t> ids(size_t(texts) * len), pos(ids.size());
    std::vector<ge_seq> seqs(static_cast<size_t>(texts));
    ge_synth_tokens(3, 2, 262144, int32_t(ids.size()), ids.data());
    for (int t = 0; t < texts; t++) {
        seqs[size_t(t)] = ge_seq{uint32_t(t * len), uint32_t(len)};
        for (int i = 0; i < len; i++) pos[size_t(t) * len + i] = i;
    }
    if (ge_batch_stage(c, ids.data(), pos.data(), int32_t(ids.size()), seqs.data(), texts) != 0) return fail(c, "stage");
    for (int r = 0; r < 2; r++) ge_batch_run(c);
    ge_sync(c);
    if (!parts) ge_profile_enable(c, "");
    ge_profile_reset(c);
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; r++)
        if (ge_batch_run(c) != 0) return fail(c, "run");
    std::vector<float> out(size_t(texts) * 768);
    if (ge_batch_read(c, out.data()) != 0) return fail(c, "read");
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / reps;
    double check = 0;
    for (float v : out) check += std::fabs(double(v));
    std::printf("%s forward, %d x %d tokens (%s): %.3f ms per forward; sum |pooled| %.6e\n",
                real_shapes ? "reference shapes" : "config 2", texts, len,
                parts ? "parts on four streams" : "one stream, every launch timed", ms, check);
    if (!parts) {
        std::printf("%-24s %9s %10s %12s\n", "kernel", "launches", "avg us", "ms/forward");
        for (int i = 0;; i++) {
            const char* name = nullptr;
            int64_t n = 0;
            double total = 0;
            if (ge_profile_get(c, i, &name, &n, &total) != 0) break;
            std::printf("%-24s %9lld %10.2f %12.4f\n", name, (long long)(n / reps), total / double(n) * 1e3, total / reps);
        }
        ge_profile_disable(c);
    }
    std::fflush(stdout);
    ge_model_free(m);
    return 0;
}

int probe_calibrate(ge_ctx* c) {
    const size_t n = size_t(1) << 28;
    void* src = ge_dev_alloc(c, 2 * n);
    void* dst = ge_dev_alloc(c, 4 * n);
    if (!src || !dst) return fail(c, "dev_alloc");
    if (ge_op_f16_to_f32(c, src, dst, n) != 0) return fail(c, "f16_to_f32");
    std::printf("ge_probe calibrate: converted %zu values (reads %zu, writes %zu bytes)\n", n, 2 * n, 4 * n);
    std::fflush(stdout);
    ge_dev_free(c, src);
    ge_dev_free(c, dst);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const char* what = argc > 1 ? argv[1] : "gate_up";
    const int reps = argc > 2 ? std::atoi(argv[2]) : 20;
    if (std::strcmp(what, "embed") == 0) return reps < 1 || reps > 10000 ? 2 : probe_embed(reps);
    if (std::strcmp(what, "reference_shapes") == 0) return reps < 1 || reps > 10000 ? 2 : probe_reference_shapes(reps);
    if (std::strcmp(what, "image_embed") == 0) return reps < 1 || reps > 10000 ? 2 : probe_image_embed(reps);
    if (std::strcmp(what, "forward") == 0 || std::strcmp(what, "reference_forward") == 0)
        return reps < 1 || reps > 10000 ? 2
                                        : probe_forward(reps, what[0] == 'r', argc > 3 && std::strcmp(argv[3], "parts") == 0);
    if (std::strcmp(what, "gate_up") != 0 && std::strcmp(what, "attention") != 0 && std::strcmp(what, "calibrate") != 0 &&
        std::strcmp(what, "vision") != 0) {
        std::fprintf(stderr, "usage: ge_probe gate_up|attention|embed|vision|reference_shapes|image_embed|forward|reference_forward [reps] | ge_probe calibrate\n");
        return 2;
    }
    if (reps < 1 || reps > 10000) {
        std::fprintf(stderr, "ge_probe: reps must be in [1, 10000]\n");
        return 2;
    }
    ge_ctx* c = nullptr;
    if (ge_create(0, &c) != 0) return fail(nullptr, "create");
    std::printf("ge_probe on %s\n", ge_device_name(c));
    std::fflush(stdout);
    const int rc = std::strcmp(what, "calibrate") == 0   ? probe_calibrate(c)
                   : std::strcmp(what, "attention") == 0 ? probe_attention(c, reps)
                   : std::strcmp(what, "vision") == 0    ? probe_vision(c, reps)
                                                         : probe_gate_up(c, reps);
    if (rc == 0) ge_destroy(c);
    return rc;
}
