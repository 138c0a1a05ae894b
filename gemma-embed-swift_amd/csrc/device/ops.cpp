// Per-op entry points for the row kernels of the forward (the reference's `Kernels`,
// Metal/MetalForward.swift:490-758): RMSNorm, the residual norms, QK norm + RoPE, the embedding
// gather and mean pooling, each running the forward's own kernel on caller device memory.
// Every entry checks the shapes its kernel assumes and validates the integer inputs it gathers
// with (token ids, positions, sequence ranges) on the host before launching.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "runtime_internal.hpp"

namespace ge {
namespace {

// Temporary device buffers of one call, freed when it returns.
struct Temps {
    std::vector<void*> ptrs;
    ~Temps() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <typename T>
    T* alloc(size_t count, const char* what) {
        void* p = dev_alloc(count * sizeof(T), what);
        ptrs.push_back(p);
        return static_cast<T*>(p);
    }
};

float* device_constant(ge_ctx* c, Temps& t, size_t n, float value) {
    std::vector<float> h(n, value);
    float* d = t.alloc<float>(n, "op constant");
    hip_check(hipMemcpy(d, h.data(), n * 4, hipMemcpyHostToDevice), "upload");
    (void)c;
    return d;
}

template <typename T>
std::vector<T> read_back(const void* src, size_t n) {
    std::vector<T> h(n);
    if (n) hip_check(hipMemcpy(h.data(), src, n * sizeof(T), hipMemcpyDeviceToHost), "read back");
    return h;
}

bool row_width_ok(int width) { return width > 0 && width % 4 == 0 && width <= 1024; }

}  // namespace
}  // namespace ge

using ge::fail;
using ge::guarded;

extern "C" {

int ge_op_rmsnorm(ge_ctx* c, const void* x, void* out, const void* w, int32_t rows, int32_t width, float eps,
                  float pre_scale) {
    return guarded(c, [&] {
        if (!x || !out || rows < 0 || !ge::row_width_ok(width))
            fail(GE_ERR_INVALID, "rmsnorm: rows >= 0 and a width that is a multiple of 4 up to 1024");
        if (rows == 0) return;
        ge::Temps t;
        // the forward's standalone norm: out = rmsnorm(x * mul * rscale[row / per_scale]) * w
        const float* one = ge::device_constant(c, t, 1, 1.0f);
        const float* wt = w ? static_cast<const float*>(w) : ge::device_constant(c, t, size_t(width), 1.0f);
        ge::launch(c, "rmsnorm", [&] {
            return ge::launch_ple_rmsnorm(c->stream, static_cast<const float*>(x), rows, width, pre_scale, one, rows, wt, eps,
                                          static_cast<float*>(out));
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_rmsnorm_residual(ge_ctx* c, void* x, const void* t16, const void* w, float scale, const void* next_w, void* h16,
                           int32_t rows, int32_t width, float eps) {
    return guarded(c, [&] {
        if (!x || !t16 || !w || rows < 0 || !ge::row_width_ok(width) || (next_w && !h16))
            fail(GE_ERR_INVALID, "rmsnorm_residual: x, t and w, h with next_w, a width that is a multiple of 4 up to 1024");
        if (rows == 0) return;
        ge::launch(c, "residual_norm", [&] {
            return ge::launch_residual_norm(c->stream, static_cast<float*>(x), static_cast<const uint16_t*>(t16), eps,
                                            static_cast<const float*>(w), scale, static_cast<const float*>(next_w), eps, rows,
                                            width, static_cast<uint16_t*>(h16));
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_qk_norm_rope(ge_ctx* c, const void* qkv, int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim,
                       const void* q_norm, const void* k_norm, float eps, const void* positions, float rope_base, void* q,
                       void* k, void* v) {
    return guarded(c, [&] {
        if (!qkv || !q_norm || !k_norm || !positions || !q || !k || !v || tokens < 0 || heads <= 0 || kv_heads <= 0 ||
            (head_dim != 128 && head_dim != 256 && head_dim != 512) || !(rope_base > 0.0f))
            fail(GE_ERR_INVALID, "qk_norm_rope: head dim 128, 256 or 512, positive head counts and RoPE base");
        if (tokens == 0) return;
        constexpr int kPositions = 8192;  // ModelConfig.supportedMaxTokens (Model/ModelConfig.swift:52)
        const std::vector<int32_t> pos = ge::read_back<int32_t>(positions, size_t(tokens));
        for (int i = 0; i < tokens; i++)
            if (pos[size_t(i)] < 0 || pos[size_t(i)] >= kPositions)
                fail(GE_ERR_INVALID, "position %d at row %d is outside [0, %d)", pos[size_t(i)], i, kPositions);
        const float* table = ge::rope_table(c, head_dim, rope_base, kPositions);
        ge::launch(c, "qk_norm_rope", [&] {
            return ge::launch_qk_norm_rope(c->stream, static_cast<const float*>(qkv), tokens, heads, kv_heads, head_dim,
                                           static_cast<const float*>(q_norm), static_cast<const float*>(k_norm), eps,
                                           static_cast<const int32_t*>(positions), table, static_cast<uint16_t*>(q),
                                           static_cast<uint16_t*>(k), static_cast<uint16_t*>(v));
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_embed(ge_ctx* c, const ge_q8_matrix* table, const void* tokens, int32_t n_tokens, float scale,
                const void* vectors, int32_t n_vectors, const void* norm_w, float eps, void* x, void* h16) {
    return guarded(c, [&] {
        if (!table || !tokens || !x || n_tokens < 0 || n_vectors < 0 || (n_vectors > 0 && !vectors) || (h16 && !norm_w))
            fail(GE_ERR_INVALID, "embed: table, tokens and x; vectors for vector rows; norm_w with h");
        const int d = table->m.cols;
        if (d % 32 || d > 1024) fail(GE_ERR_INVALID, "embed: rows of %d (a multiple of 32 up to 1024)", d);
        if (n_tokens == 0) return;
        const std::vector<int32_t> ids = ge::read_back<int32_t>(tokens, size_t(n_tokens));
        for (int i = 0; i < n_tokens; i++)
            if (ids[size_t(i)] < -n_vectors || ids[size_t(i)] >= table->m.rows)
                fail(GE_ERR_INVALID, "token %d at row %d is neither in the table [0, %d) nor one of the %d vector rows",
                     ids[size_t(i)], i, table->m.rows, n_vectors);
        ge::Temps t;
        const float* w = norm_w ? static_cast<const float*>(norm_w) : ge::device_constant(c, t, size_t(d), 1.0f);
        uint16_t* h = h16 ? static_cast<uint16_t*>(h16) : t.alloc<uint16_t>(size_t(n_tokens) * d, "embed h");
        ge::launch(c, "embed_norm", [&] {
            return ge::launch_embed_norm(c->stream, table->m, static_cast<const int32_t*>(tokens), n_tokens, scale,
                                         static_cast<const float*>(vectors), w, eps, static_cast<float*>(x), h);
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_mean_pool(ge_ctx* c, const void* x, int32_t rows, int32_t width, const void* seqs, int32_t n_seqs,
                    void* pooled) {
    return guarded(c, [&] {
        if (!x || !seqs || !pooled || rows < 0 || width <= 0 || n_seqs < 0)
            fail(GE_ERR_INVALID, "mean_pool: x, sequences and output with non-negative sizes");
        if (width % 4) fail(GE_ERR_INVALID, "mean_pool: width %d is not a multiple of 4", width);
        if (n_seqs == 0) return;
        const std::vector<ge_seq> sq = ge::read_back<ge_seq>(seqs, size_t(n_seqs));
        for (int s = 0; s < n_seqs; s++)
            if (uint64_t(sq[size_t(s)].start) + sq[size_t(s)].length > uint64_t(rows))
                fail(GE_ERR_INVALID, "sequence %d [%u, +%u) runs past the %d rows", s, sq[size_t(s)].start,
                     sq[size_t(s)].length, rows);
        ge::launch(c, "mean_pool", [&] {
            return ge::launch_mean_pool(c->stream, static_cast<const float*>(x), static_cast<const ge::SeqRange*>(seqs), n_seqs,
                                        width, static_cast<float*>(pooled));
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

}  // extern "C"
