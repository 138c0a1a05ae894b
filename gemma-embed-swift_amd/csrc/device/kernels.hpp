// Host-side launchers of the gfx950 kernels. Every launcher checks the shapes its kernel
// assumes and returns hipErrorInvalidValue instead of launching when they do not hold.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ge {

// One block of query rows of one packed sequence (AttentionWork, Shaders/Common.metal:75-79),
// plus the column of the sequence's first key in the transposed V buffer (a multiple of 8).
struct AttnWork {
    uint32_t seq_start;
    uint32_t seq_len;
    uint32_t q0;
    uint32_t vt_start;
};

struct SeqRange {
    uint32_t start;
    uint32_t length;
};

// Query rows per attention work item.
constexpr int kAttnQueries = 32;
// Rows of slack every activation buffer keeps past its last token, so tile loads of the last
// GEMM row block and of the last attention query/key block stay inside the allocation.
constexpr int kRowSlack = 256;

// A Q8_0 matrix in device memory. q / s: the row-major planes, quants [rows][cols] int8 and scales
// [rows][cols / 32] fp16 (raw bits). fh: for GEMM weights, the dequantised matrix (fp16 of q * d,
// rounded once) in MFMA fragment order: for 32-row block j and 16-wide k-step t, 512 halves at
// ((j * cols / 16) + t) * 512 where lane l's 8 halves are row 32 j + l % 32, columns
// 16 t + 8 (l / 32) + [0, 8) -- the B operand of one v_mfma_f32_32x32x16_f16.
struct Q8Dev {
    int rows = 0, cols = 0;
    int8_t* q = nullptr;
    uint16_t* s = nullptr;
    uint16_t* fh = nullptr;
};

// Device-side dequantisation of w's row-major planes into Q8Dev::fh order (fh holds rows * cols
// halves; rows a multiple of 32).
hipError_t launch_q8_fragments(hipStream_t s, const Q8Dev& w, uint16_t* fh);

enum GemmEpilogue { kEpiF32 = 0, kEpiF16 = 1, kEpiGeglu = 2, kEpiGeluBias = 3, kEpiHeads = 4 };

// Operands of the bias epilogues of the image tower. kEpiGeluBias: fp16
// y[M][N] = gelu_tanh(acc + bias) * out_scale. kEpiHeads: fp16 (acc + bias) * out_scale into three
// head-padded buffers: column n = (part * heads + head) * hd + e of the product goes to dst[part]
// at [row][head][e], row stride heads * hp; columns hd .. hp of each head are not written.
struct GemmEpiArgs {
    const float* bias = nullptr;
    uint16_t* dst[3] = {nullptr, nullptr, nullptr};
    int hd = 0, hp = 0, heads = 0;
};

// y[M][N] = (x[M][K] (fp16) * W[N][K]^T (Q8_0, through W.fh)) * out_scale; N a multiple of 64,
// K of 32. kEpiGeglu expects W's rows
// interleaved in 32-row gate/up groups and writes fp16 act[M][N / 2] = gelu_tanh(gate) * up *
// out_scale. out_scale is a power of two wherever the forward uses it, so it is exact.
// Batches of at most kSkinnyMaxRows rows (and K a multiple of 128) run on the skinny kernel,
// one wave per 32-row by 32-column block; the results are bitwise those of the tiled kernel.
// Up to 512 rows the skinny kernel is the faster of the two at every projection of the
// config-2 and real-architecture models (at 128 rows 4-6 against 8-18 us; 512 rows is about
// the crossover), since the tiled kernel's few workgroups sit on a few CUs.
constexpr int kSkinnyMaxRows = 512;
// kEpiGeluBias and kEpiHeads take their operands from ea (y is then unused by kEpiHeads).
hipError_t launch_gemm_q8(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale = 1.0f, const GemmEpiArgs* ea = nullptr);

// The QKV projection with the per-head norms and RoPE in its epilogue: the GEMM's fp32 result,
// rounded to fp16 as qkv * scale (scale a power of two; eps is eps_model * scale^2), then the
// same as launch_qk_norm_rope / launch_qkv_norm_rope_vt: q [T][H][hd], k, v [T][KV][hd] fp16,
// and when vt is set, normalised V transposed: vt [KV * hd][vt_cols], token t at column vcol[t]
// (v may then be null: row-major V is not written). W's rows are the H query heads, then KV key
// heads, then KV value heads.
struct QkvEpilogue {
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    const int32_t* positions = nullptr;
    const float* rope = nullptr;  // [position][hd / 2] (cos, sin) pairs
    uint16_t* q = nullptr;
    uint16_t* k = nullptr;
    uint16_t* v = nullptr;
    const int32_t* vcol = nullptr;
    uint16_t* vt = nullptr;
    float scale = 1.0f;
    float eps = 0.0f;
    int vt_cols = 0;
    int heads = 0;
    int kv_heads = 0;
    // fp16 scratch of at least M * N halves: lets short batches (M <= kSkinnyMaxRows) take the
    // skinny GEMM and a separate row pass, with the same results; null = always the fused kernel
    uint16_t* stage = nullptr;
};
bool gemm_qkv_supported(int hd, int H, int KV);
hipError_t launch_gemm_qkv(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, int hd, const QkvEpilogue& e);

// x = table[id] * scale (fp32 [T][d]), or row -(id + 1) of vectors (fp32 [rows][d]) unscaled for a
// negative id; h = rmsnorm(x) * w (fp16 [T][d]).
hipError_t launch_embed_norm(hipStream_t s, const Q8Dev& table, const int32_t* tokens, int T, float scale,
                             const float* vectors, const float* norm_w, float eps, float* x, uint16_t* h);

// x = (x + rmsnorm(t) * w) * out_scale; if next_w: h = rmsnorm(x) * next_w (fp16), or into h32 in
// fp32 when h32 is given (the final norm, whose rows are pooled before the output projection).
// t arrives as fp16 t16 = t * c for a power of two c, and t_eps = eps * c^2, so rmsnorm(t16)
// with t_eps is rmsnorm(t) exactly. d a multiple of 4, at most 1024.
hipError_t launch_residual_norm(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w,
                                float out_scale, const float* next_w, float eps, int T, int d, uint16_t* h,
                                float* h32 = nullptr);

// The layer's two residual steps with x stored once. launch_residual_norm_h writes only
// h = rmsnorm((x + rmsnorm(t) * w) * out_scale) * next_w and leaves x as it was;
// launch_residual_norm_two then stores x = ((x + rmsnorm(t) * w) * out_scale + rmsnorm(t2) * w2) *
// out_scale2 and h = rmsnorm(x) * next_w (or h32) from the same x and t. The sum x + rmsnorm(t) * w
// has the bits launch_residual_norm would have stored.
hipError_t launch_residual_norm_h(hipStream_t s, const float* x, const uint16_t* t16, float t_eps, const float* w,
                                  float out_scale, const float* next_w, float eps, int T, int d, uint16_t* h);
hipError_t launch_residual_norm_two(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w,
                                    float out_scale, const uint16_t* t2_16, float t2_eps, const float* w2,
                                    float out_scale2, const float* next_w, float eps, int T, int d, uint16_t* h,
                                    float* h32 = nullptr);

// h3 fp16 [T][3 d] = [hi | lo | hi] of y = rmsnorm(x) * w (hi = fp16(y), lo = fp16(y - hi)): the
// input of a split-precision GEMM against [W_hi | W_hi | W_lo]. d a multiple of 4, at most 1024.
hipError_t launch_norm_split(hipStream_t s, const float* x, const float* w, float eps, int T, int d, uint16_t* h3);

// qkv fp32 [T][(H + 2 KV) hd] -> q fp16 [T][H][hd], k, v fp16 [T][KV][hd]: weighted RMSNorm and
// NeoX RoPE on q and k, unweighted RMSNorm on v.
// With q_lo and k_lo set, q and k are also written as split pairs: q_lo = fp16(q - fp16(q)).
hipError_t launch_qk_norm_rope(hipStream_t s, const float* qkv, int T, int H, int KV, int hd, const float* q_norm,
                               const float* k_norm, float eps, const int32_t* positions, const float* rope_table,
                               uint16_t* q, uint16_t* k, uint16_t* v, uint16_t* q_lo = nullptr, uint16_t* k_lo = nullptr);

// The same as launch_qk_norm_rope (head dims 128 and 256, H + 2 KV in {3, 4, 5, 6, 8, 10}) on the
// QKV projection stored as fp16 qkv16 = qkv * c for a power of two c, with eps = eps_model * c^2;
// when vt is set it also writes normalised V transposed: vt [KV * hd][vt_cols], token t at
// column vcol[t].
bool qkv_norm_rope_vt_supported(int hd, int H, int KV);
hipError_t launch_qkv_norm_rope_vt(hipStream_t s, const uint16_t* qkv16, int T, int H, int KV, int hd,
                                   const float* q_norm, const float* k_norm, float eps, const int32_t* positions,
                                   const float* rope_table, uint16_t* q, uint16_t* k, uint16_t* v, const int32_t* vcol,
                                   int vt_cols, uint16_t* vt);

// Flash-style bidirectional attention over packed sequences.
hipError_t launch_attention(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                            const AttnWork* work, int n_work, int H, int KV, int hd, int half_window, float scale);

// Attention with K/V copied straight into LDS (head dims 128 and 256 with at most 4 query heads
// per KV head, and head dim 512 with exactly 4): work items of item_queries query rows (kAttnQueriesV2, or 32 for up to 3 query heads
// per KV head: twice the workgroups for a small batch; a query's result is the same either way);
// V given transposed, vt [KV * hd][vt_cols], each sequence's keys starting at its work items'
// vt_start.
constexpr int kAttnQueriesV2 = 64;
bool attention_v2_supported(int hd, int H, int KV);
hipError_t launch_attention_v2(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, int vt_cols,
                               uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hd, int half_window,
                               float scale, int item_queries = kAttnQueriesV2);

// Attention with split-precision scores for the split-precision layers: q and k as fp16 pairs
// (hi, lo) with hi + lo their fp32 values, same layouts as q and k; scores q_hi.k_hi + q_lo.k_hi +
// q_hi.k_lo. Head dim 512 with 4 query heads per KV head; work items of item_queries (16, 32 or
// 64) query rows with vt_start as for launch_attention_v2.
bool attention_split_supported(int hd, int H, int KV);
hipError_t launch_attention_split(hipStream_t s, const uint16_t* q, const uint16_t* q_lo, const uint16_t* k,
                                  const uint16_t* k_lo, const uint16_t* vt, int vt_cols, uint16_t* o, const AttnWork* work,
                                  int n_work, int H, int KV, int hd, int half_window, float scale, int item_queries);

// The same attention over heads stored padded: q [T][H][hp], k [T][KV][hp] and vt [KV * hp][vt_cols]
// hold hd real dims per head and zeros past them; out [T][H][hd]. Supported: hp 96 with hd 72
// (the image tower's heads), one query head per KV head, no window (half_window 0), work items
// of 64 or 256 queries (a query's result is the same either way).
bool attention_padded_supported(int hp, int hd, int H, int KV);
hipError_t launch_attention_padded(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, int vt_cols,
                                   uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hp, int hd,
                                   int half_window, float scale, int item_queries);

// v [T][width] fp16 -> vt [width][vt_cols] with token t at column vcol[t]; width a multiple of 64.
hipError_t launch_v_transpose(hipStream_t s, const uint16_t* v, int T, int width, const int32_t* vcol, int vt_cols,
                              uint16_t* vt);

// pooled[s] = mean of the sequence's rows of x [*][width].
hipError_t launch_mean_pool(hipStream_t s, const float* x, const SeqRange* seqs, int n_seqs, int width, float* pooled);

// out[r][n] = sum over k of in[r][k] * W[n][k], W = d * q from w's Q8_0 planes, all in fp32 (the
// output projection of pooled rows; w.cols = width, a multiple of 32 up to 1024).
hipError_t launch_pooled_projection(hipStream_t s, const float* in, int n_rows, int width, const Q8Dev& w, float* out);

// ---- per-layer-input branch (ple.hip); widths a multiple of 4, at most 1024.
// out[r] = rmsnorm(in[r] * mul * rscale[r / per_scale]) * w for rows of `width` (in may be out).
hipError_t launch_ple_rmsnorm(hipStream_t s, const float* in, int rows, int width, float mul, const float* rscale,
                              int per_scale, const float* w, float eps, float* out);
// x16[r] = fp16(x[r] / s_r), rscale[r] = s_r: the power of two >= 1 that brings ||x[r]||_2 under 2^14.
hipError_t launch_ple_input(hipStream_t s, const float* x, int T, int d, uint16_t* x16, float* rscale);
// x = x + rmsnorm(t16) * w (t16 = t * c, t_eps = eps * c^2), then x16 / rscale as launch_ple_input.
hipError_t launch_ple_residual_input(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w, int T,
                                     int d, uint16_t* x16, float* rscale);
// g = gelu_tanh(graw[r] * rscale[r]) * ple[r][layer] (ple fp32 [T][layers][pl]); g16 = fp16(g / s2_r),
// rscale2[r] = s2_r, chosen as in launch_ple_input.
hipError_t launch_ple_gate(hipStream_t s, const float* graw, const float* rscale, const float* ple, int layer, int layers,
                           int T, int pl, uint16_t* g16, float* rscale2);
// x = (x + rmsnorm(praw[r] * rscale2[r]) * w) * out_scale; if next_w: h = rmsnorm(x) * next_w (fp16),
// or into h32 in fp32 when h32 is given.
hipError_t launch_ple_residual_norm(hipStream_t s, float* x, const float* praw, const float* rscale2, const float* w,
                                    float out_scale, const float* next_w, float eps, int T, int d, uint16_t* h,
                                    float* h32 = nullptr);

// ---- image tower row kernels (vision.hip); widths a multiple of 4, at most kVitMaxWidth.
constexpr int kVitMaxWidth = 2048;
// x = ((t + bias) + pos[px]) + pos[npos + py] (fp32 [T][d]), h = LayerNorm(x) * w + b (fp16).
hipError_t launch_vit_embed(hipStream_t s, const float* t, const float* bias, const float* pos, int npos,
                            const int32_t* px, const int32_t* py, int T, int d, const float* w, const float* b, float eps,
                            float* x, uint16_t* h);
// The layer's two residual steps with x stored once; o16 (the attention output) and t16 (the
// down projection) are fp16 times 1 / o_inv and 1 / t_inv (powers of two). mode 0:
// h = LayerNorm(x + (o o_inv + bo)) * w + b, x unchanged; mode 1: the same, and
// x = x + (o o_inv + bo) stored; mode 2: x = (x + (o o_inv + bo)) + (t t_inv + bt) stored and,
// with w, h = LayerNorm(x) * w + b.
hipError_t launch_vit_residual2_ln(hipStream_t s, int mode, float* x, const uint16_t* o16, float o_inv, const float* bo,
                                   const uint16_t* t16, float t_inv, const float* bt, const float* w, const float* b,
                                   float eps, int T, int d, uint16_t* h);
// Token i: the mean of LayerNorm(x) * pw + pb over rows row0[i] + dy gx[i] + dx (dy, dx < merge)
// into pooled (fp32 [n][d]), and RMSNorm(mean) * nw into out (fp16 [n][d]).
hipError_t launch_vit_pool(hipStream_t s, const float* x, const int32_t* row0, const int32_t* gx, int n_tokens, int merge,
                           int d, const float* pw, const float* pb, float eps, const float* nw, float* pooled,
                           uint16_t* out);

// Per-device kernel attributes (dynamic LDS limits); call once per device before launching.
hipError_t configure_kernels();
hipError_t gemm_configure();

hipError_t launch_f32_to_f16(hipStream_t s, const float* src, uint16_t* dst, size_t n);
hipError_t launch_f16_to_f32(hipStream_t s, const uint16_t* src, float* dst, size_t n);

}  // namespace ge
