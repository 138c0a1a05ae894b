// Declarations shared by the runtime's translation units: runtime.cpp (context, text encoder,
// per-op entry points) and vision.cpp (the image tower). Internal: not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "gemmaembed.h"
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

struct Fail {
    int code;
    std::string msg;
};

[[noreturn]] void fail(int code, const char* fmt, ...);
void hip_check(hipError_t e, const char* what);
float host_h2f(uint16_t h);

// ---------------------------------------------------------------- device model

struct DevLayer {
    bool sliding = false;
    bool attn_v2 = false;  // attention with Q/K/V copied into LDS and V transposed
    bool qkv_gn = false;   // QKV projection stored as scaled fp16 and read by the fused norm kernel
    bool qkv_fused = false;  // QKV projection with the norms, RoPE and V^T in its epilogue
    // Split-precision QKV projection (layers of head dim >= kPreciseHeadDim): the normed input as
    // fp16 [hi | lo | hi] (launch_norm_split) against wqkv3 = [W_hi | W_hi | W_lo] over 3 hidden
    // columns, fp32 out, so q and k reach their norms at about fp32 precision.
    bool precise = false;
    // Projections stored in fp16 before an RMSNorm are multiplied by these powers of two, chosen
    // from load-time bounds so the values stay inside fp16's range; the norm then uses
    // eps * c^2, which makes it exact for the scaled values.
    float qkv_c = 1, o_c = 1, down_c = 1;
    double act_norm_bound = 0;  // bound on ||gelu(gate) * up||_2 of one row
    int kv_heads = 0, head_dim = 0, qd = 0, kvd = 0;
    float rope_base = 0, out_scale = 1;
    // act is stored in fp16 as gelu(gate) * up * act_scale; the down projection multiplies by
    // 1 / act_scale. Both are powers of two, so the round trip is exact.
    float act_scale = 1, down_scale = 1;
    Q8Dev wqkv, wo, wgu, wd;  // wqkv rows: q | k | v; wgu rows: gate/up interleaved in 32-row groups
    Q8Dev wqkv3;              // precise layers: fragments of [W_hi | W_hi | W_lo], [q | k | v rows][3 hidden]
    Q8Dev inp_gate, proj;     // per-layer-input branch (per_layer_input > 0)
    float* post_norm = nullptr;
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *post_attn = nullptr, *ffn_norm = nullptr,
          *post_ffw = nullptr;
    const float* rope = nullptr;
};

struct DevModel {
    int layers = 0, hidden = 0, heads = 0, ff = 0, out_dims = 0, pl = 0, vocab = 0, window = 0, max_tokens = 8192;
    float eps = 1e-6f, emb_scale = 1, pl_scale = 1;
    Q8Dev tok_embd, output;
    Q8Dev pl_proj;  // per_layer_model_proj as fp16 fragments [layers * pl][hidden] (per_layer_input > 0)
    float* pl_norm = nullptr;
    float* out_norm = nullptr;
    std::vector<DevLayer> layer;
    int max_qd = 0, max_kvd = 0, max_qkv = 0, max_kv_heads = 1;
    bool any_v2 = false;
    bool any_precise = false;
    bool all_v2 = true;  // every layer: the LDS-copy attention (a large pack may then run in parts)
    bool items32_ok = true;  // every LDS-copy attention layer takes 32-query work items (<= 3 heads per KV head)
};

struct Workspace {
    int rows = 0;  // capacity in rows, slack included
    // qkv and t hold fp16 (scaled, see DevLayer::qkv_c) where the layer's kernels take it
    float *x = nullptr, *qkv = nullptr, *t = nullptr, *out = nullptr;
    uint16_t *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *act = nullptr;
    int32_t *tokens = nullptr, *positions = nullptr;
    int seq_cap = 0, work_cap = 0;
    SeqRange* seqs = nullptr;
    AttnWork* work = nullptr;
    float* pooled = nullptr;
    // transposed V for the LDS-copy attention: vt [max_kvd][vt_cap], token t at column vcol[t];
    // its 64-query work list
    int vt_cap = 0, work2_cap = 0;
    uint16_t* vt = nullptr;
    int32_t* vcol = nullptr;
    AttnWork* work2 = nullptr;
    // per-layer-input branch: the per-layer inputs fp32 [T][layers][pl], row-scaled fp16 GEMM
    // inputs (x16 [T][hidden], g16 [T][pl]) with their row scales, and an fp32 GEMM output
    // [T][max(pl, hidden)]
    float *ple = nullptr, *ple_t = nullptr, *rs = nullptr, *rs2 = nullptr;
    uint16_t *x16 = nullptr, *g16 = nullptr;
    // split-precision QKV input [T][3 hidden] (any precise layer)
    uint16_t* h3 = nullptr;
    // the final norm's rows in fp32 [T][hidden] and their per-sequence means [seq_cap][hidden],
    // the input of the output projection
    float *hn = nullptr, *pooled_n = nullptr;
    // their q and k as split pairs: the low halves beside w.q / w.k (same layouts)
    uint16_t *q_lo = nullptr, *k_lo = nullptr;
};

struct ProfStat {
    int64_t launches = 0;
    double ms = 0;
};

struct PendingEvent {
    std::string name;
    hipEvent_t a, b;
};

struct StopPoint {
    std::string name;
    int layer = -1;
    bool hit = false;
};

// Layers whose heads are at least this wide take the split-precision QKV projection. Their
// scores are dot products of two RMS-normed vectors of that width at attention scale 1, so they
// reach several hundred, and fp16 rounding of the projection's operands (2^-11 relative per
// element) moved them enough to put the attention output of the reference's global layers
// (head dim 512) at 1.1e-2 max relative error against the fp32 oracle.
constexpr int kPreciseHeadDim = 512;

// Streams a large batch is split over (measured 2, 3, 4: 5.93, 5.93, 5.85 ms at config 2; with
// 8192-row parts' gate/up launches ending in half tiles, 2 parts 6.18 against 4 parts 6.15 ms).
constexpr int kMaxParts = 4;

// A short pack's forward captured as a HIP graph, keyed by everything its launches' arguments
// depend on (see run_graph); exec is null while the shape has been seen only once.
struct ShortGraph {
    int key[6] = {};
    hipGraphExec_t exec = nullptr;
};

struct VisionState;
// Frees the image tower's weights and workspace (vision.cpp).
void free_vision(ge_ctx* c);

}  // namespace ge

// A Q8_0 matrix of the per-op entry points (ge_op_q8_create).
struct ge_q8_matrix {
    ge::Q8Dev m;
};

struct ge_ctx {
    int device = 0;
    // Layers of at least this head dim (and a query/KV grouping attention_split_kernel supports)
    // run the split-precision QKV projection and scores; set before ge_upload_model.
    int split_head_dim = ge::kPreciseHeadDim;
    hipStream_t stream = nullptr;
    // Part p > 0 of a split batch runs its layers on part_stream[p] (see stage()).
    hipStream_t part_stream[ge::kMaxParts] = {};
    hipEvent_t part_join[ge::kMaxParts] = {};
    hipEvent_t ev_start = nullptr, ev_stop = nullptr, ev_fork = nullptr;
    // Pinned host staging of a batch's small arrays (ids, positions, ranges, work lists, V^T
    // columns): their uploads are asynchronous, and the next batch waits for staged_copy before
    // writing the buffer again.
    void* pinned = nullptr;
    size_t pinned_cap = 0;
    hipEvent_t staged_copy = nullptr;
    bool staged_copy_recorded = false;
    std::string err, name;
    bool has_model = false;
    ge::DevModel model;
    std::vector<void*> weight_allocs;
    std::map<std::pair<int, float>, float*> rope_tables;
    ge::Workspace ws;
    // staged batch
    int staged_tokens = -1, staged_seqs = 0, staged_work = 0, staged_work2 = 0, staged_vt_cols = 0;
    int attn_items = ge::kAttnQueriesV2;  // query rows per LDS-copy attention work item of the staged batch
    // Split batch: part p is rows [part_row[p], part_row[p + 1]) with work2 items
    // [part_work[p], part_work[p + 1]); n_parts 1 = not split.
    int n_parts = 1;
    int part_row[ge::kMaxParts + 1] = {}, part_work[ge::kMaxParts + 1] = {};
    // profiling
    bool prof = false;
    std::string prof_prefix;
    std::vector<std::pair<std::string, ge::ProfStat>> prof_stats;
    std::vector<ge::PendingEvent> prof_pending;
    std::vector<hipEvent_t> event_pool;
    // short packs replayed as HIP graphs (run_graph); dropped whenever the workspace or the
    // model changes, since the graphs hold their addresses
    std::vector<ge::ShortGraph> graphs;
    // the image tower, when one is uploaded (vision.cpp)
    ge::VisionState* vision = nullptr;
    // Vector rows (ge_set_vectors): fp32 [vec_rows][vec_width] in HBM, referenced by token ids
    // -(r + 1). staged_vectors: the rows the staged batch reads (these or the image tower's
    // output), null when it has none.
    float* vec_buf = nullptr;
    size_t vec_cap = 0;
    int vec_rows = 0, vec_width = 0;
    const float* staged_vectors = nullptr;
    // One past the largest vector row the staged batch reads (0 when it reads none).
    int staged_vec_rows = 0;
    // This device's copy of the no-allocation forward's scratch array (noalloc.cpp).
    void* scratch = nullptr;
};

namespace ge {

int set_error(ge_ctx* c, const Fail& f);

template <typename F>
int guarded(ge_ctx* c, F&& f) {
    if (!c) return GE_ERR_INVALID;
    try {
        hipError_t e = hipSetDevice(c->device);
        if (e != hipSuccess) fail(GE_ERR_GPU, "GPU execution failed: hipSetDevice: %s", hipGetErrorString(e));
        f();
        return GE_OK;
    } catch (const Fail& fl) {
        return set_error(c, fl);
    } catch (const std::bad_alloc&) {
        c->err = "out of host memory";
        return GE_ERR_GPU;
    } catch (const std::exception& ex) {
        c->err = ex.what();
        return GE_ERR_INVALID;
    }
}

void* dev_alloc(size_t bytes, const char* what);
hipEvent_t take_event(ge_ctx* c);

// Runs one launch. When profiling covers `name`, the kernel's dispatch records a start and a
// stop event itself (hipExtLaunchKernelGGL), so the measured time is the kernel's own.
template <typename F>
void launch(ge_ctx* c, const char* name, F&& f) {
    const bool prof = c->prof && std::strncmp(name, c->prof_prefix.c_str(), c->prof_prefix.size()) == 0;
    hipEvent_t a = nullptr, b = nullptr;
    if (prof) {
        a = take_event(c);
        b = take_event(c);
        launch_events() = LaunchEvents{a, b};
    }
    hipError_t e = f();
    launch_events() = LaunchEvents{};
    if (e != hipSuccess) fail(e == hipErrorInvalidValue ? GE_ERR_INVALID : GE_ERR_GPU, "GPU execution failed: %s: %s", name, hipGetErrorString(e));
    if (prof) c->prof_pending.push_back({name, a, b});
}

// Weight-file tensors (GGUFTensorInfo, GGUF/GGUFValue.swift:117-131).
int64_t tensor_rows(const ge_tensor_desc* t);
size_t tensor_bytes(const ge_tensor_desc* t);
const uint8_t* tensor_ptr(const ge_tensor_desc* t, const void* base, size_t len);
void check_shape(const ge_tensor_desc* t, int64_t cols, int64_t rows);

// A Q8_0 matrix's rows, split into an int8 quant plane and an fp16 scale plane.
struct HostQ8 {
    int rows = 0, cols = 0;
    std::vector<int8_t> q;
    std::vector<uint16_t> s;
};

void repack_rows(const uint8_t* src, int rows, int cols, HostQ8* dst, int dst_row0);
HostQ8 host_q8(int rows, int cols);
// Quant and scale planes, plus (for GEMM weights) the dequantised fragment-order copy.
Q8Dev upload_q8(ge_ctx* c, const HostQ8& h, const char* what, bool gemm_weight = true);
// A [cols, rows] weight tensor of any accepted type (F32, F16, BF16, Q8_0) as fp16 MFMA fragments
// (Q8Dev::fh order only, no quant planes), columns zero-padded to cols_pad; the allocation is
// appended to allocs. With row_norm, *row_norm = max_j ||W_j||_2 of the fp16 rows uploaded.
Q8Dev upload_fragments(const ge_tensor_desc* t, int64_t cols, int64_t rows, int cols_pad, const void* base, size_t len,
                       std::vector<void*>& allocs, double* row_norm = nullptr);
// max_j ||W_j||_2 of repacked Q8_0 rows.
double max_row_norm(const HostQ8& h);
// The power of two c <= 1 that brings `bound` under 2^15 (half of fp16's largest finite value).
float fp16_range_scale(double bound);
// Copies `rows` x `width` of a device buffer (fp32 or fp16, row stride `stride`) starting at
// column `col0` into out as fp32, after the context's stream has drained.
void copy_out(ge_ctx* c, const void* src, bool f16, int rows, int stride, int col0, int width, float* out);

// Packed text batches (runtime.cpp): validate and upload (a negative id -(r + 1) names row r of
// `vectors`, device fp32 [n_vectors][hidden]); enqueue the forward (record_start: time from here,
// else from an ev_start the caller recorded); wait and copy the pooled vectors out.
// Transposed-V layout of a packed batch: each sequence's keys start at a column that is a
// multiple of 8 (16-byte aligned copies); cols leaves a key block of slack past the end.
struct VtLayout {
    std::vector<uint32_t> start;  // per sequence
    std::vector<int32_t> vcol;    // per token
    int cols = 0;
};

// A validated packed batch, planned on the host: sequence ranges, attention work lists (32-query
// items; LDS-copy attention items of `items` queries with V^T columns), the V^T layout and the
// split into parts.
struct BatchPlan {
    std::vector<SeqRange> sr;
    std::vector<AttnWork> work, work2;
    VtLayout vl;
    int items = kAttnQueriesV2;
    int n_parts = 1;
    int part_row[kMaxParts + 1] = {0}, part_work[kMaxParts + 1] = {0};
    bool any_vector = false;
    int vec_rows_read = 0;
};
BatchPlan plan_batch(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int n, const ge_seq* seqs, int n_seqs,
                     const float* vectors, int n_vectors);
void set_staged(ge_ctx* c, const BatchPlan& b, int n, int n_seqs, const float* vectors);
// The rows ge_set_vectors uploaded, when they are as wide as the model's residual stream.
const float* own_vectors(ge_ctx* c);
int own_vector_rows(ge_ctx* c);
// MetalForward.encode (Metal/MetalForward.swift:364-423) of the staged batch on the context's
// stream, one launch after another (sp: stop after the op producing a traced tensor; null = all).
struct StopPoint;
void encode(ge_ctx* c, StopPoint* sp);
// Waits for every stream of the context.
void drain(ge_ctx* c);
// Packs of at least this many tokens (of two or more sequences) run as parts on several streams.
constexpr int kSplitMinTokens = 4096;
// Takes the device address of the no-allocation forward's scratch array on the context's device
// (noalloc.cpp); called once per context at creation.
void noalloc_init(ge_ctx* c);

// RopeTable (Model/RopeTable.swift:16-31) for (hd, base) over `positions` positions, cached on the
// context with the model's weights (freed with them).
const float* rope_table(ge_ctx* c, int hd, float base, int positions);

void stage(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int n, const ge_seq* seqs, int n_seqs,
           const float* vectors, int n_vectors);
void run_forward(ge_ctx* c, double* gpu_seconds, bool record_start = true);
void read_pooled(ge_ctx* c, float* out);

}  // namespace ge
