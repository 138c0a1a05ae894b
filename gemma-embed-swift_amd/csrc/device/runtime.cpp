// Device runtime behind the C-ABI: context, weight upload with Q8_0 repacking, grow-only
// workspace, the per-layer forward encode, named-tensor tracing, HIP-event profiling and the
// per-op entry points. Replaces Sources/GemmaEmbed/Metal/MetalContext.swift and
// Metal/MetalForward.swift (execute :310-360, encode :364-423, Kernels :427-759).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "runtime_internal.hpp"

namespace ge {


[[noreturn]] void fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    throw Fail{code, buf};
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(GE_ERR_GPU, "GPU execution failed: %s: %s", what, hipGetErrorString(e));
}


// ---------------------------------------------------------------- half conversion (host)
float host_h2f(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400u));
            bits = sign | (uint32_t(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace ge

namespace ge {

LaunchEvents& launch_events() {
    static thread_local LaunchEvents ev;
    return ev;
}

thread_local std::string g_create_error;

int set_error(ge_ctx* c, const Fail& f) {
    if (c) c->err = f.msg;
    return f.code;
}


void* dev_alloc(size_t bytes, const char* what) {
    void* p = nullptr;
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) fail(GE_ERR_GPU, "GPU execution failed: hipMalloc(%zu) for %s: %s", bytes, what, hipGetErrorString(e));
    return p;
}

// ---------------------------------------------------------------- profiling

hipEvent_t take_event(ge_ctx* c) {
    if (!c->event_pool.empty()) {
        hipEvent_t e = c->event_pool.back();
        c->event_pool.pop_back();
        return e;
    }
    hipEvent_t e;
    hip_check(hipEventCreate(&e), "hipEventCreate");
    return e;
}

// Waits for every stream of the context: its own and the part streams of split forwards.
void drain(ge_ctx* c) {
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    for (int p = 0; p < kMaxParts; p++)
        if (c->part_stream[p] && c->part_stream[p] != c->stream)
            hip_check(hipStreamSynchronize(c->part_stream[p]), "hipStreamSynchronize");
}

void resolve_profile(ge_ctx* c) {
    for (auto& p : c->prof_pending) {
        hip_check(hipEventSynchronize(p.b), "hipEventSynchronize");
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, p.a, p.b), "hipEventElapsedTime");
        auto it = std::find_if(c->prof_stats.begin(), c->prof_stats.end(), [&](auto& s) { return s.first == p.name; });
        if (it == c->prof_stats.end()) {
            c->prof_stats.push_back({p.name, ProfStat{}});
            it = c->prof_stats.end() - 1;
        }
        it->second.launches++;
        it->second.ms += ms;
        c->event_pool.push_back(p.a);
        c->event_pool.push_back(p.b);
    }
    c->prof_pending.clear();
}


// ---------------------------------------------------------------- upload

const ge_tensor_desc* find(const ge_model_desc* d, const std::string& name, bool optional = false) {
    for (int i = 0; i < d->n_tensors; i++)
        if (d->tensors[i].name && name == d->tensors[i].name) return &d->tensors[i];
    if (!optional) fail(GE_ERR_MODEL, "weight file lacks tensor %s", name.c_str());
    return nullptr;
}

int64_t tensor_rows(const ge_tensor_desc* t) {
    int64_t r = 1;
    for (int i = 1; i < t->ndim; i++) r *= t->shape[i];
    return r;
}

size_t tensor_bytes(const ge_tensor_desc* t) {
    const int64_t n = t->shape[0] * tensor_rows(t);
    switch (t->type) {
    case GE_TYPE_F32: return size_t(n) * 4;
    case GE_TYPE_F16:
    case GE_TYPE_BF16: return size_t(n) * 2;
    case GE_TYPE_Q8_0: return size_t(n) / 32 * 34;
    default: return 0;
    }
}

const uint8_t* tensor_ptr(const ge_tensor_desc* t, const void* base, size_t len) {
    const size_t b = tensor_bytes(t);
    if (b == 0) fail(GE_ERR_MODEL, "tensor %s uses unsupported storage type %d", t->name, t->type);
    if (t->offset > len || b > len - t->offset) fail(GE_ERR_GGUF, "invalid GGUF file: tensor %s extends past the end of the file", t->name);
    return static_cast<const uint8_t*>(base) + t->offset;
}

void check_shape(const ge_tensor_desc* t, int64_t cols, int64_t rows) {
    if (t->shape[0] != cols || tensor_rows(t) != rows)
        fail(GE_ERR_MODEL, "tensor %s has shape [%lld, %lld], expected [%lld, %lld]", t->name, (long long)t->shape[0],
             (long long)tensor_rows(t), (long long)cols, (long long)rows);
}


void repack_rows(const uint8_t* src, int rows, int cols, HostQ8* dst, int dst_row0) {
    const int kb = cols / 32;
    for (int r = 0; r < rows; r++) {
        const uint8_t* row = src + (size_t)r * kb * 34;
        int8_t* q = dst->q.data() + (size_t)(dst_row0 + r) * cols;
        uint16_t* s = dst->s.data() + (size_t)(dst_row0 + r) * kb;
        for (int b = 0; b < kb; b++) {
            s[b] = uint16_t(row[b * 34] | (row[b * 34 + 1] << 8));
            std::memcpy(q + b * 32, row + b * 34 + 2, 32);
        }
    }
}

HostQ8 host_q8(int rows, int cols) {
    HostQ8 h;
    h.rows = rows;
    h.cols = cols;
    h.q.resize((size_t)rows * cols);
    h.s.resize((size_t)rows * (cols / 32));
    return h;
}

// The GEMMs read the dequantised fragment-order copy; it needs whole 32-row fragment blocks.
bool wants_fragments(const Q8Dev& d) { return d.rows % 32 == 0 && d.cols % 32 == 0; }

void build_fragments(hipStream_t s, Q8Dev* d, const char* what) {
    d->fh = static_cast<uint16_t*>(dev_alloc((size_t)d->rows * d->cols * 2, what));
    hip_check(launch_q8_fragments(s, *d, d->fh), "q8 fragment order");
}

// Quant and scale planes, plus (for GEMM weights) the dequantised fragment-order copy.
Q8Dev upload_q8(ge_ctx* c, const HostQ8& h, const char* what, bool gemm_weight) {
    Q8Dev d;
    d.rows = h.rows;
    d.cols = h.cols;
    d.q = static_cast<int8_t*>(dev_alloc(h.q.size(), what));
    c->weight_allocs.push_back(d.q);
    d.s = static_cast<uint16_t*>(dev_alloc(h.s.size() * 2, what));
    c->weight_allocs.push_back(d.s);
    hip_check(hipMemcpy(d.q, h.q.data(), h.q.size(), hipMemcpyHostToDevice), "hipMemcpy weights");
    hip_check(hipMemcpy(d.s, h.s.data(), h.s.size() * 2, hipMemcpyHostToDevice), "hipMemcpy weights");
    if (gemm_weight && wants_fragments(d)) {
        build_fragments(c->stream, &d, what);
        c->weight_allocs.push_back(d.fh);
        hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    }
    return d;
}

float half_bits_to_float(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }

Q8Dev upload_dense_fragments(const std::vector<uint16_t>& dense, int rows, int cols, const char* what,
                             std::vector<void*>& allocs);

// A [cols, rows] weight of any accepted type as fp16 MFMA fragments (Q8Dev::fh order) with the
// columns zero-padded to cols_pad: values are rounded to fp16 once (Q8_0: fp16 of q * d, as the
// device dequantisation does; F16 as stored; F32 and BF16 rounded to nearest even).
Q8Dev upload_fragments(const ge_tensor_desc* t, int64_t cols, int64_t rows, int cols_pad, const void* base, size_t len,
                       std::vector<void*>& allocs, double* row_norm) {
    check_shape(t, cols, rows);
    if (rows % 32 || cols_pad % 32 || cols_pad < cols) fail(GE_ERR_MODEL, "tensor %s: shape does not tile", t->name);
    const uint8_t* p = tensor_ptr(t, base, len);
    std::vector<float> row(size_t(cols), 0.0f);
    std::vector<uint16_t> dense(size_t(rows) * cols_pad, 0);
    if (row_norm) *row_norm = 0;
    for (int64_t r = 0; r < rows; r++) {
        switch (t->type) {
        case GE_TYPE_F32: std::memcpy(row.data(), p + size_t(r) * cols * 4, size_t(cols) * 4); break;
        case GE_TYPE_F16:
            for (int64_t i = 0; i < cols; i++) {
                uint16_t b;
                std::memcpy(&b, p + (size_t(r) * cols + i) * 2, 2);
                row[size_t(i)] = half_bits_to_float(b);
            }
            break;
        case GE_TYPE_BF16:
            for (int64_t i = 0; i < cols; i++) {
                uint16_t b;
                std::memcpy(&b, p + (size_t(r) * cols + i) * 2, 2);
                const uint32_t bits = uint32_t(b) << 16;
                std::memcpy(&row[size_t(i)], &bits, 4);
            }
            break;
        case GE_TYPE_Q8_0: {
            if (cols % 32) fail(GE_ERR_MODEL, "tensor %s: Q8_0 rows must be a multiple of 32 wide", t->name);
            const uint8_t* rp = p + size_t(r) * (cols / 32) * 34;
            for (int64_t b = 0; b < cols / 32; b++) {
                const float sc = half_bits_to_float(uint16_t(rp[b * 34] | (rp[b * 34 + 1] << 8)));
                for (int e = 0; e < 32; e++) row[size_t(b * 32 + e)] = sc * float(int8_t(rp[b * 34 + 2 + e]));
            }
            break;
        }
        default: fail(GE_ERR_MODEL, "tensor %s uses unsupported storage type %d", t->name, t->type);
        }
        double ss = 0;
        for (int64_t i = 0; i < cols; i++) {
            const _Float16 w = _Float16(row[size_t(i)]);
            dense[size_t(r) * cols_pad + i] = __builtin_bit_cast(uint16_t, w);
            ss += double(w) * double(w);
        }
        if (row_norm) *row_norm = std::max(*row_norm, std::sqrt(ss));
    }
    return upload_dense_fragments(dense, int(rows), cols_pad, t->name, allocs);
}

// A dense row-major fp16 matrix [rows][cols] (rows a multiple of 32, cols of 16) uploaded in
// fragment order: 32-row block j, 16-wide k-step s: 512 halves, lane l's 8 halves are row
// 32 j + l % 32, columns 16 s + 8 (l / 32) + [0, 8).
Q8Dev upload_dense_fragments(const std::vector<uint16_t>& dense, int rows, int cols, const char* what,
                             std::vector<void*>& allocs) {
    const int KT = cols / 16;
    std::vector<uint16_t> fh(dense.size());
    for (int64_t j = 0; j < rows / 32; j++)
        for (int s = 0; s < KT; s++)
            for (int l = 0; l < 64; l++)
                for (int e = 0; e < 8; e++)
                    fh[((size_t(j) * KT + s) * 64 + l) * 8 + e] = dense[size_t(32 * j + l % 32) * cols + 16 * s + 8 * (l / 32) + e];
    Q8Dev m;
    m.rows = rows;
    m.cols = cols;
    m.fh = static_cast<uint16_t*>(dev_alloc(fh.size() * 2, what));
    allocs.push_back(m.fh);
    hip_check(hipMemcpy(m.fh, fh.data(), fh.size() * 2, hipMemcpyHostToDevice), "hipMemcpy weights");
    return m;
}

// The split-precision copy of a Q8_0 matrix W [rows][cols]: fragments of [W_hi | W_hi | W_lo]
// ([rows][3 cols]) with W_hi = fp16(q d), the value of the plain fragment copy, and
// W_lo = fp16(q d - W_hi). q d has at most 18 significant bits, so W_hi + W_lo is q d up to the
// fp16 subnormal step of W_lo (2^-25 absolute).
Q8Dev upload_split_fragments(ge_ctx* c, const HostQ8& h, const char* what) {
    const int K = h.cols, kb = K / 32;
    std::vector<uint16_t> dense(size_t(h.rows) * 3 * K);
    for (int r = 0; r < h.rows; r++)
        for (int k = 0; k < K; k++) {
            const float wv = host_h2f(h.s[size_t(r) * kb + k / 32]) * float(h.q[size_t(r) * K + k]);
            const _Float16 hi = _Float16(wv);
            const _Float16 lo = _Float16(wv - float(hi));
            uint16_t* row = dense.data() + size_t(r) * 3 * K;
            row[k] = row[K + k] = __builtin_bit_cast(uint16_t, hi);
            row[2 * K + k] = __builtin_bit_cast(uint16_t, lo);
        }
    return upload_dense_fragments(dense, h.rows, 3 * K, what, c->weight_allocs);
}

const uint8_t* q8_tensor(const ge_model_desc* d, const std::string& name, int64_t cols, int64_t rows, const void* base,
                         size_t len) {
    const ge_tensor_desc* t = find(d, name);
    check_shape(t, cols, rows);
    if (t->type != GE_TYPE_Q8_0)
        fail(GE_ERR_MODEL, "tensor %s uses storage type %d; the MI355X GEMMs take Q8_0 projection weights", t->name, t->type);
    if (cols % 32) fail(GE_ERR_MODEL, "tensor %s: Q8_0 rows must be a multiple of 32 wide", t->name);
    return tensor_ptr(t, base, len);
}

float* upload_f32(ge_ctx* c, const ge_model_desc* d, const std::string& name, int64_t n, const void* base, size_t len) {
    const ge_tensor_desc* t = find(d, name);
    check_shape(t, n, 1);
    if (t->type != GE_TYPE_F32) fail(GE_ERR_MODEL, "tensor %s uses unsupported storage type %d", t->name, t->type);
    const uint8_t* p = tensor_ptr(t, base, len);
    float* dptr = static_cast<float*>(dev_alloc(size_t(n) * 4, t->name));
    c->weight_allocs.push_back(dptr);
    hip_check(hipMemcpy(dptr, p, size_t(n) * 4, hipMemcpyHostToDevice), "hipMemcpy norm");
    return dptr;
}

// RopeTable (Model/RopeTable.swift:16-31): cos/sin of pos * base^(-2i/hd) in fp64, stored fp32.
const float* rope_table(ge_ctx* c, int hd, float base, int positions) {
    auto key = std::make_pair(hd, base);
    auto it = c->rope_tables.find(key);
    if (it != c->rope_tables.end()) return it->second;
    const int pairs = hd / 2;
    std::vector<float> t((size_t)positions * pairs * 2);
    for (int i = 0; i < pairs; i++) {
        const double inv = std::pow(double(base), -2.0 * double(i) / double(hd));
        for (int p = 0; p < positions; p++) {
            const double th = double(p) * inv;
            t[((size_t)p * pairs + i) * 2] = float(std::cos(th));
            t[((size_t)p * pairs + i) * 2 + 1] = float(std::sin(th));
        }
    }
    float* dptr = static_cast<float*>(dev_alloc(t.size() * 4, "rope table"));
    c->weight_allocs.push_back(dptr);
    hip_check(hipMemcpy(dptr, t.data(), t.size() * 4, hipMemcpyHostToDevice), "hipMemcpy rope");
    c->rope_tables[key] = dptr;
    return dptr;
}

// Bounds |act| = |gelu_tanh(h . g_j) * (h . u_j)| <= |h . g_j| |h . u_j| over any input: h is an
// RMS-normalised row times the ffn_norm weight, so ||h||_2 <= sqrt(d) max|w|, and by Cauchy-Schwarz
// |act_j| <= d max|w|^2 ||g_j||_2 ||u_j||_2. The shift keeps that bound under 2^15, half of fp16's
// largest finite value, leaving room for the fp16 rounding of h and of the dequantised weights.
void choose_act_scale(ge_ctx*, const ge_model_desc* d, const std::string& b, const uint8_t* g, const uint8_t* u, int D,
                      int ff, const void* base, size_t len, DevLayer* L) {
    const ge_tensor_desc* nt = find(d, b + "ffn_norm.weight");
    check_shape(nt, D, 1);
    const float* w = reinterpret_cast<const float*>(tensor_ptr(nt, base, len));
    double wmax = 0;
    for (int i = 0; i < D; i++) wmax = std::max(wmax, double(std::fabs(w[i])));
    const size_t rb = size_t(D / 32) * 34;
    double worst = 0, sumsq = 0;
    for (int j = 0; j < ff; j++) {
        double gg = 0, uu = 0;
        for (int blk = 0; blk < D / 32; blk++) {
            const uint8_t* gp = g + (size_t)j * rb + (size_t)blk * 34;
            const uint8_t* up = u + (size_t)j * rb + (size_t)blk * 34;
            const double gd = host_h2f(uint16_t(gp[0] | (gp[1] << 8))), ud = host_h2f(uint16_t(up[0] | (up[1] << 8)));
            double gs = 0, us = 0;
            for (int e = 0; e < 32; e++) {
                gs += double(int8_t(gp[2 + e])) * int8_t(gp[2 + e]);
                us += double(int8_t(up[2 + e])) * int8_t(up[2 + e]);
            }
            gg += gd * gd * gs;
            uu += ud * ud * us;
        }
        worst = std::max(worst, std::sqrt(gg * uu));
        sumsq += gg * uu;
    }
    const double bound = double(D) * wmax * wmax * worst;
    L->act_norm_bound = double(D) * wmax * wmax * std::sqrt(sumsq);
    int shift = 0;
    while (bound * std::ldexp(1.0, -shift) > 32768.0 && shift < 60) shift++;
    L->act_scale = float(std::ldexp(1.0, -shift));
    L->down_scale = float(std::ldexp(1.0, shift));
}

// max_j ||W_j||_2 of repacked Q8_0 rows.
double max_row_norm(const HostQ8& h) {
    const int kb = h.cols / 32;
    double worst = 0;
    for (int r = 0; r < h.rows; r++) {
        double ss = 0;
        for (int b = 0; b < kb; b++) {
            const double d = host_h2f(h.s[(size_t)r * kb + b]);
            double qq = 0;
            for (int e = 0; e < 32; e++) {
                const double q = h.q[(size_t)r * h.cols + b * 32 + e];
                qq += q * q;
            }
            ss += d * d * qq;
        }
        worst = std::max(worst, ss);
    }
    return std::sqrt(worst);
}

// The power of two c <= 1 that brings `bound` under 2^15 (half of fp16's largest finite value).
float fp16_range_scale(double bound) {
    int shift = 0;
    while (bound * std::ldexp(1.0, -shift) > 32768.0 && shift < 60) shift++;
    return float(std::ldexp(1.0, -shift));
}

double max_abs(const ge_model_desc* d, const std::string& name, int n, const void* base, size_t len) {
    const ge_tensor_desc* t = find(d, name);
    check_shape(t, n, 1);
    const float* w = reinterpret_cast<const float*>(tensor_ptr(t, base, len));
    double m = 0;
    for (int i = 0; i < n; i++) m = std::max(m, double(std::fabs(w[i])));
    return m;
}

void drop_graphs(ge_ctx* c) {
    for (ShortGraph& g : c->graphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    c->graphs.clear();
}

void free_model(ge_ctx* c) {
    drop_graphs(c);
    for (void* p : c->weight_allocs) (void)hipFree(p);
    c->weight_allocs.clear();
    c->rope_tables.clear();
    c->model = DevModel{};
    c->has_model = false;
}

void free_workspace(ge_ctx* c) {
    drop_graphs(c);
    Workspace& w = c->ws;
    void* ps[] = {w.x, w.qkv, w.t, w.out, w.h, w.q, w.k, w.v, w.attn, w.act, w.tokens, w.positions, w.seqs, w.work, w.pooled,
                  w.vt, w.vcol, w.work2, w.ple, w.ple_t, w.rs, w.rs2, w.x16, w.g16, w.h3, w.q_lo, w.k_lo, w.hn,
                  w.pooled_n};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    c->ws = Workspace{};
    c->staged_tokens = -1;
}

void upload(ge_ctx* c, const ge_model_desc* d, const void* base, size_t len) {
    if (!d || !base) fail(GE_ERR_INVALID, "null model descriptor or file base");
    if (d->layers <= 0 || d->hidden <= 0 || d->heads <= 0 || d->feed_forward <= 0 || d->out_dims <= 0 || d->vocab <= 0)
        fail(GE_ERR_MODEL, "model descriptor has a non-positive size");
    if (d->per_layer_input < 0 || d->per_layer_input % 64 || d->per_layer_input > 1024)
        fail(GE_ERR_MODEL, "per-layer input width %d: the kernels need a multiple of 64 up to 1024", d->per_layer_input);
    if (d->hidden % 64 || d->hidden > 1024) fail(GE_ERR_MODEL, "hidden size %d: the kernels need a multiple of 64 up to 1024", d->hidden);
    if (d->feed_forward % 32) fail(GE_ERR_MODEL, "feed_forward_length %d is not a multiple of 32", d->feed_forward);
    if (d->out_dims % 64) fail(GE_ERR_MODEL, "embedding_length_out %d is not a multiple of 64", d->out_dims);
    drain(c);  // nothing queued may still read the old weights or workspace
    free_model(c);
    free_workspace(c);
    DevModel& m = c->model;
    m.layers = d->layers;
    m.hidden = d->hidden;
    m.heads = d->heads;
    m.ff = d->feed_forward;
    m.out_dims = d->out_dims;
    m.pl = d->per_layer_input;
    m.vocab = d->vocab;
    m.window = d->sliding_window;
    m.max_tokens = d->max_tokens > 0 ? d->max_tokens : 8192;
    m.eps = d->eps;
    m.emb_scale = d->embedding_scale;
    m.pl_scale = d->per_layer_scale;
    const int D = m.hidden;

    {
        HostQ8 h = host_q8(m.vocab, D);
        repack_rows(q8_tensor(d, "token_embd.weight", D, m.vocab, base, len), m.vocab, D, &h, 0);
        m.tok_embd = upload_q8(c, h, "token_embd", false);
    }
    {
        HostQ8 h = host_q8(m.out_dims, D);
        repack_rows(q8_tensor(d, "output.weight", D, m.out_dims, base, len), m.out_dims, D, &h, 0);
        m.output = upload_q8(c, h, "output", false);  // projected from its Q8_0 planes (pooled_projection_kernel)
    }
    m.out_norm = upload_f32(c, d, "output_norm.weight", D, base, len);
    if (m.pl > 0) {
        // per_layer_model_proj (BF16 in the reference's file) as fp16 fragments
        m.pl_proj = upload_fragments(find(d, "per_layer_model_proj.weight"), D, int64_t(m.pl) * m.layers, D, base, len,
                                     c->weight_allocs);
        m.pl_norm = upload_f32(c, d, "per_layer_proj_norm.weight", m.pl, base, len);
    }
    for (int i = 0; i < m.layers; i++) {
        DevLayer L;
        L.sliding = d->sliding[i] != 0;
        L.kv_heads = d->kv_heads[i];
        L.head_dim = d->head_dim[i];
        L.rope_base = d->rope_base[i];
        L.out_scale = d->out_scale ? d->out_scale[i] : 1.0f;
        const int hd = L.head_dim;
        if (L.kv_heads <= 0 || m.heads % L.kv_heads || m.heads / L.kv_heads > 4)
            fail(GE_ERR_MODEL, "layer %d: %d query heads over %d KV heads (the attention kernel takes groups of 1 to 4)", i, m.heads, L.kv_heads);
        if (hd != 128 && hd != 256 && hd != 512) fail(GE_ERR_MODEL, "layer %d: head dim %d (supported: 128, 256, 512)", i, hd);
        L.qd = m.heads * hd;
        L.kvd = L.kv_heads * hd;
        const std::string b = "blk." + std::to_string(i) + ".";
        {
            const int n = L.qd + 2 * L.kvd;
            HostQ8 h = host_q8(n, D);
            repack_rows(q8_tensor(d, b + "attn_q.weight", D, L.qd, base, len), L.qd, D, &h, 0);
            repack_rows(q8_tensor(d, b + "attn_k.weight", D, L.kvd, base, len), L.kvd, D, &h, L.qd);
            repack_rows(q8_tensor(d, b + "attn_v.weight", D, L.kvd, base, len), L.kvd, D, &h, L.qd + L.kvd);
            L.precise = hd >= c->split_head_dim && attention_split_supported(hd, m.heads, L.kv_heads);
            // a precise layer's GEMMs read only the split copy
            L.wqkv = upload_q8(c, h, "attn_qkv", !L.precise);
            if (L.precise) L.wqkv3 = upload_split_fragments(c, h, "attn_qkv split");
            // |qkv_j| <= ||h|| ||W_j||, ||h|| <= sqrt(D) max|attn_norm|
            const double hn = std::sqrt(double(D)) * max_abs(d, b + "attn_norm.weight", D, base, len);
            L.qkv_c = fp16_range_scale(hn * max_row_norm(h));
        }
        {
            HostQ8 h = host_q8(D, L.qd);
            repack_rows(q8_tensor(d, b + "attn_output.weight", L.qd, D, base, len), D, L.qd, &h, 0);
            L.wo = upload_q8(c, h, "attn_output");
            // each head's output is a convex combination of RMS-normalised V rows: norm <= sqrt(hd)
            L.o_c = fp16_range_scale(std::sqrt(double(L.qd)) * max_row_norm(h));
        }
        {
            HostQ8 h = host_q8(2 * m.ff, D);
            const uint8_t* g = q8_tensor(d, b + "ffn_gate.weight", D, m.ff, base, len);
            const uint8_t* u = q8_tensor(d, b + "ffn_up.weight", D, m.ff, base, len);
            const size_t rb = size_t(D / 32) * 34;
            for (int jb = 0; jb < m.ff / 32; jb++) {
                repack_rows(g + (size_t)jb * 32 * rb, 32, D, &h, jb * 64);
                repack_rows(u + (size_t)jb * 32 * rb, 32, D, &h, jb * 64 + 32);
            }
            L.wgu = upload_q8(c, h, "ffn_gate_up");
            choose_act_scale(c, d, b, g, u, D, m.ff, base, len, &L);
        }
        {
            HostQ8 h = host_q8(D, m.ff);
            repack_rows(q8_tensor(d, b + "ffn_down.weight", m.ff, D, base, len), D, m.ff, &h, 0);
            L.wd = upload_q8(c, h, "ffn_down");
            L.down_c = fp16_range_scale(L.act_norm_bound * max_row_norm(h));
        }
        L.attn_norm = upload_f32(c, d, b + "attn_norm.weight", D, base, len);
        L.q_norm = upload_f32(c, d, b + "attn_q_norm.weight", hd, base, len);
        L.k_norm = upload_f32(c, d, b + "attn_k_norm.weight", hd, base, len);
        L.post_attn = upload_f32(c, d, b + "post_attention_norm.weight", D, base, len);
        L.ffn_norm = upload_f32(c, d, b + "ffn_norm.weight", D, base, len);
        L.post_ffw = upload_f32(c, d, b + "post_ffw_norm.weight", D, base, len);
        L.rope = rope_table(c, hd, L.rope_base, m.max_tokens);
        if (m.pl > 0) {
            HostQ8 g = host_q8(m.pl, D);
            repack_rows(q8_tensor(d, b + "inp_gate.weight", D, m.pl, base, len), m.pl, D, &g, 0);
            L.inp_gate = upload_q8(c, g, "inp_gate");
            HostQ8 pj = host_q8(D, m.pl);
            repack_rows(q8_tensor(d, b + "proj.weight", m.pl, D, base, len), D, m.pl, &pj, 0);
            L.proj = upload_q8(c, pj, "proj");
            L.post_norm = upload_f32(c, d, b + "post_norm.weight", D, base, len);
        }
        m.max_qd = std::max(m.max_qd, L.qd);
        m.max_kvd = std::max(m.max_kvd, L.kvd);
        m.max_kv_heads = std::max(m.max_kv_heads, L.kv_heads);
        L.attn_v2 = attention_v2_supported(L.head_dim, m.heads, L.kv_heads);
        L.qkv_gn = qkv_norm_rope_vt_supported(L.head_dim, m.heads, L.kv_heads);
        // The fused epilogue stages one 128 x 256 tile in the GEMM's own LDS, so it also takes
        // layouts the separate kernel's V^T staging cannot hold (2 KV heads of 256); a trace of the
        // raw projection of such a layer runs the fp32 path.
        L.qkv_fused = gemm_qkv_supported(L.head_dim, m.heads, L.kv_heads);
        if (L.precise) L.qkv_gn = L.qkv_fused = false;  // fp32 projection, separate norm kernel
        m.any_precise = m.any_precise || L.precise;
        m.any_v2 = m.any_v2 || L.attn_v2;
        m.all_v2 = m.all_v2 && L.attn_v2;
        if (L.attn_v2 && m.heads / L.kv_heads > 3) m.items32_ok = false;
        m.max_qkv = std::max(m.max_qkv, L.qd + 2 * L.kvd);
        m.layer.push_back(L);
    }
    c->has_model = true;
}

// ---------------------------------------------------------------- workspace

// A zero-filled workspace buffer. The fill is queued on the context's stream, ahead of the batch
// copies and kernels that follow there: the context's streams are created non-blocking, so a
// plain hipMemset (the null stream) would not be ordered before them, and a fill that landed late
// would overwrite the staged batch with zeros.
template <typename T>
T* ws_alloc(hipStream_t s, size_t rows, size_t width, const char* what) {
    const size_t bytes = rows * width * sizeof(T);
    void* p = dev_alloc(bytes, what);
    hip_check(hipMemsetAsync(p, 0, bytes, s), "hipMemsetAsync workspace");
    return static_cast<T*>(p);
}

// Whether ensure_workspace would reallocate any buffer for a batch of this size.
bool workspace_grows(const ge_ctx* c, int tokens, int seqs, int work, int work2, int vt_cols) {
    const Workspace& w = c->ws;
    const DevModel& m = c->model;
    const int rows = (tokens + 63) / 64 * 64 + kRowSlack;
    return rows > w.rows || seqs > w.seq_cap || !w.seqs || work > w.work_cap || !w.work ||
           (m.any_v2 && (work2 > w.work2_cap || !w.work2 || vt_cols > w.vt_cap || !w.vt));
}

void ensure_workspace_impl(ge_ctx* c, int tokens, int seqs, int work, int work2, int vt_cols);

// Grows the workspace for a batch. If an allocation fails, the whole workspace is freed before
// the error propagates, so no capacity is ever recorded for a buffer that does not exist.
void ensure_workspace(ge_ctx* c, int tokens, int seqs, int work, int work2, int vt_cols) {
    if (!workspace_grows(c, tokens, seqs, work, work2, vt_cols)) return;
    drop_graphs(c);
    try {
        ensure_workspace_impl(c, tokens, seqs, work, work2, vt_cols);
    } catch (...) {
        free_workspace(c);
        throw;
    }
}

void ensure_workspace_impl(ge_ctx* c, int tokens, int seqs, int work, int work2, int vt_cols) {
    Workspace& w = c->ws;
    const DevModel& m = c->model;
    const int rows = (tokens + 63) / 64 * 64 + kRowSlack;
    if (rows > w.rows) {
        const int keep_seq = w.seq_cap, keep_work = w.work_cap;
        free_workspace(c);
        w.seq_cap = keep_seq;
        w.work_cap = keep_work;
        w.rows = rows;
        w.x = ws_alloc<float>(c->stream, rows, m.hidden, "x");
        w.h = ws_alloc<uint16_t>(c->stream, rows, m.hidden, "h");
        w.qkv = ws_alloc<float>(c->stream, rows, m.max_qkv, "qkv");
        w.q = ws_alloc<uint16_t>(c->stream, rows, m.max_qd, "q");
        w.k = ws_alloc<uint16_t>(c->stream, rows, m.max_kvd, "k");
        w.v = ws_alloc<uint16_t>(c->stream, rows, m.max_kvd, "v");
        w.attn = ws_alloc<uint16_t>(c->stream, rows, m.max_qd, "attn");
        w.t = ws_alloc<float>(c->stream, rows, m.hidden, "t");
        w.act = ws_alloc<uint16_t>(c->stream, rows, m.ff, "act");
        w.out = ws_alloc<float>(c->stream, rows, m.out_dims, "out");
        w.hn = ws_alloc<float>(c->stream, rows, m.hidden, "final norm");
        w.tokens = ws_alloc<int32_t>(c->stream, rows, 1, "tokens");
        w.positions = ws_alloc<int32_t>(c->stream, rows, 1, "positions");
        w.vcol = ws_alloc<int32_t>(c->stream, rows, 1, "vt columns");
        if (m.any_precise) {
            w.h3 = ws_alloc<uint16_t>(c->stream, rows, 3 * size_t(m.hidden), "split-precision input");
            w.q_lo = ws_alloc<uint16_t>(c->stream, rows, m.max_qd, "q low halves");
            w.k_lo = ws_alloc<uint16_t>(c->stream, rows, m.max_kvd, "k low halves");
        }
        if (m.pl > 0) {
            w.ple = ws_alloc<float>(c->stream, rows, size_t(m.layers) * m.pl, "per-layer inputs");
            w.ple_t = ws_alloc<float>(c->stream, rows, size_t(std::max(m.pl, m.hidden)), "per-layer projection");
            w.rs = ws_alloc<float>(c->stream, rows, 1, "row scales");
            w.rs2 = ws_alloc<float>(c->stream, rows, 1, "row scales");
            w.x16 = ws_alloc<uint16_t>(c->stream, rows, m.hidden, "scaled residual");
            w.g16 = ws_alloc<uint16_t>(c->stream, rows, m.pl, "per-layer gate");
        }
        w.seqs = nullptr;
        w.work = nullptr;
        w.pooled = nullptr;
        w.pooled_n = nullptr;
        w.seq_cap = 0;
        w.work_cap = 0;
        w.vt = nullptr;
        w.work2 = nullptr;
        w.vt_cap = 0;
        w.work2_cap = 0;
    }
    if (seqs > w.seq_cap || !w.seqs) {
        if (w.seqs) (void)hipFree(w.seqs);
        if (w.pooled) (void)hipFree(w.pooled);
        if (w.pooled_n) (void)hipFree(w.pooled_n);
        w.seqs = nullptr;
        w.pooled = w.pooled_n = nullptr;
        w.seq_cap = std::max(seqs, 1);
        w.seqs = ws_alloc<SeqRange>(c->stream, w.seq_cap, 1, "sequences");
        w.pooled = ws_alloc<float>(c->stream, w.seq_cap, m.out_dims, "pooled");
        w.pooled_n = ws_alloc<float>(c->stream, w.seq_cap, m.hidden, "pooled rows");
    }
    if (work > w.work_cap || !w.work) {
        if (w.work) (void)hipFree(w.work);
        w.work_cap = std::max(work, 1);
        w.work = ws_alloc<AttnWork>(c->stream, w.work_cap, 1, "attention work");
    }
    if (m.any_v2 && (work2 > w.work2_cap || !w.work2)) {
        if (w.work2) (void)hipFree(w.work2);
        w.work2_cap = std::max(work2, 1);
        w.work2 = ws_alloc<AttnWork>(c->stream, w.work2_cap, 1, "attention work");
    }
    // Zero-filled once: columns no token writes (alignment gaps, slack) stay finite, and keys
    // read from them are masked, so they contribute exact zeros.
    if (m.any_v2 && (vt_cols > w.vt_cap || !w.vt)) {
        if (w.vt) (void)hipFree(w.vt);
        // grow by half, in whole 64-column steps: the copies and the kernels' checks need
        // 16-byte aligned rows (a multiple of 8 columns)
        w.vt_cap = (std::max(vt_cols, w.vt_cap + w.vt_cap / 2) + 63) / 64 * 64;
        w.vt = ws_alloc<uint16_t>(c->stream, size_t(m.max_kvd), size_t(w.vt_cap), "transposed v");
    }
}

// Below this many 64-query workgroups (one per CU), use 32-query items. Measured at config 2's
// sliding layers: a 8192-token pack (128 items) 36.5 -> 31.0 us per attention launch; a 16384-token
// pack (256 items) 41.0 -> 57.0 us, so it keeps 64-query items.
constexpr int kAttnSmallItems = 256;


VtLayout vt_layout(int n_tokens, const ge_seq* seqs, int n_seqs) {
    VtLayout v;
    v.start.resize(size_t(n_seqs));
    v.vcol.assign(size_t(n_tokens), -1);
    uint32_t col = 0;
    for (int s = 0; s < n_seqs; s++) {
        v.start[size_t(s)] = col;
        for (uint32_t i = 0; i < seqs[s].length; i++) v.vcol[seqs[s].start + i] = int32_t(col + i);
        col += (seqs[s].length + 7) / 8 * 8;
    }
    v.cols = int(col) + 64;
    // tokens outside every sequence write to the last slack column, which no key block reaches
    for (auto& x : v.vcol)
        if (x < 0) x = v.cols - 1;
    return v;
}

// ---------------------------------------------------------------- batch staging

// Validates a packed batch and builds its attention work lists, V^T layout and split into parts
// (PackedBatch and AttentionWork.items, Metal/MetalForward.swift:8-58; execute :326-334). Host only.
BatchPlan plan_batch(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int n, const ge_seq* seqs, int n_seqs,
                     const float* vectors, int n_vectors) {
    if (!c->has_model) fail(GE_ERR_STATE, "no model has been uploaded");
    if (n <= 0 || !tokens || !positions) fail(GE_ERR_INVALID, "a batch needs at least one token");
    if (n_seqs <= 0 || !seqs) fail(GE_ERR_INVALID, "a batch needs at least one sequence");
    const DevModel& m = c->model;
    if (!vectors) n_vectors = 0;
    BatchPlan b;
    for (int i = 0; i < n; i++) {
        if (tokens[i] < -n_vectors || tokens[i] >= m.vocab)
            fail(GE_ERR_INVALID, "token %d at row %d is neither in the vocabulary [0, %d) nor one of the %d vector rows",
                 tokens[i], i, m.vocab, n_vectors);
        b.any_vector |= tokens[i] < 0;
        if (tokens[i] < 0) b.vec_rows_read = std::max(b.vec_rows_read, -tokens[i]);
        if (positions[i] < 0 || positions[i] >= m.max_tokens)
            fail(GE_ERR_INVALID, "position %d at row %d is outside [0, %d)", positions[i], i, m.max_tokens);
    }
    b.sr.resize(size_t(n_seqs));
    for (int s = 0; s < n_seqs; s++) {
        const uint64_t end = uint64_t(seqs[s].start) + seqs[s].length;
        if (end > uint64_t(n)) fail(GE_ERR_INVALID, "sequence %d [%u, +%u) runs past the %d tokens", s, seqs[s].start, seqs[s].length, n);
        if (seqs[s].length > uint32_t(m.max_tokens)) fail(GE_ERR_INVALID, "sequence %d has %u tokens, more than %d", s, seqs[s].length, m.max_tokens);
        b.sr[size_t(s)] = SeqRange{seqs[s].start, seqs[s].length};
        for (uint32_t q0 = 0; q0 < seqs[s].length; q0 += kAttnQueries)
            b.work.push_back(AttnWork{seqs[s].start, seqs[s].length, q0, 0});
    }
    // Sequences may not share tokens: each token's key and value belong to one sequence.
    {
        std::vector<std::pair<uint32_t, uint32_t>> iv;
        for (int s = 0; s < n_seqs; s++)
            if (seqs[s].length) iv.push_back({seqs[s].start, seqs[s].start + seqs[s].length});
        std::sort(iv.begin(), iv.end());
        for (size_t i = 1; i < iv.size(); i++)
            if (iv[i].first < iv[i - 1].second) fail(GE_ERR_INVALID, "sequences overlap at token %u", iv[i].first);
    }
    if (m.any_v2) {
        b.vl = vt_layout(n, seqs, n_seqs);
        // A batch whose 64-query items would give fewer than kAttnSmallItems workgroups (a pack of
        // 8192 tokens: 128) takes 32-query items: twice the workgroups, the same results (a query's
        // wave sees the same key blocks; blocks outside its window add exact zeros).
        int64_t items64 = 0;
        for (int s = 0; s < n_seqs; s++) items64 += (seqs[s].length + kAttnQueriesV2 - 1) / kAttnQueriesV2;
        if (m.items32_ok && items64 * m.max_kv_heads < kAttnSmallItems) b.items = 32;
        for (int s = 0; s < n_seqs; s++)
            for (uint32_t q0 = 0; q0 < seqs[s].length; q0 += uint32_t(b.items))
                b.work2.push_back(AttnWork{seqs[s].start, seqs[s].length, q0, b.vl.start[size_t(s)]});
    }
    // Split a large batch of several sequences into parts of whole sequences, cut at the
    // sequence starts nearest to p n / P, whose layers run on their own streams: one part's
    // memory-bound kernels and its kernels' start and end phases overlap the others' work.
    if (m.all_v2 && n >= kSplitMinTokens && n_seqs >= 2) {
        const int want = kMaxParts;
        std::vector<int> starts;
        for (int s = 0; s < n_seqs; s++)
            if (seqs[s].length && seqs[s].start > 0) starts.push_back(int(seqs[s].start));
        std::sort(starts.begin(), starts.end());
        std::vector<int> cuts;
        for (int p = 1; p < want; p++) {
            const int target = int((int64_t)n * p / want);
            int best = -1;
            for (int r : starts)
                if (r > (cuts.empty() ? 0 : cuts.back()) && (best < 0 || std::abs(r - target) < std::abs(best - target)))
                    best = r;
            if (best > 0 && best < n) cuts.push_back(best);
        }
        if (!cuts.empty()) {
            b.n_parts = int(cuts.size()) + 1;
            for (int p = 1; p < b.n_parts; p++) b.part_row[p] = cuts[size_t(p) - 1];
            b.part_row[b.n_parts] = n;
            auto part_of = [&](const AttnWork& a) {
                int p = 0;
                while (p + 1 < b.n_parts && int(a.seq_start) >= b.part_row[p + 1]) p++;
                return p;
            };
            std::stable_sort(b.work2.begin(), b.work2.end(), [&](const AttnWork& x, const AttnWork& y) { return part_of(x) < part_of(y); });
            for (const AttnWork& a : b.work2) b.part_work[part_of(a) + 1]++;
            for (int p = 0; p < b.n_parts; p++) b.part_work[p + 1] += b.part_work[p];
            for (int p = 0; p < b.n_parts; p++)
                if (b.part_work[p + 1] == b.part_work[p]) b.n_parts = 1;  // a part without work: do not split
        }
    }
    return b;
}

// Records a planned batch as the context's staged batch (its arrays already on their way to the
// workspace the forward reads).
void set_staged(ge_ctx* c, const BatchPlan& b, int n, int n_seqs, const float* vectors) {
    c->staged_tokens = n;
    c->staged_vectors = b.any_vector ? vectors : nullptr;
    c->staged_vec_rows = b.vec_rows_read;
    c->staged_seqs = n_seqs;
    c->staged_work = int(b.work.size());
    c->staged_work2 = int(b.work2.size());
    c->staged_vt_cols = b.vl.cols;
    c->attn_items = b.items;
    c->n_parts = b.n_parts;
    std::copy(b.part_row, b.part_row + kMaxParts + 1, c->part_row);
    std::copy(b.part_work, b.part_work + kMaxParts + 1, c->part_work);
}

// Validates and uploads a packed batch into the context's workspace, grown as needed.
void stage(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int n, const ge_seq* seqs, int n_seqs,
           const float* vectors, int n_vectors) {
    const BatchPlan b = plan_batch(c, tokens, positions, n, seqs, n_seqs, vectors, n_vectors);
    // The workspace may be reallocated below: nothing queued may still use it.
    if (workspace_grows(c, n, n_seqs, int(b.work.size()), int(b.work2.size()), b.vl.cols)) drain(c);
    ensure_workspace(c, n, n_seqs, int(b.work.size()), int(b.work2.size()), b.vl.cols);
    Workspace& w = c->ws;
    // The small arrays go through one pinned buffer: asynchronous copies, no wait for them here
    // (the forward's kernels follow them on the same stream).
    struct Piece {
        void* dst;
        const void* src;
        size_t bytes;
    };
    const Piece pieces[] = {{w.tokens, tokens, size_t(n) * 4},
                            {w.positions, positions, size_t(n) * 4},
                            {w.seqs, b.sr.data(), b.sr.size() * sizeof(SeqRange)},
                            {w.work, b.work.data(), b.work.size() * sizeof(AttnWork)},
                            {w.work2, b.work2.data(), b.work2.size() * sizeof(AttnWork)},
                            {w.vcol, b.vl.vcol.data(), b.work2.empty() ? 0 : size_t(n) * 4}};
    size_t total = 0;
    for (const Piece& pc : pieces) total += (pc.bytes + 255) / 256 * 256;
    if (c->staged_copy_recorded) hip_check(hipEventSynchronize(c->staged_copy), "hipEventSynchronize");
    if (total > c->pinned_cap) {
        if (c->pinned) hip_check(hipHostFree(c->pinned), "hipHostFree");
        c->pinned = nullptr;
        c->pinned_cap = 0;
        const size_t cap = std::max(total, size_t(1) << 20);
        hip_check(hipHostMalloc(&c->pinned, cap, hipHostMallocDefault), "hipHostMalloc");
        c->pinned_cap = cap;
    }
    size_t off = 0;
    for (const Piece& pc : pieces) {
        if (pc.bytes == 0) continue;
        unsigned char* h = static_cast<unsigned char*>(c->pinned) + off;
        std::memcpy(h, pc.src, pc.bytes);
        hip_check(hipMemcpyAsync(pc.dst, h, pc.bytes, hipMemcpyHostToDevice, c->stream), "upload batch");
        off += (pc.bytes + 255) / 256 * 256;
    }
    hip_check(hipEventRecord(c->staged_copy, c->stream), "hipEventRecord");
    c->staged_copy_recorded = true;
    set_staged(c, b, n, n_seqs, vectors);
}

// ---------------------------------------------------------------- forward

bool at(StopPoint* sp, const char* name, int layer) {
    if (!sp || sp->hit) return false;
    if (sp->name == name && sp->layer == layer) {
        sp->hit = true;
        return true;
    }
    return false;
}

// The output (CPUReference.swift:272-282): the mean of each sequence's final-norm rows (fp32),
// then the output projection of those means. The reference projects every token and averages
// the projections; the mean and the projection are both linear, so the order does not change
// the result beyond fp32 rounding, and here the projection runs once per sequence, in fp32.
void encode_tail(ge_ctx* c, hipStream_t s) {
    const DevModel& m = c->model;
    Workspace& w = c->ws;
    launch(c, "mean_pool", [&] { return launch_mean_pool(s, w.hn, w.seqs, c->staged_seqs, m.hidden, w.pooled_n); });
    launch(c, "output_projection", [&] {
        return launch_pooled_projection(s, w.pooled_n, c->staged_seqs, m.hidden, m.output, w.pooled);
    });
}

// MetalForward.encode (Metal/MetalForward.swift:364-423) for the text path without the
// per-layer-input branch: 7 launches per layer. Returns early after the op producing the stop point.
void encode(ge_ctx* c, StopPoint* sp) {
    const DevModel& m = c->model;
    Workspace& w = c->ws;
    const int T = c->staged_tokens;
    hipStream_t s = c->stream;
    const int D = m.hidden;
    launch(c, "embed_norm", [&] {
        return launch_embed_norm(s, m.tok_embd, w.tokens, T, m.emb_scale, c->staged_vectors, m.layer[0].attn_norm, m.eps, w.x, w.h);
    });
    if (at(sp, "inp_scaled", -1) || at(sp, "attn_norm", 0)) return;
    if (m.pl > 0) {
        // CPUReference.swift:206-210: the per-layer inputs from the scaled embedding rows
        launch(c, "ple_input", [&] { return launch_ple_input(s, w.x, T, D, w.x16, w.rs); });
        launch(c, "gemm_ple_model_proj", [&] { return launch_gemm_q8(s, m.pl_proj, w.x16, T, w.ple, kEpiF32); });
        launch(c, "ple_norm", [&] {
            return launch_ple_rmsnorm(s, w.ple, T * m.layers, m.pl, m.pl_scale, w.rs, m.layers, m.pl_norm, m.eps, w.ple);
        });
        if (at(sp, "inp_per_layer", -1)) return;
    }
    for (int l = 0; l < m.layers; l++) {
        const DevLayer& L = m.layer[size_t(l)];
        // The raw projection (trace points Qcur / Kcur / Vcur) only exists on the unfused path.
        const bool raw_qkv = sp && sp->layer == l && (sp->name == "Qcur" || sp->name == "Kcur" || sp->name == "Vcur");
        if (L.qkv_fused && !raw_qkv) {
            launch(c, "gemm_qkv", [&] {
                QkvEpilogue e;
                e.q_norm = L.q_norm;
                e.k_norm = L.k_norm;
                e.positions = w.positions;
                e.rope = L.rope;
                e.q = w.q;
                e.k = w.k;
                // Row-major V is read only by the attention without V^T and by traces.
                e.v = L.attn_v2 && !sp ? nullptr : w.v;
                e.vcol = w.vcol;
                e.vt = L.attn_v2 ? w.vt : nullptr;
                e.vt_cols = w.vt_cap;
                e.scale = L.qkv_c;
                e.eps = m.eps * L.qkv_c * L.qkv_c;
                e.heads = m.heads;
                e.kv_heads = L.kv_heads;
                e.stage = reinterpret_cast<uint16_t*>(w.qkv);  // [rows][max_qkv] fp32: room for fp16 [T][N]
                return launch_gemm_qkv(s, L.wqkv, w.h, T, L.head_dim, e);
            });
        } else if (L.precise) {
            launch(c, "norm_split", [&] { return launch_norm_split(s, w.x, L.attn_norm, m.eps, T, D, w.h3); });
            launch(c, "gemm_qkv", [&] { return launch_gemm_q8(s, L.wqkv3, w.h3, T, w.qkv, kEpiF32); });
            if (at(sp, "Qcur", l) || at(sp, "Kcur", l) || at(sp, "Vcur", l)) return;
            launch(c, "qk_norm_rope", [&] {
                return launch_qk_norm_rope(s, w.qkv, T, m.heads, L.kv_heads, L.head_dim, L.q_norm, L.k_norm, m.eps,
                                           w.positions, L.rope, w.q, w.k, w.v, w.q_lo, w.k_lo);
            });
        } else {
            launch(c, "gemm_qkv", [&] {
                return L.qkv_gn ? launch_gemm_q8(s, L.wqkv, w.h, T, w.qkv, kEpiF16, L.qkv_c)
                                : launch_gemm_q8(s, L.wqkv, w.h, T, w.qkv, kEpiF32);
            });
            if (at(sp, "Qcur", l) || at(sp, "Kcur", l) || at(sp, "Vcur", l)) return;
            launch(c, "qk_norm_rope", [&] {
                if (L.qkv_gn)
                    return launch_qkv_norm_rope_vt(s, reinterpret_cast<const uint16_t*>(w.qkv), T, m.heads, L.kv_heads,
                                                   L.head_dim, L.q_norm, L.k_norm, m.eps * L.qkv_c * L.qkv_c, w.positions,
                                                   L.rope, w.q, w.k, w.v, w.vcol, w.vt_cap, L.attn_v2 ? w.vt : nullptr);
                return launch_qk_norm_rope(s, w.qkv, T, m.heads, L.kv_heads, L.head_dim, L.q_norm, L.k_norm, m.eps,
                                           w.positions, L.rope, w.q, w.k, w.v);
            });
        }
        // The fused kernels also write V^T for the LDS-copy attention: the QKV GEMM's epilogue, or
        // the fp16 path's norm kernel.
        const bool fused_vt = (L.qkv_fused && !raw_qkv) || L.qkv_gn;
        if (at(sp, "Qcur_pos", l) || at(sp, "Kcur_pos", l) || at(sp, "Vcur_normed", l)) return;
        const int hw = L.sliding ? m.window / 2 : 0;  // halfWindow = slidingWindow / 2 (MetalForward.swift:399)
        if (L.attn_v2) {
            if (!fused_vt) launch(c, "v_transpose", [&] { return launch_v_transpose(s, w.v, T, L.kvd, w.vcol, w.vt_cap, w.vt); });
            launch(c, "attention", [&] {
                if (L.precise)
                    return launch_attention_split(s, w.q, w.q_lo, w.k, w.k_lo, w.vt, w.vt_cap, w.attn, w.work2, c->staged_work2,
                                                  m.heads, L.kv_heads, L.head_dim, hw, 1.0f, c->attn_items);
                return launch_attention_v2(s, w.q, w.k, w.vt, w.vt_cap, w.attn, w.work2, c->staged_work2, m.heads, L.kv_heads,
                                           L.head_dim, hw, 1.0f, c->attn_items);
            });
        } else {
            launch(c, "attention", [&] {
                return launch_attention(s, w.q, w.k, w.v, w.attn, w.work, c->staged_work, m.heads, L.kv_heads, L.head_dim, hw, 1.0f);
            });
        }
        if (at(sp, "kqv_out", l)) return;
        // t (fp32 [T][D]) holds two fp16 [T][D] halves: the o projection in the second, the down
        // projection in the first. Without the per-layer-input branch x is stored once per layer:
        // the attention residual's kernel writes only the FFN input h, and the FFN residual's
        // kernel sums both residuals into x (the sum after attention is stored only for its trace).
        uint16_t* t16 = reinterpret_cast<uint16_t*>(w.t);
        uint16_t* const o16 = t16 + size_t(T) * D;
        const bool x_once = m.pl == 0 && !(sp && !sp->hit && sp->layer == l && sp->name == "attn_out");
        launch(c, "gemm_o", [&] { return launch_gemm_q8(s, L.wo, w.attn, T, o16, kEpiF16, L.o_c); });
        if (x_once)
            launch(c, "residual_norm_h", [&] {
                return launch_residual_norm_h(s, w.x, o16, m.eps * L.o_c * L.o_c, L.post_attn, 1.0f, L.ffn_norm, m.eps, T, D, w.h);
            });
        else
            launch(c, "residual_norm", [&] {
                return launch_residual_norm(s, w.x, o16, m.eps * L.o_c * L.o_c, L.post_attn, 1.0f, L.ffn_norm, m.eps, T, D, w.h);
            });
        if (at(sp, "attn_out", l) || at(sp, "ffn_norm", l)) return;
        launch(c, "gemm_gate_up", [&] { return launch_gemm_q8(s, L.wgu, w.h, T, w.act, kEpiGeglu, L.act_scale); });
        if (at(sp, "ffn_geglu", l)) return;
        launch(c, "gemm_down", [&] { return launch_gemm_q8(s, L.wd, w.act, T, t16, kEpiF16, L.down_scale * L.down_c); });
        if (at(sp, "ffn_out", l)) return;
        const float* next = l + 1 < m.layers ? m.layer[size_t(l) + 1].attn_norm : m.out_norm;
        float* const h32 = l + 1 < m.layers ? nullptr : w.hn;  // the final norm stays fp32
        if (m.pl > 0) {
            // CPUReference.swift:259-269: x += rmsnorm(proj(gelu(inp_gate(x)) * ple_l), post_norm), then
            // the layer output scale; the unnormalised inputs of both projections go row-scaled
            launch(c, "ple_residual_input", [&] {
                return launch_ple_residual_input(s, w.x, t16, m.eps * L.down_c * L.down_c, L.post_ffw, T, D, w.x16, w.rs);
            });
            if (at(sp, "pe_in", l)) return;
            launch(c, "gemm_ple_gate", [&] { return launch_gemm_q8(s, L.inp_gate, w.x16, T, w.ple_t, kEpiF32); });
            launch(c, "ple_gate", [&] { return launch_ple_gate(s, w.ple_t, w.rs, w.ple, l, m.layers, T, m.pl, w.g16, w.rs2); });
            // the projection (fp32 [T][hidden]) goes to t, free once the FFN residual has read it
            launch(c, "gemm_ple_proj", [&] { return launch_gemm_q8(s, L.proj, w.g16, T, w.t, kEpiF32); });
            launch(c, "ple_residual_norm", [&] {
                return launch_ple_residual_norm(s, w.x, w.t, w.rs2, L.post_norm, L.out_scale, next, m.eps, T, D, w.h, h32);
            });
            if (at(sp, "l_out", l) || at(sp, "attn_norm", l + 1)) return;
            continue;
        }
        if (x_once)
            launch(c, "residual_norm_two", [&] {
                return launch_residual_norm_two(s, w.x, o16, m.eps * L.o_c * L.o_c, L.post_attn, 1.0f, t16,
                                                m.eps * L.down_c * L.down_c, L.post_ffw, L.out_scale, next, m.eps, T, D, w.h,
                                                h32);
            });
        else
            launch(c, "residual_norm", [&] {
                return launch_residual_norm(s, w.x, t16, m.eps * L.down_c * L.down_c, L.post_ffw, L.out_scale, next, m.eps, T, D,
                                            w.h, h32);
            });
        if (at(sp, "pe_in", l) || at(sp, "l_out", l) || at(sp, "attn_norm", l + 1)) return;
    }
    if (at(sp, "result_norm", -1)) return;
    if (sp && !sp->hit && sp->name == "result_embd") {
        // the reference's per-token projection, traced only: every row through the same projection
        launch(c, "output_projection", [&] { return launch_pooled_projection(s, w.hn, T, D, m.output, w.out); });
        at(sp, "result_embd", -1);
        return;
    }
    encode_tail(c, s);
}

// The forward of a split batch (see stage()): every layer's kernels run for each part's rows
// on the part's stream, launched part after part, so the parts' kernels overlap. The same kernels
// and arguments per row as encode(), so a token's values do not depend on the split; every layer
// must use the LDS-copy attention, whose work list stage() orders by part.
void encode_split(ge_ctx* c) {
    const DevModel& m = c->model;
    Workspace& w = c->ws;
    const int D = m.hidden;
    struct Half {
        hipStream_t s;
        int r0, T;
        const AttnWork* work;
        int n_work;
    };
    std::vector<Half> halves;
    for (int p = 0; p < c->n_parts; p++)
        halves.push_back(Half{c->part_stream[p], c->part_row[p], c->part_row[p + 1] - c->part_row[p],
                              w.work2 + c->part_work[p], c->part_work[p + 1] - c->part_work[p]});
    hip_check(hipEventRecord(c->ev_fork, c->stream), "hipEventRecord");
    for (int p = 0; p < c->n_parts; p++)
        if (c->part_stream[p] != c->stream) hip_check(hipStreamWaitEvent(c->part_stream[p], c->ev_fork, 0), "hipStreamWaitEvent");
    // The parts run unsynchronised, so one may be a layer ahead of another: each part owns the
    // slice of a buffer that starts at row r0 times the buffer's allocated width, whatever width a
    // layer uses (head dims differ between layers), and fp16 t16 lives in the part's slice of fp32 t.
    // The attention kernels index absolute rows: they take the base at which row r0 lands at its
    // part's slice (part_base), and rows past a sequence's end, which they read and mask, stay
    // inside the buffer.
    uint16_t* t16 = reinterpret_cast<uint16_t*>(w.t);
    auto rows = [](auto* base, int r0, size_t width) { return base + size_t(r0) * width; };
    auto part_base = [](auto* base, int r0, size_t width, size_t alloc_width) {
        return base + size_t(r0) * (alloc_width - width);
    };
    for (const Half& H : halves)
        launch(c, "embed_norm", [&] {
            return launch_embed_norm(H.s, m.tok_embd, w.tokens + H.r0, H.T, m.emb_scale, c->staged_vectors, m.layer[0].attn_norm, m.eps,
                                     rows(w.x, H.r0, D), rows(w.h, H.r0, D));
        });
    if (m.pl > 0) {
        const size_t LP = size_t(m.layers) * m.pl;
        for (const Half& H : halves)
            launch(c, "ple_input", [&] {
                return launch_ple_input(H.s, rows(w.x, H.r0, D), H.T, D, rows(w.x16, H.r0, D), w.rs + H.r0);
            });
        for (const Half& H : halves)
            launch(c, "gemm_ple_model_proj", [&] {
                return launch_gemm_q8(H.s, m.pl_proj, rows(w.x16, H.r0, D), H.T, rows(w.ple, H.r0, LP), kEpiF32);
            });
        for (const Half& H : halves)
            launch(c, "ple_norm", [&] {
                return launch_ple_rmsnorm(H.s, rows(w.ple, H.r0, LP), H.T * m.layers, m.pl, m.pl_scale, w.rs + H.r0, m.layers,
                                          m.pl_norm, m.eps, rows(w.ple, H.r0, LP));
            });
    }
    for (int l = 0; l < m.layers; l++) {
        const DevLayer& L = m.layer[size_t(l)];
        if (L.qkv_fused) {
            for (const Half& H : halves)
                launch(c, "gemm_qkv", [&] {
                    QkvEpilogue e;
                    e.q_norm = L.q_norm;
                    e.k_norm = L.k_norm;
                    e.positions = w.positions + H.r0;
                    e.rope = L.rope;
                    e.q = rows(w.q, H.r0, m.max_qd);
                    e.k = rows(w.k, H.r0, m.max_kvd);
                    e.v = nullptr;
                    e.vcol = w.vcol + H.r0;
                    e.vt = w.vt;
                    e.vt_cols = w.vt_cap;
                    e.scale = L.qkv_c;
                    e.eps = m.eps * L.qkv_c * L.qkv_c;
                    e.heads = m.heads;
                    e.kv_heads = L.kv_heads;
                    return launch_gemm_qkv(H.s, L.wqkv, rows(w.h, H.r0, D), H.T, L.head_dim, e);
                });
        } else {
            // the projection, then the norms and RoPE (fp16 kernel with V^T where the layout allows,
            // else fp32 and a separate transpose), as encode() does
            if (L.precise) {
                for (const Half& H : halves)
                    launch(c, "norm_split", [&] {
                        return launch_norm_split(H.s, rows(w.x, H.r0, D), L.attn_norm, m.eps, H.T, D, rows(w.h3, H.r0, 3 * size_t(D)));
                    });
                for (const Half& H : halves)
                    launch(c, "gemm_qkv", [&] {
                        return launch_gemm_q8(H.s, L.wqkv3, rows(w.h3, H.r0, 3 * size_t(D)), H.T, rows(w.qkv, H.r0, m.max_qkv),
                                              kEpiF32);
                    });
            } else {
                for (const Half& H : halves)
                    launch(c, "gemm_qkv", [&] {
                        return L.qkv_gn ? launch_gemm_q8(H.s, L.wqkv, rows(w.h, H.r0, D), H.T, rows(w.qkv, H.r0, m.max_qkv),
                                                         kEpiF16, L.qkv_c)
                                        : launch_gemm_q8(H.s, L.wqkv, rows(w.h, H.r0, D), H.T, rows(w.qkv, H.r0, m.max_qkv),
                                                         kEpiF32);
                    });
            }
            for (const Half& H : halves)
                launch(c, "qk_norm_rope", [&] {
                    if (L.qkv_gn)
                        return launch_qkv_norm_rope_vt(H.s, reinterpret_cast<const uint16_t*>(rows(w.qkv, H.r0, m.max_qkv)), H.T,
                                                       m.heads, L.kv_heads, L.head_dim, L.q_norm, L.k_norm,
                                                       m.eps * L.qkv_c * L.qkv_c, w.positions + H.r0, L.rope,
                                                       rows(w.q, H.r0, m.max_qd), rows(w.k, H.r0, m.max_kvd), rows(w.v, H.r0, m.max_kvd),
                                                       w.vcol + H.r0, w.vt_cap, w.vt);
                    return launch_qk_norm_rope(H.s, rows(w.qkv, H.r0, m.max_qkv), H.T, m.heads, L.kv_heads, L.head_dim, L.q_norm,
                                               L.k_norm, m.eps, w.positions + H.r0, L.rope, rows(w.q, H.r0, m.max_qd),
                                               rows(w.k, H.r0, m.max_kvd), rows(w.v, H.r0, m.max_kvd),
                                               L.precise ? rows(w.q_lo, H.r0, m.max_qd) : nullptr,
                                               L.precise ? rows(w.k_lo, H.r0, m.max_kvd) : nullptr);
                });
            if (!L.qkv_gn)
                for (const Half& H : halves)
                    launch(c, "v_transpose", [&] {
                        return launch_v_transpose(H.s, rows(w.v, H.r0, m.max_kvd), H.T, L.kvd, w.vcol + H.r0, w.vt_cap, w.vt);
                    });
        }
        const int hw = L.sliding ? m.window / 2 : 0;
        for (const Half& H : halves)
            launch(c, "attention", [&] {
                if (L.precise)
                    return launch_attention_split(H.s, part_base(w.q, H.r0, L.qd, m.max_qd), part_base(w.q_lo, H.r0, L.qd, m.max_qd),
                                                  part_base(w.k, H.r0, L.kvd, m.max_kvd), part_base(w.k_lo, H.r0, L.kvd, m.max_kvd),
                                                  w.vt, w.vt_cap, part_base(w.attn, H.r0, L.qd, m.max_qd), H.work, H.n_work, m.heads,
                                                  L.kv_heads, L.head_dim, hw, 1.0f, c->attn_items);
                return launch_attention_v2(H.s, part_base(w.q, H.r0, L.qd, m.max_qd), part_base(w.k, H.r0, L.kvd, m.max_kvd),
                                           w.vt, w.vt_cap, part_base(w.attn, H.r0, L.qd, m.max_qd), H.work, H.n_work, m.heads, L.kv_heads,
                                           L.head_dim, hw, 1.0f, c->attn_items);
            });
        // a part's rows of t hold its down projection (fp16) in their first half and its o
        // projection in the second, as encode() lays them out for the whole pack
        auto o16 = [&](const Half& H) { return rows(t16, H.r0, 2 * size_t(D)) + size_t(H.T) * D; };
        const bool x_once = m.pl == 0;
        for (const Half& H : halves)
            launch(c, "gemm_o", [&] {
                return launch_gemm_q8(H.s, L.wo, rows(w.attn, H.r0, m.max_qd), H.T, o16(H), kEpiF16, L.o_c);
            });
        for (const Half& H : halves) {
            if (x_once)
                launch(c, "residual_norm_h", [&] {
                    return launch_residual_norm_h(H.s, rows(w.x, H.r0, D), o16(H), m.eps * L.o_c * L.o_c, L.post_attn, 1.0f,
                                                  L.ffn_norm, m.eps, H.T, D, rows(w.h, H.r0, D));
                });
            else
                launch(c, "residual_norm", [&] {
                    return launch_residual_norm(H.s, rows(w.x, H.r0, D), o16(H), m.eps * L.o_c * L.o_c, L.post_attn, 1.0f,
                                                L.ffn_norm, m.eps, H.T, D, rows(w.h, H.r0, D));
                });
        }
        for (const Half& H : halves)
            launch(c, "gemm_gate_up", [&] {
                return launch_gemm_q8(H.s, L.wgu, rows(w.h, H.r0, D), H.T, rows(w.act, H.r0, m.ff), kEpiGeglu, L.act_scale);
            });
        for (const Half& H : halves)
            launch(c, "gemm_down", [&] {
                return launch_gemm_q8(H.s, L.wd, rows(w.act, H.r0, m.ff), H.T, rows(t16, H.r0, 2 * size_t(D)), kEpiF16,
                                      L.down_scale * L.down_c);
            });
        const float* next = l + 1 < m.layers ? m.layer[size_t(l) + 1].attn_norm : m.out_norm;
        const bool last = l + 1 == m.layers;  // the final norm stays fp32
        if (m.pl > 0) {
            const size_t LP = size_t(m.layers) * m.pl;
            for (const Half& H : halves)
                launch(c, "ple_residual_input", [&] {
                    return launch_ple_residual_input(H.s, rows(w.x, H.r0, D), rows(t16, H.r0, 2 * size_t(D)), m.eps * L.down_c * L.down_c,
                                                     L.post_ffw, H.T, D, rows(w.x16, H.r0, D), w.rs + H.r0);
                });
            for (const Half& H : halves)
                launch(c, "gemm_ple_gate", [&] {
                    return launch_gemm_q8(H.s, L.inp_gate, rows(w.x16, H.r0, D), H.T, rows(w.ple_t, H.r0, m.pl), kEpiF32);
                });
            for (const Half& H : halves)
                launch(c, "ple_gate", [&] {
                    return launch_ple_gate(H.s, rows(w.ple_t, H.r0, m.pl), w.rs + H.r0, rows(w.ple, H.r0, LP), l, m.layers,
                                           H.T, m.pl, rows(w.g16, H.r0, m.pl), w.rs2 + H.r0);
                });
            for (const Half& H : halves)
                launch(c, "gemm_ple_proj", [&] {
                    return launch_gemm_q8(H.s, L.proj, rows(w.g16, H.r0, m.pl), H.T, rows(w.t, H.r0, D), kEpiF32);
                });
            for (const Half& H : halves)
                launch(c, "ple_residual_norm", [&] {
                    return launch_ple_residual_norm(H.s, rows(w.x, H.r0, D), rows(w.t, H.r0, D), w.rs2 + H.r0, L.post_norm,
                                                    L.out_scale, next, m.eps, H.T, D, rows(w.h, H.r0, D),
                                                    last ? rows(w.hn, H.r0, D) : nullptr);
                });
            continue;
        }
        for (const Half& H : halves)
            launch(c, "residual_norm_two", [&] {
                return launch_residual_norm_two(H.s, rows(w.x, H.r0, D), o16(H), m.eps * L.o_c * L.o_c, L.post_attn, 1.0f,
                                                rows(t16, H.r0, 2 * size_t(D)), m.eps * L.down_c * L.down_c, L.post_ffw,
                                                L.out_scale, next, m.eps, H.T, D, rows(w.h, H.r0, D),
                                                last ? rows(w.hn, H.r0, D) : nullptr);
            });
    }
    for (int p = 0; p < c->n_parts; p++)
        if (c->part_stream[p] != c->stream) {
            hip_check(hipEventRecord(c->part_join[p], c->part_stream[p]), "hipEventRecord");
            hip_check(hipStreamWaitEvent(c->stream, c->part_join[p], 0), "hipStreamWaitEvent");
        }
    encode_tail(c, c->stream);
}

// Packs of at most this many tokens replay their forward as a HIP graph from the second run of
// the same shape on.
constexpr int kGraphMaxTokens = 64;
constexpr size_t kMaxGraphs = 32;

// A short pack's forward is ~170 launches of a few microseconds of work each, so launch latency,
// not the kernels, sets its time. The first run of a pack shape is eager and records the shape;
// the second captures the launches (encode) into a graph, which that run and every later one
// replays with one launch. The key holds everything the launches' arguments depend on besides
// the workspace and model addresses, and every graph is dropped when those change.
// GE_NO_GRAPHS=1 in the environment runs short packs eagerly, launch by launch, as on their
// first run: the same kernels and bits, for tools that trace kernel dispatches but not graph
// launches.
static bool graphs_disabled() {
    static const bool off = [] {
        const char* v = std::getenv("GE_NO_GRAPHS");
        return v && *v && std::strcmp(v, "0") != 0;
    }();
    return off;
}

void run_graph(ge_ctx* c) {
    const int key[6] = {c->staged_tokens, c->staged_seqs, c->staged_work, c->staged_work2, c->ws.vt_cap, c->attn_items};
    ShortGraph* g = nullptr;
    for (ShortGraph& x : c->graphs)
        if (std::equal(key, key + 6, x.key)) g = &x;
    if (!g) {
        if (c->graphs.size() >= kMaxGraphs) {
            // a launch of the oldest graph may still be queued (ge_batch_run returns before the
            // GPU is done): its executable is destroyed only once the streams are idle
            if (c->graphs.front().exec) {
                drain(c);
                (void)hipGraphExecDestroy(c->graphs.front().exec);
            }
            c->graphs.erase(c->graphs.begin());
        }
        ShortGraph n;
        std::copy(key, key + 6, n.key);
        c->graphs.push_back(n);
        encode(c, nullptr);
        return;
    }
    if (!g->exec) {
        hipGraph_t graph = nullptr;
        hip_check(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            encode(c, nullptr);
        } catch (...) {
            (void)hipStreamEndCapture(c->stream, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        hip_check(hipStreamEndCapture(c->stream, &graph), "hipStreamEndCapture");
        const hipError_t e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) g->exec = nullptr;
        hip_check(e, "hipGraphInstantiate");
    }
    hip_check(hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
}

// The rows ge_set_vectors uploaded, when they are as wide as the model's residual stream.
const float* own_vectors(ge_ctx* c) { return c->vec_rows && c->vec_width == c->model.hidden ? c->vec_buf : nullptr; }
int own_vector_rows(ge_ctx* c) { return own_vectors(c) ? c->vec_rows : 0; }

// Copies `rows` vector rows (fp32 [rows][width]) into the context's buffer, growing it when needed.
void set_vectors(ge_ctx* c, const float* rows, int n_rows, int width) {
    if (n_rows < 0 || (n_rows > 0 && (!rows || width <= 0))) fail(GE_ERR_INVALID, "bad vector rows");
    const size_t bytes = size_t(n_rows) * size_t(std::max(width, 0)) * 4;
    drain(c);  // queued work may read the rows
    // A staged batch that reads these rows stays valid only while the new rows still cover the
    // ones it names, at the residual stream's width, in the same buffer.
    if (c->staged_vectors && c->staged_vectors == c->vec_buf &&
        (bytes > c->vec_cap || n_rows < c->staged_vec_rows || width != c->model.hidden)) {
        c->staged_tokens = -1;
        c->staged_vectors = nullptr;
    }
    if (bytes > c->vec_cap) {
        if (c->vec_buf) hip_check(hipFree(c->vec_buf), "hipFree");
        c->vec_buf = nullptr;
        c->vec_cap = 0;
        c->vec_rows = 0;
        hip_check(hipMalloc(reinterpret_cast<void**>(&c->vec_buf), bytes), "hipMalloc vector rows");
        c->vec_cap = bytes;
    }
    if (bytes) hip_check(hipMemcpy(c->vec_buf, rows, bytes, hipMemcpyHostToDevice), "upload vector rows");
    c->vec_rows = n_rows;
    c->vec_width = width;
}

void run_forward(ge_ctx* c, double* gpu_seconds, bool record_start) {
    if (c->staged_tokens < 0) fail(GE_ERR_STATE, "no batch is staged");
    if (record_start) hip_check(hipEventRecord(c->ev_start, c->stream), "hipEventRecord");
    if (c->n_parts > 1 && !c->prof)
        encode_split(c);
    else if (!c->prof && !graphs_disabled() && c->staged_tokens <= kGraphMaxTokens && !c->staged_vectors)  // graphs hold no vector source
        run_graph(c);
    else
        encode(c, nullptr);
    hip_check(hipEventRecord(c->ev_stop, c->stream), "hipEventRecord");
    if (gpu_seconds) {
        hip_check(hipEventSynchronize(c->ev_stop), "hipEventSynchronize");
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, c->ev_start, c->ev_stop), "hipEventElapsedTime");
        *gpu_seconds = ms * 1e-3;
    }
}

void read_pooled(ge_ctx* c, float* out) {
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->prof) resolve_profile(c);
    hip_check(hipMemcpy(out, c->ws.pooled, size_t(c->staged_seqs) * c->model.out_dims * 4, hipMemcpyDeviceToHost), "read pooled");
}

// Copies `rows` x `width` of a device buffer (fp32 or fp16, row stride `stride`) starting at
// column `col0` into out as fp32.
void copy_out(ge_ctx* c, const void* src, bool f16, int rows, int stride, int col0, int width, float* out) {
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    const size_t es = f16 ? 2 : 4;
    std::vector<uint8_t> host((size_t)rows * stride * es);
    hip_check(hipMemcpy(host.data(), src, host.size(), hipMemcpyDeviceToHost), "trace copy");
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < width; i++) {
            const size_t idx = (size_t)r * stride + col0 + i;
            float v;
            if (f16) {
                uint16_t h;
                std::memcpy(&h, host.data() + idx * 2, 2);
                v = host_h2f(h);
            } else {
                std::memcpy(&v, host.data() + idx * 4, 4);
            }
            out[(size_t)r * width + i] = v;
        }
}

void trace(ge_ctx* c, const char* name, int layer, float* out, size_t cap, size_t* needed) {
    const DevModel& m = c->model;
    const Workspace& w = c->ws;
    const int T = c->staged_tokens;
    if (!name) fail(GE_ERR_INVALID, "null tensor name");
    if (layer < -1 || layer >= m.layers) fail(GE_ERR_INVALID, "layer %d out of range", layer);
    const DevLayer* L = layer >= 0 ? &m.layer[size_t(layer)] : nullptr;
    const std::string n = name;
    // Which buffer holds the tensor, its element type, row stride, column range.
    const void* buf = nullptr;
    float unscale = 1;  // a tensor stored scaled (DevLayer::qkv_c, down_c) is multiplied back
    bool f16 = false;
    int stride = 0, col0 = 0, width = 0;
    auto need_layer = [&] {
        if (!L) fail(GE_ERR_INVALID, "tensor %s needs a layer index", name);
    };
    if (n == "inp_scaled" || n == "attn_out" || n == "pe_in" || n == "l_out") {
        if (n != "inp_scaled") need_layer();
        buf = w.x; stride = width = m.hidden;
    } else if (n == "attn_norm" || n == "ffn_norm") {
        need_layer();
        buf = w.h; f16 = true; stride = width = m.hidden;
    } else if (n == "result_norm") {
        buf = w.hn; stride = width = m.hidden;
    } else if (n == "Qcur" || n == "Kcur" || n == "Vcur") {
        need_layer();
        buf = w.qkv; stride = L->qd + 2 * L->kvd;
        if (L->qkv_gn) { f16 = true; unscale = 1.0f / L->qkv_c; }
        if (n == "Qcur") { col0 = 0; width = L->qd; }
        else if (n == "Kcur") { col0 = L->qd; width = L->kvd; }
        else { col0 = L->qd + L->kvd; width = L->kvd; }
    } else if (n == "Qcur_pos") {
        need_layer();
        buf = w.q; f16 = true; stride = width = L->qd;
    } else if (n == "Kcur_pos" || n == "Vcur_normed") {
        need_layer();
        buf = n == "Kcur_pos" ? w.k : w.v; f16 = true; stride = width = L->kvd;
    } else if (n == "kqv_out") {
        need_layer();
        buf = w.attn; f16 = true; stride = width = L->qd;
    } else if (n == "ffn_geglu") {
        need_layer();
        buf = w.act; f16 = true; stride = width = m.ff;
        unscale = 1.0f / L->act_scale;  // stored times the power of two act_scale
    } else if (n == "ffn_out") {
        need_layer();
        buf = w.t; stride = width = m.hidden;
        f16 = true;
        unscale = 1.0f / L->down_c;
    } else if (n == "result_embd") {
        buf = w.out; stride = width = m.out_dims;
    } else if (n == "inp_per_layer" && m.pl > 0) {
        buf = w.ple; stride = width = m.layers * m.pl;
    } else {
        fail(GE_ERR_INVALID, "unknown trace tensor %s", name);
    }
    const size_t count = (size_t)T * width;
    if (needed) *needed = count;
    if (!out) return;
    if (cap < count) fail(GE_ERR_INVALID, "trace buffer holds %zu floats, %s needs %zu", cap, name, count);
    StopPoint sp{n, (n == "inp_scaled" || n == "result_norm" || n == "result_embd" || n == "inp_per_layer") ? -1 : layer,
                 false};
    encode(c, &sp);
    if (!sp.hit) fail(GE_ERR_INVALID, "tensor %s at layer %d is not produced by this forward", name, layer);
    copy_out(c, buf, f16, T, stride, col0, width, out);
    if (unscale != 1.0f)
        for (size_t i = 0; i < count; i++) out[i] *= unscale;
}

}  // namespace ge

using ge::Fail;
using ge::fail;
using ge::guarded;

extern "C" {

int ge_create(int device, ge_ctx** out) {
    if (!out) return GE_ERR_INVALID;
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) {
        ge::g_create_error = std::string("no HIP device is available: ") + hipGetErrorString(e);
        return GE_ERR_NO_DEVICE;
    }
    if (device < 0 || device >= count) {
        ge::g_create_error = "device " + std::to_string(device) + " does not exist (" + std::to_string(count) + " present)";
        return GE_ERR_INVALID;
    }
    std::unique_ptr<ge_ctx> c(new ge_ctx);
    c->device = device;
    int rc = guarded(c.get(), [&] {
        ge::hip_check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
        c->part_stream[0] = c->stream;
        for (int p = 0; p < ge::kMaxParts; p++) {
            if (p > 0) ge::hip_check(hipStreamCreateWithFlags(&c->part_stream[p], hipStreamNonBlocking), "hipStreamCreate");
            ge::hip_check(hipEventCreateWithFlags(&c->part_join[p], hipEventDisableTiming), "hipEventCreate");
        }
        ge::hip_check(hipEventCreate(&c->ev_start), "hipEventCreate");
        ge::hip_check(hipEventCreate(&c->ev_stop), "hipEventCreate");
        ge::hip_check(hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming), "hipEventCreate");
        ge::hip_check(hipEventCreateWithFlags(&c->staged_copy, hipEventDisableTiming), "hipEventCreate");

        hipDeviceProp_t prop;
        ge::hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        c->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            fail(GE_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 (MI355X)", device, prop.gcnArchName);
        ge::hip_check(ge::configure_kernels(), "configure kernels");
        ge::noalloc_init(c.get());
    });
    if (rc != GE_OK) {
        ge::g_create_error = c->err;
        for (int p = 0; p < ge::kMaxParts; p++) {
            if (c->part_stream[p] && c->part_stream[p] != c->stream) (void)hipStreamDestroy(c->part_stream[p]);
            if (c->part_join[p]) (void)hipEventDestroy(c->part_join[p]);
        }
        if (c->stream) (void)hipStreamDestroy(c->stream);
        for (hipEvent_t e : {c->ev_start, c->ev_stop, c->ev_fork, c->staged_copy})
            if (e) (void)hipEventDestroy(e);
        return rc;
    }
    *out = c.release();
    return GE_OK;
}

void ge_destroy(ge_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    // Every stream that may still run kernels on the buffers below drains first: the context's
    // stream, and the part streams, whose work the context's stream joins only when a forward
    // ends normally (a forward that failed between the fork and the join leaves theirs unjoined).
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (int p = 0; p < ge::kMaxParts; p++)
        if (c->part_stream[p] && c->part_stream[p] != c->stream) (void)hipStreamSynchronize(c->part_stream[p]);
    ge::free_workspace(c);
    ge::free_model(c);
    ge::free_vision(c);
    if (c->vec_buf) (void)hipFree(c->vec_buf);
    for (auto& p : c->prof_pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    for (auto e : c->event_pool) (void)hipEventDestroy(e);
    if (c->ev_start) (void)hipEventDestroy(c->ev_start);
    if (c->ev_stop) (void)hipEventDestroy(c->ev_stop);
    if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
    if (c->staged_copy) (void)hipEventDestroy(c->staged_copy);
    if (c->pinned) (void)hipHostFree(c->pinned);
    for (int p = 0; p < ge::kMaxParts; p++) {
        if (c->part_stream[p] && c->part_stream[p] != c->stream) (void)hipStreamDestroy(c->part_stream[p]);
        if (c->part_join[p]) (void)hipEventDestroy(c->part_join[p]);
    }
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char* ge_last_error(const ge_ctx* c) { return c ? c->err.c_str() : "null context"; }
const char* ge_create_error(void) { return ge::g_create_error.c_str(); }
const char* ge_device_name(const ge_ctx* c) { return c ? c->name.c_str() : ""; }

int ge_set_split_scores(ge_ctx* c, int32_t min_head_dim) {
    return guarded(c, [&] {
        if (min_head_dim < 0) fail(GE_ERR_INVALID, "split-score head dim %d is negative", min_head_dim);
        c->split_head_dim = min_head_dim;
    });
}

int ge_upload_model(ge_ctx* c, const ge_model_desc* desc, const void* base, size_t len) {
    return guarded(c, [&] {
        try {
            ge::upload(c, desc, base, len);
        } catch (...) {
            ge::free_model(c);
            throw;
        }
    });
}

int ge_forward(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int32_t n, const ge_seq* seqs, int32_t n_seqs,
               float* pooled, double* gpu_seconds) {
    return guarded(c, [&] {
        if (!pooled) fail(GE_ERR_INVALID, "null output");
        ge::stage(c, tokens, positions, n, seqs, n_seqs, ge::own_vectors(c), ge::own_vector_rows(c));
        ge::run_forward(c, gpu_seconds);
        ge::read_pooled(c, pooled);
    });
}

int ge_forward_trace(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int32_t n, const ge_seq* seqs,
                     int32_t n_seqs, const char* name, int32_t layer, float* out, size_t cap, size_t* needed) {
    return guarded(c, [&] {
        ge::stage(c, tokens, positions, n, seqs, n_seqs, ge::own_vectors(c), ge::own_vector_rows(c));
        ge::trace(c, name, layer, out, cap, needed);
    });
}

int ge_batch_stage(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int32_t n, const ge_seq* seqs, int32_t n_seqs) {
    return guarded(c, [&] { ge::stage(c, tokens, positions, n, seqs, n_seqs, ge::own_vectors(c), ge::own_vector_rows(c)); });
}

int ge_set_vectors(ge_ctx* c, const float* rows, int32_t n_rows, int32_t width) {
    return guarded(c, [&] { ge::set_vectors(c, rows, n_rows, width); });
}

int ge_batch_run(ge_ctx* c) {
    return guarded(c, [&] { ge::run_forward(c, nullptr); });
}

int ge_batch_read(ge_ctx* c, float* pooled) {
    return guarded(c, [&] {
        if (!pooled) fail(GE_ERR_INVALID, "null output");
        if (c->staged_tokens < 0) fail(GE_ERR_STATE, "no batch is staged");
        ge::read_pooled(c, pooled);
    });
}

int ge_sync(ge_ctx* c) {
    return guarded(c, [&] {
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        if (c->prof) ge::resolve_profile(c);
    });
}

int ge_profile_enable(ge_ctx* c, const char* prefix) {
    return guarded(c, [&] {
        c->prof = true;
        c->prof_prefix = prefix ? prefix : "";
    });
}

int ge_profile_disable(ge_ctx* c) {
    return guarded(c, [&] {
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        ge::resolve_profile(c);
        c->prof = false;
    });
}

int ge_profile_reset(ge_ctx* c) {
    return guarded(c, [&] {
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        ge::resolve_profile(c);
        c->prof_stats.clear();
    });
}

int ge_profile_get(ge_ctx* c, int32_t i, const char** name, int64_t* launches, double* total_ms) {
    return guarded(c, [&] {
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        ge::resolve_profile(c);
        if (i < 0 || size_t(i) >= c->prof_stats.size()) fail(GE_ERR_INVALID, "no kernel class %d", i);
        if (name) *name = c->prof_stats[size_t(i)].first.c_str();
        if (launches) *launches = c->prof_stats[size_t(i)].second.launches;
        if (total_ms) *total_ms = c->prof_stats[size_t(i)].second.ms;
    });
}

void* ge_dev_alloc(ge_ctx* c, size_t bytes) {
    void* p = nullptr;
    int rc = guarded(c, [&] {
        p = ge::dev_alloc(bytes, "ge_dev_alloc");
        // zeroed before the pointer is returned, whichever stream the caller uses next
        ge::hip_check(hipMemsetAsync(p, 0, bytes ? bytes : 16, c->stream), "hipMemsetAsync");
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
    return rc == GE_OK ? p : nullptr;
}

int ge_dev_free(ge_ctx* c, void* p) {
    return guarded(c, [&] { ge::hip_check(hipFree(p), "hipFree"); });
}

int ge_dev_upload(ge_ctx* c, void* dst, const void* src, size_t bytes) {
    return guarded(c, [&] { ge::hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D"); });
}

int ge_dev_download(ge_ctx* c, void* dst, const void* src, size_t bytes) {
    return guarded(c, [&] {
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        ge::hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    });
}

int ge_op_f32_to_f16(ge_ctx* c, const void* src, void* dst, size_t n) {
    return guarded(c, [&] {
        ge::launch(c, "f32_to_f16", [&] { return ge::launch_f32_to_f16(c->stream, static_cast<const float*>(src), static_cast<uint16_t*>(dst), n); });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_f16_to_f32(ge_ctx* c, const void* src, void* dst, size_t n) {
    return guarded(c, [&] {
        ge::launch(c, "f16_to_f32", [&] { return ge::launch_f16_to_f32(c->stream, static_cast<const uint16_t*>(src), static_cast<float*>(dst), n); });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_q8_create(ge_ctx* c, const void* rows_q8, int32_t rows, int32_t cols, ge_q8_matrix** out) {
    if (out) *out = nullptr;
    std::unique_ptr<ge_q8_matrix> m(new ge_q8_matrix);
    int rc = guarded(c, [&] {
        if (!rows_q8 || !out || rows <= 0 || cols <= 0 || cols % 32) fail(GE_ERR_INVALID, "Q8_0 matrix needs rows > 0 and cols a multiple of 32");
        ge::HostQ8 h = ge::host_q8(rows, cols);
        ge::repack_rows(static_cast<const uint8_t*>(rows_q8), rows, cols, &h, 0);
        m->m.rows = rows;
        m->m.cols = cols;
        m->m.q = static_cast<int8_t*>(ge::dev_alloc(h.q.size(), "q8 matrix"));
        m->m.s = static_cast<uint16_t*>(ge::dev_alloc(h.s.size() * 2, "q8 matrix"));
        ge::hip_check(hipMemcpy(m->m.q, h.q.data(), h.q.size(), hipMemcpyHostToDevice), "hipMemcpy");
        ge::hip_check(hipMemcpy(m->m.s, h.s.data(), h.s.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
        if (ge::wants_fragments(m->m)) {
            ge::build_fragments(c->stream, &m->m, "q8 matrix");
            ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        }
    });
    if (rc != GE_OK) {
        if (m->m.q) (void)hipFree(m->m.q);
        if (m->m.s) (void)hipFree(m->m.s);
        if (m->m.fh) (void)hipFree(m->m.fh);
        return rc;
    }
    *out = m.release();
    return GE_OK;
}

int ge_op_q8_destroy(ge_ctx* c, ge_q8_matrix* m) {
    if (!m) return GE_OK;
    int rc = guarded(c, [&] {
        ge::hip_check(hipFree(m->m.q), "hipFree");
        ge::hip_check(hipFree(m->m.s), "hipFree");
        if (m->m.fh) ge::hip_check(hipFree(m->m.fh), "hipFree");
    });
    delete m;
    return rc;
}

int ge_op_gemm_q8(ge_ctx* c, const ge_q8_matrix* w, const void* x, int32_t m, void* y, int32_t y_f16) {
    return guarded(c, [&] {
        if (!w) fail(GE_ERR_INVALID, "null matrix");
        ge::launch(c, "gemm", [&] {
            return ge::launch_gemm_q8(c->stream, w->m, static_cast<const uint16_t*>(x), m, y, y_f16 ? ge::kEpiF16 : ge::kEpiF32);
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int ge_op_gemm_q8_geglu(ge_ctx* c, const ge_q8_matrix* gate, const ge_q8_matrix* up, const void* x, int32_t m, void* act) {
    return guarded(c, [&] {
        if (!gate || !up) fail(GE_ERR_INVALID, "null matrix");
        if (gate->m.rows != up->m.rows || gate->m.cols != up->m.cols || gate->m.rows % 32)
            fail(GE_ERR_INVALID, "gate and up must have the same shape, rows a multiple of 32");
        // Interleave the two matrices' rows in 32-row groups on the device.
        const int F = gate->m.rows, K = gate->m.cols;
        ge::Q8Dev gu;
        gu.rows = 2 * F;
        gu.cols = K;
        gu.q = static_cast<int8_t*>(ge::dev_alloc((size_t)gu.rows * K, "geglu"));
        gu.s = static_cast<uint16_t*>(ge::dev_alloc((size_t)gu.rows * (K / 32) * 2, "geglu"));
        struct Free {
            ge::Q8Dev* p;
            ~Free() {
                (void)hipFree(p->q);
                (void)hipFree(p->s);
                if (p->fh) (void)hipFree(p->fh);
            }
        } guard{&gu};
        for (int jb = 0; jb < F / 32; jb++) {
            for (int half = 0; half < 2; half++) {
                const ge::Q8Dev& src = half ? up->m : gate->m;
                ge::hip_check(hipMemcpyAsync(gu.q + (size_t)(jb * 64 + half * 32) * K, src.q + (size_t)jb * 32 * K, (size_t)32 * K,
                                             hipMemcpyDeviceToDevice, c->stream), "hipMemcpy");
                ge::hip_check(hipMemcpyAsync(gu.s + (size_t)(jb * 64 + half * 32) * (K / 32), src.s + (size_t)jb * 32 * (K / 32),
                                             (size_t)32 * (K / 32) * 2, hipMemcpyDeviceToDevice, c->stream), "hipMemcpy");
            }
        }
        if (ge::wants_fragments(gu)) ge::build_fragments(c->stream, &gu, "geglu");
        ge::launch(c, "gemm_geglu", [&] {
            return ge::launch_gemm_q8(c->stream, gu, static_cast<const uint16_t*>(x), m, act, ge::kEpiGeglu);
        });
        ge::hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    });
}

int32_t ge_attention_queries(void) { return ge::kAttnQueries; }

}  // extern "C"

namespace ge {

// Kernels.attention on device memory (ge_op_attention, ge_op_attention_split): with q_lo and k_lo
// set, the split-precision scores.
void op_attention(ge_ctx* c, const void* q, const void* q_lo, const void* k, const void* k_lo, const void* v, void* out,
                  const void* work, int n_work, int heads, int kv_heads, int head_dim, int half_window, float scale) {
    if (n_work < 0 || (n_work > 0 && !work)) fail(GE_ERR_INVALID, "bad attention work list");
    const bool split = q_lo || k_lo;
    if (split && (!q_lo || !k_lo || !attention_split_supported(head_dim, heads, kv_heads)))
        fail(GE_ERR_INVALID, "split-precision attention takes q_lo and k_lo, and head dim 512 with 4 query heads per KV head or 256 with 3");
    if (n_work == 0) return;
    // The ABI's work items (ge_attention_work) come in; the kernels take ge::AttnWork.
    std::vector<ge_attention_work> items(static_cast<size_t>(n_work), ge_attention_work{});
    hip_check(hipMemcpy(items.data(), work, items.size() * sizeof(ge_attention_work), hipMemcpyDeviceToHost), "read work");
    std::vector<void*> temps;
    struct Free {
        std::vector<void*>* p;
        ~Free() {
            for (void* x : *p) (void)hipFree(x);
        }
    } guard{&temps};
    auto temp = [&](size_t bytes) {
        void* p = dev_alloc(bytes, "attention op");
        temps.push_back(p);
        return p;
    };
    if (split || attention_v2_supported(head_dim, heads, kv_heads)) {
        // The sequences behind the work items, in order; V transposed into their layout.
        std::vector<ge_seq> seqs;
        int T = 0;
        for (const auto& it : items) {
            if (seqs.empty() || seqs.back().start != it.seq_start || seqs.back().length != it.seq_len)
                if (it.q0 == 0) seqs.push_back(ge_seq{it.seq_start, it.seq_len});
            T = std::max(T, int(it.seq_start + it.seq_len));
        }
        const VtLayout vl = vt_layout(T, seqs.data(), int(seqs.size()));
        std::vector<AttnWork> w2;
        for (size_t s = 0; s < seqs.size(); s++)
            for (uint32_t q0 = 0; q0 < seqs[s].length; q0 += kAttnQueriesV2)
                w2.push_back(AttnWork{seqs[s].start, seqs[s].length, q0, vl.start[s]});
        const int kvd = kv_heads * head_dim;
        auto* vt = static_cast<uint16_t*>(temp(size_t(kvd) * vl.cols * 2));
        auto* vcol = static_cast<int32_t*>(temp(size_t(T) * 4));
        auto* dw = static_cast<AttnWork*>(temp(w2.size() * sizeof(AttnWork)));
        hip_check(hipMemsetAsync(vt, 0, size_t(kvd) * vl.cols * 2, c->stream), "hipMemset");
        hip_check(hipMemcpyAsync(vcol, vl.vcol.data(), size_t(T) * 4, hipMemcpyHostToDevice, c->stream), "upload");
        hip_check(hipMemcpyAsync(dw, w2.data(), w2.size() * sizeof(AttnWork), hipMemcpyHostToDevice, c->stream), "upload");
        launch(c, "v_transpose", [&] {
            return launch_v_transpose(c->stream, static_cast<const uint16_t*>(v), T, kvd, vcol, vl.cols, vt);
        });
        launch(c, "attention", [&] {
            const auto* qh = static_cast<const uint16_t*>(q);
            const auto* kh = static_cast<const uint16_t*>(k);
            if (split)
                return launch_attention_split(c->stream, qh, static_cast<const uint16_t*>(q_lo), kh,
                                              static_cast<const uint16_t*>(k_lo), vt, vl.cols, static_cast<uint16_t*>(out), dw,
                                              int(w2.size()), heads, kv_heads, head_dim, half_window, scale, kAttnQueriesV2);
            return launch_attention_v2(c->stream, qh, kh, vt, vl.cols, static_cast<uint16_t*>(out), dw, int(w2.size()), heads,
                                       kv_heads, head_dim, half_window, scale);
        });
    } else {
        std::vector<AttnWork> w1;
        for (const auto& it : items) w1.push_back(AttnWork{it.seq_start, it.seq_len, it.q0, 0});
        auto* dw = static_cast<AttnWork*>(temp(w1.size() * sizeof(AttnWork)));
        hip_check(hipMemcpyAsync(dw, w1.data(), w1.size() * sizeof(AttnWork), hipMemcpyHostToDevice, c->stream), "upload");
        launch(c, "attention", [&] {
            return launch_attention(c->stream, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                    static_cast<const uint16_t*>(v), static_cast<uint16_t*>(out), dw, n_work, heads, kv_heads,
                                    head_dim, half_window, scale);
        });
    }
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

}  // namespace ge

extern "C" {

int ge_op_attention(ge_ctx* c, const void* q, const void* k, const void* v, void* out, const void* work, int32_t n_work,
                    int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t half_window, float scale) {
    return guarded(c, [&] {
        ge::op_attention(c, q, nullptr, k, nullptr, v, out, work, n_work, heads, kv_heads, head_dim, half_window, scale);
    });
}

int ge_op_attention_split(ge_ctx* c, const void* q, const void* q_lo, const void* k, const void* k_lo, const void* v,
                          void* out, const void* work, int32_t n_work, int32_t heads, int32_t kv_heads, int32_t head_dim,
                          int32_t half_window, float scale) {
    return guarded(c, [&] {
        if (!q_lo || !k_lo) ge::fail(GE_ERR_INVALID, "split-precision attention needs q_lo and k_lo");
        ge::op_attention(c, q, q_lo, k, k_lo, v, out, work, n_work, heads, kv_heads, head_dim, half_window, scale);
    });
}

}  // extern "C"
