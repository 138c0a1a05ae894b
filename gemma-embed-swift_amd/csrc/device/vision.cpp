// The image tower on the device: weight upload from an image-encoder GGUF's tensor directory,
// staging of a batch of images (patches plus pool grids), the forward and named-tensor traces.
// Plays the role of the reference's Metal/VisionTower.swift (VisionBatch :8-34, VisionWorkspace
// :38-82, upload :113-140, encode :143-185) for BASELINE config 5's encoder: LayerNorm with bias
// before attention and MLP, biased projections, a non-gated gelu_tanh MLP, heads of 72, learned
// column and row position tables (the reference's table layout), a final LayerNorm, 3x3 mean
// pooling, the projector's weighted RMSNorm and a Q8_0 projection into the text space.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "runtime_internal.hpp"

namespace ge {

struct VitLayer {
    Q8Dev wqkv, wo, wup, wdown;  // wup rows padded to ff_pad; wdown columns padded to ff_pad
    float *ln1_w = nullptr, *ln1_b = nullptr, *bqkv = nullptr, *bo = nullptr;
    float *ln2_w = nullptr, *ln2_b = nullptr, *bup = nullptr, *bdown = nullptr;
    // q, k, v are stored in fp16 times qkv_c, the MLP activation times act_c, the attention
    // output projection times o_c and the MLP down projection times down_c (powers of two from
    // load-time bounds, so the values stay inside fp16's range; their consumers divide back).
    float qkv_c = 1, act_c = 1, o_c = 1, down_c = 1;
};

struct VisionState {
    int layers = 0, hidden = 0, heads = 0, hd = 0, hp = 0, ff = 0, ff_pad = 0, patch = 0, area = 0, merge = 0;
    int proj = 0, npos = 0;
    float eps = 1e-6f;
    Q8Dev patch_w, proj_w;
    float *patch_b = nullptr, *pos = nullptr, *post_w = nullptr, *post_b = nullptr, *norm_w = nullptr;
    std::vector<VitLayer> layer;
    std::vector<void*> weights;
    // workspace (grow-only), rows with kRowSlack of slack
    int rows = 0, tok_rows = 0, work_cap = 0, vt_cap = 0;
    float *patches32 = nullptr, *x = nullptr, *t = nullptr, *pooled = nullptr, *out = nullptr;
    uint16_t *patches16 = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *vt = nullptr;
    uint16_t *attn = nullptr, *act = nullptr, *pooled16 = nullptr, *o16 = nullptr;
    int32_t *px = nullptr, *py = nullptr, *vcol = nullptr, *tok_row0 = nullptr, *tok_gx = nullptr;
    AttnWork* work = nullptr;
    // staged batch
    int staged_patches = -1, staged_tokens = 0, staged_work = 0;
    int items = kAttnQueriesV2;  // query rows per attention work item of the staged batch
};

namespace {

// Smallest count of 256-query attention workgroups for which a batch takes them (one per CU).
constexpr int64_t kVitWideItems = 256;

VisionState& vision_of(ge_ctx* c) {
    if (!c->vision) fail(GE_ERR_STATE, "no image encoder has been uploaded");
    return *c->vision;
}

void free_vision_workspace(VisionState& v) {
    void* ps[] = {v.patches32, v.x, v.t, v.pooled, v.out, v.patches16, v.h, v.q, v.k, v.v, v.vt, v.attn, v.act,
                  v.pooled16, v.o16, v.px, v.py, v.vcol, v.tok_row0, v.tok_gx, v.work};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    v.patches32 = v.x = v.t = v.pooled = v.out = nullptr;
    v.patches16 = v.h = v.q = v.k = v.v = v.vt = v.attn = v.act = v.pooled16 = v.o16 = nullptr;
    v.px = v.py = v.vcol = v.tok_row0 = v.tok_gx = nullptr;
    v.work = nullptr;
    v.rows = v.tok_rows = v.work_cap = v.vt_cap = 0;
    v.staged_patches = -1;
}

const ge_tensor_desc* vfind(const ge_vision_desc* d, const std::string& name) {
    for (int i = 0; i < d->n_tensors; i++)
        if (d->tensors[i].name && name == d->tensors[i].name) return &d->tensors[i];
    fail(GE_ERR_MODEL, "image encoder file lacks tensor %s", name.c_str());
}

float* upload_floats(VisionState& v, const std::vector<float>& h, const char* what) {
    float* p = static_cast<float*>(dev_alloc(h.size() * 4, what));
    v.weights.push_back(p);
    hip_check(hipMemcpy(p, h.data(), h.size() * 4, hipMemcpyHostToDevice), "hipMemcpy weights");
    return p;
}

// An F32 vector tensor of n elements, zero-padded to n_pad.
std::vector<float> f32_vector(const ge_vision_desc* d, const std::string& name, int64_t n, const void* base, size_t len,
                              int64_t n_pad = -1) {
    const ge_tensor_desc* t = vfind(d, name);
    check_shape(t, n, 1);
    if (t->type != GE_TYPE_F32) fail(GE_ERR_MODEL, "tensor %s uses storage type %d; vectors must be F32", t->name, t->type);
    const float* p = reinterpret_cast<const float*>(tensor_ptr(t, base, len));
    std::vector<float> out(size_t(n_pad < 0 ? n : n_pad), 0.0f);
    std::memcpy(out.data(), p, size_t(n) * 4);
    return out;
}

double max_abs(const std::vector<float>& v) {
    double m = 0;
    for (float x : v) m = std::max(m, double(std::fabs(x)));
    return m;
}

double l2(const std::vector<float>& v) {
    double s = 0;
    for (float x : v) s += double(x) * x;
    return std::sqrt(s);
}

// A Q8_0 [cols, rows] tensor's rows, zero rows appended up to rows_pad.
HostQ8 q8_rows(const ge_vision_desc* d, const std::string& name, int64_t cols, int64_t rows, const void* base, size_t len,
               int rows_pad) {
    const ge_tensor_desc* t = vfind(d, name);
    check_shape(t, cols, rows);
    if (t->type != GE_TYPE_Q8_0)
        fail(GE_ERR_MODEL, "tensor %s uses storage type %d; the image tower's projections take Q8_0", t->name, t->type);
    if (cols % 32) fail(GE_ERR_MODEL, "tensor %s: Q8_0 rows must be a multiple of 32 wide", t->name);
    HostQ8 h = host_q8(rows_pad, int(cols));
    repack_rows(tensor_ptr(t, base, len), int(rows), int(cols), &h, 0);
    return h;
}

// A [cols, rows] weight of any accepted type as fp16 MFMA fragments, columns zero-padded.
Q8Dev fragments_any(VisionState& v, const ge_vision_desc* d, const std::string& name, int64_t cols, int64_t rows,
                    int cols_pad, const void* base, size_t len, double* row_norm = nullptr) {
    return upload_fragments(vfind(d, name), cols, rows, cols_pad, base, len, v.weights, row_norm);
}

Q8Dev upload_vision_q8(ge_ctx* c, VisionState& v, const HostQ8& h, const char* what) {
    // upload_q8 records its allocations on the context; move them to the tower's list
    const size_t before = c->weight_allocs.size();
    Q8Dev d = upload_q8(c, h, what);
    v.weights.insert(v.weights.end(), c->weight_allocs.begin() + long(before), c->weight_allocs.end());
    c->weight_allocs.resize(before);
    return d;
}

void vision_upload(ge_ctx* c, const ge_vision_desc* d, const void* base, size_t len) {
    if (!d || !base) fail(GE_ERR_INVALID, "null image encoder descriptor or file base");
    if (d->layers <= 0 || d->hidden <= 0 || d->heads <= 0 || d->feed_forward <= 0 || d->patch_size <= 0 ||
        d->merge <= 0 || d->proj_dims <= 0 || d->positions <= 0)
        fail(GE_ERR_MODEL, "image encoder descriptor has a non-positive size");
    if (d->hidden % 64 || d->hidden > kVitMaxWidth)
        fail(GE_ERR_MODEL, "vision width %d: the kernels need a multiple of 64 up to %d", d->hidden, kVitMaxWidth);
    if (d->hidden % d->heads) fail(GE_ERR_MODEL, "vision width %d does not split into %d heads", d->hidden, d->heads);
    if (d->proj_dims % 64) fail(GE_ERR_MODEL, "projection_dim %d is not a multiple of 64", d->proj_dims);
    const int hd = d->hidden / d->heads;
    int hp = 0;
    if (attention_padded_supported(96, hd, d->heads, d->heads))
        hp = 96;
    else if (attention_v2_supported(hd, d->heads, d->heads))
        hp = hd;
    else
        fail(GE_ERR_MODEL, "vision head dim %d is not supported (72, 128 and 256 are)", hd);
    const int area = 3 * d->patch_size * d->patch_size;
    if (area % 32) fail(GE_ERR_MODEL, "patch area %d is not a multiple of 32", area);
    std::unique_ptr<VisionState> vs(new VisionState);
    VisionState& v = *vs;
    try {
        v.layers = d->layers;
        v.hidden = d->hidden;
        v.heads = d->heads;
        v.hd = hd;
        v.hp = hp;
        v.ff = d->feed_forward;
        v.ff_pad = (d->feed_forward + 63) / 64 * 64;
        v.patch = d->patch_size;
        v.area = area;
        v.merge = d->merge;
        v.proj = d->proj_dims;
        v.npos = d->positions;
        v.eps = d->eps;
        const int D = v.hidden;
        const double rD = std::sqrt(double(D));
        v.patch_w = upload_vision_q8(c, v, q8_rows(d, "v.patch_embd.weight", area, D, base, len, D), "v.patch_embd");
        v.patch_b = upload_floats(v, f32_vector(d, "v.patch_embd.bias", D, base, len), "v.patch_embd.bias");
        {
            const ge_tensor_desc* t = vfind(d, "v.position_embd.weight");
            check_shape(t, D, 2 * int64_t(v.npos));
            if (t->type != GE_TYPE_F32) fail(GE_ERR_MODEL, "tensor %s uses storage type %d; it must be F32", t->name, t->type);
            const float* p = reinterpret_cast<const float*>(tensor_ptr(t, base, len));
            v.pos = upload_floats(v, std::vector<float>(p, p + size_t(2) * v.npos * D), "v.position_embd");
        }
        // An fp16 LayerNorm output h satisfies |h_i| <= sqrt(D) |w_i| + |b_i| and
        // ||h||_2 <= sqrt(D) max|w| + ||b||_2.
        auto ln_bounds = [&](const std::vector<float>& w, const std::vector<float>& b, const std::string& name) {
            const double elem = rD * max_abs(w) + max_abs(b);
            if (elem >= 65504.0) fail(GE_ERR_MODEL, "%s: LayerNorm outputs may leave fp16's range", name.c_str());
            return rD * max_abs(w) + l2(b);
        };
        for (int l = 0; l < v.layers; l++) {
            VitLayer L;
            const std::string b = "v.blk." + std::to_string(l) + ".";
            const auto ln1w = f32_vector(d, b + "ln1.weight", D, base, len), ln1b = f32_vector(d, b + "ln1.bias", D, base, len);
            const auto ln2w = f32_vector(d, b + "ln2.weight", D, base, len), ln2b = f32_vector(d, b + "ln2.bias", D, base, len);
            const double hn1 = ln_bounds(ln1w, ln1b, b + "ln1"), hn2 = ln_bounds(ln2w, ln2b, b + "ln2");
            double qkv_bound = 0, act_bound = 0;
            {
                HostQ8 h = host_q8(3 * D, D);
                const char* parts[3] = {"attn_q", "attn_k", "attn_v"};
                std::vector<float> bias;
                for (int p = 0; p < 3; p++) {
                    const HostQ8 one = q8_rows(d, b + parts[p] + ".weight", D, D, base, len, D);
                    std::copy(one.q.begin(), one.q.end(), h.q.begin() + long(p) * D * D);
                    std::copy(one.s.begin(), one.s.end(), h.s.begin() + long(p) * D * (D / 32));
                    const auto bp = f32_vector(d, b + parts[p] + ".bias", D, base, len);
                    bias.insert(bias.end(), bp.begin(), bp.end());
                }
                L.wqkv = upload_vision_q8(c, v, h, "v.attn_qkv");
                L.bqkv = upload_floats(v, bias, "v.attn_qkv.bias");
                // |q_j| <= ||h|| ||W_j|| + |b_j|
                qkv_bound = hn1 * max_row_norm(h) + max_abs(bias);
                L.qkv_c = fp16_range_scale(qkv_bound);
            }
            {
                // an attention output row mixes v rows (|a_e| <= the v bound), so
                // |o_j| <= sqrt(heads hd) * bound * ||W_o,j||
                const HostQ8 h = q8_rows(d, b + "attn_out.weight", D, D, base, len, D);
                L.o_c = fp16_range_scale(std::sqrt(double(D)) * qkv_bound * max_row_norm(h));
                L.wo = upload_vision_q8(c, v, h, "v.attn_out");
            }
            L.bo = upload_floats(v, f32_vector(d, b + "attn_out.bias", D, base, len), "v.attn_out.bias");
            {
                const HostQ8 h = q8_rows(d, b + "ffn_up.weight", D, v.ff, base, len, v.ff_pad);
                L.wup = upload_vision_q8(c, v, h, "v.ffn_up");
                const auto bu = f32_vector(d, b + "ffn_up.bias", v.ff, base, len, v.ff_pad);
                L.bup = upload_floats(v, bu, "v.ffn_up.bias");
                // |gelu(z)| <= |z| and |z_j| <= ||h|| ||W_j|| + |b_j|
                act_bound = hn2 * max_row_norm(h) + max_abs(bu);
                L.act_c = fp16_range_scale(act_bound);
            }
            {
                // |d_j| <= ||a|| ||W_down,j|| with every activation a_e within the bound above
                double wn = 0;
                L.wdown = fragments_any(v, d, b + "ffn_down.weight", v.ff, D, v.ff_pad, base, len, &wn);
                L.down_c = fp16_range_scale(std::sqrt(double(v.ff)) * act_bound * wn);
            }
            L.bdown = upload_floats(v, f32_vector(d, b + "ffn_down.bias", D, base, len), "v.ffn_down.bias");
            L.ln1_w = upload_floats(v, ln1w, "v.ln1");
            L.ln1_b = upload_floats(v, ln1b, "v.ln1");
            L.ln2_w = upload_floats(v, ln2w, "v.ln2");
            L.ln2_b = upload_floats(v, ln2b, "v.ln2");
            v.layer.push_back(L);
        }
        v.post_w = upload_floats(v, f32_vector(d, "v.post_ln.weight", D, base, len), "v.post_ln");
        v.post_b = upload_floats(v, f32_vector(d, "v.post_ln.bias", D, base, len), "v.post_ln");
        {
            const auto nw = f32_vector(d, "mm.soft_emb_norm.weight", D, base, len);
            if (rD * max_abs(nw) >= 65504.0) fail(GE_ERR_MODEL, "mm.soft_emb_norm: outputs may leave fp16's range");
            v.norm_w = upload_floats(v, nw, "mm.soft_emb_norm");
        }
        v.proj_w = upload_vision_q8(c, v, q8_rows(d, "mm.input_projection.weight", D, v.proj, base, len, v.proj),
                                    "mm.input_projection");
    } catch (...) {
        for (void* p : v.weights) (void)hipFree(p);
        throw;
    }
    free_vision(c);
    c->vision = vs.release();
}

// ---------------------------------------------------------------- staging

// A zero-filled workspace buffer, the fill queued on the context's stream (see ws_alloc): the
// image batch's copies and the tower's kernels come after it there.
template <typename T>
T* vws_alloc(hipStream_t s, size_t rows, size_t width, const char* what) {
    const size_t bytes = rows * width * sizeof(T);
    void* p = dev_alloc(bytes, what);
    hip_check(hipMemsetAsync(p, 0, bytes, s), "hipMemsetAsync workspace");
    return static_cast<T*>(p);
}

void alloc_vision_workspace(hipStream_t s, VisionState& v, int r, int tr, int wc, int vc);

void ensure_vision_workspace(ge_ctx* c, VisionState& v, int patches, int tokens, int work, int vt_cols) {
    const int rows = (patches + 63) / 64 * 64 + kRowSlack, tok_rows = (tokens + 63) / 64 * 64 + kRowSlack;
    const bool grow = rows > v.rows || tok_rows > v.tok_rows || work > v.work_cap || vt_cols > v.vt_cap;
    if (!grow) return;
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    const int r = std::max(rows, v.rows), tr = std::max(tok_rows, v.tok_rows), wc = std::max(std::max(work, 1), v.work_cap);
    const int vc = (std::max(vt_cols, v.vt_cap + v.vt_cap / 2) + 63) / 64 * 64;
    free_vision_workspace(v);
    try {
        alloc_vision_workspace(c->stream, v, r, tr, wc, vc);
    } catch (...) {
        free_vision_workspace(v);  // no capacity is recorded for buffers that do not exist
        throw;
    }
    v.rows = r;
    v.tok_rows = tr;
    v.work_cap = wc;
    v.vt_cap = vc;
}

void alloc_vision_workspace(hipStream_t s, VisionState& v, int r, int tr, int wc, int vc) {
    const size_t D = size_t(v.hidden), HP = size_t(v.heads) * v.hp;
    v.patches32 = vws_alloc<float>(s, r, v.area, "patches");
    v.patches16 = vws_alloc<uint16_t>(s, r, v.area, "patches");
    v.x = vws_alloc<float>(s, r, D, "x");
    v.t = vws_alloc<float>(s, r, D, "t");
    v.h = vws_alloc<uint16_t>(s, r, D, "h");
    v.o16 = vws_alloc<uint16_t>(s, r, D, "attention output");
    // q, k, v keep zeros in each head's padding columns: the epilogue never writes them
    v.q = vws_alloc<uint16_t>(s, r, HP, "q");
    v.k = vws_alloc<uint16_t>(s, r, HP, "k");
    v.v = vws_alloc<uint16_t>(s, r, HP, "v");
    v.vt = vws_alloc<uint16_t>(s, HP, size_t(vc), "transposed v");
    v.attn = vws_alloc<uint16_t>(s, r, size_t(v.heads) * v.hd, "attn");
    v.act = vws_alloc<uint16_t>(s, r, size_t(v.ff_pad), "act");
    v.pooled = vws_alloc<float>(s, tr, D, "pooled");
    v.pooled16 = vws_alloc<uint16_t>(s, tr, D, "pooled");
    v.out = vws_alloc<float>(s, tr, size_t(v.proj), "vectors");
    v.px = vws_alloc<int32_t>(s, r, 1, "patch x");
    v.py = vws_alloc<int32_t>(s, r, 1, "patch y");
    v.vcol = vws_alloc<int32_t>(s, r, 1, "vt columns");
    v.tok_row0 = vws_alloc<int32_t>(s, tr, 1, "pool windows");
    v.tok_gx = vws_alloc<int32_t>(s, tr, 1, "pool windows");
    v.work = vws_alloc<AttnWork>(s, size_t(wc), 1, "attention work");
}

// VisionBatch.init (VisionTower.swift:17-33) and VisionTower.upload (:113-140): images back to
// back as patch rows (patch i of an image at column i % gx, row i / gx), each image one attention
// sequence, pooled tokens back to back in (oy, ox) order.
void vision_stage(ge_ctx* c, const float* patches, int n_patches, const ge_image_grid* grids, int n_images) {
    VisionState& v = vision_of(c);
    if (n_images <= 0 || !grids) fail(GE_ERR_INVALID, "a batch needs at least one image");
    if (!patches) fail(GE_ERR_INVALID, "null patches");
    std::vector<int32_t> px, py, row0, gxs, vcol;
    std::vector<AttnWork> work;
    int64_t P = 0;
    uint32_t col = 0;
    // 256-query work items when they still give at least kVitWideItems workgroups (eight waves
    // of two query tiles share a K/V block: a quarter of the L2 reads per query, half the LDS
    // reads); 64 for small batches. Same results either way.
    int64_t items256 = 0;
    for (int i = 0; i < n_images; i++) items256 += (int64_t(grids[i].grid_x) * grids[i].grid_y + 255) / 256;
    const int items = v.hp != v.hd && items256 * v.heads >= kVitWideItems ? 256 : kAttnQueriesV2;
    for (int i = 0; i < n_images; i++) {
        const int gx = grids[i].grid_x, gy = grids[i].grid_y;
        if (gx <= 0 || gy <= 0 || gx % v.merge || gy % v.merge)
            fail(GE_ERR_INVALID, "image %d: grid %d x %d is not a positive multiple of the merge size %d", i, gx, gy, v.merge);
        if (gx > v.npos || gy > v.npos)
            fail(GE_ERR_INVALID, "image %d: grid %d x %d exceeds the %d position rows", i, gx, gy, v.npos);
        const int n = gx * gy;
        if (P + n > (int64_t(1) << 24)) fail(GE_ERR_INVALID, "batch has too many patches");
        for (int p = 0; p < n; p++) {
            px.push_back(p % gx);
            py.push_back(p / gx);
            vcol.push_back(int32_t(col + uint32_t(p)));
        }
        for (uint32_t q0 = 0; q0 < uint32_t(n); q0 += uint32_t(items))
            work.push_back(AttnWork{uint32_t(P), uint32_t(n), q0, col});
        for (int oy = 0; oy < gy / v.merge; oy++)
            for (int ox = 0; ox < gx / v.merge; ox++) {
                row0.push_back(int32_t(P + int64_t(oy) * v.merge * gx + int64_t(ox) * v.merge));
                gxs.push_back(gx);
            }
        col += (uint32_t(n) + 7) / 8 * 8;
        P += n;
    }
    if (P != n_patches) fail(GE_ERR_INVALID, "the grids hold %lld patches, the batch %d", (long long)P, n_patches);
    const int vt_cols = int(col) + 64;
    const int tokens = int(row0.size());
    ensure_vision_workspace(c, v, n_patches, tokens, int(work.size()), vt_cols);
    struct Piece {
        void* dst;
        const void* src;
        size_t bytes;
    };
    const Piece pieces[] = {{v.patches32, patches, size_t(n_patches) * v.area * 4},
                            {v.px, px.data(), px.size() * 4},
                            {v.py, py.data(), py.size() * 4},
                            {v.vcol, vcol.data(), vcol.size() * 4},
                            {v.tok_row0, row0.data(), row0.size() * 4},
                            {v.tok_gx, gxs.data(), gxs.size() * 4},
                            {v.work, work.data(), work.size() * sizeof(AttnWork)}};
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    for (const Piece& pc : pieces)
        if (pc.bytes) hip_check(hipMemcpy(pc.dst, pc.src, pc.bytes, hipMemcpyHostToDevice), "upload image batch");
    v.staged_patches = n_patches;
    v.staged_tokens = tokens;
    v.staged_work = int(work.size());
    v.items = items;
}

// ---------------------------------------------------------------- forward

struct VitStop {
    std::string name;
    int layer = -1;
    bool hit = false;
    bool at(const char* n, int l) {
        if (hit || name != n || layer != l) return false;
        hit = true;
        return true;
    }
};

// VisionTower.encode (VisionTower.swift:143-185) for config 5's encoder: 8 launches per layer.
void vision_encode(ge_ctx* c, VitStop* sp) {
    VisionState& v = vision_of(c);
    if (v.staged_patches < 0) fail(GE_ERR_STATE, "no image batch is staged");
    const int P = v.staged_patches, T = v.staged_tokens, D = v.hidden;
    hipStream_t s = c->stream;
    auto stop = [&](const char* n, int l) { return sp && sp->at(n, l); };
    launch(c, "vit_patches_f16", [&] { return launch_f32_to_f16(s, v.patches32, v.patches16, size_t(P) * v.area); });
    launch(c, "vit_gemm_patch", [&] { return launch_gemm_q8(s, v.patch_w, v.patches16, P, v.t, kEpiF32); });
    if (stop("inp", -1)) return;
    launch(c, "vit_embed", [&] {
        return launch_vit_embed(s, v.t, v.patch_b, v.pos, v.npos, v.px, v.py, P, D, v.layer[0].ln1_w, v.layer[0].ln1_b,
                                v.eps, v.x, v.h);
    });
    if (stop("pos_embd", -1) || stop("layer_inp_normed", 0)) return;
    // softmax(q k^T / sqrt(hd)); q and k arrive multiplied by qkv_c
    const float att_scale = 1.0f / std::sqrt(float(v.hd));
    for (int l = 0; l < v.layers; l++) {
        const VitLayer& L = v.layer[size_t(l)];
        launch(c, "vit_gemm_qkv", [&] {
            GemmEpiArgs ea;
            ea.bias = L.bqkv;
            ea.dst[0] = v.q;
            ea.dst[1] = v.k;
            ea.dst[2] = v.v;
            ea.hd = v.hd;
            ea.hp = v.hp;
            ea.heads = v.heads;
            return launch_gemm_q8(s, L.wqkv, v.h, P, nullptr, kEpiHeads, L.qkv_c, &ea);
        });
        if (stop("Qcur", l) || stop("Kcur", l) || stop("Vcur", l)) return;
        launch(c, "v_transpose", [&] { return launch_v_transpose(s, v.v, P, v.heads * v.hp, v.vcol, v.vt_cap, v.vt); });
        launch(c, "vit_attention", [&] {
            const float sc = att_scale / (L.qkv_c * L.qkv_c);
            if (v.hp != v.hd)
                return launch_attention_padded(s, v.q, v.k, v.vt, v.vt_cap, v.attn, v.work, v.staged_work, v.heads, v.heads,
                                               v.hp, v.hd, 0, sc, v.items);
            return launch_attention_v2(s, v.q, v.k, v.vt, v.vt_cap, v.attn, v.work, v.staged_work, v.heads, v.heads, v.hd, 0,
                                       sc);
        });
        if (stop("kqv_out", l)) return;
        // The attention output in fp16 (times o_c). x is stored once per layer: the attention
        // residual's launch writes only the MLP input h (and x only when a trace wants the sum after
        // attention), and the MLP residual's launch recomputes that sum beside its own.
        launch(c, "vit_gemm_o", [&] { return launch_gemm_q8(s, L.wo, v.attn, P, v.o16, kEpiF16, L.o_c / L.qkv_c); });
        if (stop("attn_out", l)) return;
        const bool store_sum = sp && !sp->hit && sp->layer == l && sp->name == "ffn_inp";
        launch(c, "vit_residual_ln_h", [&] {
            return launch_vit_residual2_ln(s, store_sum ? 1 : 0, v.x, v.o16, 1.0f / L.o_c, L.bo, nullptr, 1.0f, nullptr,
                                           L.ln2_w, L.ln2_b, v.eps, P, D, v.h);
        });
        if (stop("ffn_inp", l) || stop("ffn_inp_normed", l)) return;
        launch(c, "vit_gemm_up", [&] {
            GemmEpiArgs ea;
            ea.bias = L.bup;
            return launch_gemm_q8(s, L.wup, v.h, P, v.act, kEpiGeluBias, L.act_c, &ea);
        });
        if (stop("ffn_gelu", l)) return;
        // the down projection in fp16 (times down_c) over the start of t
        uint16_t* const d16 = reinterpret_cast<uint16_t*>(v.t);
        launch(c, "vit_gemm_down", [&] { return launch_gemm_q8(s, L.wdown, v.act, P, d16, kEpiF16, L.down_c / L.act_c); });
        if (stop("ffn_out", l)) return;
        const bool last = l + 1 == v.layers;
        launch(c, "vit_residual_ln_two", [&] {
            const VitLayer* N = last ? nullptr : &v.layer[size_t(l) + 1];
            return launch_vit_residual2_ln(s, 2, v.x, v.o16, 1.0f / L.o_c, L.bo, d16, 1.0f / L.down_c, L.bdown,
                                           N ? N->ln1_w : nullptr, N ? N->ln1_b : nullptr, v.eps, P, D, v.h);
        });
        if (stop("layer_out", l) || stop("layer_inp_normed", l + 1)) return;
    }
    launch(c, "vit_pool", [&] {
        return launch_vit_pool(s, v.x, v.tok_row0, v.tok_gx, T, v.merge, D, v.post_w, v.post_b, v.eps, v.norm_w, v.pooled,
                               v.pooled16);
    });
    if (stop("pooled", -1) || stop("pooled_normed", -1)) return;
    launch(c, "vit_gemm_proj", [&] { return launch_gemm_q8(s, v.proj_w, v.pooled16, T, v.out, kEpiF32); });
}

void vision_read(ge_ctx* c, float* out, size_t cap) {
    VisionState& v = vision_of(c);
    if (v.staged_patches < 0) fail(GE_ERR_STATE, "no image batch is staged");
    const size_t need = size_t(v.staged_tokens) * v.proj;
    if (cap < need) fail(GE_ERR_INVALID, "vector buffer holds %zu floats, the staged images need %zu", cap, need);
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    hip_check(hipMemcpy(out, v.out, size_t(v.staged_tokens) * v.proj * 4, hipMemcpyDeviceToHost), "read vectors");
}

void vision_trace(ge_ctx* c, const char* name, int layer, float* out, size_t cap, size_t* needed) {
    VisionState& v = vision_of(c);
    if (!name) fail(GE_ERR_INVALID, "null tensor name");
    if (layer < -1 || layer >= v.layers) fail(GE_ERR_INVALID, "layer %d out of range", layer);
    const std::string n = name;
    const int P = v.staged_patches, T = v.staged_tokens, D = v.hidden, HD = v.heads * v.hd;
    const VitLayer* L = layer >= 0 ? &v.layer[size_t(layer)] : nullptr;
    const bool global = n == "inp" || n == "pos_embd" || n == "pooled" || n == "pooled_normed" || n == "projected";
    if (global != (layer < 0)) fail(GE_ERR_INVALID, "tensor %s %s a layer index", name, global ? "takes no" : "needs");
    const void* buf = nullptr;
    bool f16 = false, heads = false;
    int rows = P, stride = D, width = D;
    float unscale = 1;
    if (n == "attn_out") {
        buf = v.o16; f16 = true; unscale = 1.0f / L->o_c;
    } else if (n == "ffn_out") {
        buf = v.t; f16 = true; unscale = 1.0f / L->down_c;
    } else if (n == "inp") {
        buf = v.t;
    } else if (n == "pos_embd" || n == "ffn_inp" || n == "layer_out") {
        buf = v.x;
    } else if (n == "layer_inp_normed" || n == "ffn_inp_normed") {
        buf = v.h; f16 = true;
    } else if (n == "Qcur" || n == "Kcur" || n == "Vcur") {
        buf = n == "Qcur" ? v.q : n == "Kcur" ? v.k : v.v;
        f16 = heads = true; stride = v.heads * v.hp; width = HD; unscale = 1.0f / L->qkv_c;
    } else if (n == "kqv_out") {
        buf = v.attn; f16 = true; stride = width = HD; unscale = 1.0f / L->qkv_c;
    } else if (n == "ffn_gelu") {
        buf = v.act; f16 = true; stride = v.ff_pad; width = v.ff; unscale = 1.0f / L->act_c;
    } else if (n == "pooled") {
        buf = v.pooled; rows = T;
    } else if (n == "pooled_normed") {
        buf = v.pooled16; f16 = true; rows = T;
    } else if (n == "projected") {
        buf = v.out; rows = T; stride = width = v.proj;
    } else {
        fail(GE_ERR_INVALID, "unknown image encoder trace tensor %s", name);
    }
    const size_t count = size_t(rows) * width;
    if (needed) *needed = count;
    if (!out) return;
    if (cap < count) fail(GE_ERR_INVALID, "trace buffer holds %zu floats, %s needs %zu", cap, name, count);
    VitStop sp{n, layer, false};
    if (n != "projected") {
        vision_encode(c, &sp);
        if (!sp.hit) fail(GE_ERR_INVALID, "tensor %s at layer %d is not produced by this forward", name, layer);
    } else {
        vision_encode(c, nullptr);
    }
    if (heads) {
        // [rows][heads][hp] -> [rows][heads][hd]
        std::vector<float> full(size_t(rows) * stride);
        copy_out(c, buf, true, rows, stride, 0, stride, full.data());
        for (int r = 0; r < rows; r++)
            for (int h = 0; h < v.heads; h++)
                for (int e = 0; e < v.hd; e++)
                    out[(size_t(r) * v.heads + h) * v.hd + e] = full[size_t(r) * stride + size_t(h) * v.hp + e];
    } else {
        copy_out(c, buf, f16, rows, stride, 0, width, out);
    }
    if (unscale != 1.0f)
        for (size_t i = 0; i < count; i++) out[i] *= unscale;
}

}  // namespace

// The image forward (MetalForward.run(images:), Metal/MetalForward.swift:213-219 with imageBatches
// :285-294): the tower over every image, then the text tower over each image's
// [bos, begin, v_1 .. v_n, end, eos] (Model/InputRow.swift:52-56), whose vector rows are the
// tower's output rows in HBM (MetalForward.swift:23-32), on one stream with no host round trip.
void image_forward(ge_ctx* c, const float* patches, int n_patches, const ge_image_grid* grids, int n_images,
                   const int32_t* markers, float* pooled, double* gpu_seconds) {
    if (!pooled || !markers) fail(GE_ERR_INVALID, "null argument");
    if (!c->has_model) fail(GE_ERR_STATE, "no text model has been uploaded");
    VisionState& v = vision_of(c);
    if (v.proj != c->model.hidden)
        fail(GE_ERR_INVALID, "the image tower's %d-wide vectors do not fit the text model's %d-wide rows", v.proj,
             c->model.hidden);
    // The markers are vocabulary ids (InputRow.swift SpanMarkers); a negative id would name a
    // vector row instead.
    for (int i = 0; i < 4; i++)
        if (markers[i] < 0 || markers[i] >= c->model.vocab)
            fail(GE_ERR_INVALID, "marker %d (%d) is outside the vocabulary [0, %d)", i, markers[i], c->model.vocab);
    // The text batch staged below reads the tower's buffers, which the next image batch may
    // replace: it is dropped on every exit, a failed one included.
    struct DropStaged {
        ge_ctx* c;
        ~DropStaged() {
            c->staged_tokens = -1;
            c->staged_vectors = nullptr;
            c->staged_vec_rows = 0;
        }
    } drop{c};
    vision_stage(c, patches, n_patches, grids, n_images);
    std::vector<int32_t> ids, pos;
    std::vector<ge_seq> seqs;
    int row = 0;
    for (int i = 0; i < n_images; i++) {
        const int rows = (grids[i].grid_x / v.merge) * (grids[i].grid_y / v.merge);
        if (rows + 4 > c->model.max_tokens)
            fail(GE_ERR_INVALID, "image %d: %d vector rows and 4 markers exceed the %d-token context", i, rows,
                 c->model.max_tokens);
        seqs.push_back(ge_seq{uint32_t(ids.size()), uint32_t(rows + 4)});
        ids.push_back(markers[0]);
        ids.push_back(markers[1]);
        for (int r = 0; r < rows; r++) ids.push_back(-(row + r) - 1);
        ids.push_back(markers[2]);
        ids.push_back(markers[3]);
        row += rows;
    }
    for (size_t t = 0, s = 0; s < seqs.size(); s++)
        for (uint32_t p = 0; p < seqs[s].length; p++, t++) pos.push_back(int32_t(p));
    stage(c, ids.data(), pos.data(), int(ids.size()), seqs.data(), n_images, v.out, v.staged_tokens);
    hip_check(hipEventRecord(c->ev_start, c->stream), "hipEventRecord");
    vision_encode(c, nullptr);
    run_forward(c, gpu_seconds, false);
    read_pooled(c, pooled);
}

void free_vision(ge_ctx* c) {
    if (!c->vision) return;
    VisionState& v = *c->vision;
    free_vision_workspace(v);
    for (void* p : v.weights) (void)hipFree(p);
    delete c->vision;
    c->vision = nullptr;
}

}  // namespace ge

extern "C" {

int ge_upload_vision(ge_ctx* c, const ge_vision_desc* desc, const void* base, size_t len) {
    return ge::guarded(c, [&] { ge::vision_upload(c, desc, base, len); });
}

int ge_vision_stage(ge_ctx* c, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images) {
    return ge::guarded(c, [&] { ge::vision_stage(c, patches, n_patches, grids, n_images); });
}

int ge_vision_run(ge_ctx* c) {
    return ge::guarded(c, [&] { ge::vision_encode(c, nullptr); });
}

int ge_vision_read(ge_ctx* c, float* vectors, size_t vectors_count) {
    if (!vectors) return GE_ERR_INVALID;
    return ge::guarded(c, [&] { ge::vision_read(c, vectors, vectors_count); });
}

int ge_vision_get_info(ge_ctx* c, ge_vision_info* info) {
    if (!info) return GE_ERR_INVALID;
    return ge::guarded(c, [&] {
        const ge::VisionState& v = ge::vision_of(c);
        info->layers = v.layers;
        info->hidden = v.hidden;
        info->heads = v.heads;
        info->patch_size = v.patch;
        info->patch_area = v.area;
        info->merge = v.merge;
        info->proj_dims = v.proj;
        info->positions = v.npos;
    });
}

int32_t ge_vision_tokens(ge_ctx* c) {
    if (!c || !c->vision || c->vision->staged_patches < 0) return -1;
    return c->vision->staged_tokens;
}

int ge_vision_encode(ge_ctx* c, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images,
                     float* vectors, size_t vectors_count, double* gpu_seconds) {
    if (!vectors) return GE_ERR_INVALID;
    return ge::guarded(c, [&] {
        ge::vision_stage(c, patches, n_patches, grids, n_images);
        ge::hip_check(hipEventRecord(c->ev_start, c->stream), "hipEventRecord");
        ge::vision_encode(c, nullptr);
        ge::hip_check(hipEventRecord(c->ev_stop, c->stream), "hipEventRecord");
        if (gpu_seconds) {
            ge::hip_check(hipEventSynchronize(c->ev_stop), "hipEventSynchronize");
            float ms = 0;
            ge::hip_check(hipEventElapsedTime(&ms, c->ev_start, c->ev_stop), "hipEventElapsedTime");
            *gpu_seconds = ms * 1e-3;
        }
        ge::vision_read(c, vectors, vectors_count);
    });
}

int ge_image_forward(ge_ctx* c, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images,
                     const int32_t* markers, float* pooled, double* gpu_seconds) {
    return ge::guarded(c, [&] { ge::image_forward(c, patches, n_patches, grids, n_images, markers, pooled, gpu_seconds); });
}

int ge_vision_trace(ge_ctx* c, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images,
                    const char* tensor_name, int32_t layer, float* out, size_t out_count, size_t* needed) {
    return ge::guarded(c, [&] {
        ge::vision_stage(c, patches, n_patches, grids, n_images);
        ge::vision_trace(c, tensor_name, layer, out, out_count, needed);
    });
}

}  // extern "C"
