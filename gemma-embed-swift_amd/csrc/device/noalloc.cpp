// The forward of one packed batch with every device buffer in a file-scope device array, for
// callers that cannot allocate device memory (tight serving loops, harnesses that forbid
// hipMalloc). No counterpart in the reference. The call is synchronous like ge_forward: it clears
// its region with hipMemsetAsync, waits for its stream and reads the pooled vectors back with a
// blocking copy, so it is not meant to be captured into a HIP graph.
//
// The workspace the forward's kernels read and write (activations, the staged token ids,
// positions, sequence ranges and attention work lists, transposed V, the pooled output) is carved
// out of `scratch` instead of hipMalloc'd buffers; the kernels and their launches are the
// forward's own (encode), so a batch's vectors are bitwise those of ge_forward. The entry point
// calls no hipMalloc, hipFree, hipHostMalloc or other allocating HIP routine: the token ids,
// positions and small arrays are copied from the caller's host arrays straight into the array.
//
// Every call on one GPU uses that GPU's copy of the array, which keeps the last call's contents:
// the used region is cleared at the start of each call, and calls that overlap on one GPU (from
// two contexts on two threads) race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "runtime_internal.hpp"

namespace ge {

constexpr size_t kScratchBytes = size_t(64) << 20;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// The array's device address per device, taken once per device (each GPU holds its own copy).
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;

// A bump allocator over the array (base null: only counts the bytes).
struct Carver {
    unsigned char* base;
    size_t used = 0;
    template <typename T>
    T* take(size_t count) {
        T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
        used += (count * sizeof(T) + 255) / 256 * 256;
        return p;
    }
};

// The forward's workspace (ensure_workspace's buffers and widths) for a planned batch of n tokens,
// carved out of `base`.
Workspace carve(const DevModel& m, const BatchPlan& b, int n, int n_seqs, Carver& cv) {
    Workspace w;
    const size_t R = size_t((n + 63) / 64 * 64 + kRowSlack);
    w.rows = int(R);
    w.x = cv.take<float>(R * m.hidden);
    w.h = cv.take<uint16_t>(R * m.hidden);
    w.qkv = cv.take<float>(R * m.max_qkv);
    w.q = cv.take<uint16_t>(R * m.max_qd);
    w.k = cv.take<uint16_t>(R * m.max_kvd);
    w.v = cv.take<uint16_t>(R * m.max_kvd);
    w.attn = cv.take<uint16_t>(R * m.max_qd);
    w.t = cv.take<float>(R * m.hidden);
    w.act = cv.take<uint16_t>(R * m.ff);
    w.out = nullptr;  // only a trace of the per-token projection (result_embd) writes it; this forward never traces
    w.hn = cv.take<float>(R * m.hidden);
    w.tokens = cv.take<int32_t>(R);
    w.positions = cv.take<int32_t>(R);
    w.vcol = cv.take<int32_t>(R);
    if (m.pl > 0) {
        w.ple = cv.take<float>(R * size_t(m.layers) * m.pl);
        w.ple_t = cv.take<float>(R * size_t(std::max(m.pl, m.hidden)));
        w.rs = cv.take<float>(R);
        w.rs2 = cv.take<float>(R);
        w.x16 = cv.take<uint16_t>(R * m.hidden);
        w.g16 = cv.take<uint16_t>(R * m.pl);
    }
    if (m.any_precise) {
        w.h3 = cv.take<uint16_t>(R * 3 * size_t(m.hidden));
        w.q_lo = cv.take<uint16_t>(R * m.max_qd);
        w.k_lo = cv.take<uint16_t>(R * m.max_kvd);
    }
    w.seq_cap = n_seqs;
    w.seqs = cv.take<SeqRange>(size_t(n_seqs));
    w.pooled = cv.take<float>(size_t(n_seqs) * m.out_dims);
    w.pooled_n = cv.take<float>(size_t(n_seqs) * m.hidden);
    // the producer-wave attention's work list, read only by layers off the LDS-copy attention
    w.work_cap = m.all_v2 ? 0 : std::max(int(b.work.size()), 1);
    w.work = m.all_v2 ? nullptr : cv.take<AttnWork>(size_t(w.work_cap));
    if (m.any_v2) {
        w.work2_cap = std::max(int(b.work2.size()), 1);
        w.work2 = cv.take<AttnWork>(size_t(w.work2_cap));
        w.vt_cap = (b.vl.cols + 63) / 64 * 64;
        w.vt = cv.take<uint16_t>(size_t(m.max_kvd) * w.vt_cap);
    }
    return w;
}

void forward_noalloc(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int n, const ge_seq* seqs, int n_seqs,
                     float* pooled, double* gpu_seconds) {
    if (!pooled) fail(GE_ERR_INVALID, "null output");
    if (!c->scratch) fail(GE_ERR_STATE, "the no-allocation scratch of device %d is not set up", c->device);
    if (c->prof) fail(GE_ERR_STATE, "the no-allocation forward does not run while profiling is enabled");
    if (n >= kSplitMinTokens) fail(GE_ERR_INVALID, "the no-allocation forward takes packs below %d tokens", kSplitMinTokens);
    const BatchPlan b = plan_batch(c, tokens, positions, n, seqs, n_seqs, own_vectors(c), own_vector_rows(c));
    if (b.n_parts != 1) fail(GE_ERR_STATE, "a pack below %d tokens was split into parts", kSplitMinTokens);
    Carver count{nullptr};
    carve(c->model, b, n, n_seqs, count);
    if (count.used > kScratchBytes)
        fail(GE_ERR_INVALID, "this pack of %d tokens needs %zu bytes of device scratch; the no-allocation forward holds %zu",
             n, count.used, kScratchBytes);
    Carver cv{static_cast<unsigned char*>(c->scratch)};
    const Workspace w = carve(c->model, b, n, n_seqs, cv);
    hipStream_t s = c->stream;
    // The array keeps the previous call's contents: zero the region this call uses (alignment
    // gaps and slack rows of V^T and the activations must read as finite values).
    hip_check(hipMemsetAsync(c->scratch, 0, cv.used, s), "clear scratch");
    hip_check(hipMemcpyAsync(w.tokens, tokens, size_t(n) * 4, hipMemcpyHostToDevice, s), "upload tokens");
    hip_check(hipMemcpyAsync(w.positions, positions, size_t(n) * 4, hipMemcpyHostToDevice, s), "upload positions");
    hip_check(hipMemcpyAsync(w.seqs, b.sr.data(), b.sr.size() * sizeof(SeqRange), hipMemcpyHostToDevice, s), "upload");
    if (w.work)
        hip_check(hipMemcpyAsync(w.work, b.work.data(), b.work.size() * sizeof(AttnWork), hipMemcpyHostToDevice, s), "upload");
    if (!b.work2.empty()) {
        hip_check(hipMemcpyAsync(w.work2, b.work2.data(), b.work2.size() * sizeof(AttnWork), hipMemcpyHostToDevice, s),
                  "upload");
        hip_check(hipMemcpyAsync(w.vcol, b.vl.vcol.data(), size_t(n) * 4, hipMemcpyHostToDevice, s), "upload");
    }
    // The forward reads the context's workspace and staged batch: point them at the array for
    // this call and put the context's own back on every exit (its buffers are untouched).
    struct Restore {
        ge_ctx* c;
        Workspace ws;
        int tokens, seqs, work, work2, vt_cols, items, parts, vec_rows;
        const float* vectors;
        int part_row[kMaxParts + 1], part_work[kMaxParts + 1];
        ~Restore() {
            c->ws = ws;
            c->staged_tokens = tokens;
            c->staged_seqs = seqs;
            c->staged_work = work;
            c->staged_work2 = work2;
            c->staged_vt_cols = vt_cols;
            c->attn_items = items;
            c->n_parts = parts;
            c->staged_vec_rows = vec_rows;
            c->staged_vectors = vectors;
            std::copy(part_row, part_row + kMaxParts + 1, c->part_row);
            std::copy(part_work, part_work + kMaxParts + 1, c->part_work);
        }
    } restore{c, c->ws, c->staged_tokens, c->staged_seqs, c->staged_work, c->staged_work2, c->staged_vt_cols,
              c->attn_items, c->n_parts, c->staged_vec_rows, c->staged_vectors, {}, {}};
    std::copy(c->part_row, c->part_row + kMaxParts + 1, restore.part_row);
    std::copy(c->part_work, c->part_work + kMaxParts + 1, restore.part_work);
    c->ws = w;
    set_staged(c, b, n, n_seqs, own_vectors(c));
    hip_check(hipEventRecord(c->ev_start, s), "hipEventRecord");
    try {
        encode(c, nullptr);
    } catch (...) {
        (void)hipStreamSynchronize(s);  // nothing queued may outlive the call's view of the array
        throw;
    }
    hip_check(hipEventRecord(c->ev_stop, s), "hipEventRecord");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (gpu_seconds) {
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, c->ev_start, c->ev_stop), "hipEventElapsedTime");
        *gpu_seconds = ms * 1e-3;
    }
    hip_check(hipMemcpy(pooled, w.pooled, size_t(n_seqs) * c->model.out_dims * 4, hipMemcpyDeviceToHost), "read pooled");
}

}  // namespace

// At context creation, with the context's device current: the array's address on that device.
void noalloc_init(ge_ctx* c) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr.size() <= size_t(c->device)) g_scratch_ptr.resize(size_t(c->device) + 1, nullptr);
    if (!g_scratch_ptr[size_t(c->device)]) {
        void* p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) fail(GE_ERR_GPU, "no device address for the no-allocation scratch");
        g_scratch_ptr[size_t(c->device)] = p;
    }
    c->scratch = g_scratch_ptr[size_t(c->device)];
}

}  // namespace ge

extern "C" {

int ge_forward_noalloc(ge_ctx* c, const int32_t* tokens, const int32_t* positions, int32_t n_tokens, const ge_seq* seqs,
                       int32_t n_seqs, float* pooled_out, double* gpu_seconds) {
    return ge::guarded(c, [&] { ge::forward_noalloc(c, tokens, positions, n_tokens, seqs, n_seqs, pooled_out, gpu_seconds); });
}

}  // extern "C"
