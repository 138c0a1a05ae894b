// Bidirectional flash attention over packed sequences on gfx950 MFMA.
//
// One workgroup of 4 waves per (work item of 32 query rows, KV head). Waves 0..G-1 (G = query
// heads per KV head) each own one query head; every K/V block staged in LDS serves the whole
// group. Keys stream in blocks of 64 with an online softmax in fp32 (reference
// Shaders/Attention.metal:25-170).
//
// Pipelining: when G < 4 the remaining waves are producers. While the compute waves work on key
// block i from one LDS buffer, the producers load block i + 1 from HBM/L2 into the other buffer,
// issuing eight 16-byte loads before their first LDS store so the load latency is paid once per
// eight loads instead of once per load. One workgroup barrier per block separates the roles.
// With G = 4 (or a head dim whose double buffer does not fit LDS) every wave stages the next
// block after computing the current one.
//
// Both products run transposed so a query is an accumulator column, owned by lane l % 32:
//   S^T[key][query] = K[key][:] . Q[query][:]    (A = K from LDS, B = Q fragments in registers)
//   O^T[d][query]  += V^T[d][key] . P^T[key][query] (A = V^T from LDS, B = P from the S registers)
// so the softmax max / sum over keys is a reduction over a lane's own registers plus its
// partner lane l ^ 32, and the rescale by alpha is per lane. For the second product the 16
// keys of a k-step are split between the two lane halves in the order the S accumulator
// already holds them (keys 4h..4h+3 and 8+4h..8+4h+3 for half h); V^T is read in that order.
// Scores are kept in the log2 domain (s * scale * log2 e) so the exponentials are v_exp_f32.
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

namespace attn {
constexpr int BKV = 64;
constexpr int LDV = BKV + 8;
constexpr int WAVES = 4;
constexpr int BATCH = 8;  // 16-byte loads a producer thread keeps in flight
constexpr int BATCH_INLINE = 2;  // the same when compute waves stage between blocks
}  // namespace attn

// Stages key block [kb, kb + 64) of one KV head: K as [64][HD + 8] and V^T as [DS][64 + 8].
// `t` is this thread's index among the `nt` staging threads. Chunks go in full batches of BATCH
// loads with no per-load condition, so the batch's loads are all in flight before the first
// LDS store; a guarded tail takes what the batches leave.
__device__ __forceinline__ void attn_store_vt(uint32_t* dst, const uint4& a, const uint4& b) {
    constexpr int ROW = attn::LDV / 2;  // one V^T row in 32-bit words
    dst[0 * ROW] = (a.x & 0xffffu) | (b.x << 16);
    dst[1 * ROW] = (a.x >> 16) | (b.x & 0xffff0000u);
    dst[2 * ROW] = (a.y & 0xffffu) | (b.y << 16);
    dst[3 * ROW] = (a.y >> 16) | (b.y & 0xffff0000u);
    dst[4 * ROW] = (a.z & 0xffffu) | (b.z << 16);
    dst[5 * ROW] = (a.z >> 16) | (b.z & 0xffff0000u);
    dst[6 * ROW] = (a.w & 0xffffu) | (b.w << 16);
    dst[7 * ROW] = (a.w >> 16) | (b.w & 0xffff0000u);
}

template <int HD, int DS, int BATCH, int nt>
__device__ __forceinline__ void attn_stage(_Float16* __restrict__ Ks, _Float16* __restrict__ Vt,
                                           const _Float16* __restrict__ kbase, const _Float16* __restrict__ vbase,
                                           int kb, int kvStride, int t) {
    using namespace attn;
    constexpr int LDK = HD + 8;
    constexpr int KCH = BKV * HD / 8;          // 16-byte K chunks: (key, 8 columns)
    constexpr int VCH = (BKV / 2) * (DS / 8);  // V chunks: (key pair, 8 columns)
    constexpr int KFULL = KCH / (nt * BATCH), VB = BATCH / 2, VFULL = VCH / (nt * VB);
    auto kaddr = [&](int c) { return kbase + (size_t)(kb + c / (HD / 8)) * kvStride + (c % (HD / 8)) * 8; };
    auto klds = [&](int c) { return reinterpret_cast<uint4*>(&Ks[(c / (HD / 8)) * LDK + (c % (HD / 8)) * 8]); };
    auto vaddr = [&](int c) { return vbase + (size_t)(kb + 2 * (c % (BKV / 2))) * kvStride + (c / (BKV / 2)) * 8; };
    auto vlds = [&](int c) { return reinterpret_cast<uint32_t*>(&Vt[(c / (BKV / 2)) * 8 * LDV + 2 * (c % (BKV / 2))]); };
#pragma unroll 1
    for (int bi = 0; bi < KFULL; bi++) {
        uint4 r[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; j++) r[j] = *reinterpret_cast<const uint4*>(kaddr(t + (bi * BATCH + j) * nt));
#pragma unroll
        for (int j = 0; j < BATCH; j++) *klds(t + (bi * BATCH + j) * nt) = r[j];
    }
    for (int c = t + KFULL * BATCH * nt; c < KCH; c += nt) *klds(c) = *reinterpret_cast<const uint4*>(kaddr(c));
#pragma unroll 1
    for (int bi = 0; bi < VFULL; bi++) {
        uint4 a[VB], b[VB];
#pragma unroll
        for (int j = 0; j < VB; j++) {
            const _Float16* p = vaddr(t + (bi * VB + j) * nt);
            a[j] = *reinterpret_cast<const uint4*>(p);
            b[j] = *reinterpret_cast<const uint4*>(p + kvStride);
        }
#pragma unroll
        for (int j = 0; j < VB; j++) attn_store_vt(vlds(t + (bi * VB + j) * nt), a[j], b[j]);
    }
    for (int c = t + VFULL * VB * nt; c < VCH; c += nt) {
        const _Float16* p = vaddr(c);
        attn_store_vt(vlds(c), *reinterpret_cast<const uint4*>(p), *reinterpret_cast<const uint4*>(p + kvStride));
    }
}

template <int HD, int DS, int G>
__global__ __launch_bounds__(256) void attention_kernel(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kg,
                                                        const uint16_t* __restrict__ Vg, uint16_t* __restrict__ Og,
                                                        const AttnWork* __restrict__ work, int H, int KV, int hw,
                                                        float scale_log2) {
    using namespace attn;
    constexpr int LDK = HD + 8;
    constexpr int BUF = BKV * LDK + DS * LDV;  // halves per K + V^T buffer
    constexpr bool PIPE = G < WAVES && HD <= 256;
    constexpr int NP = PIPE ? (WAVES - G) * 64 : WAVES * 64;  // staging threads
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const AttnWork wi = work[blockIdx.x];
    const int kvh = blockIdx.y, slice = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool computes = wave < G;
    const int h = kvh * G + wave;
    const int len = int(wi.seq_len), q0 = int(wi.q0);
    // A work item of an empty sequence has nothing to attend; leaving before any access also keeps
    // the (len - 1) in the buffer ranges and row clamps below from wrapping around.
    if (len <= 0) return;
    const int qStride = H * HD, kvStride = KV * HD;
    const int d0 = slice * DS;
    const int qi = q0 + (lane & 31);
    const bool qvalid = computes && qi < len;

    int kstart = 0, kend = len;
    if (hw > 0) {
        kstart = q0 - hw > 0 ? q0 - hw : 0;
        const int hi = q0 + kAttnQueries + hw;
        kend = hi < len ? hi : len;
    }
    kstart = kstart / BKV * BKV;
    const int nblocks = (kend - kstart + BKV - 1) / BKV;

    const _Float16* kbase = reinterpret_cast<const _Float16*>(Kg) + (size_t)wi.seq_start * kvStride + kvh * HD;
    const _Float16* vbase = reinterpret_cast<const _Float16*>(Vg) + (size_t)wi.seq_start * kvStride + kvh * HD + d0;
    // Producers: the waves past G when pipelined; everyone otherwise.
    const int pt = PIPE ? tid - G * 64 : tid;

    half8_t qf[HD / 16];
    if (computes) {
        const _Float16* qp = reinterpret_cast<const _Float16*>(Qg) + (size_t)(wi.seq_start + qi) * qStride + h * HD + (lane >> 5) * 8;
#pragma unroll
        for (int ks = 0; ks < HD / 16; ks++) {
            if (qvalid)
                qf[ks] = *reinterpret_cast<const half8_t*>(qp + ks * 16);
            else
#pragma unroll
                for (int j = 0; j < 8; j++) qf[ks][j] = _Float16(0.0f);
        }
    }

    float16_t o[DS / 32];
#pragma unroll
    for (int i = 0; i < DS / 32; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    if (PIPE && !computes) {
        // Producer waves: block 0, then block it + 1 while the compute waves work on block it.
        // They pass the same number of barriers as the compute waves.
        if (nblocks > 0) attn_stage<HD, DS, BATCH, NP>(lds, lds + BKV * LDK, kbase, vbase, kstart, kvStride, pt);
        __syncthreads();
        for (int it = 0; it < nblocks; it++) {
            if (it + 1 < nblocks) {
                _Float16* nK = lds + ((it + 1) & 1) * BUF;
                attn_stage<HD, DS, BATCH, NP>(nK, nK + BKV * LDK, kbase, vbase, kstart + (it + 1) * BKV, kvStride, pt);
            }
            __syncthreads();
        }
        return;
    }
    if (!PIPE && nblocks > 0) attn_stage<HD, DS, BATCH_INLINE, NP>(lds, lds + BKV * LDK, kbase, vbase, kstart, kvStride, pt);
    __syncthreads();
    for (int it = 0; it < nblocks; it++) {
        const int kb = kstart + it * BKV;
        _Float16* Ks = lds + (PIPE ? (it & 1) * BUF : 0);
        _Float16* Vt = Ks + BKV * LDK;
        if (computes) {
            float16_t s[2];
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int r = 0; r < 16; r++) s[kt][r] = 0.0f;
                const _Float16* kp = &Ks[(kt * 32 + (lane & 31)) * LDK + (lane >> 5) * 8];
#pragma unroll
                for (int ks = 0; ks < HD / 16; ks++) {
                    const half8_t a = *reinterpret_cast<const half8_t*>(kp + ks * 16);
                    s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], s[kt], 0, 0, 0);
                }
            }
            float bmax = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = kb + kt * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                    bool valid = key < len;
                    if (hw > 0) valid = valid && abs(qi - key) <= hw;
                    const float val = valid ? s[kt][r] * scale_log2 : -INFINITY;
                    s[kt][r] = val;
                    bmax = fmaxf(bmax, val);
                }
            bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
            const float m_new = fmaxf(m_run, bmax);
            float alpha = 1.0f, sum = 0.0f;
            if (m_new == -INFINITY) {
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) s[kt][r] = 0.0f;
            } else {
                alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float p = __builtin_amdgcn_exp2f(s[kt][r] - m_new);
                        s[kt][r] = p;
                        sum += p;
                    }
            }
            sum += __shfl_xor(sum, 32, 64);
            l_run = l_run * alpha + sum;
            m_run = m_new;
            if (alpha != 1.0f) {
#pragma unroll
                for (int i = 0; i < DS / 32; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[i][r] *= alpha;
            }
#pragma unroll
            for (int ks = 0; ks < BKV / 16; ks++) {
                half8_t pb;
#pragma unroll
                for (int j = 0; j < 8; j++) pb[j] = _Float16(s[ks >> 1][(ks & 1) * 8 + j]);
                const _Float16* vp = &Vt[(lane & 31) * LDV + ks * 16 + (lane >> 5) * 4];
#pragma unroll
                for (int dt = 0; dt < DS / 32; dt++) {
                    const half4_t lo4 = *reinterpret_cast<const half4_t*>(vp + dt * 32 * LDV);
                    const half4_t hi4 = *reinterpret_cast<const half4_t*>(vp + dt * 32 * LDV + 8);
                    const half8_t a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[dt], 0, 0, 0);
                }
            }
        }
        __syncthreads();
        if (!PIPE && it + 1 < nblocks) {
            attn_stage<HD, DS, BATCH_INLINE, NP>(lds, lds + BKV * LDK, kbase, vbase, kb + BKV, kvStride, pt);
            __syncthreads();
        }
    }
    if (!qvalid) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    _Float16* op = reinterpret_cast<_Float16*>(Og) + (size_t)(wi.seq_start + qi) * qStride + h * HD + d0 + (lane >> 5) * 4;
#pragma unroll
    for (int dt = 0; dt < DS / 32; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            half4_t v4;
#pragma unroll
            for (int j = 0; j < 4; j++) v4[j] = _Float16(o[dt][g * 4 + j] * inv);
            *reinterpret_cast<half4_t*>(op + dt * 32 + g * 8) = v4;
        }
}

// ============================================================================ attention, Q/K/V copied straight into LDS
//
// One workgroup of 2 G waves per (work item of 64 query rows, KV head): wave w owns query head
// kvh * G + w % G for the query half w / G (32 rows). Q, K and V move from global memory into
// LDS with buffer_load ... lds copies -- no register or producer wave carries them. Each wave's
// 32 query rows sit in LDS for the whole kernel (so the fp32 output accumulators, 32 x hd per
// wave, are the only large register array); keys stream in blocks of 32 through two LDS
// buffers, the next block's copy in flight while the current one is multiplied. V arrives
// transposed (V^T [kv head][d][key], written by the QKV epilogue or launch_v_transpose).
//
// Everything in LDS is stored in MFMA fragment order: a 1 KB chunk holds one operand fragment
// of v_mfma_f32_32x32x16_f16, lane l's 16 bytes at 16 l. The copies gather the fragments
// (lane l of a chunk reads 16 bytes of row l % 32, columns 8 (l / 32) .. + 8 of the k-step), so
// every fragment read is base + 16 lane + a constant: no per-k-step address registers and no
// bank conflicts.
//   Q (per wave): chunk ks = query rows q0 .. q0 + 31, head dims 16 ks .. 16 ks + 15.
//   K (per block): chunk ks = S^T rows (keys, permuted as below), head dims 16 ks ...
//   V^T (per block): chunk ks2 * DT + dt = head dims 32 dt .. + 31, keys 16 ks2 .. + 15.
//
// The rows of the S^T tile are taken from the key block in the order 0-3, 8-11, 4-7, 12-15
// within each 16 keys. The accumulator then holds, for lane half h, keys 8h .. 8h + 7 of each
// 16-key step in consecutive registers: the B operand of the P.V product is the accumulator
// itself, converted to fp16.
namespace attn2 {
constexpr int QB = 64;   // query rows per work item
constexpr int BKV = 32;  // keys per block
}  // namespace attn2

template <int HD, int G>
constexpr int attention_v2_lds_bytes() { return 2 * G * 32 * HD * 2 + 2 * (2 * attn2::BKV * HD * 2); }

template <int HD, int G>
__global__ __launch_bounds__(2 * G * 64) void attention_v2_kernel(const uint16_t* __restrict__ Qg,
                                                                  const uint16_t* __restrict__ Kg,
                                                                  const uint16_t* __restrict__ VTg,
                                                                  uint16_t* __restrict__ Og,
                                                                  const AttnWork* __restrict__ work, int H, int KV,
                                                                  int vt_cols, int hw, float scale_log2) {
    using namespace attn2;
    constexpr int NW = 2 * G, KSQ = HD / 16, DT = HD / 32;
    constexpr int Q_BYTES = 32 * HD * 2;              // one wave's query rows
    constexpr int K_BYTES = BKV * HD * 2, STAGE = 2 * K_BYTES;
    constexpr int KCH = K_BYTES / 1024, CH = 2 * KCH;  // 1 KB chunks per key block (K, then V^T)
    static_assert(KCH == KSQ && KCH == 2 * DT, "chunk counts");
    extern __shared__ __attribute__((aligned(1024))) unsigned char ldsb[];
    unsigned char* const kv = ldsb + NW * Q_BYTES;

    // XCD-aware order: workgroup b runs on XCD b % 8, so giving each XCD a contiguous run of work
    // items keeps a sequence's K and V^T in one XCD's L2.
    const int nb = int(gridDim.x), full = nb / 8 * 8, bx = int(blockIdx.x);
    const AttnWork wi = work[bx < full ? (bx % 8) * (full / 8) + bx / 8 : bx];
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = kvh * G + wave % G;
    const int len = int(wi.seq_len), q0 = int(wi.q0) + (wave / G) * 32;
    // A work item of an empty sequence has nothing to attend; leaving before any access also keeps
    // the (len - 1) in the buffer ranges and row clamps below from wrapping around.
    if (len <= 0) return;
    const int qi = q0 + (lane & 31), half = lane >> 5;
    const int qStride = H * HD, kvStride = KV * HD;

    int kstart = 0, kend = len;
    if (hw > 0) {
        kstart = max(int(wi.q0) - hw, 0);
        kend = min(int(wi.q0) + QB + hw, len);
    }
    kstart = kstart / BKV * BKV;
    const int nblocks = (kend - kstart + BKV - 1) / BKV;

    // Buffer resources over this sequence's rows of the wave's query head and of the KV head, and
    // over the KV head's V^T rows from the sequence's first column on: copies past them read
    // zeros.
    const __amdgpu_buffer_rsrc_t qr =
        buffer_rsrc(Qg + (size_t)wi.seq_start * qStride + h * HD, uint32_t(((len - 1) * qStride + HD) * 2));
    const __amdgpu_buffer_rsrc_t kr =
        buffer_rsrc(Kg + (size_t)wi.seq_start * kvStride + kvh * HD, uint32_t(((len - 1) * kvStride + HD) * 2));
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(VTg + (size_t)kvh * HD * vt_cols + wi.vt_start,
                                                  uint32_t(((HD - 1) * vt_cols + (vt_cols - int(wi.vt_start))) * 2));

    // This wave's query fragments (rows past the sequence re-read its last row; their outputs
    // are never stored).
    unsigned char* const qs = ldsb + wave * Q_BYTES;
    {
        const uint32_t qo = uint32_t((min(qi, len - 1) * qStride + 8 * half) * 2);
#pragma unroll
        for (int c = 0; c < KSQ; c++) lds_copy16(qr, qs + c * 1024, qo + c * 32, 0);
    }

    // S^T row i (lane i % 32 of the A operand) reads key (i / 16) * 16 + perm(i % 16): 0-3,
    // 8-11, 4-7, 12-15.
    const int i16 = lane & 15;
    const int krow = (lane & 16) + (i16 < 4 || i16 >= 12 ? i16 : (i16 < 8 ? i16 + 4 : i16 - 4));

    // This wave's copies of a key block: chunks wave, wave + NW, ... (at most CPW). The lane part
    // of each source offset is fixed; a block adds its key offset.
    constexpr int CPW = (CH + NW - 1) / NW;
    uint32_t coff[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int c = wave + i * NW;
        if (c < KCH) {
            coff[i] = uint32_t((krow * kvStride + 16 * c + 8 * half) * 2);
        } else {
            const int ks2 = (c - KCH) / DT, dt = (c - KCH) % DT;
            coff[i] = uint32_t(((dt * 32 + (lane & 31)) * vt_cols + 16 * ks2 + 8 * half) * 2);
        }
    }
#define A2_ISSUE(kb, b)                                                                                    \
    do {                                                                                                   \
        const uint32_t ko_ = uint32_t((kb) * kvStride * 2), vo_ = uint32_t((kb) * 2);                      \
        _Pragma("unroll") for (int i = 0; i < CPW; i++) {                                                  \
            const int c = wave + i * NW;                                                                   \
            if (c < KCH)                                                                                   \
                lds_copy16(kr, kv + (b) * STAGE + c * 1024, coff[i] + ko_, 0);                            \
            else if (c < CH)                                                                               \
                lds_copy16(vr, kv + (b) * STAGE + c * 1024, coff[i] + vo_, 0);                            \
        }                                                                                                  \
    } while (0)

    float16_t o[DT];
#pragma unroll
    for (int i = 0; i < DT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    if (nblocks > 0) A2_ISSUE(kstart, 0);
    wait_vmcnt<0>();
    workgroup_barrier();
    const unsigned char* const qf = qs + lane * 16;
    for (int it = 0; it < nblocks; it++) {
        const int kb = kstart + it * BKV, b = it & 1;
        if (it + 1 < nblocks) A2_ISSUE(kb + BKV, b ^ 1);
        // Every wave computes, also one whose query rows all lie past the sequence (they read
        // the clamped last row; nothing of theirs is stored): no branch around the block.
        const unsigned char* const kf = kv + b * STAGE + lane * 16;
        const unsigned char* const vf = kf + K_BYTES;
        // S^T = K Q^T over the head dims, two accumulation chains; fragments read PF k-steps
        // ahead through a ring of PF + 1 registers, so LDS latency overlaps the MFMAs.
        constexpr int PF = 3, RING = PF + 1;
        float16_t sc, sc1;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = sc1[r] = 0.0f;
        half8_t ka[RING], qa[RING];
#pragma unroll
        for (int f = 0; f < PF; f++) {
            ka[f] = *reinterpret_cast<const half8_t*>(kf + f * 1024);
            qa[f] = *reinterpret_cast<const half8_t*>(qf + f * 1024);
        }
#pragma unroll
        for (int ks = 0; ks < KSQ; ks++) {
            if (ks + PF < KSQ) {
                ka[(ks + PF) % RING] = *reinterpret_cast<const half8_t*>(kf + (ks + PF) * 1024);
                qa[(ks + PF) % RING] = *reinterpret_cast<const half8_t*>(qf + (ks + PF) * 1024);
            }
            // keep the reads ahead of the MFMA (the scheduler would otherwise sink them)
            __builtin_amdgcn_sched_barrier(0);
            if (ks & 1)
                sc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks % RING], qa[ks % RING], sc1, 0, 0, 0);
            else
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks % RING], qa[ks % RING], sc, 0, 0, 0);
        }
        // the first V^T fragments are read while the softmax runs
        half8_t va[RING];
#pragma unroll
        for (int f = 0; f < PF; f++) va[f] = *reinterpret_cast<const half8_t*>(vf + f * 1024);
        sc += sc1;
        // key of accumulator element r for this lane: kb + 16 (r / 8) + 8 half + r % 8
        const bool inside = kb + BKV <= len && (hw == 0 || (kb >= q0 + 31 - hw && kb + BKV - 1 <= q0 + hw));
        float bmax = -INFINITY;
        if (inside) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                sc[r] *= scale_log2;
                bmax = fmaxf(bmax, sc[r]);
            }
        } else {
            // keys past the sequence, and (sliding window) keys farther than hw from the query
            const int lim = hw > 0 ? hw : 1 << 30;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = kb + (r >> 3) * 16 + half * 8 + (r & 7);
                const bool valid = key < len && abs(qi - key) <= lim;
                const float val = valid ? sc[r] * scale_log2 : -INFINITY;
                sc[r] = val;
                bmax = fmaxf(bmax, val);
            }
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        // Lazy rescaling: the reference point m_run moves only when a score exceeds it by more
        // than 2^8 (log2 domain), so P stays below 256 -- exact in fp16 to the same relative
        // precision -- and the o *= alpha pass runs only on the rare blocks that move it.
        // o / l is unchanged by the choice of reference point.
        if (__builtin_amdgcn_ballot_w64(bmax > m_run + 8.0f)) {
            const float m_new = fmaxf(m_run, bmax);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < DT; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[i][r] *= alpha;
            m_run = m_new;
        }
        // m_run is -inf only while every key seen so far is masked (all scores -inf): the
        // reference point 0 then gives p = 0.
        const float m_ref = m_run == -INFINITY ? 0.0f : m_run;
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p = __builtin_amdgcn_exp2f(sc[r] - m_ref);
            sc[r] = p;
            sum += p;
        }
        sum += __shfl_xor(sum, 32, 64);
        l_run += sum;
        // O^T += V^T P^T: 16-key steps ks2, head-dim tiles dt; V^T fragments PF steps ahead.
#pragma unroll
        for (int ks2 = 0; ks2 < BKV / 16; ks2++) {
            half8_t pb;
#pragma unroll
            for (int j = 0; j < 8; j++) pb[j] = _Float16(sc[ks2 * 8 + j]);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int f = ks2 * DT + dt;
                if (f + PF < 2 * DT) va[(f + PF) % RING] = *reinterpret_cast<const half8_t*>(vf + (f + PF) * 1024);
                __builtin_amdgcn_sched_barrier(0);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[f % RING], pb, o[dt], 0, 0, 0);
            }
        }
        wait_vmcnt<0>();
        wait_lgkmcnt0();
        workgroup_barrier();
    }
#undef A2_ISSUE
    if (qi >= len) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    _Float16* op = reinterpret_cast<_Float16*>(Og) + (size_t)(wi.seq_start + qi) * qStride + h * HD + half * 4;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            half4_t v4;
#pragma unroll
            for (int j = 0; j < 4; j++) v4[j] = _Float16(o[dt][g * 4 + j] * inv);
            *reinterpret_cast<half4_t*>(op + dt * 32 + g * 8) = v4;
        }
}

// ============================================================================ attention, 16-query waves
//
// The same work item (64 query rows of one sequence, one KV head) and the same K / V^T stream as
// attention_v2_kernel, with 4 G waves of 16 queries each (wave w: query head kvh * G + w % G,
// rows q0 + 16 (w / G) .. + 15) on v_mfma_f32_16x16x32_f16. A wave's accumulators shrink to
// 16 queries x hd (64 registers at hd 256) and its queries' fragments fit in registers (32),
// so nothing but K and V^T lives in LDS and G = 3 gives 12 waves, three per SIMD: while one
// wave is in its softmax, the SIMD's other waves keep the MFMA pipe busy.
//
// LDS per stage (one block of 32 keys), in fragment order (1 KB chunk = one operand fragment,
// lane l's 16 bytes at 16 l):
//   K chunk (ks, m), m = 0, 1: A operand of S^T tile m over head dims 32 ks .. + 31; lane l
//     holds key 8 ((l % 16) / 4) + 4 m + l % 4, head dims 32 ks + 8 (l / 16) + [0, 8);
//   V^T chunk dt: A operand of O^T rows 16 dt .. + 15; lane l holds head dim 16 dt + l % 16,
//     keys 8 (l / 16) + [0, 8).
// With that key order, lane l's accumulators of the two S^T tiles (rows 4 (l / 16) + r) are
// keys 8 (l / 16) + [0, 8) of query l % 16: exactly the B operand of the P.V product, so P
// goes from the S accumulators to the MFMA with only the fp16 conversion. A query's 32 scores
// sit in lanes q, q + 16, q + 32, q + 48; its softmax reductions are two lane exchanges.
// Max and sum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four key groups of a query in the
// 16x16 MFMA layouts) with the gfx950 row-swap instructions: VALU operations, where a shuffle
// would be an LDS round trip.
__device__ __forceinline__ float max_over_key_groups(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_over_key_groups(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

namespace attn3 {
constexpr int NS = 2;     // key blocks in LDS
constexpr int BKV = 32;   // keys per block
}  // namespace attn3

template <int HD>
constexpr int attention_v3_lds_bytes() { return attn3::NS * 2 * attn3::BKV * HD * 2; }

// ONE: one query head per workgroup (grid y over the H query heads, QW waves) instead of the G
// heads of a KV head (grid y over the KV heads, QW G waves). For the smallest batches: each
// workgroup's key-block loop then carries a G-th of the work, on G times as many CUs. A head's
// waves run the same operations either way, so the outputs are the same bits.
template <int HD, int G, int QW, bool ONE = false>
__global__ __launch_bounds__(QW * (ONE ? 1 : G) * 64) void attention_v3_kernel(const uint16_t* __restrict__ Qg,
                                                                  const uint16_t* __restrict__ Kg,
                                                                  const uint16_t* __restrict__ VTg,
                                                                  uint16_t* __restrict__ Og,
                                                                  const AttnWork* __restrict__ work, int H, int KV,
                                                                  int vt_cols, int hw, float scale_log2) {
    using namespace attn3;
    constexpr int QB = 16 * QW, NW = QW * (ONE ? 1 : G), KS = HD / 32, DT = HD / 16;
    constexpr int K_BYTES = BKV * HD * 2, STAGE = 2 * K_BYTES;
    constexpr int KCH = K_BYTES / 1024, CH = 2 * KCH;  // K chunks (ks, m), then V^T chunks dt
    static_assert(KCH == 2 * KS && KCH == DT, "chunk counts");
    constexpr int CPW = (CH + NW - 1) / NW;  // copies per wave per block (some waves repeat one)
    static_assert(NW <= CH, "a wave past the last chunk repeats its own chunk index");
    extern __shared__ __attribute__((aligned(1024))) unsigned char ldsa[];

    // XCD-aware order, as in attention_v2_kernel.
    const int nb = int(gridDim.x), full = nb / 8 * 8, bx = int(blockIdx.x);
    const int widx = bx < full ? (bx % 8) * (full / 8) + bx / 8 : bx;
    const int seq_start = __builtin_amdgcn_readfirstlane(int(work[widx].seq_start));
    const int len = __builtin_amdgcn_readfirstlane(int(work[widx].seq_len));
    // A work item of an empty sequence has nothing to attend; leaving before any access also keeps
    // the (len - 1) in the buffer ranges and row clamps below from wrapping around.
    if (len <= 0) return;
    // grid z splits a work item into parts of QB queries (head dim 512: 32-query workgroups over
    // 64-query items)
    const int wq0 = __builtin_amdgcn_readfirstlane(int(work[widx].q0)) + int(blockIdx.z) * QB;
    const int vt_start = __builtin_amdgcn_readfirstlane(int(work[widx].vt_start));
    const int kvh = ONE ? int(blockIdx.y) / G : int(blockIdx.y);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int h = ONE ? int(blockIdx.y) : kvh * G + wave % G;
    const int q0 = wq0 + (ONE ? wave : wave / G) * 16;
    const int l16 = lane & 15, g4 = lane >> 4;  // query column, lane group
    const int qi = q0 + l16;
    const int qStride = H * HD, kvStride = KV * HD;

    int kstart = 0, kend = len;
    if (hw > 0) {
        kstart = max(wq0 - hw, 0);
        kend = min(wq0 + QB + hw, len);
    }
    kstart = kstart / BKV * BKV;
    const int nblocks = (kend - kstart + BKV - 1) / BKV;

    // Buffer resources over the sequence's rows of the KV head and over the head's V^T rows from
    // the sequence's first column on: copies past them read zeros.
    const __amdgpu_buffer_rsrc_t kr =
        buffer_rsrc(Kg + (size_t)seq_start * kvStride + kvh * HD, uint32_t(((len - 1) * kvStride + HD) * 2));
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(VTg + (size_t)kvh * HD * vt_cols + vt_start,
                                                  uint32_t(((HD - 1) * vt_cols + (vt_cols - vt_start)) * 2));
    const uint32_t klane = uint32_t(((8 * (l16 >> 2) + (lane & 3)) * kvStride + 8 * g4) * 2);
    const uint32_t vlane = uint32_t((l16 * vt_cols + 8 * g4) * 2);
    // Every wave issues CPW copies per block (the waves past the last chunk repeat their first
    // one), so one vmcnt count fits every wave.
#define A3_ISSUE(kb, b)                                                                                    \
    do {                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < CPW; i++) {                                                  \
            int c = wave + i * NW;                                                                         \
            if (c >= CH) c = wave;                                                                         \
            unsigned char* dst_ = ldsa + (b) * STAGE + c * 1024;                                           \
            if (c < KCH) {                                                                                 \
                const int ks_ = c >> 1, m_ = c & 1;                                                        \
                lds_copy16(kr, dst_, klane + uint32_t(((kb) + 4 * m_) * kvStride * 2 + ks_ * 64), 0);      \
            } else {                                                                                       \
                lds_copy16(vr, dst_, vlane + uint32_t((c - KCH) * 16 * vt_cols * 2 + (kb) * 2), 0);        \
            }                                                                                              \
        }                                                                                                  \
    } while (0)

    // This wave's query fragments (B operand of S^T = K Q^T): lane l: query qi (rows past the
    // sequence re-read its last row; their outputs are never stored), head dims 32 ks + 8 (l / 16).
    half8_t qa[KS];
    {
        const __amdgpu_buffer_rsrc_t qr =
            buffer_rsrc(Qg + (size_t)seq_start * qStride + h * HD, uint32_t(((len - 1) * qStride + HD) * 2));
        const uint32_t qo = uint32_t((min(qi, len - 1) * qStride + 8 * g4) * 2);
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
            qa[ks] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(qr, qo + ks * 64, 0, 0));
    }

    float4_t o[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) o[i] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < nblocks) A3_ISSUE(kstart + s * BKV, s);
    int b = 0;
    for (int it = 0; it < nblocks; it++) {
        const int kb = kstart + it * BKV;
        // Block it has landed once at most the later blocks' copies are in flight (min(NS - 2,
        // blocks left) of them, CPW copies each); the barrier then covers every wave's copies,
        // and (after each wave's LDS reads) frees the buffer the next copies overwrite.
        static_assert(NS >= 2 && NS <= 4, "the waits below cover two to four stages");
        const int ahead = min(NS - 2, nblocks - 1 - it);
        if (ahead >= 2)
            wait_vmcnt<2 * CPW>();
        else if (ahead == 1)
            wait_vmcnt<CPW>();
        else
            wait_vmcnt<0>();
        wait_lgkmcnt0();
        workgroup_barrier();
        if (it + NS - 1 < nblocks) A3_ISSUE(kstart + (it + NS - 1) * BKV, b == 0 ? NS - 1 : b - 1);
        const unsigned char* const kf = ldsa + b * STAGE + lane * 16;
        const unsigned char* const vf = kf + K_BYTES;
        // S^T tiles m = 0, 1 over the head dims; K fragments read PF k-steps ahead
        constexpr int PF = 2, RING = PF + 1;
        float4_t s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
        half8_t ka[RING][2];
#pragma unroll
        for (int f = 0; f < PF; f++) {
            ka[f][0] = *reinterpret_cast<const half8_t*>(kf + (2 * f) * 1024);
            ka[f][1] = *reinterpret_cast<const half8_t*>(kf + (2 * f + 1) * 1024);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks + PF < KS) {
                ka[(ks + PF) % RING][0] = *reinterpret_cast<const half8_t*>(kf + (2 * (ks + PF)) * 1024);
                ka[(ks + PF) % RING][1] = *reinterpret_cast<const half8_t*>(kf + (2 * (ks + PF) + 1) * 1024);
            }
            // keep the reads ahead of the MFMAs (the scheduler would otherwise sink them)
            __builtin_amdgcn_sched_barrier(0);
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks % RING][0], qa[ks], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks % RING][1], qa[ks], s1, 0, 0, 0);
        }
        // the first V^T fragments are read while the softmax runs
        half8_t va[RING];
#pragma unroll
        for (int f = 0; f < PF; f++) va[f] = *reinterpret_cast<const half8_t*>(vf + f * 1024);
        // this lane's scores: keys kb + 8 g4 + e, e = 0..7
        float sc[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        const bool inside = kb + BKV <= len && (hw == 0 || (kb >= q0 + 15 - hw && kb + BKV - 1 <= q0 + hw));
        if (!inside) {
            // keys past the sequence, and (sliding window) keys farther than hw from the query
            const int lim = hw > 0 ? hw : 1 << 30;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int key = kb + 8 * g4 + e;
                const bool valid = (key < len) & (abs(qi - key) <= lim);
                sc[e] = valid ? sc[e] : -INFINITY;
            }
        }
        // this lane's max in the raw score domain (scale > 0)
        const float lmax =
            fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
        // Lazy rescaling, as in attention_v2_kernel: the reference point moves only when a
        // score exceeds it by more than 2^8, so P stays below 256. A lane's own scores decide
        // whether the wave takes the update; the query's block max (over its four key groups)
        // is formed only then.
        if (__builtin_amdgcn_ballot_w64(lmax * scale_log2 > m_run + 8.0f)) {
            const float bmax = max_over_key_groups(lmax) * scale_log2;
            const float m_new = fmaxf(m_run, bmax);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < DT; i++) o[i] *= alpha;
            m_run = m_new;
        }
        const float m_ref = m_run == -INFINITY ? 0.0f : m_run;
        float sum = 0.0f;
        half8_t pb;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], scale_log2, -m_ref));
            sum += p;
            pb[e] = _Float16(p);
        }
        l_run += sum;  // this lane's keys only; the key groups are summed once, at the end
        // O^T += V^T P^T: head-dim tiles dt of 16 rows, the block's 32 keys as one k-step
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            if (dt + PF < DT) va[(dt + PF) % RING] = *reinterpret_cast<const half8_t*>(vf + (dt + PF) * 1024);
            __builtin_amdgcn_sched_barrier(0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt % RING], pb, o[dt], 0, 0, 0);
        }
        b = b + 1 == NS ? 0 : b + 1;
    }
#undef A3_ISSUE
    wait_vmcnt<0>();
    l_run = sum_over_key_groups(l_run);
    if (qi >= len) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    // o[dt], lane l: head dims 16 dt + 4 (l / 16) + r of query qi
    _Float16* op = reinterpret_cast<_Float16*>(Og) + (size_t)(seq_start + qi) * qStride + h * HD + 4 * g4;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        half4_t v4;
#pragma unroll
        for (int r = 0; r < 4; r++) v4[r] = _Float16(o[dt][r] * inv);
        *reinterpret_cast<half4_t*>(op + dt * 16) = v4;
    }
}

// Batches of fewer workgroups than this (one per work item and KV head: a text of up to about 250
// tokens) run one query head per workgroup. One 64-token text's attention: 9.2 -> 7.1 us per
// layer (config-2 model); at 16 work items and more it gained nothing (one 512-token text) or
// lost (eight: 26.7 -> 34.5 us).
constexpr int kAttnOneHeadWork = 16;

template <int HD, int G>
static hipError_t attention_v3_dispatch(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                                        int vt_cols, uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hw,
                                        float scale, int item_queries) {
    const float scale_log2 = scale * 1.4426950408889634f;
    const uint32_t lds = uint32_t(attention_v3_lds_bytes<HD>());
    if (G > 1 && n_work * KV < kAttnOneHeadWork) {
        if (item_queries == 32)
            launch_kernel(attention_v3_kernel<HD, G, 2, true>, dim3(n_work, H), dim3(2 * 64), lds, s, q, k, vt, o, work, H, KV,
                          vt_cols, hw, scale_log2);
        else
            launch_kernel(attention_v3_kernel<HD, G, 4, true>, dim3(n_work, H), dim3(4 * 64), lds, s, q, k, vt, o, work, H, KV,
                          vt_cols, hw, scale_log2);
    } else if (item_queries == 32) {
        launch_kernel(attention_v3_kernel<HD, G, 2>, dim3(n_work, KV), dim3(2 * G * 64), lds, s, q, k, vt, o, work, H, KV, vt_cols,
                      hw, scale_log2);
    } else {
        launch_kernel(attention_v3_kernel<HD, G, 4>, dim3(n_work, KV), dim3(4 * G * 64), lds, s, q, k, vt, o, work, H, KV, vt_cols,
                      hw, scale_log2);
    }
    return hipGetLastError();
}

template <int HD, int G>
static hipError_t attention_v2_dispatch(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                                        int vt_cols, uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hw,
                                        float scale) {
    const float scale_log2 = scale * 1.4426950408889634f;
    launch_kernel(attention_v2_kernel<HD, G>, dim3(n_work, KV), dim3(2 * G * 64), uint32_t(attention_v2_lds_bytes<HD, G>()), s,
                  q, k, vt, o, work, H, KV, vt_cols, hw, scale_log2);
    return hipGetLastError();
}

template <int HD>
static hipError_t attention_v2_dispatch_g(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                                          int vt_cols, uint16_t* o, const AttnWork* work, int n_work, int H, int KV,
                                          int hw, float scale, int item_queries) {
    switch (H / KV) {
    // groups of up to 3 query heads: 16-query waves (item_queries / 16 per head)
    case 1: return attention_v3_dispatch<HD, 1>(s, q, k, vt, vt_cols, o, work, n_work, H, KV, hw, scale, item_queries);
    case 2: return attention_v3_dispatch<HD, 2>(s, q, k, vt, vt_cols, o, work, n_work, H, KV, hw, scale, item_queries);
    case 3: return attention_v3_dispatch<HD, 3>(s, q, k, vt, vt_cols, o, work, n_work, H, KV, hw, scale, item_queries);
    case 4:
        if (item_queries != 64) return hipErrorInvalidValue;
        if constexpr (attention_v2_lds_bytes<HD, 4>() <= 160 * 1024)
            return attention_v2_dispatch<HD, 4>(s, q, k, vt, vt_cols, o, work, n_work, H, KV, hw, scale);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

bool attention_v2_supported(int hd, int H, int KV) {
    if (hd == 512) return KV > 0 && H == 4 * KV;  // attention_v3_kernel<512, 4, 2>
    if (!((hd == 128 || hd == 256) && KV > 0 && H % KV == 0 && H / KV >= 1 && H / KV <= 4)) return false;
    const int G = H / KV;
    return 2 * G * 32 * hd * 2 + 2 * (2 * attn2::BKV * hd * 2) <= 160 * 1024;  // LDS of one workgroup
}

hipError_t launch_attention_v2(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, int vt_cols,
                               uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hd, int half_window,
                               float scale, int item_queries) {
    if (n_work < 0 || !attention_v2_supported(hd, H, KV) || half_window < 0 || vt_cols <= 0 || vt_cols % 8 ||
        (item_queries != 64 && !(item_queries == 32 && (H / KV <= 3 || hd == 512))))
        return hipErrorInvalidValue;
    if (n_work == 0) return hipSuccess;
    if (hd == 512) {
        // 8 waves (4 query heads x 2 query tiles) of 252 registers, K/V blocks of 64 KB in LDS: a
        // workgroup takes 32 queries, grid z the halves of a 64-query item
        const float scale_log2 = scale * 1.4426950408889634f;
        launch_kernel(attention_v3_kernel<512, 4, 2>, dim3(n_work, KV, item_queries / 32), dim3(8 * 64),
                      uint32_t(attention_v3_lds_bytes<512>()), s, q, k, vt, o, work, H, KV, vt_cols, half_window, scale_log2);
        return hipGetLastError();
    }
    if (hd == 128)
        return attention_v2_dispatch_g<128>(s, q, k, vt, vt_cols, o, work, n_work, H, KV, half_window, scale, item_queries);
    return attention_v2_dispatch_g<256>(s, q, k, vt, vt_cols, o, work, n_work, H, KV, half_window, scale, item_queries);
}

// ============================================================================ attention, split-precision scores
//
// For the layers whose QKV projection runs at split precision (head dim 512): q and k arrive as
// fp16 pairs with hi + lo the fp32 value (hi = fp16(x), lo = fp16(x - hi)), and a score is
// q_hi.k_hi + q_lo.k_hi + q_hi.k_lo on v_mfma_f32_16x16x32_f16 (the dropped q_lo.k_lo is below
// 2^-22 of it). Scores of two RMS-normed 512-wide vectors at attention scale 1 reach several
// hundred; with plain fp16 operands (2^-11 relative per element) they move by ~0.02, which
// shifts the weights of two nearly tied keys by a few percent (reference: fp32 scores,
// Shaders/Attention.metal:172-188, Model/CPUReference.swift:129-160).
//
// The fragment layouts, the key order of the S^T tiles, the masks and the lazily rescaled
// log2-domain softmax are attention_v3_kernel's. One 16-query tile per wave, the G query heads
// of one KV head as the workgroup's G waves: a wave's q_hi and q_lo fragments (16 x 512 each)
// and its 16 x 512 output accumulators take 256 registers, so a SIMD runs one wave. LDS holds
// K_hi and K_lo of a 32-key block in two stages (block it + 1 copies while block it is used)
// and V^T of one block in one buffer, refilled after the P.V product while the next block's
// scores are computed: 2 x 64 KB + 32 KB at head dim 512, 2 x 32 KB + 16 KB at head dim 256 (three
// query heads per KV head there, for contexts that ask for split scores on every layer).
namespace attns {
constexpr int BKV = 32;  // keys per block
}  // namespace attns

template <int HD>
constexpr int attention_split_lds_bytes() { return 2 * (2 * attns::BKV * HD * 2) + attns::BKV * HD * 2; }

template <int HD, int G>
__global__ __launch_bounds__(G * 64) void attention_split_kernel(const uint16_t* __restrict__ Qg,
                                                                 const uint16_t* __restrict__ QLg,
                                                                 const uint16_t* __restrict__ Kg,
                                                                 const uint16_t* __restrict__ KLg,
                                                                 const uint16_t* __restrict__ VTg,
                                                                 uint16_t* __restrict__ Og,
                                                                 const AttnWork* __restrict__ work, int H, int KV,
                                                                 int vt_cols, int hw, float scale_log2) {
    constexpr int BKV = attns::BKV, KS = HD / 32, DT = HD / 16;
    constexpr int K_BYTES = BKV * HD * 2;  // one plane (K_hi or K_lo) of a block
    constexpr int KCH = K_BYTES / 1024;    // its chunks (ks, m)
    constexpr int KSTAGE = 2 * K_BYTES;    // K_hi, then K_lo
    // copies per wave per block (K planes, V^T), rounded up: where G does not divide the chunk
    // count, a wave past the last chunk repeats its own previous chunk (same data, same wave), so
    // every wave issues the same number of copies and the vmcnt waits below hold for each
    constexpr int KPW = (2 * KCH + G - 1) / G, VPW = (DT + G - 1) / G;
    static_assert(KCH == 2 * KS && 2 * KCH >= G && DT >= G, "chunk counts");
    static_assert(KPW + VPW < 64 && KS * 2 + KPW + VPW < 64, "outstanding copies fit the vmcnt counter");
    extern __shared__ __attribute__((aligned(1024))) unsigned char ldss[];
    unsigned char* const vbuf = ldss + 2 * KSTAGE;

    // XCD-aware order, as in attention_v2_kernel.
    const int nb = int(gridDim.x), full = nb / 8 * 8, bx = int(blockIdx.x);
    const int widx = bx < full ? (bx % 8) * (full / 8) + bx / 8 : bx;
    const int seq_start = __builtin_amdgcn_readfirstlane(int(work[widx].seq_start));
    const int len = __builtin_amdgcn_readfirstlane(int(work[widx].seq_len));
    // A work item of an empty sequence has nothing to attend; leaving before any access also keeps
    // the (len - 1) in the buffer ranges and row clamps below from wrapping around.
    if (len <= 0) return;
    const int q0 = __builtin_amdgcn_readfirstlane(int(work[widx].q0)) + int(blockIdx.z) * 16;
    const int vt_start = __builtin_amdgcn_readfirstlane(int(work[widx].vt_start));
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int h = kvh * G + wave;
    const int l16 = lane & 15, g4 = lane >> 4;
    const int qi = q0 + l16;
    const int qStride = H * HD, kvStride = KV * HD;

    int kstart = 0, kend = len;
    if (hw > 0) {
        kstart = max(q0 - hw, 0);
        kend = min(q0 + 16 + hw, len);
    }
    kstart = kstart / BKV * BKV;
    const int nblocks = (kend - kstart + BKV - 1) / BKV;

    // Buffer resources over the sequence's rows (reads past them return zeros).
    const uint32_t kbytes = uint32_t(((len - 1) * kvStride + HD) * 2);
    const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(Kg + (size_t)seq_start * kvStride + kvh * HD, kbytes);
    const __amdgpu_buffer_rsrc_t klr = buffer_rsrc(KLg + (size_t)seq_start * kvStride + kvh * HD, kbytes);
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(VTg + (size_t)kvh * HD * vt_cols + vt_start,
                                                  uint32_t(((HD - 1) * vt_cols + (vt_cols - vt_start)) * 2));
    const uint32_t klane = uint32_t(((8 * (l16 >> 2) + (lane & 3)) * kvStride + 8 * g4) * 2);
    const uint32_t vlane = uint32_t((l16 * vt_cols + 8 * g4) * 2);
    // K chunk c of a block: plane c / KCH (hi, lo), (ks, m) = (c % KCH / 2, c % 2); wave w copies
    // chunks w, w + G, ...; V^T chunk dt likewise.
#define AS_KISSUE(kb, b)                                                                                   \
    do {                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < KPW; i++) {                                                  \
            const int c0 = wave + i * G, c = c0 < 2 * KCH ? c0 : c0 - G, pl = c / KCH, cc = c % KCH;       \
            lds_copy16(pl ? klr : kr, ldss + (b) * KSTAGE + pl * K_BYTES + cc * 1024,                      \
                       klane + uint32_t(((kb) + 4 * (cc & 1)) * kvStride * 2 + (cc >> 1) * 64), 0);        \
        }                                                                                                  \
    } while (0)
#define AS_VISSUE(kb)                                                                                      \
    do {                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < VPW; i++) {                                                  \
            const int c0 = wave + i * G, c = c0 < DT ? c0 : c0 - G;                                        \
            lds_copy16(vr, vbuf + c * 1024, vlane + uint32_t(c * 16 * vt_cols * 2 + (kb) * 2), 0);        \
        }                                                                                                  \
    } while (0)

    // This wave's query fragments, hi and lo (B operands of S^T = K Q^T): lane l: query qi (rows
    // past the sequence re-read its last row; their outputs are never stored), head dims
    // 32 ks + 8 (l / 16).
    half8_t qh[KS], ql[KS];
    {
        const uint32_t qbytes = uint32_t(((len - 1) * qStride + HD) * 2);
        const __amdgpu_buffer_rsrc_t qr = buffer_rsrc(Qg + (size_t)seq_start * qStride + h * HD, qbytes);
        const __amdgpu_buffer_rsrc_t qlr = buffer_rsrc(QLg + (size_t)seq_start * qStride + h * HD, qbytes);
        const uint32_t qo = uint32_t((min(qi, len - 1) * qStride + 8 * g4) * 2);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            qh[ks] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(qr, qo + ks * 64, 0, 0));
            ql[ks] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(qlr, qo + ks * 64, 0, 0));
        }
    }

    float4_t o[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) o[i] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    if (nblocks > 0) {
        AS_KISSUE(kstart, 0);
        AS_VISSUE(kstart);
    }
    for (int it = 0; it < nblocks; it++) {
        const int kb = kstart + it * BKV, b = it & 1;
        const bool more = it + 1 < nblocks;
        // K(it) has landed once only V(it)'s copies (issued after it) may be in flight; the
        // barrier covers every wave's copies and frees the other K stage (read in block it - 1).
        wait_vmcnt<VPW>();
        wait_lgkmcnt0();
        workgroup_barrier();
        if (more) AS_KISSUE(kb + BKV, b ^ 1);
        const unsigned char* const kf = ldss + b * KSTAGE + lane * 16;
        // S^T tiles m = 0, 1: the hi.hi products in one chain, the two correction products in
        // another; K fragments (hi and lo) read PF k-steps ahead
        constexpr int PF = 2, RING = PF + 1;
        float4_t s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0, c0 = s0, c1 = s0;
        half8_t kh[RING][2], kl[RING][2];
#pragma unroll
        for (int f = 0; f < PF; f++)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                kh[f][m] = *reinterpret_cast<const half8_t*>(kf + (2 * f + m) * 1024);
                kl[f][m] = *reinterpret_cast<const half8_t*>(kf + K_BYTES + (2 * f + m) * 1024);
            }
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks + PF < KS)
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    kh[(ks + PF) % RING][m] = *reinterpret_cast<const half8_t*>(kf + (2 * (ks + PF) + m) * 1024);
                    kl[(ks + PF) % RING][m] = *reinterpret_cast<const half8_t*>(kf + K_BYTES + (2 * (ks + PF) + m) * 1024);
                }
            __builtin_amdgcn_sched_barrier(0);
            const int r = ks % RING;
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[r][0], qh[ks], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[r][1], qh[ks], s1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[r][0], ql[ks], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[r][1], ql[ks], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl[r][0], qh[ks], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl[r][1], qh[ks], c1, 0, 0, 0);
        }
        s0 += c0;
        s1 += c1;
        // this lane's scores: keys kb + 8 g4 + e, e = 0..7
        float sc[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        const bool inside = kb + BKV <= len && (hw == 0 || (kb >= q0 + 15 - hw && kb + BKV - 1 <= q0 + hw));
        if (!inside) {
            const int lim = hw > 0 ? hw : 1 << 30;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int key = kb + 8 * g4 + e;
                const bool valid = (key < len) & (abs(qi - key) <= lim);
                sc[e] = valid ? sc[e] : -INFINITY;
            }
        }
        const float lmax =
            fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
        // lazy rescaling, as in attention_v3_kernel
        if (__builtin_amdgcn_ballot_w64(lmax * scale_log2 > m_run + 8.0f)) {
            const float bmax = max_over_key_groups(lmax) * scale_log2;
            const float m_new = fmaxf(m_run, bmax);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < DT; i++) o[i] *= alpha;
            m_run = m_new;
        }
        const float m_ref = m_run == -INFINITY ? 0.0f : m_run;
        float sum = 0.0f;
        half8_t pb;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], scale_log2, -m_ref));
            sum += p;
            pb[e] = _Float16(p);
        }
        l_run += sum;
        // V(it) has landed once only K(it + 1)'s copies may be in flight.
        if (more)
            wait_vmcnt<KPW>();
        else
            wait_vmcnt<0>();
        wait_lgkmcnt0();
        workgroup_barrier();
        const unsigned char* const vf = vbuf + lane * 16;
        half8_t va[RING];
#pragma unroll
        for (int f = 0; f < PF; f++) va[f] = *reinterpret_cast<const half8_t*>(vf + f * 1024);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            if (dt + PF < DT) va[(dt + PF) % RING] = *reinterpret_cast<const half8_t*>(vf + (dt + PF) * 1024);
            __builtin_amdgcn_sched_barrier(0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt % RING], pb, o[dt], 0, 0, 0);
        }
        if (more) {
            // every wave's V^T reads are done before the buffer is refilled
            wait_lgkmcnt0();
            workgroup_barrier();
            AS_VISSUE(kb + BKV);
        }
    }
#undef AS_KISSUE
#undef AS_VISSUE
    wait_vmcnt<0>();
    l_run = sum_over_key_groups(l_run);
    if (qi >= len) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    _Float16* op = reinterpret_cast<_Float16*>(Og) + (size_t)(seq_start + qi) * qStride + h * HD + 4 * g4;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        half4_t v4;
#pragma unroll
        for (int r = 0; r < 4; r++) v4[r] = _Float16(o[dt][r] * inv);
        *reinterpret_cast<half4_t*>(op + dt * 16) = v4;
    }
}

bool attention_split_supported(int hd, int H, int KV) {
    return KV > 0 && ((hd == 512 && H == 4 * KV) || (hd == 256 && H == 3 * KV));
}

hipError_t launch_attention_split(hipStream_t s, const uint16_t* q, const uint16_t* q_lo, const uint16_t* k,
                                  const uint16_t* k_lo, const uint16_t* vt, int vt_cols, uint16_t* o, const AttnWork* work,
                                  int n_work, int H, int KV, int hd, int half_window, float scale, int item_queries) {
    if (n_work < 0 || !attention_split_supported(hd, H, KV) || half_window < 0 || vt_cols <= 0 || vt_cols % 8 ||
        (item_queries != 16 && item_queries != 32 && item_queries != 64) || !q || !q_lo || !k || !k_lo || !vt || !o || !work)
        return hipErrorInvalidValue;
    if (n_work == 0) return hipSuccess;
    const float scale_log2 = scale * 1.4426950408889634f;
    const dim3 grid(n_work, KV, item_queries / 16);
    if (hd == 512)
        launch_kernel(attention_split_kernel<512, 4>, grid, dim3(4 * 64), uint32_t(attention_split_lds_bytes<512>()), s, q, q_lo,
                      k, k_lo, vt, o, work, H, KV, vt_cols, half_window, scale_log2);
    else
        launch_kernel(attention_split_kernel<256, 3>, grid, dim3(3 * 64), uint32_t(attention_split_lds_bytes<256>()), s, q, q_lo,
                      k, k_lo, vt, o, work, H, KV, vt_cols, half_window, scale_log2);
    return hipGetLastError();
}

// The image tower's attention: one query head per KV head, no window, heads stored padded (HD
// dims of which the first HO are real). Each wave owns 32 queries of one head on
// v_mfma_f32_32x32x16_f16: on gfx950 the 16x16x32 form issues no faster than this one (14.3
// against 14.8 ns per instruction per SIMD in a register-only loop), so these 32x32 tiles do twice
// the work per MFMA cycle. S^T = K Q^T over HS dims (the real HO rounded up to 16: 80 for 72, where
// 16x16x32 steps needed 96), O^T = V^T P^T over the stored HD dims in 32-dim tiles.
//
// LDS per block of 32 keys, filled by coalesced copies (each copy instruction reads whole key rows
// of K and whole key runs of V^T, not one 16-byte piece of 64 rows; with 16-byte pieces per row the
// texture units' return path was busy 78% of the kernel):
//   K: key-major rows of HS / 8 + 1 16-byte pieces (the last a pad, never read; the odd row
//     stride makes the fragment reads conflict-free). The S^T MFMA's A operand for k-step ks is
//     lane l: key pi(l % 32), piece 2 ks + l / 32, where pi swaps the 4s and 8s bits of the row.
//     With that key order, register r of a lane's S^T tile holds key 16 (r / 8) + 8 (l / 32) + r % 8
//     of query l % 32, so registers 8 t .. 8 t + 7 are the B operand of the P.V k-step t (keys
//     16 t + 8 (l / 32) + [0, 8)) with no data exchange;
//   V^T: dim-major rows of 5 pieces (32 keys, a pad) for the HO real dims. The P.V MFMA's A operand
//     (dt, t) is lane l: dim 32 dt + l % 32, piece 2 t + l / 32. Dims HO .. HD - 1 come from a
//     constant area written once: zeros, except dim HO, all ones, so that row HO of O^T is the sum
//     of the fp16 P the products used, the softmax denominator, with no VALU additions.
// A query's 32 scores of a block sit in lanes q and q + 32: its block max is one lane swap.
__device__ __forceinline__ float max_over_lane_halves(float v) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_over_lane_halves(float v) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

namespace attnp {
constexpr int NS = 2;    // key blocks in LDS
constexpr int BKV = 32;  // keys per block
}  // namespace attnp

// Pieces per K row and per V^T row, and the 1 KB chunks a block's copies fill.
template <int HS>
constexpr int mq_k_chunks() { return (attnp::BKV * (HS / 8 + 1) + 63) / 64; }
template <int HO>
constexpr int mq_v_chunks() { return (HO * (attnp::BKV / 8 + 1) + 63) / 64; }
template <int HD, int HS, int HO>
constexpr int attention_mq_lds_bytes() {
    return attnp::NS * (mq_k_chunks<HS>() + mq_v_chunks<HO>()) * 1024 + (HD - HO) * (attnp::BKV / 8 + 1) * 16;
}

template <int HD, int HS, int QW, int HO>
__global__ __launch_bounds__(QW * 64) void attention_mq_kernel(const uint16_t* __restrict__ Qg,
                                                               const uint16_t* __restrict__ Kg,
                                                               const uint16_t* __restrict__ VTg,
                                                               uint16_t* __restrict__ Og,
                                                               const AttnWork* __restrict__ work, int H, int vt_cols,
                                                               float scale_log2) {
    using namespace attnp;
    constexpr int KSS = HS / 16, DT = HD / 32;
    constexpr int KP = HS / 8 + 1, KPIECES = BKV * KP, KCH = mq_k_chunks<HS>();
    constexpr int VP = BKV / 8 + 1, VPIECES = HO * VP, VCH = mq_v_chunks<HO>();
    constexpr int CH = KCH + VCH, STAGE = CH * 1024, VOFF = KCH * 1024;
    constexpr int CPW = (CH + QW - 1) / QW;  // copies per wave per block (some waves repeat one)
    constexpr int CONST_OFF = NS * STAGE, CONST_BYTES = (HD - HO) * VP * 16;
    static_assert(HO <= HS && HS <= HD && HS % 16 == 0 && HD % 32 == 0 && HO % 32 == 8, "head dims (row sum in register 4)");
    static_assert(QW <= CH, "a wave past the last chunk repeats its own chunk index");
    extern __shared__ __attribute__((aligned(1024))) unsigned char ldsm[];

    const int nb = int(gridDim.x), full = nb / 8 * 8, bx = int(blockIdx.x);
    const int widx = bx < full ? (bx % 8) * (full / 8) + bx / 8 : bx;
    const int seq_start = __builtin_amdgcn_readfirstlane(int(work[widx].seq_start));
    const int len = __builtin_amdgcn_readfirstlane(int(work[widx].seq_len));
    // A work item of an empty sequence has nothing to attend; leaving before any access also keeps
    // the (len - 1) in the buffer ranges and row clamps below from wrapping around.
    if (len <= 0) return;
    const int wq0 = __builtin_amdgcn_readfirstlane(int(work[widx].q0));
    const int vt_start = __builtin_amdgcn_readfirstlane(int(work[widx].vt_start));
    const int h = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int l32 = lane & 31, hi = lane >> 5;
    const int q0 = wq0 + wave * 32, qi = q0 + l32;
    const int stride = H * HD;
    const int nblocks = (len + BKV - 1) / BKV;

    // Keys past the sequence read as zeros (the resource ends at its last row); their scores are
    // masked below.
    const __amdgpu_buffer_rsrc_t kr =
        buffer_rsrc(Kg + (size_t)seq_start * stride + h * HD, uint32_t(((len - 1) * stride + HD) * 2));
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(VTg + (size_t)h * HD * vt_cols + vt_start,
                                                  uint32_t(((HD - 1) * vt_cols + (vt_cols - vt_start)) * 2));
    // This wave's chunks and each lane's source at block 0: piece p of the block's K rows or V^T
    // rows; a pad piece (and a lane past the last piece) re-reads its row's first piece into a
    // place no fragment read touches.
    uint32_t src[CPW];
    int chk[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        int c = wave + i * QW;
        if (c >= CH) c = wave;
        chk[i] = c;
        if (c < KCH) {
            const int pz = c * 64 + lane, key = pz < KPIECES ? pz / KP : 0, pc = pz < KPIECES ? pz % KP : 0;
            src[i] = uint32_t((key * stride + 8 * (pc < KP - 1 ? pc : 0)) * 2);
        } else {
            const int pz = (c - KCH) * 64 + lane, dim = pz < VPIECES ? pz / VP : 0, pc = pz < VPIECES ? pz % VP : 0;
            src[i] = uint32_t((dim * vt_cols + 8 * (pc < VP - 1 ? pc : 0)) * 2);
        }
    }
#define MQ_ISSUE(kb, b)                                                                                    \
    do {                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < CPW; i++) {                                                  \
            unsigned char* dst_ = ldsm + (b) * STAGE + chk[i] * 1024;                                      \
            if (chk[i] < KCH) lds_copy16(kr, dst_, src[i] + uint32_t((kb) * stride * 2), 0);               \
            else lds_copy16(vr, dst_, src[i] + uint32_t((kb) * 2), 0);                                     \
        }                                                                                                  \
    } while (0)

    // the constant V^T rows HO .. HD - 1 (ones in row HO, keys and pad), read after the first barrier
    for (int i = int(threadIdx.x); i < CONST_BYTES / 4; i += QW * 64)
        reinterpret_cast<uint32_t*>(ldsm + CONST_OFF)[i] = i < VP * 4 ? 0x3c003c00u : 0u;

    // This wave's query fragments (B operand of S^T = K Q^T): lane l: query qi (rows past the
    // sequence re-read its last row; their outputs are never stored), dims 16 ks + 8 (l / 32).
    half8_t qa[KSS];
    {
        const __amdgpu_buffer_rsrc_t qr =
            buffer_rsrc(Qg + (size_t)seq_start * stride + h * HD, uint32_t(((len - 1) * stride + HD) * 2));
        const uint32_t qo = uint32_t((min(qi, len - 1) * stride + 8 * hi) * 2);
#pragma unroll
        for (int ks = 0; ks < KSS; ks++)
            qa[ks] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(qr, qo + ks * 32, 0, 0));
    }
    // fragment offsets in a block's buffer: K (key pi(l % 32), piece hi), V^T (dim 32 dt + l % 32,
    // piece hi; dims past HO in the constant area, offsets from the start of LDS)
    const int krow = (l32 & 16) | ((l32 & 4) << 1) | ((l32 & 8) >> 1) | (l32 & 3);  // pi(l % 32)
    const int koff = (krow * KP + hi) * 16;
    int voff[DT];
    bool vconst[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        const int dim = 32 * dt + l32;
        vconst[dt] = dim >= HO;
        voff[dt] = dim < HO ? VOFF + (dim * VP + hi) * 16 : CONST_OFF + ((dim - HO) * VP + hi) * 16;
    }
    float16_t o[DT];
#pragma unroll
    for (int i = 0; i < DT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    float m_run = -INFINITY;

    MQ_ISSUE(0, 0);
    int b = 0;
    for (int it = 0; it < nblocks; it++) {
        const int kb = it * BKV;
        // block it has landed (every wave's copies: the barrier), and every wave is done reading
        // the buffer the next copies overwrite
        wait_vmcnt<0>();
        wait_lgkmcnt0();
        workgroup_barrier();
        if (it + 1 < nblocks) MQ_ISSUE(kb + BKV, b ^ 1);
        const unsigned char* const kb_lds = ldsm + b * STAGE;
        float16_t s;
#pragma unroll
        for (int r = 0; r < 16; r++) s[r] = 0.0f;
        half8_t ka[KSS];
#pragma unroll
        for (int f = 0; f < KSS; f++) ka[f] = *reinterpret_cast<const half8_t*>(kb_lds + koff + f * 32);
#pragma unroll
        for (int ks = 0; ks < KSS; ks++) {
            // keep the reads ahead of the MFMAs (the scheduler would otherwise sink them)
            __builtin_amdgcn_sched_barrier(0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks], qa[ks], s, 0, 0, 0);
        }
        // the V^T fragments are read while the softmax runs
        half8_t va[DT * 2];
#pragma unroll
        for (int f = 0; f < DT * 2; f++) {
            const int dt = f >> 1, t = f & 1;
            va[f] = *reinterpret_cast<const half8_t*>((vconst[dt] ? ldsm : kb_lds) + voff[dt] + t * 32);
        }
        // register r: key kb + 16 (r / 8) + 8 (l / 32) + r % 8 of query qi
        float sc[16];
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = s[r];
        if (kb + BKV > len) {
#pragma unroll
            for (int r = 0; r < 16; r++) sc[r] = kb + 16 * (r >> 3) + 8 * hi + (r & 7) < len ? sc[r] : -INFINITY;
        }
        float lmax = sc[0];
#pragma unroll
        for (int r = 1; r < 16; r++) lmax = fmaxf(lmax, sc[r]);
        // lazy rescaling, as in attention_v3_kernel: the reference point moves only when a score
        // exceeds it by more than 2^8, so P stays below 256; rescaling O^T rescales its row-sum row
        if (__builtin_amdgcn_ballot_w64(lmax * scale_log2 > m_run + 8.0f)) {
            const float bmax = max_over_lane_halves(lmax) * scale_log2;
            const float m_new = fmaxf(m_run, bmax);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
            for (int i = 0; i < DT; i++) o[i] *= alpha;
            m_run = m_new;
        }
        const float m_ref = m_run == -INFINITY ? 0.0f : m_run;
        half8_t pb[2];
#pragma unroll
        for (int r = 0; r < 16; r++)
            pb[r >> 3][r & 7] = _Float16(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, -m_ref)));
        // O^T += V^T P^T: 32-dim tiles dt, the block's keys as two k-steps t of 16
#pragma unroll
        for (int f = 0; f < DT * 2; f++) {
            const int dt = f >> 1, t = f & 1;
            __builtin_amdgcn_sched_barrier(0);
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[f], pb[t], o[dt], 0, 0, 0);
        }
        b ^= 1;
    }
#undef MQ_ISSUE
    wait_vmcnt<0>();
    // o[dt] register 4 g + e: dim 32 dt + 8 g + 4 (l / 32) + e of query qi, so the row sum (dim HO,
    // register 4 of tile HO / 32) sits in lane qi % 32
    const float lsum = __shfl(o[HO / 32][4], l32, 64);
    if (qi >= len) return;
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    // outputs [rows][H][HO]
    _Float16* op = reinterpret_cast<_Float16*>(Og) + (size_t)(seq_start + qi) * (H * HO) + h * HO + 4 * hi;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            if (32 * dt + 8 * g >= HO) continue;
            half4_t v4;
#pragma unroll
            for (int e = 0; e < 4; e++) v4[e] = _Float16(o[dt][4 * g + e] * inv);
            *reinterpret_cast<half4_t*>(op + 32 * dt + 8 * g) = v4;
        }
}

bool attention_padded_supported(int hp, int hd, int H, int KV) { return hp == 96 && hd == 72 && H > 0 && KV == H; }

hipError_t launch_attention_padded(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, int vt_cols,
                                   uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hp, int hd,
                                   int half_window, float scale, int item_queries) {
    if (n_work < 0 || !attention_padded_supported(hp, hd, H, KV) || half_window != 0 || vt_cols <= 0 || vt_cols % 8 ||
        (item_queries != 64 && item_queries != 256))
        return hipErrorInvalidValue;
    if (n_work == 0) return hipSuccess;
    const float scale_log2 = scale * 1.4426950408889634f;
    // 256-query items: eight waves of 32 queries share each K/V block copied into LDS; 64-query
    // items (small batches): two
    constexpr uint32_t lds = uint32_t(attention_mq_lds_bytes<96, 80, 72>());
    if (item_queries == 256)
        launch_kernel(attention_mq_kernel<96, 80, 8, 72>, dim3(n_work, KV), dim3(8 * 64), lds, s, q, k, vt, o, work, H, vt_cols,
                      scale_log2);
    else
        launch_kernel(attention_mq_kernel<96, 80, 2, 72>, dim3(n_work, KV), dim3(2 * 64), lds, s, q, k, vt, o, work, H, vt_cols,
                      scale_log2);
    return hipGetLastError();
}

// V [T][KV][hd] fp16 -> V^T [KV * hd][vt_cols] at column vcol[t]. A workgroup transposes 64
// tokens through LDS: reads are 16-byte row pieces, writes are one d row of 64 tokens per wave
// instruction (consecutive columns within a sequence).
__global__ __launch_bounds__(256) void v_transpose_kernel(const uint16_t* __restrict__ v, int T, int width,
                                                          const int32_t* __restrict__ vcol, int vt_cols,
                                                          uint16_t* __restrict__ vt) {
    __shared__ uint16_t tile[64][64 + 2];
    const int t0 = blockIdx.x * 64, c0 = blockIdx.y * 64, tid = threadIdx.x;
    for (int i = tid; i < 64 * 8; i += 256) {
        const int r = i / 8, cc = (i % 8) * 8;
        if (t0 + r < T) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(v + (size_t)(t0 + r) * width + c0 + cc);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                tile[r][cc + 2 * j] = uint16_t(w[j] & 0xffffu);
                tile[r][cc + 2 * j + 1] = uint16_t(w[j] >> 16);
            }
        }
    }
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6;
    if (t0 + lane >= T) return;
    const int col = vcol[t0 + lane];
    for (int d = wave; d < 64; d += 4) vt[(size_t)(c0 + d) * vt_cols + col] = tile[lane][d];
}

hipError_t launch_v_transpose(hipStream_t s, const uint16_t* v, int T, int width, const int32_t* vcol, int vt_cols,
                              uint16_t* vt) {
    if (T < 0 || width <= 0 || width % 64 || !v || !vcol || !vt) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    launch_kernel(v_transpose_kernel, dim3((T + 63) / 64, width / 64), dim3(256), 0, s, v, T, width, vcol, vt_cols, vt);
    return hipGetLastError();
}

static size_t attention_lds_bytes(int hd, int ds, bool pipe) {
    return (size_t)(pipe ? 2 : 1) * (attn::BKV * (hd + 8) + ds * attn::LDV) * sizeof(_Float16);
}

template <int HD, int DS, int G>
static hipError_t attention_configure() {
    constexpr bool pipe = G < attn::WAVES && HD <= 256;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<HD, DS, G>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(attention_lds_bytes(HD, DS, pipe)));
}

template <int HD, int DS>
static hipError_t attention_configure_all() {
    hipError_t e = attention_configure<HD, DS, 1>();
    if (e == hipSuccess) e = attention_configure<HD, DS, 2>();
    if (e == hipSuccess) e = attention_configure<HD, DS, 3>();
    if (e == hipSuccess) e = attention_configure<HD, DS, 4>();
    return e;
}

template <int HD, int G>
static hipError_t attention_v2_configure() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_v2_kernel<HD, G>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, attention_v2_lds_bytes<HD, G>());
}

template <int HD, int G>
static hipError_t attention_v3_configure() {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_v3_kernel<HD, G, 4>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, attention_v3_lds_bytes<HD>());
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_v3_kernel<HD, G, 2>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, attention_v3_lds_bytes<HD>());
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_v3_kernel<HD, G, 4, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, attention_v3_lds_bytes<HD>());
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_v3_kernel<HD, G, 2, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, attention_v3_lds_bytes<HD>());
    return e;
}

hipError_t configure_kernels() {
    hipError_t e = gemm_configure();
    if (e == hipSuccess) e = attention_configure_all<128, 128>();
    if (e == hipSuccess) e = attention_v2_configure<128, 1>();
    if (e == hipSuccess) e = attention_v2_configure<128, 2>();
    if (e == hipSuccess) e = attention_v2_configure<128, 3>();
    if (e == hipSuccess) e = attention_v2_configure<128, 4>();
    if (e == hipSuccess) e = attention_v2_configure<256, 1>();
    if (e == hipSuccess) e = attention_v2_configure<256, 2>();
    if (e == hipSuccess) e = attention_v2_configure<256, 3>();
    if (e == hipSuccess) e = attention_v3_configure<128, 1>();
    if (e == hipSuccess) e = attention_v3_configure<128, 2>();
    if (e == hipSuccess) e = attention_v3_configure<128, 3>();
    if (e == hipSuccess) e = attention_v3_configure<256, 1>();
    if (e == hipSuccess) e = attention_v3_configure<256, 2>();
    if (e == hipSuccess) e = attention_v3_configure<256, 3>();
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_v3_kernel<512, 4, 2>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, attention_v3_lds_bytes<512>());
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_split_kernel<512, 4>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, attention_split_lds_bytes<512>());
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_split_kernel<256, 3>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, attention_split_lds_bytes<256>());
    if (e == hipSuccess) e = attention_configure_all<256, 256>();
    if (e == hipSuccess) e = attention_configure_all<512, 256>();
    return e;
}

template <int HD, int DS, int G>
static hipError_t attention_dispatch(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hw,
                                     float scale) {
    constexpr bool pipe = G < attn::WAVES && HD <= 256;
    const size_t lds = attention_lds_bytes(HD, DS, pipe);
    dim3 grid(n_work, KV, HD / DS);
    const float scale_log2 = scale * 1.4426950408889634f;
    launch_kernel(attention_kernel<HD, DS, G>, grid, 64 * attn::WAVES, lds, s, q, k, v, o, work, H, KV, hw, scale_log2);
    return hipGetLastError();
}

template <int HD, int DS>
static hipError_t attention_dispatch_g(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hw,
                                       float scale) {
    switch (H / KV) {
    case 1: return attention_dispatch<HD, DS, 1>(s, q, k, v, o, work, n_work, H, KV, hw, scale);
    case 2: return attention_dispatch<HD, DS, 2>(s, q, k, v, o, work, n_work, H, KV, hw, scale);
    case 3: return attention_dispatch<HD, DS, 3>(s, q, k, v, o, work, n_work, H, KV, hw, scale);
    case 4: return attention_dispatch<HD, DS, 4>(s, q, k, v, o, work, n_work, H, KV, hw, scale);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attention(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                            const AttnWork* work, int n_work, int H, int KV, int hd, int half_window, float scale) {
    if (n_work < 0 || H <= 0 || KV <= 0 || H % KV != 0 || H / KV > attn::WAVES || half_window < 0)
        return hipErrorInvalidValue;
    if (n_work == 0) return hipSuccess;
    switch (hd) {
    case 128: return attention_dispatch_g<128, 128>(s, q, k, v, o, work, n_work, H, KV, half_window, scale);
    case 256: return attention_dispatch_g<256, 256>(s, q, k, v, o, work, n_work, H, KV, half_window, scale);
    case 512: return attention_dispatch_g<512, 256>(s, q, k, v, o, work, n_work, H, KV, half_window, scale);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ge
