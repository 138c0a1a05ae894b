/*
 * CPU oracle for the GemmaEmbed text-encoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C fp32 restatement of
 * /root/reference/Sources/GemmaEmbed/Model/CPUReference.swift, the reference's own oracle,
 * with its GGUF reading (GGUF/GGUFFile.swift), configuration (Model/ModelConfig.swift),
 * weights (Model/Weights.swift) and RoPE table (Model/RopeTable.swift). It is the checker of
 * the HIP path and the CPU baseline, never part of the product.
 *
 * Deliberate differences from the reference, each with its reason:
 *  - vDSP_mmul / vDSP_mtrans (Apple Accelerate) are replaced by a blocked fp32 dot-product
 *    matmul. The fp32 summation order of vDSP is not published, so it is not reproduced.
 *  - Attention is computed one query row at a time (scores, mask, softmax, P.V) rather than as
 *    a T x T matrix product; the arithmetic per row is the reference's.
 *  - RoPE tables are keyed by (head dim, base). The reference keys them by head dim alone
 *    (CPUReference.swift:21-28), which is the same thing on its model, where the two layer
 *    kinds differ in head dim; on a model whose layer kinds share a head dim, keying by base too
 *    gives each layer kind its own base (rope.freq_base vs rope.freq_base_swa).
 *  - The per-layer-input (PLE) branch is optional: without `per_layer_model_proj.weight` the
 *    lines CPUReference.swift:206-210 and :259-268 are skipped and the layer output is
 *    `x * layer_output_scale` (1 when that tensor is absent).
 */
#define _GNU_SOURCE
#include "ge_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define ORA_MAX_LAYERS 64
#define ORA_MAX_TOKENS 8192 /* ModelConfig.swift:52 */

/* ---------------------------------------------------------------- fp16 / bf16 */

/* IEEE 754 binary16 -> binary32, exact (Weights.swift:27,37 use Float(Float16(bitPattern:))). */
float ora_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (used by the test-side generator checks). */
uint16_t ora_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0));
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
    if (absx < 0x38800000u) {                                    /* result subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign;           /* < 2^-25 rounds to 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* 14 - (e - 127) + 13 - 1 ... value = m * 2^(e-150); unit 2^-24 */
        /* number of half ulps: m * 2^(e - 150 + 24) = m >> (126 - e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 127 + 15;
    uint32_t m = absx & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

/* Weights.swift:19-43: one row of a tensor widened to fp32. Q8_0 blocks are an fp16 scale
 * followed by 32 int8 values (34 bytes); element = scale * q. */
void ora_dequant_row(int type, const void* row, int cols, float* out) {
    const uint8_t* p = (const uint8_t*)row;
    switch (type) {
    case ORA_F32:
        memcpy(out, p, (size_t)cols * 4);
        break;
    case ORA_F16:
        for (int i = 0; i < cols; i++) out[i] = ora_half_to_float((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
        break;
    case ORA_BF16:
        for (int i = 0; i < cols; i++) {
            uint32_t bits = (uint32_t)(p[2 * i] | (p[2 * i + 1] << 8)) << 16;
            memcpy(&out[i], &bits, 4);
        }
        break;
    case ORA_Q8_0:
        for (int b = 0; b < cols / 32; b++) {
            const uint8_t* bp = p + (size_t)b * 34;
            float scale = ora_half_to_float((uint16_t)(bp[0] | (bp[1] << 8)));
            for (int j = 0; j < 32; j++) out[b * 32 + j] = scale * (float)(int8_t)bp[2 + j];
        }
        break;
    default:
        memset(out, 0, (size_t)cols * 4);
    }
}

/* ---------------------------------------------------------------- primitives */

typedef float v8f __attribute__((vector_size(32)));

static inline float hsum8(v8f v) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

/* CPUReference.swift:63-74 (vDSP_mmul over a transposed weight): y[M,N] = x[M,K] * W[N,K]^T,
 * fp32 products and sums. Here W stays [N][K] (the reference transposes it so vDSP can read it
 * column-major; the product is the same). Each output is 8 interleaved fp32 partial sums over K
 * followed by a fixed-order combine, so the result does not depend on the thread count. */
void ora_matmul(const float* x, int m, int k, const float* w, int n, float* y, int threads) {
    const int kv = k / 8 * 8;
    if (threads <= 0) threads = omp_get_max_threads();
    const int RB = 4, CB = 4;
    const int mb = (m + RB - 1) / RB, nb = (n + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads)
    for (long t = 0; t < (long)mb * nb; t++) {
        const int r0 = (int)(t / nb) * RB, c0 = (int)(t % nb) * CB;
        const int rn = r0 + RB <= m ? RB : m - r0, cn = c0 + CB <= n ? CB : n - c0;
        if (rn == RB && cn == CB) {
            v8f acc[4][4];
            memset(acc, 0, sizeof(acc));
            for (int kk = 0; kk < kv; kk += 8) {
                v8f xv[4], wv[4];
                for (int i = 0; i < 4; i++) memcpy(&xv[i], x + (size_t)(r0 + i) * k + kk, 32);
                for (int j = 0; j < 4; j++) memcpy(&wv[j], w + (size_t)(c0 + j) * k + kk, 32);
                for (int i = 0; i < 4; i++)
                    for (int j = 0; j < 4; j++) acc[i][j] += xv[i] * wv[j];
            }
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 4; j++) {
                    float s = hsum8(acc[i][j]);
                    for (int kk = kv; kk < k; kk++) s += x[(size_t)(r0 + i) * k + kk] * w[(size_t)(c0 + j) * k + kk];
                    y[(size_t)(r0 + i) * n + c0 + j] = s;
                }
        } else {
            for (int i = 0; i < rn; i++)
                for (int j = 0; j < cn; j++) {
                    v8f acc = {0, 0, 0, 0, 0, 0, 0, 0};
                    const float* xr = x + (size_t)(r0 + i) * k;
                    const float* wr = w + (size_t)(c0 + j) * k;
                    for (int kk = 0; kk < kv; kk += 8) {
                        v8f a, b;
                        memcpy(&a, xr + kk, 32);
                        memcpy(&b, wr + kk, 32);
                        acc += a * b;
                    }
                    float s = hsum8(acc);
                    for (int kk = kv; kk < k; kk++) s += xr[kk] * wr[kk];
                    y[(size_t)(r0 + i) * n + c0 + j] = s;
                }
        }
    }
}

/* CPUReference.swift:77-90: out = x * inv * w with inv = 1 / sqrt(mean(x^2) + eps), the sum of
 * squares accumulated in order. prescale multiplies x first (the GPU kernels' preScale,
 * Shaders/Elementwise.metal:37); the forward applies its one pre-scale explicitly instead. */
void ora_rmsnorm(const float* x, int rows, int width, const float* weight, float eps, float prescale, float* out) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * width;
        float* o = out + (size_t)r * width;
        float ss = 0;
        for (int i = 0; i < width; i++) {
            float v = xr[i] * prescale;
            ss += v * v;
        }
        float inv = 1.0f / sqrtf(ss / (float)width + eps);
        for (int i = 0; i < width; i++) {
            float v = xr[i] * prescale * inv;
            o[i] = weight ? v * weight[i] : v;
        }
    }
}

/* CPUReference.swift:92-95, ggml's constants (Model/Architecture.md:45). */
float ora_gelu_tanh(float x) {
    const float c = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + 0.044715f * x * x)));
}

/* RopeTable.swift:16-31: [position][pair] -> (cos, sin) of pos * base^(-2i/hd), in fp64. */
void ora_rope_table(int head_dim, float base, int positions, float* out) {
    const int pairs = head_dim / 2;
    for (int i = 0; i < pairs; i++) {
        double inv_freq = pow((double)base, -2.0 * (double)i / (double)head_dim);
        for (int pos = 0; pos < positions; pos++) {
            double theta = (double)pos * inv_freq;
            out[((size_t)pos * pairs + i) * 2] = (float)cos(theta);
            out[((size_t)pos * pairs + i) * 2 + 1] = (float)sin(theta);
        }
    }
}

/* CPUReference.swift:98-113: NeoX rotation of (i, i + hd/2) over [tokens][heads][hd]. */
void ora_rope(float* x, int tokens, int heads, int head_dim, const float* table, const int32_t* positions) {
    const int half = head_dim / 2;
    for (int t = 0; t < tokens; t++) {
        const int pos = positions[t];
        for (int h = 0; h < heads; h++) {
            float* v = x + ((size_t)t * heads + h) * head_dim;
            for (int i = 0; i < half; i++) {
                const float c = table[((size_t)pos * half + i) * 2];
                const float s = table[((size_t)pos * half + i) * 2 + 1];
                const float a = v[i], b = v[i + half];
                v[i] = a * c - b * s;
                v[i + half] = a * s + b * c;
            }
        }
    }
}

/* CPUReference.swift:117-174: bidirectional attention over one sequence. q is [T][H][hd], k and
 * v are [T][KV][hd]; head h reads kv head h / (H / KV). window > 0 masks |i - j| > window / 2
 * (:144). Per row: scale, max over unmasked, expf(s - max) (0 where masked), 1 / sum, P.V. */
void ora_attention(const float* q, const float* k, const float* v, int tokens, int heads, int kv_heads,
                   int head_dim, float scale, int window, float* out, int threads) {
    const int group = heads / kv_heads;
    const int hd = head_dim;
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
    {
        float* s = (float*)malloc((size_t)tokens * sizeof(float));
        float* acc = (float*)malloc((size_t)hd * sizeof(float));
#pragma omp for schedule(dynamic, 8)
        for (long idx = 0; idx < (long)heads * tokens; idx++) {
            const int h = (int)(idx / tokens), i = (int)(idx % tokens);
            const int kh = h / group;
            const float* qi = q + ((size_t)i * heads + h) * hd;
            float maxs = -INFINITY;
            for (int j = 0; j < tokens; j++) {
                if (window > 0 && abs(i - j) > window / 2) {
                    s[j] = -INFINITY;
                } else {
                    const float* kj = k + ((size_t)j * kv_heads + kh) * hd;
                    v8f a8 = {0, 0, 0, 0, 0, 0, 0, 0};
                    int d = 0;
                    for (; d + 8 <= hd; d += 8) {
                        v8f a, b;
                        memcpy(&a, qi + d, 32);
                        memcpy(&b, kj + d, 32);
                        a8 += a * b;
                    }
                    float dot = hsum8(a8);
                    for (; d < hd; d++) dot += qi[d] * kj[d];
                    s[j] = dot * scale;
                    if (s[j] > maxs) maxs = s[j];
                }
            }
            float sum = 0;
            for (int j = 0; j < tokens; j++) {
                const float e = s[j] == -INFINITY ? 0.0f : expf(s[j] - maxs);
                s[j] = e;
                sum += e;
            }
            const float inv = 1.0f / sum;
            for (int j = 0; j < tokens; j++) s[j] *= inv;
            for (int d = 0; d < hd; d++) acc[d] = 0;
            for (int j = 0; j < tokens; j++) {
                if (s[j] == 0.0f) continue;
                const float* vj = v + ((size_t)j * kv_heads + kh) * hd;
                const float p = s[j];
                for (int d = 0; d < hd; d++) acc[d] += p * vj[d];
            }
            float* o = out + ((size_t)i * heads + h) * hd;
            for (int d = 0; d < hd; d++) o[d] = acc[d];
        }
        free(s);
        free(acc);
    }
}

/* ---------------------------------------------------------------- GGUF (GGUFFile.swift) */

typedef struct {
    char name[96];
    int ndim;
    int64_t shape[4];
    int type;
    uint64_t offset;
} ora_tensor;

typedef struct {
    char key[96];
    int vtype;      /* GGUF value type */
    int64_t ival;   /* integer scalars */
    double fval;    /* float scalars */
    int arr_type;   /* element type for arrays */
    int64_t arr_len;
    const uint8_t* arr_data; /* element data for fixed-size arrays */
    char sval[96];
} ora_kv;

typedef struct {
    int index, sliding, kv_heads, head_dim;
    float rope_base, out_scale;
    const float *attn_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffw, *post_norm;
    float *wq, *wk, *wv, *wo, *wg, *wu, *wd, *inp_gate, *proj; /* dequantized [rows][cols] */
    const float* rope; /* table for this layer */
} ora_layer;

struct ora_model {
    uint8_t* map;
    size_t size;
    ora_kv* kv;
    int nkv;
    ora_tensor* tensors;
    int ntensors;
    size_t data_offset;
    /* config (ModelConfig.swift:54-112) */
    int layers, hidden, heads, out_dims, ff, pl, vocab, window;
    float eps, emb_scale, pl_scale;
    int has_ple;
    ora_layer layer[ORA_MAX_LAYERS];
    const ora_tensor* tok_embd;
    float *pl_proj, *output;
    const float *pl_norm, *out_norm;
    float* tables[8];
    int table_hd[8];
    float table_base[8];
    int ntables;
};

typedef struct {
    const uint8_t* p;
    size_t n, pos;
    int bad;
} cur_t;

static int need(cur_t* c, size_t k) {
    if (c->bad || c->pos + k > c->n) {
        c->bad = 1;
        return 0;
    }
    return 1;
}
static uint64_t rd(cur_t* c, int bytes) {
    uint64_t v = 0;
    if (!need(c, (size_t)bytes)) return 0;
    memcpy(&v, c->p + c->pos, (size_t)bytes);
    c->pos += (size_t)bytes;
    return v;
}

static int type_size(int t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

static void read_scalar(cur_t* c, int t, ora_kv* kv) {
    switch (t) {
    case 0: kv->ival = (uint8_t)rd(c, 1); break;
    case 1: kv->ival = (int8_t)rd(c, 1); break;
    case 2: kv->ival = (uint16_t)rd(c, 2); break;
    case 3: kv->ival = (int16_t)rd(c, 2); break;
    case 4: kv->ival = (uint32_t)rd(c, 4); break;
    case 5: kv->ival = (int32_t)rd(c, 4); break;
    case 6: { uint32_t b = (uint32_t)rd(c, 4); float f; memcpy(&f, &b, 4); kv->fval = f; break; }
    case 7: kv->ival = rd(c, 1) != 0; break;
    case 10: kv->ival = (int64_t)rd(c, 8); break;
    case 11: kv->ival = (int64_t)rd(c, 8); break;
    case 12: { uint64_t b = rd(c, 8); double d; memcpy(&d, &b, 8); kv->fval = d; break; }
    default: c->bad = 1;
    }
}

static void skip_string(cur_t* c, char* dst, size_t cap) {
    uint64_t n = rd(c, 8);
    if (!need(c, n)) return;
    if (dst) {
        size_t k = n < cap - 1 ? n : cap - 1;
        memcpy(dst, c->p + c->pos, k);
        dst[k] = 0;
    }
    c->pos += n;
}

static void skip_value(cur_t* c, int t) {
    if (t == 8) {
        skip_string(c, NULL, 0);
    } else if (t == 9) {
        int et = (int)rd(c, 4);
        uint64_t n = rd(c, 8);
        for (uint64_t i = 0; i < n && !c->bad; i++) skip_value(c, et);
    } else {
        int s = type_size(t);
        if (!s) { c->bad = 1; return; }
        if (need(c, (size_t)s)) c->pos += (size_t)s;
    }
}

static const ora_kv* find_kv(const ora_model* m, const char* key) {
    for (int i = 0; i < m->nkv; i++)
        if (strcmp(m->kv[i].key, key) == 0) return &m->kv[i];
    return NULL;
}
static int kv_is_int(const ora_kv* kv) {
    return kv && ((kv->vtype >= 0 && kv->vtype <= 5 && kv->vtype != 6) || kv->vtype == 10 || kv->vtype == 11 || kv->vtype == 7);
}
static const ora_tensor* find_tensor(const ora_model* m, const char* name) {
    for (int i = 0; i < m->ntensors; i++)
        if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i];
    return NULL;
}

static size_t tensor_bytes(const ora_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    switch (t->type) {
    case ORA_F32: return (size_t)n * 4;
    case ORA_F16: case ORA_BF16: return (size_t)n * 2;
    case ORA_Q8_0: return (size_t)n / 32 * 34;
    default: return 0;
    }
}

static const uint8_t* tensor_data(const ora_model* m, const ora_tensor* t) {
    return m->map + m->data_offset + t->offset;
}

static int row_bytes(const ora_tensor* t) {
    int cols = (int)t->shape[0];
    switch (t->type) {
    case ORA_F32: return cols * 4;
    case ORA_F16: case ORA_BF16: return cols * 2;
    case ORA_Q8_0: return cols / 32 * 34;
    default: return 0;
    }
}

static float* dequant(const ora_model* m, const ora_tensor* t) {
    int cols = (int)t->shape[0];
    int64_t rows = 1;
    for (int i = 1; i < t->ndim; i++) rows *= t->shape[i];
    float* out = (float*)malloc((size_t)rows * cols * sizeof(float));
    const uint8_t* p = tensor_data(m, t);
    int rb = row_bytes(t);
    for (int64_t r = 0; r < rows; r++) ora_dequant_row(t->type, p + (size_t)r * rb, cols, out + (size_t)r * cols);
    return out;
}

static void set_err(char* err, int errlen, const char* fmt, ...) {
    if (!err || errlen <= 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, (size_t)errlen, fmt, ap);
    va_end(ap);
}

static int parse(ora_model* m, char* err, int errlen) {
    cur_t c = {m->map, m->size, 0, 0};
    uint32_t magic = (uint32_t)rd(&c, 4);
    if (c.bad || magic != 0x46554747u) { set_err(err, errlen, "invalid GGUF file: bad magic"); return -1; }
    uint32_t version = (uint32_t)rd(&c, 4);
    if (version != 2 && version != 3) { set_err(err, errlen, "invalid GGUF file: unsupported version %u", version); return -1; }
    uint64_t nt = rd(&c, 8), nkv = rd(&c, 8);
    if (c.bad || nt > 100000 || nkv > 100000) { set_err(err, errlen, "invalid GGUF file: truncated header"); return -1; }
    m->kv = (ora_kv*)calloc(nkv ? nkv : 1, sizeof(ora_kv));
    m->nkv = (int)nkv;
    for (uint64_t i = 0; i < nkv && !c.bad; i++) {
        ora_kv* kv = &m->kv[i];
        skip_string(&c, kv->key, sizeof(kv->key));
        kv->vtype = (int)rd(&c, 4);
        if (kv->vtype == 8) {
            skip_string(&c, kv->sval, sizeof(kv->sval));
        } else if (kv->vtype == 9) {
            kv->arr_type = (int)rd(&c, 4);
            kv->arr_len = (int64_t)rd(&c, 8);
            int es = type_size(kv->arr_type);
            if (kv->arr_type != 8 && es > 0) {
                if (!need(&c, (size_t)kv->arr_len * es)) break;
                kv->arr_data = c.p + c.pos;
                c.pos += (size_t)kv->arr_len * es;
            } else {
                for (int64_t j = 0; j < kv->arr_len && !c.bad; j++) skip_value(&c, kv->arr_type);
            }
        } else {
            read_scalar(&c, kv->vtype, kv);
        }
    }
    if (c.bad) { set_err(err, errlen, "invalid GGUF file: truncated header at byte %zu", c.pos); return -1; }
    m->tensors = (ora_tensor*)calloc(nt ? nt : 1, sizeof(ora_tensor));
    m->ntensors = (int)nt;
    for (uint64_t i = 0; i < nt && !c.bad; i++) {
        ora_tensor* t = &m->tensors[i];
        skip_string(&c, t->name, sizeof(t->name));
        t->ndim = (int)rd(&c, 4);
        if (t->ndim > 4) { set_err(err, errlen, "invalid GGUF file: tensor %s has %d dimensions", t->name, t->ndim); return -1; }
        for (int d = 0; d < t->ndim; d++) t->shape[d] = (int64_t)rd(&c, 8);
        t->type = (int)rd(&c, 4);
        if (t->type != ORA_F32 && t->type != ORA_F16 && t->type != ORA_Q8_0 && t->type != ORA_BF16) {
            set_err(err, errlen, "tensor %s uses unsupported storage type %d", t->name, t->type);
            return -1;
        }
        t->offset = rd(&c, 8);
    }
    if (c.bad) { set_err(err, errlen, "invalid GGUF file: truncated header at byte %zu", c.pos); return -1; }
    const ora_kv* al = find_kv(m, "general.alignment");
    size_t align = al && kv_is_int(al) ? (size_t)al->ival : 32;
    m->data_offset = (c.pos + align - 1) / align * align;
    for (int i = 0; i < m->ntensors; i++) {
        if (m->data_offset + m->tensors[i].offset + tensor_bytes(&m->tensors[i]) > m->size) {
            set_err(err, errlen, "invalid GGUF file: tensor %s extends past the end of the file", m->tensors[i].name);
            return -1;
        }
    }
    return 0;
}

static int meta_int(const ora_model* m, const char* arch, const char* key, int* out, char* err, int errlen) {
    char full[160];
    snprintf(full, sizeof(full), "%s.%s", arch, key);
    const ora_kv* kv = find_kv(m, full);
    if (!kv || !kv_is_int(kv)) { set_err(err, errlen, "weight file lacks metadata key %s", full); return -1; }
    *out = (int)kv->ival;
    return 0;
}
static int meta_float(const ora_model* m, const char* arch, const char* key, float* out, char* err, int errlen) {
    char full[160];
    snprintf(full, sizeof(full), "%s.%s", arch, key);
    const ora_kv* kv = find_kv(m, full);
    if (!kv) { set_err(err, errlen, "weight file lacks metadata key %s", full); return -1; }
    *out = (kv->vtype == 6 || kv->vtype == 12) ? (float)kv->fval : (float)kv->ival;
    return 0;
}

/* Shape/type checked tensor lookup (Weights.swift:93-98). cols/rows < 0 skips that check. */
static const ora_tensor* tensor_checked(const ora_model* m, const char* name, int64_t cols, int64_t rows, int f32_only,
                                        int optional, char* err, int errlen, int* failed) {
    const ora_tensor* t = find_tensor(m, name);
    if (!t) {
        if (!optional) { set_err(err, errlen, "weight file lacks tensor %s", name); *failed = 1; }
        return NULL;
    }
    int64_t r = 1;
    for (int i = 1; i < t->ndim; i++) r *= t->shape[i];
    if (t->shape[0] != cols || (rows >= 0 && r != rows)) {
        set_err(err, errlen, "tensor %s has shape [%lld, %lld], expected [%lld, %lld]", name, (long long)t->shape[0],
                (long long)r, (long long)cols, (long long)rows);
        *failed = 1;
        return NULL;
    }
    if (f32_only && t->type != ORA_F32) {
        set_err(err, errlen, "tensor %s uses unsupported storage type %d", name, t->type);
        *failed = 1;
        return NULL;
    }
    return t;
}

static const float* rope_for(ora_model* m, int hd, float base) {
    for (int i = 0; i < m->ntables; i++)
        if (m->table_hd[i] == hd && m->table_base[i] == base) return m->tables[i];
    if (m->ntables >= 8) return NULL;
    float* t = (float*)malloc((size_t)ORA_MAX_TOKENS * (hd / 2) * 2 * sizeof(float));
    ora_rope_table(hd, base, ORA_MAX_TOKENS, t);
    m->tables[m->ntables] = t;
    m->table_hd[m->ntables] = hd;
    m->table_base[m->ntables] = base;
    m->ntables++;
    return t;
}

ora_model* ora_open(const char* path, char* err, int errlen) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { set_err(err, errlen, "cannot read %s", path); return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        set_err(err, errlen, "invalid GGUF file: too short");
        return NULL;
    }
    void* p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (p == MAP_FAILED) { set_err(err, errlen, "cannot map %s", path); return NULL; }
    ora_model* m = (ora_model*)calloc(1, sizeof(ora_model));
    m->map = (uint8_t*)p;
    m->size = (size_t)st.st_size;
    if (parse(m, err, errlen) != 0) { ora_close(m); return NULL; }

    /* ModelConfig.swift:54-112 */
    const ora_kv* archkv = find_kv(m, "general.architecture");
    const char* arch = archkv && archkv->vtype == 8 ? archkv->sval : "";
    if (strcmp(arch, "gemma-embedding2") != 0) {
        set_err(err, errlen, "unsupported architecture '%s'", arch);
        ora_close(m);
        return NULL;
    }
    int hd_global, hd_swa, vl, vls;
    if (meta_int(m, arch, "block_count", &m->layers, err, errlen) || meta_int(m, arch, "embedding_length", &m->hidden, err, errlen) ||
        meta_int(m, arch, "attention.head_count", &m->heads, err, errlen) ||
        meta_int(m, arch, "attention.key_length", &hd_global, err, errlen) ||
        meta_int(m, arch, "attention.key_length_swa", &hd_swa, err, errlen) ||
        meta_int(m, arch, "attention.value_length", &vl, err, errlen) ||
        meta_int(m, arch, "attention.value_length_swa", &vls, err, errlen) ||
        meta_int(m, arch, "embedding_length_out", &m->out_dims, err, errlen) ||
        meta_int(m, arch, "feed_forward_length", &m->ff, err, errlen) ||
        meta_int(m, arch, "attention.sliding_window", &m->window, err, errlen) ||
        meta_float(m, arch, "attention.layer_norm_rms_epsilon", &m->eps, err, errlen)) {
        ora_close(m);
        return NULL;
    }
    if (vl != hd_global || vls != hd_swa) { set_err(err, errlen, "invalid GGUF file: key and value head sizes differ"); ora_close(m); return NULL; }
    if (m->layers > ORA_MAX_LAYERS) { set_err(err, errlen, "too many layers"); ora_close(m); return NULL; }
    float rope_global, rope_swa;
    if (meta_float(m, arch, "rope.freq_base", &rope_global, err, errlen)) { ora_close(m); return NULL; }
    char k2[160];
    snprintf(k2, sizeof(k2), "%s.rope.freq_base_swa", arch);
    rope_swa = find_kv(m, k2) ? (float)(find_kv(m, k2)->vtype == 6 || find_kv(m, k2)->vtype == 12 ? find_kv(m, k2)->fval : find_kv(m, k2)->ival) : rope_global;
    snprintf(k2, sizeof(k2), "%s.attention.head_count_kv", arch);
    const ora_kv* kvh = find_kv(m, k2);
    snprintf(k2, sizeof(k2), "%s.attention.sliding_window_pattern", arch);
    const ora_kv* pat = find_kv(m, k2);
    if (!kvh || kvh->vtype != 9 || kvh->arr_type != 5 || kvh->arr_len != m->layers) {
        set_err(err, errlen, "weight file lacks metadata key %s.attention.head_count_kv", arch); ora_close(m); return NULL;
    }
    if (!pat || pat->vtype != 9 || pat->arr_type != 7 || pat->arr_len != m->layers) {
        set_err(err, errlen, "weight file lacks metadata key %s.attention.sliding_window_pattern", arch); ora_close(m); return NULL;
    }
    const ora_kv* toks = find_kv(m, "tokenizer.ggml.tokens");
    if (!toks || toks->vtype != 9 || toks->arr_type != 8) { set_err(err, errlen, "weight file lacks metadata key tokenizer.ggml.tokens"); ora_close(m); return NULL; }
    m->vocab = (int)toks->arr_len;
    m->has_ple = find_tensor(m, "per_layer_model_proj.weight") != NULL;
    if (m->has_ple && meta_int(m, arch, "embedding_length_per_layer_input", &m->pl, err, errlen)) { ora_close(m); return NULL; }
    m->emb_scale = sqrtf((float)m->hidden);
    m->pl_scale = 1.0f / sqrtf((float)m->hidden);

    /* Weights.swift:92-132 */
    int failed = 0;
    const int d = m->hidden;
    m->tok_embd = tensor_checked(m, "token_embd.weight", d, m->vocab, 0, 0, err, errlen, &failed);
    const ora_tensor* t_on = tensor_checked(m, "output_norm.weight", d, 1, 1, 0, err, errlen, &failed);
    const ora_tensor* t_out = failed ? NULL : tensor_checked(m, "output.weight", d, m->out_dims, 0, 0, err, errlen, &failed);
    if (failed) { ora_close(m); return NULL; }
    m->out_norm = (const float*)tensor_data(m, t_on);
    m->output = dequant(m, t_out);
    if (m->has_ple) {
        const ora_tensor* t = tensor_checked(m, "per_layer_model_proj.weight", d, (int64_t)m->pl * m->layers, 0, 0, err, errlen, &failed);
        const ora_tensor* n = failed ? NULL : tensor_checked(m, "per_layer_proj_norm.weight", m->pl, 1, 1, 0, err, errlen, &failed);
        if (failed) { ora_close(m); return NULL; }
        m->pl_proj = dequant(m, t);
        m->pl_norm = (const float*)tensor_data(m, n);
    }
    const int8_t* pattern = (const int8_t*)pat->arr_data;
    const int32_t* kvheads = (const int32_t*)kvh->arr_data;
    for (int l = 0; l < m->layers && !failed; l++) {
        ora_layer* L = &m->layer[l];
        L->index = l;
        L->sliding = pattern[l] != 0;
        L->kv_heads = kvheads[l];
        L->head_dim = L->sliding ? hd_swa : hd_global;
        L->rope_base = L->sliding ? rope_swa : rope_global;
        const int hd = L->head_dim, qd = m->heads * hd, kvd = L->kv_heads * hd;
        char nm[96];
#define T_(suffix, c, r, f32, opt) (snprintf(nm, sizeof(nm), "blk.%d." suffix, l), tensor_checked(m, nm, c, r, f32, opt, err, errlen, &failed))
        const ora_tensor *an = T_("attn_norm.weight", d, 1, 1, 0), *wq = T_("attn_q.weight", d, qd, 0, 0),
                         *wk = T_("attn_k.weight", d, kvd, 0, 0), *wv = T_("attn_v.weight", d, kvd, 0, 0),
                         *wo = T_("attn_output.weight", qd, d, 0, 0), *qn = T_("attn_q_norm.weight", hd, 1, 1, 0),
                         *kn = T_("attn_k_norm.weight", hd, 1, 1, 0), *pan = T_("post_attention_norm.weight", d, 1, 1, 0),
                         *fn = T_("ffn_norm.weight", d, 1, 1, 0), *wg = T_("ffn_gate.weight", d, m->ff, 0, 0),
                         *wu = T_("ffn_up.weight", d, m->ff, 0, 0), *wd = T_("ffn_down.weight", m->ff, d, 0, 0),
                         *pfn = T_("post_ffw_norm.weight", d, 1, 1, 0), *os = T_("layer_output_scale.weight", 1, 1, 1, 1);
        if (failed) break;
        L->attn_norm = (const float*)tensor_data(m, an);
        L->q_norm = (const float*)tensor_data(m, qn);
        L->k_norm = (const float*)tensor_data(m, kn);
        L->post_attn = (const float*)tensor_data(m, pan);
        L->ffn_norm = (const float*)tensor_data(m, fn);
        L->post_ffw = (const float*)tensor_data(m, pfn);
        L->out_scale = os ? *(const float*)tensor_data(m, os) : 1.0f;
        L->wq = dequant(m, wq); L->wk = dequant(m, wk); L->wv = dequant(m, wv); L->wo = dequant(m, wo);
        L->wg = dequant(m, wg); L->wu = dequant(m, wu); L->wd = dequant(m, wd);
        if (m->has_ple) {
            const ora_tensor *ig = T_("inp_gate.weight", d, m->pl, 0, 0), *pj = T_("proj.weight", m->pl, d, 0, 0),
                             *pn = T_("post_norm.weight", d, 1, 1, 0);
            if (failed) break;
            L->inp_gate = dequant(m, ig);
            L->proj = dequant(m, pj);
            L->post_norm = (const float*)tensor_data(m, pn);
        }
#undef T_
        L->rope = rope_for(m, hd, L->rope_base);
    }
    if (failed) { ora_close(m); return NULL; }
    return m;
}

void ora_close(ora_model* m) {
    if (!m) return;
    for (int l = 0; l < ORA_MAX_LAYERS; l++) {
        ora_layer* L = &m->layer[l];
        free(L->wq); free(L->wk); free(L->wv); free(L->wo); free(L->wg); free(L->wu); free(L->wd);
        free(L->inp_gate); free(L->proj);
    }
    for (int i = 0; i < m->ntables; i++) free(m->tables[i]);
    free(m->pl_proj);
    free(m->output);
    free(m->kv);
    free(m->tensors);
    if (m->map) munmap(m->map, m->size);
    free(m);
}

int ora_hidden(const ora_model* m) { return m->hidden; }
int ora_output_dims(const ora_model* m) { return m->out_dims; }
int ora_layers(const ora_model* m) { return m->layers; }
int ora_vocab(const ora_model* m) { return m->vocab; }

/* ---------------------------------------------------------------- forward */

static void trace_emit(ora_trace_fn fn, void* user, const char* name, int layer, const float* p, size_t n) {
    if (fn) fn(user, name, layer, p, n);
}

/* CPUReference.swift:183-283 for one sequence of token and vector rows. Positions are 0..T-1
 * (:188). A token id -(r + 1) stands for row r of `vectors` ([n_vectors][hidden]), entered into the
 * residual stream unscaled (:197-199; the packed-batch convention of Metal/MetalForward.swift:6-7). */
int ora_forward_rows(ora_model* m, const int32_t* tokens, int T, const float* vectors, int n_vectors, float* pooled,
                     ora_trace_fn trace, void* user, int threads) {
    if (T <= 0 || T > ORA_MAX_TOKENS) return -1;
    const int d = m->hidden;
    const float eps = m->eps;
    int32_t* pos = (int32_t*)malloc((size_t)T * sizeof(int32_t));
    for (int t = 0; t < T; t++) pos[t] = t;
    int maxq = 0, maxkv = 0;
    for (int l = 0; l < m->layers; l++) {
        int q = m->heads * m->layer[l].head_dim, kv = m->layer[l].kv_heads * m->layer[l].head_dim;
        if (q > maxq) maxq = q;
        if (kv > maxkv) maxkv = kv;
    }
    const size_t Td = (size_t)T * d;
    float* x = (float*)calloc(Td, sizeof(float));
    float* h = (float*)malloc(Td * sizeof(float));
    float* q = (float*)malloc((size_t)T * maxq * sizeof(float));
    float* qn = (float*)malloc((size_t)T * maxq * sizeof(float));
    float* k = (float*)malloc((size_t)T * maxkv * sizeof(float));
    float* kn = (float*)malloc((size_t)T * maxkv * sizeof(float));
    float* v = (float*)malloc((size_t)T * maxkv * sizeof(float));
    float* vn = (float*)malloc((size_t)T * maxkv * sizeof(float));
    float* attn = (float*)malloc((size_t)T * maxq * sizeof(float));
    float* o = (float*)malloc(Td * sizeof(float));
    float* on = (float*)malloc(Td * sizeof(float));
    float* gate = (float*)malloc((size_t)T * m->ff * sizeof(float));
    float* up = (float*)malloc((size_t)T * m->ff * sizeof(float));
    float* per_layer = NULL;
    float* g = NULL;
    if (m->has_ple) {
        per_layer = (float*)malloc((size_t)T * m->pl * m->layers * sizeof(float));
        g = (float*)malloc((size_t)T * m->pl * sizeof(float));
    }

    /* :190-204 token rows: dequantised embedding row times sqrt(d) */
    const uint8_t* emb = tensor_data(m, m->tok_embd);
    const int erb = row_bytes(m->tok_embd);
    for (int t = 0; t < T; t++) {
        float* dst = x + (size_t)t * d;
        if (tokens[t] < 0) {
            const int r = -(tokens[t] + 1);
            if (!vectors || r >= n_vectors) { T = -1; break; }
            memcpy(dst, vectors + (size_t)r * d, (size_t)d * sizeof(float));
            continue;
        }
        if (tokens[t] >= m->vocab) { T = -1; break; }
        ora_dequant_row(m->tok_embd->type, emb + (size_t)tokens[t] * erb, d, dst);
        for (int i = 0; i < d; i++) dst[i] *= m->emb_scale;
    }
    int rc = 0;
    if (T < 0) { rc = -2; goto done; }
    trace_emit(trace, user, "inp_scaled", -1, x, Td);

    if (m->has_ple) { /* :206-210 */
        const int pld = m->pl * m->layers;
        ora_matmul(x, T, d, m->pl_proj, pld, per_layer, threads);
        for (size_t i = 0; i < (size_t)T * pld; i++) per_layer[i] *= m->pl_scale;
        ora_rmsnorm(per_layer, T * m->layers, m->pl, m->pl_norm, eps, 1.0f, per_layer);
        trace_emit(trace, user, "inp_per_layer", -1, per_layer, (size_t)T * pld);
    }

    for (int l = 0; l < m->layers; l++) { /* :212-271 */
        const ora_layer* L = &m->layer[l];
        const int H = m->heads, KV = L->kv_heads, hd = L->head_dim, qd = H * hd, kvd = KV * hd;
        ora_rmsnorm(x, T, d, L->attn_norm, eps, 1.0f, h);
        trace_emit(trace, user, "attn_norm", l, h, Td);
        ora_matmul(h, T, d, L->wq, qd, q, threads);
        ora_matmul(h, T, d, L->wk, kvd, k, threads);
        ora_matmul(h, T, d, L->wv, kvd, v, threads);
        trace_emit(trace, user, "Qcur", l, q, (size_t)T * qd);
        trace_emit(trace, user, "Kcur", l, k, (size_t)T * kvd);
        trace_emit(trace, user, "Vcur", l, v, (size_t)T * kvd);
        ora_rmsnorm(q, T * H, hd, L->q_norm, eps, 1.0f, qn);
        ora_rmsnorm(k, T * KV, hd, L->k_norm, eps, 1.0f, kn);
        ora_rmsnorm(v, T * KV, hd, NULL, eps, 1.0f, vn);
        trace_emit(trace, user, "Qcur_normed", l, qn, (size_t)T * qd);
        trace_emit(trace, user, "Kcur_normed", l, kn, (size_t)T * kvd);
        trace_emit(trace, user, "Vcur_normed", l, vn, (size_t)T * kvd);
        ora_rope(qn, T, H, hd, L->rope, pos);
        ora_rope(kn, T, KV, hd, L->rope, pos);
        trace_emit(trace, user, "Qcur_pos", l, qn, (size_t)T * qd);
        trace_emit(trace, user, "Kcur_pos", l, kn, (size_t)T * kvd);
        ora_attention(qn, kn, vn, T, H, KV, hd, 1.0f, L->sliding ? m->window : 0, attn, threads);
        trace_emit(trace, user, "kqv_out", l, attn, (size_t)T * qd);
        ora_matmul(attn, T, qd, L->wo, d, o, threads);
        ora_rmsnorm(o, T, d, L->post_attn, eps, 1.0f, on);
        trace_emit(trace, user, "attn_post_norm", l, on, Td);
        for (size_t i = 0; i < Td; i++) x[i] += on[i];
        trace_emit(trace, user, "attn_out", l, x, Td);

        ora_rmsnorm(x, T, d, L->ffn_norm, eps, 1.0f, h);
        trace_emit(trace, user, "ffn_norm", l, h, Td);
        ora_matmul(h, T, d, L->wg, m->ff, gate, threads);
        ora_matmul(h, T, d, L->wu, m->ff, up, threads);
        for (size_t i = 0; i < (size_t)T * m->ff; i++) gate[i] = ora_gelu_tanh(gate[i]) * up[i];
        trace_emit(trace, user, "ffn_geglu", l, gate, (size_t)T * m->ff);
        ora_matmul(gate, T, m->ff, L->wd, d, o, threads);
        trace_emit(trace, user, "ffn_out", l, o, Td);
        ora_rmsnorm(o, T, d, L->post_ffw, eps, 1.0f, on);
        trace_emit(trace, user, "ffn_post_norm", l, on, Td);
        for (size_t i = 0; i < Td; i++) x[i] += on[i];
        trace_emit(trace, user, "pe_in", l, x, Td);

        if (m->has_ple) { /* :259-269 */
            const int pl = m->pl;
            ora_matmul(x, T, d, L->inp_gate, pl, g, threads);
            for (int t = 0; t < T; t++)
                for (int i = 0; i < pl; i++) {
                    size_t idx = (size_t)t * pl + i;
                    g[idx] = ora_gelu_tanh(g[idx]) * per_layer[((size_t)t * m->layers + l) * pl + i];
                }
            ora_matmul(g, T, pl, L->proj, d, o, threads);
            ora_rmsnorm(o, T, d, L->post_norm, eps, 1.0f, on);
            trace_emit(trace, user, "per_layer_embd_out", l, on, Td);
            for (size_t i = 0; i < Td; i++) x[i] = (x[i] + on[i]) * L->out_scale;
        } else if (L->out_scale != 1.0f) {
            for (size_t i = 0; i < Td; i++) x[i] *= L->out_scale;
        }
        trace_emit(trace, user, "l_out", l, x, Td);
    }

    { /* :273-282 */
        ora_rmsnorm(x, T, d, m->out_norm, eps, 1.0f, h);
        trace_emit(trace, user, "result_norm", -1, h, Td);
        float* proj = (float*)malloc((size_t)T * m->out_dims * sizeof(float));
        ora_matmul(h, T, d, m->output, m->out_dims, proj, threads);
        trace_emit(trace, user, "result_embd", -1, proj, (size_t)T * m->out_dims);
        for (int i = 0; i < m->out_dims; i++) pooled[i] = 0;
        for (int t = 0; t < T; t++)
            for (int i = 0; i < m->out_dims; i++) pooled[i] += proj[(size_t)t * m->out_dims + i];
        for (int i = 0; i < m->out_dims; i++) pooled[i] /= (float)T;
        free(proj);
    }
done:
    free(pos); free(x); free(h); free(q); free(qn); free(k); free(kn); free(v); free(vn); free(attn);
    free(o); free(on); free(gate); free(up); free(per_layer); free(g);
    return rc;
}

/* A sequence of token rows only. */
int ora_forward(ora_model* m, const int32_t* tokens, int T, float* pooled, ora_trace_fn trace, void* user, int threads) {
    return ora_forward_rows(m, tokens, T, NULL, 0, pooled, trace, user, threads);
}

/* ================================================================ image tower (config 5)
 *
 * BASELINE config 5's encoder, restated the way CPUVisionReference.forward
 * (Model/CPUVisionReference.swift:89-165) runs the reference's gemma4v tower: the same stage
 * order (patch projection, position rows, per-layer attention and MLP blocks with residual adds,
 * pooling over merge x merge windows, a norm and the projection), the same position-table layout
 * (column rows, then row rows, :99-107) and trace names. Config 5's architecture differs from
 * gemma4v where BASELINE says so: LayerNorm with bias (pre-LN), biased projections, a non-gated
 * gelu_tanh MLP of width feed_forward, scaled dot-product attention (1 / sqrt(hd), no q/k norms,
 * no RoPE), a final LayerNorm before pooling, and the projector's weighted RMSNorm. */

#define ORA_VIT_MAX_LAYERS 64

typedef struct {
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b, *bq, *bk, *bv, *bo, *bup, *bdown;
    float *wq, *wk, *wv, *wo, *wup, *wdown; /* dequantised [rows][cols] */
} ora_vit_layer;

struct ora_vision {
    ora_model* file; /* the mapping and its parsed directory */
    int layers, hidden, heads, ff, patch, merge, proj, npos;
    float eps;
    float *patch_w, *proj_w;
    const float *patch_b, *pos, *post_w, *post_b, *norm_w;
    ora_vit_layer layer[ORA_VIT_MAX_LAYERS];
};

/* LayerNorm per row: mean, then the mean of squared deviations, out = (x - mean) * rstd * w + b
 * with rstd = 1 / sqrt(var + eps), sums in element order. */
void ora_layernorm(const float* x, int rows, int width, const float* w, const float* b, float eps, float* out) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * width;
        float* o = out + (size_t)r * width;
        float s = 0;
        for (int i = 0; i < width; i++) s += xr[i];
        const float mean = s / (float)width;
        float ss = 0;
        for (int i = 0; i < width; i++) {
            const float t = xr[i] - mean;
            ss += t * t;
        }
        const float rstd = 1.0f / sqrtf(ss / (float)width + eps);
        for (int i = 0; i < width; i++) o[i] = (xr[i] - mean) * rstd * w[i] + b[i];
    }
}

/* Mean of each merge x merge window of a grid_x x grid_y grid of rows (CPUVisionReference.pool):
 * token oy * (grid_x / merge) + ox sums rows (merge oy + dy) * grid_x + merge ox + dx in (dy, dx)
 * order, then scales by 1 / merge^2. */
void ora_pool(const float* x, int grid_x, int grid_y, int merge, int width, float* out) {
    const int tx = grid_x / merge, ty = grid_y / merge;
    const float inv = 1.0f / (float)(merge * merge);
    for (int oy = 0; oy < ty; oy++)
        for (int ox = 0; ox < tx; ox++) {
            float* o = out + ((size_t)oy * tx + ox) * width;
            for (int i = 0; i < width; i++) o[i] = 0;
            for (int dy = 0; dy < merge; dy++)
                for (int dx = 0; dx < merge; dx++) {
                    const float* xr = x + ((size_t)(merge * oy + dy) * grid_x + merge * ox + dx) * width;
                    for (int i = 0; i < width; i++) o[i] += xr[i];
                }
            for (int i = 0; i < width; i++) o[i] *= inv;
        }
}

static int vmeta_int(const ora_model* m, const char* key, int* out, char* err, int errlen) {
    const ora_kv* kv = find_kv(m, key);
    if (!kv || !kv_is_int(kv)) { set_err(err, errlen, "image encoder file lacks metadata key %s", key); return -1; }
    *out = (int)kv->ival;
    return 0;
}

ora_vision* ora_vision_open(const char* path, char* err, int errlen) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { set_err(err, errlen, "cannot read %s", path); return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) { close(fd); set_err(err, errlen, "invalid GGUF file: too short"); return NULL; }
    void* p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (p == MAP_FAILED) { set_err(err, errlen, "cannot map %s", path); return NULL; }
    ora_vision* v = (ora_vision*)calloc(1, sizeof(ora_vision));
    v->file = (ora_model*)calloc(1, sizeof(ora_model));
    v->file->map = (uint8_t*)p;
    v->file->size = (size_t)st.st_size;
    ora_model* m = v->file;
    if (parse(m, err, errlen) != 0) { ora_vision_close(v); return NULL; }
    const ora_kv* arch = find_kv(m, "general.architecture");
    if (!arch || arch->vtype != 8 || strcmp(arch->sval, "clip") != 0) {
        set_err(err, errlen, "image encoder architecture is not clip"); ora_vision_close(v); return NULL;
    }
    const ora_kv* pt = find_kv(m, "clip.vision.projector_type");
    if (!pt || pt->vtype != 8 || strcmp(pt->sval, "gemma3") != 0) {
        set_err(err, errlen, "image projector is not gemma3"); ora_vision_close(v); return NULL;
    }
    const ora_kv* eps = find_kv(m, "clip.vision.attention.layer_norm_epsilon");
    if (vmeta_int(m, "clip.vision.block_count", &v->layers, err, errlen) ||
        vmeta_int(m, "clip.vision.embedding_length", &v->hidden, err, errlen) ||
        vmeta_int(m, "clip.vision.attention.head_count", &v->heads, err, errlen) ||
        vmeta_int(m, "clip.vision.feed_forward_length", &v->ff, err, errlen) ||
        vmeta_int(m, "clip.vision.patch_size", &v->patch, err, errlen) ||
        vmeta_int(m, "clip.vision.projection_dim", &v->proj, err, errlen) ||
        vmeta_int(m, "clip.vision.projector.scale_factor", &v->merge, err, errlen) || !eps) {
        if (!eps) set_err(err, errlen, "image encoder file lacks metadata key clip.vision.attention.layer_norm_epsilon");
        ora_vision_close(v);
        return NULL;
    }
    v->eps = (eps->vtype == 6 || eps->vtype == 12) ? (float)eps->fval : (float)eps->ival;
    if (v->layers > ORA_VIT_MAX_LAYERS || v->hidden % v->heads) { set_err(err, errlen, "bad image encoder shape"); ora_vision_close(v); return NULL; }
    const int d = v->hidden, area = 3 * v->patch * v->patch;
    const ora_tensor* pos = find_tensor(m, "v.position_embd.weight");
    if (!pos || pos->ndim != 3 || pos->shape[0] != d || pos->shape[2] != 2 || pos->type != ORA_F32) {
        set_err(err, errlen, "image encoder file lacks a [hidden, positions, 2] F32 v.position_embd.weight");
        ora_vision_close(v);
        return NULL;
    }
    v->npos = (int)pos->shape[1];
    v->pos = (const float*)tensor_data(m, pos);
    int failed = 0;
    char nm[96];
#define VT_(name, c, r, f32) (tensor_checked(m, name, c, r, f32, 0, err, errlen, &failed))
    const ora_tensor *pw = VT_("v.patch_embd.weight", area, d, 0), *pb = VT_("v.patch_embd.bias", d, 1, 1),
                     *qw = VT_("mm.input_projection.weight", d, v->proj, 0), *nw = VT_("mm.soft_emb_norm.weight", d, 1, 1),
                     *plw = VT_("v.post_ln.weight", d, 1, 1), *plb = VT_("v.post_ln.bias", d, 1, 1);
    if (failed) { ora_vision_close(v); return NULL; }
    v->patch_w = dequant(m, pw);
    v->proj_w = dequant(m, qw);
    v->patch_b = (const float*)tensor_data(m, pb);
    v->norm_w = (const float*)tensor_data(m, nw);
    v->post_w = (const float*)tensor_data(m, plw);
    v->post_b = (const float*)tensor_data(m, plb);
    for (int l = 0; l < v->layers && !failed; l++) {
        ora_vit_layer* L = &v->layer[l];
#define VL_(suffix, c, r, f32) (snprintf(nm, sizeof(nm), "v.blk.%d." suffix, l), VT_(nm, c, r, f32))
        const ora_tensor *l1w = VL_("ln1.weight", d, 1, 1), *l1b = VL_("ln1.bias", d, 1, 1), *l2w = VL_("ln2.weight", d, 1, 1),
                         *l2b = VL_("ln2.bias", d, 1, 1), *wq = VL_("attn_q.weight", d, d, 0), *wk = VL_("attn_k.weight", d, d, 0),
                         *wv = VL_("attn_v.weight", d, d, 0), *wo = VL_("attn_out.weight", d, d, 0),
                         *bq = VL_("attn_q.bias", d, 1, 1), *bk = VL_("attn_k.bias", d, 1, 1), *bv = VL_("attn_v.bias", d, 1, 1),
                         *bo = VL_("attn_out.bias", d, 1, 1), *wu = VL_("ffn_up.weight", d, v->ff, 0),
                         *bu = VL_("ffn_up.bias", v->ff, 1, 1), *wd = VL_("ffn_down.weight", v->ff, d, 0),
                         *bd = VL_("ffn_down.bias", d, 1, 1);
#undef VL_
        if (failed) break;
        L->ln1_w = (const float*)tensor_data(m, l1w); L->ln1_b = (const float*)tensor_data(m, l1b);
        L->ln2_w = (const float*)tensor_data(m, l2w); L->ln2_b = (const float*)tensor_data(m, l2b);
        L->bq = (const float*)tensor_data(m, bq); L->bk = (const float*)tensor_data(m, bk);
        L->bv = (const float*)tensor_data(m, bv); L->bo = (const float*)tensor_data(m, bo);
        L->bup = (const float*)tensor_data(m, bu); L->bdown = (const float*)tensor_data(m, bd);
        L->wq = dequant(m, wq); L->wk = dequant(m, wk); L->wv = dequant(m, wv); L->wo = dequant(m, wo);
        L->wup = dequant(m, wu); L->wdown = dequant(m, wd);
    }
#undef VT_
    if (failed) { ora_vision_close(v); return NULL; }
    return v;
}

void ora_vision_close(ora_vision* v) {
    if (!v) return;
    for (int l = 0; l < ORA_VIT_MAX_LAYERS; l++) {
        ora_vit_layer* L = &v->layer[l];
        free(L->wq); free(L->wk); free(L->wv); free(L->wo); free(L->wup); free(L->wdown);
    }
    free(v->patch_w);
    free(v->proj_w);
    ora_close(v->file);
    free(v);
}

int ora_vision_hidden(const ora_vision* v) { return v->hidden; }
int ora_vision_proj_dims(const ora_vision* v) { return v->proj; }
int ora_vision_merge(const ora_vision* v) { return v->merge; }
int ora_vision_patch_area(const ora_vision* v) { return 3 * v->patch * v->patch; }
int ora_vision_layers(const ora_vision* v) { return v->layers; }

/* One image: patches [gx * gy][3 p^2] (patch i at column i % gx, row i / gx) -> vectors
 * [(gx / merge) * (gy / merge)][proj]. */
int ora_vision_forward(ora_vision* v, const float* patches, int grid_x, int grid_y, float* vectors, ora_trace_fn trace,
                       void* user, int threads) {
    if (grid_x <= 0 || grid_y <= 0 || grid_x % v->merge || grid_y % v->merge || grid_x > v->npos || grid_y > v->npos)
        return -1;
    const int P = grid_x * grid_y, d = v->hidden, H = v->heads, hd = d / H, ff = v->ff, area = 3 * v->patch * v->patch;
    const int T = (grid_x / v->merge) * (grid_y / v->merge);
    const size_t Pd = (size_t)P * d;
    float* x = (float*)malloc(Pd * sizeof(float));
    float* h = (float*)malloc(Pd * sizeof(float));
    float* q = (float*)malloc(Pd * sizeof(float));
    float* k = (float*)malloc(Pd * sizeof(float));
    float* vv = (float*)malloc(Pd * sizeof(float));
    float* attn = (float*)malloc(Pd * sizeof(float));
    float* o = (float*)malloc(Pd * sizeof(float));
    float* u = (float*)malloc((size_t)P * ff * sizeof(float));
    float* pooled = (float*)malloc((size_t)T * d * sizeof(float));
    float* pn = (float*)malloc((size_t)T * d * sizeof(float));

    ora_matmul(patches, P, area, v->patch_w, d, x, threads);
    trace_emit(trace, user, "inp", -1, x, Pd);
    for (int t = 0; t < P; t++) {
        const float* rx = v->pos + (size_t)(t % grid_x) * d;
        const float* ry = v->pos + (size_t)(v->npos + t / grid_x) * d;
        float* xr = x + (size_t)t * d;
        for (int i = 0; i < d; i++) xr[i] = ((xr[i] + v->patch_b[i]) + rx[i]) + ry[i];
    }
    trace_emit(trace, user, "pos_embd", -1, x, Pd);
    const float scale = 1.0f / sqrtf((float)hd);
    for (int l = 0; l < v->layers; l++) {
        const ora_vit_layer* L = &v->layer[l];
        ora_layernorm(x, P, d, L->ln1_w, L->ln1_b, v->eps, h);
        trace_emit(trace, user, "layer_inp_normed", l, h, Pd);
        ora_matmul(h, P, d, L->wq, d, q, threads);
        ora_matmul(h, P, d, L->wk, d, k, threads);
        ora_matmul(h, P, d, L->wv, d, vv, threads);
        for (int t = 0; t < P; t++)
            for (int i = 0; i < d; i++) {
                const size_t idx = (size_t)t * d + i;
                q[idx] += L->bq[i];
                k[idx] += L->bk[i];
                vv[idx] += L->bv[i];
            }
        trace_emit(trace, user, "Qcur", l, q, Pd);
        trace_emit(trace, user, "Kcur", l, k, Pd);
        trace_emit(trace, user, "Vcur", l, vv, Pd);
        ora_attention(q, k, vv, P, H, H, hd, scale, 0, attn, threads);
        trace_emit(trace, user, "kqv_out", l, attn, Pd);
        ora_matmul(attn, P, d, L->wo, d, o, threads);
        trace_emit(trace, user, "attn_out", l, o, Pd);
        for (int t = 0; t < P; t++)
            for (int i = 0; i < d; i++) x[(size_t)t * d + i] += o[(size_t)t * d + i] + L->bo[i];
        trace_emit(trace, user, "ffn_inp", l, x, Pd);
        ora_layernorm(x, P, d, L->ln2_w, L->ln2_b, v->eps, h);
        trace_emit(trace, user, "ffn_inp_normed", l, h, Pd);
        ora_matmul(h, P, d, L->wup, ff, u, threads);
        for (int t = 0; t < P; t++)
            for (int i = 0; i < ff; i++) {
                const size_t idx = (size_t)t * ff + i;
                u[idx] = ora_gelu_tanh(u[idx] + L->bup[i]);
            }
        trace_emit(trace, user, "ffn_gelu", l, u, (size_t)P * ff);
        ora_matmul(u, P, ff, L->wdown, d, o, threads);
        trace_emit(trace, user, "ffn_out", l, o, Pd);
        for (int t = 0; t < P; t++)
            for (int i = 0; i < d; i++) x[(size_t)t * d + i] += o[(size_t)t * d + i] + L->bdown[i];
        trace_emit(trace, user, "layer_out", l, x, Pd);
    }
    ora_layernorm(x, P, d, v->post_w, v->post_b, v->eps, h);
    ora_pool(h, grid_x, grid_y, v->merge, d, pooled);
    trace_emit(trace, user, "pooled", -1, pooled, (size_t)T * d);
    ora_rmsnorm(pooled, T, d, v->norm_w, v->eps, 1.0f, pn);
    trace_emit(trace, user, "pooled_normed", -1, pn, (size_t)T * d);
    ora_matmul(pn, T, d, v->proj_w, v->proj, vectors, threads);
    trace_emit(trace, user, "projected", -1, vectors, (size_t)T * v->proj);
    free(x); free(h); free(q); free(k); free(vv); free(attn); free(o); free(u); free(pooled); free(pn);
    return 0;
}
