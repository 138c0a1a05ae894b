/*
 * CPU oracle for the GemmaEmbed text-encoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C fp32 restatement of the reference's CPU
 * oracle (Sources/GemmaEmbed/Model/CPUReference.swift) used to check the HIP path. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * as the checker or the timed CPU baseline. The product library never links or calls it.
 *
 * Every function cites the reference file:line it follows. Pinning (what checks each
 * function against something other than itself) lives in tests/test_oracle.py.
 */
#ifndef GE_ORACLE_H
#define GE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types the reference accepts: Sources/GemmaEmbed/GGUF/GGUFValue.swift:84-89 */
enum { ORA_F32 = 0, ORA_F16 = 1, ORA_Q8_0 = 8, ORA_BF16 = 30 };

typedef struct ora_model ora_model;

/* Trace callback: named intermediate (llama.cpp names, CPUReference.swift:204-276).
 * layer is -1 for tensors outside the layer loop. */
typedef void (*ora_trace_fn)(void* user, const char* name, int layer, const float* data, size_t count);

/* Opens a GGUF written in the reference's layout (ModelConfig.swift:54-112, Weights.swift:92-132).
 * Returns NULL and fills err on failure. */
ora_model* ora_open(const char* path, char* err, int errlen);
void ora_close(ora_model* m);

/* Model facts for tests. */
int ora_hidden(const ora_model* m);
int ora_output_dims(const ora_model* m);
int ora_layers(const ora_model* m);
int ora_vocab(const ora_model* m);

/* One sequence -> unnormalised mean-pooled vector (CPUReference.swift:183-283).
 * threads <= 0 uses every core. Returns 0 on success. */
int ora_forward(ora_model* m, const int32_t* tokens, int T, float* pooled, ora_trace_fn trace, void* user,
                int threads);
/* The same over token and vector rows (CPUReference.swift:190-202): an id -(r + 1) selects row r of
 * `vectors` ([n_vectors][hidden] fp32), entered unscaled. Returns nonzero for a row past n_vectors. */
int ora_forward_rows(ora_model* m, const int32_t* tokens, int T, const float* vectors, int n_vectors, float* pooled,
                     ora_trace_fn trace, void* user, int threads);

/* Primitives, exposed for known-answer tests. */
void ora_dequant_row(int type, const void* row, int cols, float* out);
float ora_half_to_float(uint16_t h);
uint16_t ora_float_to_half(float f);
void ora_matmul(const float* x, int m, int k, const float* w, int n, float* y, int threads);
void ora_rmsnorm(const float* x, int rows, int width, const float* weight, float eps, float prescale, float* out);
float ora_gelu_tanh(float x);
void ora_rope_table(int head_dim, float base, int positions, float* out);
void ora_rope(float* x, int tokens, int heads, int head_dim, const float* table, const int32_t* positions);
void ora_attention(const float* q, const float* k, const float* v, int tokens, int heads, int kv_heads,
                   int head_dim, float scale, int window, float* out, int threads);

/* ---- image tower, Model/CPUVisionReference.swift:89-165 in structure. */
typedef struct ora_vision ora_vision;
ora_vision* ora_vision_open(const char* path, char* err, int errlen);
void ora_vision_close(ora_vision* v);
int ora_vision_hidden(const ora_vision* v);
int ora_vision_proj_dims(const ora_vision* v);
int ora_vision_merge(const ora_vision* v);
int ora_vision_patch_area(const ora_vision* v);
int ora_vision_layers(const ora_vision* v);
/* One image's patches [gx * gy][3 p^2] -> vectors [(gx / merge) (gy / merge)][proj]. */
int ora_vision_forward(ora_vision* v, const float* patches, int grid_x, int grid_y, float* vectors, ora_trace_fn trace,
                       void* user, int threads);
void ora_layernorm(const float* x, int rows, int width, const float* w, const float* b, float eps, float* out);
void ora_pool(const float* x, int grid_x, int grid_y, int merge, int width, float* out);

#ifdef __cplusplus
}
#endif
#endif
