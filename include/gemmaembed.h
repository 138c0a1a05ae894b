/*
 * gemmaembed.h - C-ABI of the MI355X-native GemmaEmbed text-encoder forward pass.
 *
 * Two layers, both plain C (no HIP or torch types in any signature):
 *
 *  1. The device library (ge_ctx): the replacement for the reference's Metal runtime
 *     (Sources/GemmaEmbed/Metal/MetalContext.swift, MetalForward.swift). The Swift host's
 *     EmbeddingModel would bind these through a SwiftPM C target.
 *  2. The host mirror (ge_model): EmbeddingModel.load / embed / batches / finish
 *     (Sources/GemmaEmbed/EmbeddingModel.swift) and the GGUF loader (GGUF/GGUFFile.swift),
 *     written in C++ because no Swift toolchain is available.
 *
 * Conventions (replacing Swift `throws GemmaEmbedError`, Errors.swift:6-24):
 *  - every call returns an int status, GE_OK (0) on success;
 *  - ge_last_error(ctx) / ge_model_last_error(model) give the message of the last failure;
 *  - invalid shapes and arguments return GE_ERR_INVALID instead of trapping.
 * Threading (EmbeddingModel.swift:37,274-281 serialises every call on one queue): one context
 * is externally synchronised; use one context per GPU.
 */
#ifndef GEMMAEMBED_H
#define GEMMAEMBED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Each maps onto one GemmaEmbedError case (Errors.swift:6-24). */
enum {
    GE_OK = 0,
    GE_ERR_INVALID = 1,    /* bad argument or shape (reference: precondition trap) */
    GE_ERR_GGUF = 2,       /* GemmaEmbedError.invalidGGUF / fileNotReadable */
    GE_ERR_MODEL = 3,      /* missingTensor / missingMetadata / tensorShapeMismatch / unsupportedTensorType / unsupportedArchitecture */
    GE_ERR_GPU = 4,        /* GemmaEmbedError.gpuFailure (a HIP call failed) */
    GE_ERR_OPTIONS = 5,    /* GemmaEmbedError.invalidOptions */
    GE_ERR_STATE = 6,      /* no model uploaded / no batch staged */
    GE_ERR_CANCELLED = 7,  /* GemmaEmbedError.cancelled */
    GE_ERR_NO_DEVICE = 8   /* GemmaEmbedError.noMetalDevice */
};

/* ggml tensor types the loader accepts (GGUF/GGUFValue.swift:84-89). */
enum { GE_TYPE_F32 = 0, GE_TYPE_F16 = 1, GE_TYPE_Q8_0 = 8, GE_TYPE_BF16 = 30 };

/* ===================================================================== device library */

typedef struct ge_ctx ge_ctx;

/* MetalContext(device:) (Metal/MetalContext.swift:23-44): selects HIP device `device`, creates the
 * stream and events. On failure *out is NULL and ge_create_error() holds the message. */
int ge_create(int device, ge_ctx** out);
void ge_destroy(ge_ctx* ctx);
const char* ge_last_error(const ge_ctx* ctx);
const char* ge_create_error(void);
/* Device name (ModelInfo.deviceName, Model/ModelConfig.swift:26). */
const char* ge_device_name(const ge_ctx* ctx);

/* One tensor of the weight file: name, byte offset from `file_base`, ggml type and GGUF `ne`
 * shape (fastest dimension first), as GGUFTensorInfo (GGUF/GGUFValue.swift:117-131). */
typedef struct ge_tensor_desc {
    const char* name;
    uint64_t offset;
    int32_t type;
    int32_t ndim;
    int64_t shape[4];
} ge_tensor_desc;

/* Shapes and constants of the text encoder (ModelConfig.swift:54-112, LayerConfig :34-40).
 * per_layer_input = 0 means the model has no per-layer-input branch. */
typedef struct ge_model_desc {
    int32_t layers, hidden, heads, feed_forward, out_dims, per_layer_input, vocab, sliding_window, max_tokens;
    float eps, embedding_scale, per_layer_scale;
    const int32_t* kv_heads;  /* [layers] */
    const int32_t* head_dim;  /* [layers] */
    const uint8_t* sliding;   /* [layers], 1 = sliding-window layer */
    const float* rope_base;   /* [layers] */
    const float* out_scale;   /* [layers], layer_output_scale (1 when absent) */
    const ge_tensor_desc* tensors;
    int32_t n_tensors;
} ge_model_desc;

/* Replaces MetalForward.init's no-copy MTLBuffer over the mmap (Metal/MetalForward.swift:85-112):
 * the weights are copied into HBM and Q8_0 matrices are repacked into separate int8 quant and
 * fp16 scale planes. The caller may unmap the file afterwards. */
int ge_upload_model(ge_ctx* ctx, const ge_model_desc* desc, const void* file_base, size_t len);

/* Precision of the attention scores, read by the next ge_upload_model: layers whose head dim is at
 * least `min_head_dim` run the QKV projection on hi/lo fp16 operand pairs and score
 * q_hi.k_hi + q_lo.k_hi + q_hi.k_lo (near-fp32 scores, as the reference's fp32 attention,
 * Shaders/Attention.metal:172-188), where the query grouping allows it (head dim 512 with 4 query
 * heads per KV head, 256 with 3). Default 512: the reference's global layers. 0 asks for every
 * such layer, at about twice the QKV and score work there. No counterpart in the reference, whose
 * GPU path is fp32 throughout; for callers that need its 1e-4 agreement on short texts. */
int ge_set_split_scores(ge_ctx* ctx, int32_t min_head_dim);

/* SequenceRange (Shaders/Common.metal:86-89): one packed sequence. */
typedef struct ge_seq {
    uint32_t start;
    uint32_t length;
} ge_seq;

/* MetalForward.run / timeForward (Metal/MetalForward.swift:199-209): one packed batch, tokens
 * back to back, positions restarting at 0 per sequence (PackedBatch.append :17-21). Writes the
 * unnormalised mean-pooled vectors, n_seqs x out_dims fp32, into caller-owned `pooled_out`.
 * `gpu_seconds` (nullable) receives the GPU time of the forward. Synchronous. Token ids are in
 * [0, vocab), or -(r + 1) for row r of the vector rows ge_set_vectors uploaded (PackedBatch's
 * convention, :6-7), entered into the residual stream unscaled (Shaders/Elementwise.metal:25-29). */
int ge_forward(ge_ctx* ctx, const int32_t* tokens, const int32_t* positions, int32_t n_tokens, const ge_seq* seqs,
               int32_t n_seqs, float* pooled_out, double* gpu_seconds);

/* ge_forward with no device allocation: no counterpart in the reference; for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid hipMalloc). Same arguments,
 * results bitwise those of ge_forward. The forward's workspace (activations, staged ids and work
 * lists, V^T, pooled output) lives in a 64 MiB device array of the library, one per GPU, held
 * until the process ends; its address is taken at ge_create. Packs of 4096 tokens or more are
 * refused with GE_ERR_INVALID, and so is a smaller pack whose workspace does not fit (above about
 * 2650 tokens for config 2's model, 380 for the reference's architecture with its per-layer
 * inputs), as is a call while profiling is enabled. Synchronous like ge_forward: it clears its
 * region with hipMemsetAsync, waits for its stream and reads back with a blocking copy, so it is
 * not for HIP graph capture. Calls on one GPU share the array: calls that overlap (two contexts of
 * one GPU used from two threads) race. The context's own staged batch and workspace are left as
 * they were. */
int ge_forward_noalloc(ge_ctx* ctx, const int32_t* tokens, const int32_t* positions, int32_t n_tokens,
                       const ge_seq* seqs, int32_t n_seqs, float* pooled_out, double* gpu_seconds);

/* The workspace's `vectors` buffer (Metal/MetalForward.swift:137,165), filled from the host: fp32
 * [n_rows][width] copied into HBM, where the batches of ge_forward, ge_forward_trace and
 * ge_batch_stage find the rows their negative ids name. Rows are used only while `width` equals
 * the model's hidden size; n_rows 0 clears them. Kept until replaced. A staged batch reads the
 * rows present when it runs; a replacement that needs a larger buffer drops a staged batch that
 * reads them (run it again after staging it again). */
int ge_set_vectors(ge_ctx* ctx, const float* rows, int32_t n_rows, int32_t width);

/* Per-layer parity (CPUReference.forward's trace, Model/CPUReference.swift:204-276, and
 * MetalForward.attentionInputs :278-284): runs the forward up to the op that produces the named
 * tensor at `layer` (-1 for inp_scaled, result_norm, result_embd) and copies it out as fp32
 * [n_tokens][width]. Names: inp_scaled, attn_norm, Qcur, Kcur, Vcur, Qcur_pos, Kcur_pos,
 * Vcur_normed, kqv_out, attn_out, ffn_norm, ffn_geglu, ffn_out, pe_in, l_out, result_norm,
 * result_embd, and with the per-layer-input branch inp_per_layer (pe_in is then the residual
 * before the branch, l_out after it; the reference's per_layer_embd_out is not kept on the GPU).
 * `out_count` is the capacity of `out` in floats; the needed count is written to *needed. */
int ge_forward_trace(ge_ctx* ctx, const int32_t* tokens, const int32_t* positions, int32_t n_tokens,
                     const ge_seq* seqs, int32_t n_seqs, const char* tensor_name, int32_t layer, float* out,
                     size_t out_count, size_t* needed);

/* Device-resident batches, for callers that keep inputs in HBM across calls (and the bench):
 * stage uploads tokens/positions/sequences and the attention work list once; run enqueues a
 * forward over the staged batch on the context's stream and returns without waiting; read
 * waits and copies the pooled vectors out. */
int ge_batch_stage(ge_ctx* ctx, const int32_t* tokens, const int32_t* positions, int32_t n_tokens, const ge_seq* seqs,
                   int32_t n_seqs);
int ge_batch_run(ge_ctx* ctx);
int ge_batch_read(ge_ctx* ctx, float* pooled_out);
int ge_sync(ge_ctx* ctx);

/* Kernel timing with HIP events on the context's stream (the reference's Profiler,
 * Metal/Profiler.swift:16-88). While enabled, every launch whose kernel name starts with
 * `prefix` ("" = all) is bracketed by events; stats accumulate per kernel name. */
int ge_profile_enable(ge_ctx* ctx, const char* prefix);
int ge_profile_disable(ge_ctx* ctx);
int ge_profile_reset(ge_ctx* ctx);
/* i-th kernel class: name, launch count and summed milliseconds. Returns GE_ERR_INVALID past the end. */
int ge_profile_get(ge_ctx* ctx, int32_t i, const char** name, int64_t* launches, double* total_ms);

/* ---- per-op entry points on device memory, for unit tests (the reference's `Kernels`,
 * Metal/MetalForward.swift:427-759). Device buffers come from ge_dev_alloc. */
void* ge_dev_alloc(ge_ctx* ctx, size_t bytes);
int ge_dev_free(ge_ctx* ctx, void* ptr);
int ge_dev_upload(ge_ctx* ctx, void* dst, const void* src, size_t bytes);
int ge_dev_download(ge_ctx* ctx, void* dst, const void* src, size_t bytes);

/* fp32 -> fp16 (round to nearest even) and back, elementwise on device. */
int ge_op_f32_to_f16(ge_ctx* ctx, const void* src, void* dst, size_t count);
int ge_op_f16_to_f32(ge_ctx* ctx, const void* src, void* dst, size_t count);

/* A Q8_0 weight matrix (`rows` GGUF rows of `cols` elements, 34-byte blocks, host memory)
 * repacked into device memory. Replaces WeightTensor as GEMM operand (Model/Weights.swift:6-17). */
typedef struct ge_q8_matrix ge_q8_matrix;
int ge_op_q8_create(ge_ctx* ctx, const void* q8_rows, int32_t rows, int32_t cols, ge_q8_matrix** out);
int ge_op_q8_destroy(ge_ctx* ctx, ge_q8_matrix* m);

/* Kernels.gemm (Metal/MetalForward.swift:524-557): y[M][N] = x[M][K] * W^T with x fp16 [M][K]
 * and W [N][K] Q8_0; y fp32 (y_f16 = 0) or fp16 (y_f16 = 1), row stride N. */
int ge_op_gemm_q8(ge_ctx* ctx, const ge_q8_matrix* w, const void* x, int32_t m, void* y, int32_t y_f16);
/* Kernels.gemm with the geglu epilogue (:566-569, Shaders/GEMM.metal:41-67):
 * act[M][F] = gelu_tanh(x * Wg^T) * (x * Wu^T), fp16 out. */
int ge_op_gemm_q8_geglu(ge_ctx* ctx, const ge_q8_matrix* gate, const ge_q8_matrix* up, const void* x, int32_t m,
                        void* act);

/* The forward's row kernels on device memory (fp32 unless stated; widths a multiple of 4 up to
 * 1024). Integer inputs the kernels gather with (ids, positions, sequence ranges) are checked on
 * the host first.
 *
 * Kernels.rmsNorm (Metal/MetalForward.swift:502-511; Shaders/Elementwise.metal:38-75):
 * out[r] = rmsnorm(x[r] * pre_scale) * w over `rows` rows of `width`; w nullable (no weight); out
 * may be x. */
int ge_op_rmsnorm(ge_ctx* ctx, const void* x, void* out, const void* w, int32_t rows, int32_t width, float eps,
                  float pre_scale);
/* Kernels.rmsNormResidual and rmsNormResidualNorm (Metal/MetalForward.swift:615-643;
 * Shaders/Elementwise.metal:260-354): x = (x + rmsnorm(t) * w) * scale in place, with the sublayer
 * output t in fp16 (as the forward stores it); with next_w set, also h16 = rmsnorm(x) * next_w in
 * fp16. */
int ge_op_rmsnorm_residual(ge_ctx* ctx, void* x, const void* t16, const void* w, float scale, const void* next_w,
                           void* h16, int32_t rows, int32_t width, float eps);
/* Kernels.rmsNormRope (Metal/MetalForward.swift:655-667; Shaders/Elementwise.metal:97-141) with the V
 * norm (:394), as the forward runs them on the QKV projection: qkv [tokens][(heads + 2 kv_heads)
 * head_dim] -> q fp16 [tokens][heads][head_dim] (weighted RMSNorm, NeoX RoPE), k fp16 likewise with
 * k_norm, v fp16 (unweighted RMSNorm). positions: device int32 [tokens] in [0, 8192); the RoPE
 * table of (head_dim, rope_base) is computed in fp64 (Model/RopeTable.swift:16-31). head_dim 128,
 * 256 or 512. */
int ge_op_qk_norm_rope(ge_ctx* ctx, const void* qkv, int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim,
                       const void* q_norm, const void* k_norm, float eps, const void* positions, float rope_base, void* q,
                       void* k, void* v);
/* Kernels.embed (Metal/MetalForward.swift:490-500; Shaders/Elementwise.metal:8-35), fused with the
 * first RMSNorm as the forward runs it: x[t] = dequant(table[id]) * scale for id >= 0, row
 * -(id + 1) of `vectors` (device fp32 [n_vectors][cols]) unscaled for id < 0; h16 (nullable) =
 * rmsnorm(x) * norm_w in fp16. tokens: device int32 [n_tokens] in [-n_vectors, table rows). */
int ge_op_embed(ge_ctx* ctx, const ge_q8_matrix* table, const void* tokens, int32_t n_tokens, float scale,
                const void* vectors, int32_t n_vectors, const void* norm_w, float eps, void* x, void* h16);
/* Kernels.meanPool (Metal/MetalForward.swift:751-758; Shaders/Elementwise.metal:243-256):
 * pooled[s] = mean of rows [start, start + length) of x [rows][width]; seqs: device ge_seq [n_seqs]
 * inside the rows (an empty sequence pools to 0). width a multiple of 4; x and pooled 16-byte
 * aligned. */
int ge_op_mean_pool(ge_ctx* ctx, const void* x, int32_t rows, int32_t width, const void* seqs, int32_t n_seqs,
                    void* pooled);

/* AttentionWork (Shaders/Common.metal:75-79): a block of query rows of one sequence. */
typedef struct ge_attention_work {
    uint32_t seq_start;
    uint32_t seq_len;
    uint32_t q0;
} ge_attention_work;

/* Rows of queries one attention work item covers (the reference's queriesPerGroup). */
int32_t ge_attention_queries(void);

/* Kernels.attention (Metal/MetalForward.swift:669-694; Shaders/Attention.metal:25-170): q fp16
 * [T][heads][hd], k and v fp16 [T][kv_heads][hd], out fp16 [T][heads][hd]; `work` is a device
 * array of n_work items covering each sequence's queries from q0 = 0 in steps of
 * ge_attention_queries(); half_window 0 = no window; scale multiplies the scores. q, k and v
 * must hold 64 rows of slack past the last token (key blocks are read whole). */
int ge_op_attention(ge_ctx* ctx, const void* q, const void* k, const void* v, void* out, const void* work,
                    int32_t n_work, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t half_window,
                    float scale);

/* Kernels.attention at split precision (the forward's head-dim-512 layers; reference fp32 scores,
 * Shaders/Attention.metal:172-188): q and k as fp16 pairs, q_lo = fp16(q - q_hi) beside q_hi in
 * the same layout, scores q_hi.k_hi + q_lo.k_hi + q_hi.k_lo. head_dim 512 with heads = 4 kv_heads;
 * otherwise as ge_op_attention. */
int ge_op_attention_split(ge_ctx* ctx, const void* q, const void* q_lo, const void* k, const void* k_lo, const void* v,
                          void* out, const void* work, int32_t n_work, int32_t heads, int32_t kv_heads, int32_t head_dim,
                          int32_t half_window, float scale);

/* ---- image tower, on the same context as the text encoder.
 * Replaces Metal/VisionTower.swift (VisionTower.upload :113-140, encode :143-185) for a
 * pre-LayerNorm ViT: per layer x += attn_out(attn(LN1(x))) + b, x += down(gelu_tanh(up(LN2(x)))),
 * heads of hidden / heads dims (72, 128 or 256), then a final LayerNorm, merge x merge mean pooling,
 * a weighted RMSNorm and a Q8_0 projection. Tensors (GGUF names, ne order):
 *   v.patch_embd.weight Q8_0 [3 p^2, hidden] (patch element c p^2 + ky p + kx), v.patch_embd.bias,
 *   v.position_embd.weight F32 [hidden, positions, 2] (column rows, then row rows),
 *   v.blk.N.{ln1,ln2}.{weight,bias}, v.blk.N.attn_{q,k,v,out}.{weight Q8_0, bias},
 *   v.blk.N.ffn_up.{weight Q8_0 [hidden, ff], bias}, v.blk.N.ffn_down.{weight F16/F32/BF16/Q8_0 [ff, hidden], bias},
 *   v.post_ln.{weight,bias}, mm.soft_emb_norm.weight, mm.input_projection.weight Q8_0 [hidden, proj_dims];
 * vectors F32. */
typedef struct ge_vision_desc {
    int32_t layers, hidden, heads, feed_forward, patch_size, merge, proj_dims, positions;
    float eps;
    const ge_tensor_desc* tensors;
    int32_t n_tensors;
} ge_vision_desc;
int ge_upload_vision(ge_ctx* ctx, const ge_vision_desc* desc, const void* file_base, size_t len);

/* One image of a batch: its patch grid (PreparedImage.gridX / gridY, Image/ImagePreprocessor.swift:6-61),
 * both multiples of the merge size. Images follow each other as patch rows (row-major over the
 * grid) and as pooled tokens ((grid_x / merge) * (grid_y / merge) each, row-major). */
typedef struct ge_image_grid {
    int32_t grid_x, grid_y;
} ge_image_grid;

/* The uploaded tower's shapes (VisionConfig, Model/VisionConfig.swift:44-81): patch_area =
 * 3 patch_size^2 floats per patch row, merge x merge patches pool into one output token of
 * proj_dims floats. GE_ERR_STATE without a tower. */
typedef struct ge_vision_info {
    int32_t layers, hidden, heads, patch_size, patch_area, merge, proj_dims, positions;
} ge_vision_info;
int ge_vision_get_info(ge_ctx* ctx, ge_vision_info* info);

/* VisionTower.upload + encode + read back: patches fp32 [n_patches][patch_area] -> vectors fp32
 * [tokens][proj_dims] (caller-owned, capacity vectors_count floats; tokens = sum of the images'
 * pooled tokens; GE_ERR_INVALID when it does not fit). Synchronous. */
int ge_vision_encode(ge_ctx* ctx, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images,
                     float* vectors, size_t vectors_count, double* gpu_seconds);
/* Device-resident image batches (as ge_batch_*): stage uploads the patches and descriptors, run
 * enqueues the tower without waiting, read waits and copies the vectors out (capacity
 * vectors_count floats). */
int ge_vision_stage(ge_ctx* ctx, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images);
int ge_vision_run(ge_ctx* ctx);
int ge_vision_read(ge_ctx* ctx, float* vectors, size_t vectors_count);
/* Pooled tokens of the staged image batch, or -1 when none is staged. */
int32_t ge_vision_tokens(ge_ctx* ctx);
/* Per-layer parity (CPUVisionReference.forward's trace, Model/CPUVisionReference.swift:89-165):
 * stages the batch, runs up to the named tensor and copies it out as fp32. Names (layer -1): inp
 * (patch projection, no bias), pos_embd, pooled, pooled_normed, projected; per layer:
 * layer_inp_normed, Qcur, Kcur, Vcur (with bias, [patches][heads][hd]), kqv_out, attn_out (no
 * bias), ffn_inp, ffn_inp_normed, ffn_gelu, ffn_out (no bias), layer_out. */
/* MetalForward.run(images:) (Metal/MetalForward.swift:213-219): the tower over the images, then
 * the text tower over each image's [bos, begin, its vectors, end, eos] (markers[4] = {bos, begin,
 * end, eos}: the vocabulary ids of <bos>, <|image>, <image|>, <eos>, each in [0, vocab);
 * Model/InputRow.swift:16-56), reading the
 * tower's output rows in HBM. Writes n_images x out_dims unnormalised pooled vectors into
 * `pooled_out`; `gpu_seconds` (nullable) covers both towers. Needs an uploaded text model whose
 * hidden size is the tower's projection width. Synchronous. */
int ge_image_forward(ge_ctx* ctx, const float* patches, int32_t n_patches, const ge_image_grid* grids,
                     int32_t n_images, const int32_t* markers, float* pooled_out, double* gpu_seconds);
int ge_vision_trace(ge_ctx* ctx, const float* patches, int32_t n_patches, const ge_image_grid* grids, int32_t n_images,
                    const char* tensor_name, int32_t layer, float* out, size_t out_count, size_t* needed);

/* ===================================================================== host mirror */

typedef struct ge_model ge_model;

/* LoadOptions (EmbedOptions.swift:172-203) for the text path. */
typedef struct ge_load_options {
    int32_t device;              /* HIP device ordinal */
    int32_t batch_token_budget;  /* default 8192; at least 64 (EmbeddingModel.swift:110) */
    int32_t warm_up;             /* run one small forward at load (EmbeddingModel.swift:111-114) */
    int32_t split_scores;        /* nonzero: split-precision scores on every layer that allows them
                                    (ge_set_split_scores(ctx, 0)); no counterpart in LoadOptions */
    int32_t pack_tokens;         /* largest device pack of ge_model_embed, in tokens. 0 (default) =
                                    batch_token_budget: one forward per planned batch, as
                                    EmbeddingModel.swift:157-172 runs them. Larger values run
                                    consecutive planned batches as one forward of up to this many
                                    tokens (same vectors, better GPU use); a cancel then takes
                                    effect at the next forward. No counterpart in LoadOptions. */
} ge_load_options;

/* EmbedOptions (EmbedOptions.swift:35-56), minus the task prefix: prefixes and tokenization
 * happen before the token ids reach this API. */
typedef struct ge_embed_options {
    int32_t max_tokens;  /* 2 ... max_tokens of the model; default 2048 */
    int32_t dimensions;  /* 768, 512, 256 or 128 */
    int32_t normalise;   /* L2-normalise the output */
    int32_t batch_size;  /* texts per batch; 0 = pack by token count */
} ge_embed_options;

/* ModelInfo (Model/ModelConfig.swift:6-32). */
typedef struct ge_model_info {
    char architecture[64];
    char name[128];
    int32_t layers, hidden, out_dims, feed_forward, per_layer_input, heads, vocab, sliding_window, max_tokens;
    float eps;
    char quantization[16];
    char device_name[128];
    int64_t file_size;
    int32_t bos_id, eos_id;
} ge_model_info;

/* EmbeddingProgress (EmbedOptions.swift:165-169); returning non-zero cancels between batches. */
typedef int (*ge_progress_fn)(void* user, int32_t completed_texts, int32_t total_texts, int64_t completed_tokens);

/* EmbeddingModel.load(from:options:) (EmbeddingModel.swift:40-122): GGUF parse and validation,
 * context creation, weight upload, warm forward. err receives the message on failure. */
int ge_model_load(const char* path, const ge_load_options* options, ge_model** out, char* err, size_t errlen);
void ge_model_free(ge_model* model);
const char* ge_model_last_error(const ge_model* model);
int ge_model_get_info(const ge_model* model, ge_model_info* info);
/* The model's device context, for ge_forward_trace / ge_profile_* on a loaded model. */
ge_ctx* ge_model_context(ge_model* model);

/* The GGUF reader alone, on the host (GGUFFile(url:), GGUF/GGUFFile.swift:21-67): what the
 * reference's GGUFReaderTests check against Fixtures/model.json. ge_gguf_counts: GGUF version,
 * metadata key count, tensor count, data section offset and file size (each nullable).
 * ge_gguf_tensor: tensor i in file order, offset from the data section's start; the name stays
 * valid until ge_gguf_close. ge_gguf_text_config: ModelConfig.init and the weight directory's
 * checks (Model/ModelConfig.swift:54-112, Model/Weights.swift:92-132) as a ModelInfo with an
 * empty device name. */
typedef struct ge_gguf ge_gguf;
int ge_gguf_open(const char* path, ge_gguf** out, char* err, size_t errlen);
void ge_gguf_close(ge_gguf* g);
int ge_gguf_counts(const ge_gguf* g, uint32_t* version, int64_t* kv_count, int64_t* tensor_count, uint64_t* data_offset,
                   uint64_t* file_size);
int ge_gguf_tensor(const ge_gguf* g, int64_t i, ge_tensor_desc* out);
int ge_gguf_text_config(const ge_gguf* g, ge_model_info* info, char* err, size_t errlen);

/* EmbeddingModel.embed(_:options:progress:) (EmbeddingModel.swift:145-175) over pre-tokenized
 * texts: `tokens` holds n_texts sequences back to back, `lengths[i]` ids each (BOS/EOS included,
 * as the tokenizer returns them). Truncates to max_tokens keeping EOS (:189-196), batches
 * (:200-215), runs, then Matryoshka-truncates and normalises (:260-267). `out` receives
 * n_texts x dimensions floats; token_counts and truncated (both nullable) one entry per text. */
int ge_model_embed(ge_model* model, const int32_t* tokens, const int32_t* lengths, int32_t n_texts,
                   const ge_embed_options* options, float* out, int32_t* token_counts, uint8_t* truncated,
                   ge_progress_fn progress, void* user);

/* EmbeddingModel.embedTokens (EmbeddingModel.swift:285-289): one packed batch of all the
 * sequences, unnormalised pooled out_dims vectors. */
int ge_model_embed_tokens(ge_model* model, const int32_t* tokens, const int32_t* lengths, int32_t n_texts,
                          float* out);

/* EmbeddingModel.batches (EmbeddingModel.swift:200-215): consecutive ranges of at least one
 * item, cut by count when batch_size > 0, else before the item that would take any summed cost
 * past its budget. costs is n_items x n_budgets. Writes range starts (n_ranges + 1 entries, the
 * last = n_items) into `starts` (capacity n_items + 1) and the range count into *n_ranges. */
int ge_plan_batches(const int32_t* costs, int32_t n_items, const int32_t* budgets, int32_t n_budgets,
                    int32_t batch_size, int32_t* starts, int32_t* n_ranges);

/* EmbeddingModel.finish (EmbeddingModel.swift:260-267): prefix to `dimensions`, then L2
 * normalise unless the norm is 0. */
int ge_finish(const float* vector, int32_t width, int32_t dimensions, int32_t normalise, float* out);

/* Synthetic GGUF writer for seeded test and bench models (no reference counterpart: the
 * reference's models are downloaded). Rules: q ~ U{-127..127} per Q8_0 block with fp16 scale
 * |N(0, 0.02)| * max|q| / 127; fp32 norm weights 1 + 0.1 N(0,1); SplitMix64 streams seeded per
 * tensor from (seed, tensor name). per_layer_input = 0 writes no per-layer-input tensors.
 * context_length 0 writes 8192. norm_outliers > 0 replaces that many entries (at random positions)
 * of every residual-stream norm weight (attn_norm, post_attention_norm, ffn_norm, post_ffw_norm,
 * post_norm, output_norm) with +-U(norm_outlier / 6, norm_outlier): trained models' norm weights
 * carry such outliers, which stress the fp16 range scales chosen at load. */
typedef struct ge_synth_spec {
    int32_t layers, hidden, heads, feed_forward, out_dims, per_layer_input, vocab, sliding_window;
    int32_t head_dim_swa, head_dim_global, kv_heads_swa, kv_heads_global;
    float eps, rope_base, rope_base_swa;
    const uint8_t* pattern; /* [layers], 1 = sliding */
    uint64_t seed;
    int32_t context_length;
    int32_t norm_outliers;
    float norm_outlier;
} ge_synth_spec;
int ge_synth_write_gguf(const char* path, const ge_synth_spec* spec, char* err, size_t errlen);

/* Synthetic image-encoder GGUF ("clip" architecture, projector "gemma3") in the layout
 * ge_upload_vision reads (no reference counterpart). Q8_0 matrices as above but with
 * z ~ N(0, 1 / (64 sqrt(K))) for rows of K elements; ffn_down F16 N(0, 1) / sqrt(ff) (or Q8_0 when
 * ffn_down_type is GE_TYPE_Q8_0 and ff % 32 == 0); norm weights 1 + 0.1 N(0, 1); biases
 * 0.1 N(0, 1); position rows 0.5 N(0, 1). */
typedef struct ge_synth_vision_spec {
    int32_t layers, hidden, heads, feed_forward, patch_size, merge, proj_dims, positions;
    float eps;
    int32_t ffn_down_type; /* 0 = F16 */
    uint64_t seed;
} ge_synth_vision_spec;
int ge_synth_write_vision_gguf(const char* path, const ge_synth_vision_spec* spec, char* err, size_t errlen);

/* Loads an image-encoder GGUF (VisionConfig.init, Model/VisionConfig.swift:44-81, and the
 * weight directory, Model/VisionWeights.swift) onto the context through ge_upload_vision. */
int ge_vision_load(ge_ctx* ctx, const char* path, char* err, size_t errlen);

/* SplitMix64 helpers shared by tests and the bench (the reference tests' SeededRandom,
 * Tests/GemmaEmbedTests/KernelTests.swift:9-26): `count` ids uniform in [lo, hi). */
int ge_synth_tokens(uint64_t seed, int32_t lo, int32_t hi, int32_t count, int32_t* out);
/* `count` floats uniform in [lo, hi) from SplitMix64 (53-bit uniforms), e.g. pixel values. */
int ge_synth_uniform(uint64_t seed, float lo, float hi, int64_t count, float* out);

#ifdef __cplusplus
}
#endif
#endif
