// Host mirror of the reference's public text API, over the device C-ABI:
// EmbeddingModel.load / embed / embedTokens / batches / finish
// (Sources/GemmaEmbed/EmbeddingModel.swift:40-289) with EmbedOptions / LoadOptions
// (EmbedOptions.swift:35-56, :172-203). Token ids come in already tokenized: the task prefix
// and the BPE tokenizer run before this boundary.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gemmaembed.h"
#include "gguf.hpp"

struct ge_model {
    std::unique_ptr<ge::GGUFFile> file;
    ge::ModelConfig cfg;
    ge_ctx* ctx = nullptr;
    int budget = 8192;
    int64_t pack_tokens = 8192;  // largest device pack: the budget unless the load options raise it
    std::string err;
    std::string device_name;
    ~ge_model() {
        if (ctx) ge_destroy(ctx);
    }
};

namespace ge {
namespace {

const int kAllowedDimensions[] = {768, 512, 256, 128};  // EmbedOptions.allowedDimensions (:55)

// EmbeddingModel.batches (EmbeddingModel.swift:200-215).
std::vector<int> plan_batches(const int32_t* costs, int n, const int32_t* budgets, int nb, int batch_size) {
    std::vector<int> starts;
    int start = 0;
    std::vector<int64_t> totals(size_t(nb), 0);
    for (int i = 0; i < n; i++) {
        bool full = false;
        if (batch_size > 0) {
            full = i - start >= batch_size;
        } else {
            for (int b = 0; b < nb; b++)
                if (totals[size_t(b)] + costs[size_t(i) * nb + b] > budgets[b]) full = true;
        }
        if (i > start && full) {
            starts.push_back(start);
            start = i;
            std::fill(totals.begin(), totals.end(), 0);
        }
        for (int b = 0; b < nb; b++) totals[size_t(b)] += costs[size_t(i) * nb + b];
    }
    if (start < n) starts.push_back(start);
    starts.push_back(n);
    return starts;
}

// EmbeddingModel.finish (EmbeddingModel.swift:260-267).
void finish(const float* v, int dims, bool normalise, float* out) {
    for (int i = 0; i < dims; i++) out[i] = v[i];
    if (normalise) {
        float ss = 0;
        for (int i = 0; i < dims; i++) ss += out[i] * out[i];
        const float norm = std::sqrt(ss);
        if (norm > 0)
            for (int i = 0; i < dims; i++) out[i] /= norm;
    }
}

int model_fail(ge_model* m, int code, const std::string& msg) {
    m->err = msg;
    return code;
}

// Runs one packed batch through the device (PackedBatch.append restarts positions at 0 per
// sequence, Metal/MetalForward.swift:17-21).
int run_batch(ge_model* m, const std::vector<std::vector<int32_t>>& seqs, std::vector<float>* pooled) {
    std::vector<int32_t> tokens, positions;
    std::vector<ge_seq> ranges;
    for (const auto& s : seqs) {
        ranges.push_back(ge_seq{uint32_t(tokens.size()), uint32_t(s.size())});
        for (size_t i = 0; i < s.size(); i++) {
            tokens.push_back(s[i]);
            positions.push_back(int32_t(i));
        }
    }
    pooled->assign(seqs.size() * size_t(m->cfg.out_dims), 0.0f);
    int rc = ge_forward(m->ctx, tokens.data(), positions.data(), int32_t(tokens.size()), ranges.data(),
                        int32_t(ranges.size()), pooled->data(), nullptr);
    if (rc != GE_OK) m->err = ge_last_error(m->ctx);
    return rc;
}

}  // namespace
}  // namespace ge

namespace ge {

// ModelInfo (Model/ModelConfig.swift:6-32) from a parsed configuration.
void fill_info(const ModelConfig& cfg, const GGUFFile& file, const std::string& device_name, ge_model_info* info) {
    std::memset(info, 0, sizeof(*info));
    std::snprintf(info->architecture, sizeof(info->architecture), "%s", cfg.architecture.c_str());
    std::snprintf(info->name, sizeof(info->name), "%s", cfg.name.c_str());
    std::snprintf(info->quantization, sizeof(info->quantization), "%s", cfg.quantization.c_str());
    std::snprintf(info->device_name, sizeof(info->device_name), "%s", device_name.c_str());
    info->layers = cfg.layers;
    info->hidden = cfg.hidden;
    info->out_dims = cfg.out_dims;
    info->feed_forward = cfg.feed_forward;
    info->per_layer_input = cfg.per_layer_input;
    info->heads = cfg.heads;
    info->vocab = cfg.vocab;
    info->sliding_window = cfg.sliding_window;
    info->max_tokens = cfg.max_tokens;
    info->eps = cfg.eps;
    info->file_size = int64_t(file.size());
    info->bos_id = cfg.bos_id;
    info->eos_id = cfg.eos_id;
}

}  // namespace ge

extern "C" {

int ge_model_load(const char* path, const ge_load_options* options, ge_model** out, char* err, size_t errlen) {
    auto report = [&](int code, const std::string& msg) {
        if (err && errlen) std::snprintf(err, errlen, "%s", msg.c_str());
        return code;
    };
    if (!path || !out) return report(GE_ERR_INVALID, "null argument");
    *out = nullptr;
    ge_load_options opt{0, 8192, 1, 0, 0};
    if (options) opt = *options;
    if (opt.pack_tokens < 0) return report(GE_ERR_OPTIONS, "invalid options: pack_tokens must not be negative");
    std::unique_ptr<ge_model> m(new ge_model);
    try {
        m->file.reset(new ge::GGUFFile(path));
        m->cfg = ge::read_config(*m->file);
    } catch (const ge::Error& e) {
        return report(e.code, e.what());
    } catch (const std::exception& e) {
        // no C++ exception crosses the C boundary (a corrupt file must not terminate the caller)
        return report(GE_ERR_GGUF, std::string("invalid GGUF file: ") + e.what());
    }
    int rc = ge_create(opt.device, &m->ctx);
    if (rc != GE_OK) return report(rc, ge_create_error());
    m->device_name = ge_device_name(m->ctx);
    ge::UploadDesc u;
    ge::make_upload_desc(*m->file, m->cfg, &u);
    if (opt.split_scores) rc = ge_set_split_scores(m->ctx, 0);
    if (rc == GE_OK) rc = ge_upload_model(m->ctx, &u.desc, m->file->base(), m->file->size());
    if (rc != GE_OK) return report(rc, ge_last_error(m->ctx));
    m->budget = opt.batch_token_budget > 0 ? std::max(64, opt.batch_token_budget) : 8192;
    m->pack_tokens = std::max<int64_t>(m->budget, opt.pack_tokens);
    if (opt.warm_up) {
        // EmbeddingModel.swift:111-114: one small forward before the first request.
        std::vector<std::vector<int32_t>> warm{{m->cfg.bos_id, 2 < m->cfg.vocab ? 2 : 0, m->cfg.eos_id}};
        std::vector<float> pooled;
        rc = ge::run_batch(m.get(), warm, &pooled);
        if (rc != GE_OK) return report(rc, m->err);
    }
    *out = m.release();
    return GE_OK;
}

void ge_model_free(ge_model* m) { delete m; }

const char* ge_model_last_error(const ge_model* m) { return m ? m->err.c_str() : "null model"; }

ge_ctx* ge_model_context(ge_model* m) { return m ? m->ctx : nullptr; }

int ge_model_get_info(const ge_model* m, ge_model_info* info) {
    if (!m || !info) return GE_ERR_INVALID;
    ge::fill_info(m->cfg, *m->file, m->device_name, info);
    return GE_OK;
}

// ---- the GGUF reader on its own, host only (GGUFFile, GGUF/GGUFFile.swift:21-67; ModelConfig.init)

struct ge_gguf {
    std::unique_ptr<ge::GGUFFile> file;
};

int ge_gguf_open(const char* path, ge_gguf** out, char* err, size_t errlen) {
    if (!path || !out) return GE_ERR_INVALID;
    *out = nullptr;
    try {
        std::unique_ptr<ge_gguf> g(new ge_gguf);
        g->file.reset(new ge::GGUFFile(path));
        *out = g.release();
        return GE_OK;
    } catch (const ge::Error& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return e.code;
    } catch (const std::exception& e) {
        if (err && errlen) std::snprintf(err, errlen, "invalid GGUF file: %s", e.what());
        return GE_ERR_GGUF;
    }
}

void ge_gguf_close(ge_gguf* g) { delete g; }

int ge_gguf_counts(const ge_gguf* g, uint32_t* version, int64_t* kv_count, int64_t* tensor_count, uint64_t* data_offset,
                   uint64_t* file_size) {
    if (!g) return GE_ERR_INVALID;
    if (version) *version = g->file->version();
    if (kv_count) *kv_count = int64_t(g->file->meta_count());
    if (tensor_count) *tensor_count = int64_t(g->file->tensors().size());
    if (data_offset) *data_offset = g->file->data_offset();
    if (file_size) *file_size = g->file->size();
    return GE_OK;
}

int ge_gguf_tensor(const ge_gguf* g, int64_t i, ge_tensor_desc* out) {
    if (!g || !out || i < 0 || i >= int64_t(g->file->tensors().size())) return GE_ERR_INVALID;
    const ge::TensorInfo& t = g->file->tensors()[size_t(i)];
    if (t.shape.size() > 4) return GE_ERR_GGUF;
    out->name = t.name.c_str();
    out->offset = t.offset;
    out->type = t.type;
    out->ndim = int32_t(t.shape.size());
    for (int k = 0; k < 4; k++) out->shape[k] = k < out->ndim ? t.shape[size_t(k)] : 1;
    return GE_OK;
}

int ge_gguf_text_config(const ge_gguf* g, ge_model_info* info, char* err, size_t errlen) {
    if (!g || !info) return GE_ERR_INVALID;
    try {
        ge::fill_info(ge::read_config(*g->file), *g->file, "", info);
        return GE_OK;
    } catch (const ge::Error& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return e.code;
    } catch (const std::exception& e) {
        if (err && errlen) std::snprintf(err, errlen, "invalid GGUF file: %s", e.what());
        return GE_ERR_GGUF;
    }
}

int ge_plan_batches(const int32_t* costs, int32_t n, const int32_t* budgets, int32_t nb, int32_t batch_size,
                    int32_t* starts, int32_t* n_ranges) {
    if (n < 0 || nb <= 0 || !budgets || !starts || !n_ranges || (n > 0 && !costs)) return GE_ERR_INVALID;
    std::vector<int> s = ge::plan_batches(costs, n, budgets, nb, batch_size);
    for (size_t i = 0; i < s.size(); i++) starts[i] = s[i];
    *n_ranges = int32_t(s.size()) - 1;
    return GE_OK;
}

int ge_finish(const float* v, int32_t width, int32_t dims, int32_t normalise, float* out) {
    if (!v || !out || dims <= 0 || dims > width) return GE_ERR_INVALID;
    ge::finish(v, dims, normalise != 0, out);
    return GE_OK;
}

int ge_model_embed(ge_model* m, const int32_t* tokens, const int32_t* lengths, int32_t n, const ge_embed_options* options,
                   float* out, int32_t* token_counts, uint8_t* truncated, ge_progress_fn progress, void* user) {
    if (!m) return GE_ERR_INVALID;
    ge_embed_options opt{2048, 768, 1, 0};
    if (options) opt = *options;
    bool allowed = false;
    for (int d : ge::kAllowedDimensions) allowed |= opt.dimensions == d;
    if (!allowed) return ge::model_fail(m, GE_ERR_OPTIONS, "invalid options: dimensions must be one of [768, 512, 256, 128]");
    if (opt.dimensions > m->cfg.out_dims)
        return ge::model_fail(m, GE_ERR_OPTIONS, "invalid options: dimensions exceed the model's " + std::to_string(m->cfg.out_dims));
    if (opt.max_tokens < 2 || opt.max_tokens > m->cfg.max_tokens)
        return ge::model_fail(m, GE_ERR_OPTIONS, "invalid options: maxTokens must be between 2 and " + std::to_string(m->cfg.max_tokens));
    if (opt.batch_size < 0) return ge::model_fail(m, GE_ERR_OPTIONS, "invalid options: batchSize must be at least 1");
    if (n < 0 || (n > 0 && (!tokens || !lengths || !out))) return ge::model_fail(m, GE_ERR_INVALID, "null argument");
    if (n == 0) return GE_OK;

    // prepare (EmbeddingModel.swift:189-196): keep the first maxTokens - 1 ids and end with EOS.
    std::vector<std::vector<int32_t>> prepared{size_t(n)};
    std::vector<uint8_t> cut(static_cast<size_t>(n), 0);
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        if (lengths[i] < 0) return ge::model_fail(m, GE_ERR_INVALID, "negative length");
        const int32_t* ids = tokens + off;
        off += size_t(lengths[i]);
        if (lengths[i] > opt.max_tokens) {
            prepared[size_t(i)].assign(ids, ids + opt.max_tokens - 1);
            prepared[size_t(i)].push_back(m->cfg.eos_id);
            cut[size_t(i)] = 1;
        } else {
            prepared[size_t(i)].assign(ids, ids + lengths[i]);
        }
        if (prepared[size_t(i)].empty()) return ge::model_fail(m, GE_ERR_INVALID, "text " + std::to_string(i) + " has no tokens");
    }
    std::vector<int32_t> costs(static_cast<size_t>(n));
    for (int i = 0; i < n; i++) costs[size_t(i)] = int32_t(prepared[size_t(i)].size());
    const int32_t budget = m->budget;
    std::vector<int> starts = ge::plan_batches(costs.data(), n, &budget, 1, opt.batch_size);
    int completed_texts = 0;
    int64_t completed_tokens = 0;
    std::vector<float> pooled;
    auto batch_tokens = [&](size_t r) {
        int64_t t = 0;
        for (int i = starts[r]; i < starts[r + 1]; i++) t += costs[size_t(i)];
        return t;
    };
    // By default each planned batch is one forward (EmbeddingModel.swift:157-172), so the budget
    // bounds every pack and a cancel returned after a batch stops before the next batch's GPU
    // work. With pack_tokens above the budget, consecutive planned batches run as one device pack
    // of up to pack_tokens tokens. A text's vector does not depend on the pack around it (every
    // kernel gives the same bits for its rows whatever the pack), so only the time changes;
    // progress still follows the planned batches, and a cancel takes effect at the next pack.
    for (size_t r = 0; r + 1 < starts.size();) {
        size_t r_end = r + 1;
        int64_t tok = batch_tokens(r);
        while (r_end + 1 < starts.size() && tok + batch_tokens(r_end) <= m->pack_tokens) tok += batch_tokens(r_end++);
        std::vector<std::vector<int32_t>> pack(prepared.begin() + starts[r], prepared.begin() + starts[r_end]);
        int rc = ge::run_batch(m, pack, &pooled);
        if (rc != GE_OK) return rc;
        for (size_t q = r; q < r_end; q++) {
            for (int i = starts[q]; i < starts[q + 1]; i++) {
                const size_t j = size_t(i - starts[r]);
                ge::finish(pooled.data() + j * size_t(m->cfg.out_dims), opt.dimensions, opt.normalise != 0,
                           out + size_t(i) * size_t(opt.dimensions));
                if (token_counts) token_counts[i] = costs[size_t(i)];
                if (truncated) truncated[i] = cut[size_t(i)];
                completed_tokens += costs[size_t(i)];
            }
            completed_texts = starts[q + 1];
            // EmbeddingProgress after every batch; a non-zero return cancels before the next one
            // (Task.checkCancellation, EmbeddingModel.swift:162).
            if (progress && progress(user, completed_texts, n, completed_tokens) != 0 && q + 2 < starts.size())
                return ge::model_fail(m, GE_ERR_CANCELLED, "embedding was cancelled");
        }
        r = r_end;
    }
    return GE_OK;
}

int ge_model_embed_tokens(ge_model* m, const int32_t* tokens, const int32_t* lengths, int32_t n, float* out) {
    if (!m) return GE_ERR_INVALID;
    if (n < 0 || (n > 0 && (!tokens || !lengths || !out))) return ge::model_fail(m, GE_ERR_INVALID, "null argument");
    if (n == 0) return GE_OK;
    std::vector<std::vector<int32_t>> seqs{size_t(n)};
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        if (lengths[i] <= 0) return ge::model_fail(m, GE_ERR_INVALID, "text " + std::to_string(i) + " has no tokens");
        seqs[size_t(i)].assign(tokens + off, tokens + off + lengths[i]);
        off += size_t(lengths[i]);
    }
    std::vector<float> pooled;
    int rc = ge::run_batch(m, seqs, &pooled);
    if (rc != GE_OK) return rc;
    std::memcpy(out, pooled.data(), pooled.size() * sizeof(float));
    return GE_OK;
}

}  // extern "C"
