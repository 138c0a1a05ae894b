// GGUF v2/v3 reader over a read-only shared mapping, and the model configuration and weight
// directory derived from it. Mirrors Sources/GemmaEmbed/GGUF/GGUFFile.swift,
// GGUF/GGUFValue.swift, Model/ModelConfig.swift and Model/Weights.swift.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "gemmaembed.h"

namespace ge {

// A failure with the C-ABI status it maps to (GemmaEmbedError, Errors.swift:6-24).
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

// GGUFValue (GGUF/GGUFValue.swift:6-23), keeping what the text path reads.
struct GGUFValue {
    int type = -1;            // GGUF value type
    int64_t i = 0;            // integer and bool scalars
    double f = 0;             // float scalars
    std::string s;            // strings
    int arr_type = -1;        // arrays: element type
    int64_t arr_len = 0;
    std::vector<int64_t> ints;  // integer / bool array elements
    std::vector<double> floats; // float array elements

    bool is_int() const { return (type >= 0 && type <= 5) || type == 10 || type == 11; }
    bool has_int() const { return is_int(); }
    bool has_float() const { return type == 6 || type == 12 || is_int(); }
    double as_float() const { return (type == 6 || type == 12) ? f : double(i); }
};

// GGUFTensorInfo (GGUF/GGUFValue.swift:117-131).
struct TensorInfo {
    std::string name;
    std::vector<int64_t> shape;  // ne order: fastest dimension first
    int type = 0;
    uint64_t offset = 0;         // from the start of the data section

    int64_t elements() const {
        int64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
    int64_t columns() const { return shape.empty() ? 1 : shape[0]; }
    int64_t rows() const { return elements() / columns(); }
    size_t bytes() const;
    size_t row_bytes() const;
};

size_t type_block_size(int type);
size_t type_block_bytes(int type);
const char* type_name(int type);

class GGUFFile {
public:
    explicit GGUFFile(const std::string& path);
    ~GGUFFile();
    GGUFFile(const GGUFFile&) = delete;
    GGUFFile& operator=(const GGUFFile&) = delete;

    const GGUFValue* meta(const std::string& key) const;
    const TensorInfo* tensor(const std::string& name) const;
    const uint8_t* base() const { return base_; }
    size_t size() const { return size_; }
    uint64_t file_offset(const TensorInfo& t) const { return data_offset_ + t.offset; }
    const uint8_t* data(const TensorInfo& t) const { return base_ + file_offset(t); }
    const std::vector<TensorInfo>& tensors() const { return tensors_; }
    uint32_t version() const { return version_; }
    size_t meta_count() const { return meta_.size(); }
    uint64_t data_offset() const { return data_offset_; }

private:
    uint8_t* base_ = nullptr;
    size_t size_ = 0;
    uint32_t version_ = 0;
    uint64_t data_offset_ = 0;
    std::map<std::string, GGUFValue> meta_;
    std::vector<TensorInfo> tensors_;
    std::map<std::string, size_t> index_;
};

// LayerConfig (Model/ModelConfig.swift:34-40) plus layer_output_scale.
struct LayerConfig {
    int index = 0;
    bool sliding = false;
    int kv_heads = 0;
    int head_dim = 0;
    float rope_base = 0;
    float out_scale = 1;
};

// ModelConfig (Model/ModelConfig.swift:43-112). per_layer_input is 0 when the model has no
// per-layer-input branch (`per_layer_model_proj.weight` absent).
struct ModelConfig {
    std::string architecture, name, quantization;
    int layers = 0, hidden = 0, out_dims = 0, feed_forward = 0, per_layer_input = 0, heads = 0, vocab = 0;
    int sliding_window = 0, max_tokens = 8192;
    float eps = 1e-6f, embedding_scale = 1, per_layer_scale = 1;
    int bos_id = 2, eos_id = 1;
    std::vector<LayerConfig> layer;
};

// Reads the configuration from metadata and checks every tensor's presence, shape and type
// (ModelConfig.init :54-112, ModelWeights.init Weights.swift:92-132). Throws ge::Error.
ModelConfig read_config(const GGUFFile& file);

// The tensor directory of a validated model, as the device library's upload descriptor.
struct UploadDesc {
    ge_model_desc desc{};
    std::vector<ge_tensor_desc> tensors;
    std::vector<std::string> names;
    std::vector<int32_t> kv_heads, head_dim;
    std::vector<uint8_t> sliding;
    std::vector<float> rope_base, out_scale;
};
void make_upload_desc(const GGUFFile& file, const ModelConfig& cfg, UploadDesc* out);

}  // namespace ge
