// GGUF reader, model configuration and weight validation for the text encoder.
// Follows Sources/GemmaEmbed/GGUF/GGUFFile.swift:21-177, Model/ModelConfig.swift:54-112 and
// Model/Weights.swift:92-132.
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>

namespace ge {

size_t type_block_size(int type) { return type == GE_TYPE_Q8_0 ? 32 : 1; }

size_t type_block_bytes(int type) {
    switch (type) {
    case GE_TYPE_F32: return 4;
    case GE_TYPE_F16:
    case GE_TYPE_BF16: return 2;
    case GE_TYPE_Q8_0: return 34;  // fp16 scale + 32 int8 (Shaders/Common.metal:27-29)
    default: return 0;
    }
}

const char* type_name(int type) {
    switch (type) {
    case GE_TYPE_F32: return "F32";
    case GE_TYPE_F16: return "F16";
    case GE_TYPE_Q8_0: return "Q8_0";
    case GE_TYPE_BF16: return "BF16";
    default: return "unknown";
    }
}

size_t TensorInfo::bytes() const { return size_t(elements()) / type_block_size(type) * type_block_bytes(type); }
size_t TensorInfo::row_bytes() const { return size_t(columns()) / type_block_size(type) * type_block_bytes(type); }

namespace {

// Cursor (GGUFFile.swift:92-177): bounds-checked little-endian reads.
struct Cursor {
    const uint8_t* p;
    size_t n;
    size_t pos = 0;

    void need(size_t k) {
        if (k > n - pos)
            throw Error(GE_ERR_GGUF, "invalid GGUF file: truncated header at byte " + std::to_string(pos));
    }
    // `count` elements of `es` bytes each, checked without forming count * es (which can wrap).
    void need_elements(uint64_t count, size_t es) {
        if (es == 0 || count > (n - pos) / es)
            throw Error(GE_ERR_GGUF, "invalid GGUF file: array of " + std::to_string(count) +
                                         " elements past the end of the header at byte " + std::to_string(pos));
    }
    template <typename T>
    T read() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        uint64_t len = read<uint64_t>();
        need(len);
        std::string s(reinterpret_cast<const char*>(p + pos), len);
        pos += len;
        return s;
    }
    void skip_str() {
        uint64_t len = read<uint64_t>();
        need(len);
        pos += len;
    }
};

size_t scalar_size(int t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

int64_t read_int(Cursor& c, int t) {
    switch (t) {
    case 0: return c.read<uint8_t>();
    case 1: return c.read<int8_t>();
    case 2: return c.read<uint16_t>();
    case 3: return c.read<int16_t>();
    case 4: return c.read<uint32_t>();
    case 5: return c.read<int32_t>();
    case 7: return c.read<uint8_t>() != 0;
    case 10: return int64_t(c.read<uint64_t>());
    case 11: return c.read<int64_t>();
    default: throw Error(GE_ERR_GGUF, "invalid GGUF file: unknown metadata value type " + std::to_string(t));
    }
}

// readValue (GGUFFile.swift:124-176).
GGUFValue read_value(Cursor& c, int type) {
    GGUFValue v;
    v.type = type;
    if (type == 8) {
        v.s = c.str();
    } else if (type == 6) {
        v.f = c.read<float>();
    } else if (type == 12) {
        v.f = c.read<double>();
    } else if (type == 9) {
        v.arr_type = int(c.read<uint32_t>());
        uint64_t count = c.read<uint64_t>();
        v.arr_len = int64_t(count);
        if (v.arr_type == 8) {
            for (uint64_t i = 0; i < count; i++) c.skip_str();
        } else if (v.arr_type == 6 || v.arr_type == 12) {
            c.need_elements(count, scalar_size(v.arr_type));
            v.floats.reserve(count);
            for (uint64_t i = 0; i < count; i++) v.floats.push_back(v.arr_type == 6 ? c.read<float>() : c.read<double>());
        } else if (scalar_size(v.arr_type) > 0) {
            c.need_elements(count, scalar_size(v.arr_type));
            v.ints.reserve(count);
            for (uint64_t i = 0; i < count; i++) v.ints.push_back(read_int(c, v.arr_type));
        } else {
            for (uint64_t i = 0; i < count; i++) (void)read_value(c, v.arr_type);  // nested arrays: skipped
        }
    } else {
        v.i = read_int(c, type);
    }
    return v;
}

}  // namespace

GGUFFile::GGUFFile(const std::string& path) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Error(GE_ERR_GGUF, "cannot read " + path + ": " + std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        throw Error(GE_ERR_GGUF, "cannot read " + path + ": stat failed");
    }
    size_ = size_t(st.st_size);
    if (size_ == 0) {
        ::close(fd);
        throw Error(GE_ERR_GGUF, "invalid GGUF file: empty");
    }
    void* p = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) throw Error(GE_ERR_GGUF, "cannot read " + path + ": mmap failed");
    base_ = static_cast<uint8_t*>(p);
    try {
        Cursor c{base_, size_};
        uint32_t magic = c.read<uint32_t>();
        if (magic != 0x46554747u) {
            char buf[64];
            std::snprintf(buf, sizeof(buf), "invalid GGUF file: bad magic 0x%x", magic);
            throw Error(GE_ERR_GGUF, buf);
        }
        version_ = c.read<uint32_t>();
        if (version_ != 2 && version_ != 3)
            throw Error(GE_ERR_GGUF, "invalid GGUF file: unsupported version " + std::to_string(version_));
        uint64_t tensor_count = c.read<uint64_t>();
        uint64_t kv_count = c.read<uint64_t>();
        for (uint64_t i = 0; i < kv_count; i++) {
            std::string key = c.str();
            int type = int(c.read<uint32_t>());
            meta_[key] = read_value(c, type);
        }
        for (uint64_t i = 0; i < tensor_count; i++) {
            TensorInfo t;
            t.name = c.str();
            uint32_t ndim = c.read<uint32_t>();
            if (ndim > 4) throw Error(GE_ERR_GGUF, "invalid GGUF file: tensor " + t.name + " has " + std::to_string(ndim) + " dimensions");
            for (uint32_t d = 0; d < ndim; d++) t.shape.push_back(int64_t(c.read<uint64_t>()));
            t.type = int(c.read<uint32_t>());
            if (type_block_bytes(t.type) == 0)
                throw Error(GE_ERR_MODEL, "tensor " + t.name + " uses unsupported storage type " + std::to_string(t.type));
            // Every dimension positive and the element count representable, so that elements(),
            // rows() and bytes() below cannot wrap; a Q8_0 row is whole blocks.
            int64_t elems = 1;
            for (int64_t d : t.shape) {
                if (d <= 0 || __builtin_mul_overflow(elems, d, &elems) || elems > (int64_t(1) << 56))
                    throw Error(GE_ERR_GGUF, "invalid GGUF file: tensor " + t.name + " has an invalid shape");
            }
            if (t.columns() % int64_t(type_block_size(t.type)) != 0)
                throw Error(GE_ERR_GGUF, "invalid GGUF file: tensor " + t.name + " has rows of partial blocks");
            t.offset = c.read<uint64_t>();
            index_[t.name] = tensors_.size();
            tensors_.push_back(std::move(t));
        }
        uint64_t alignment = 32;
        if (auto* a = meta("general.alignment"); a && a->is_int() && a->i > 0) alignment = uint64_t(a->i);
        data_offset_ = (c.pos + alignment - 1) / alignment * alignment;
        if (data_offset_ > size_) throw Error(GE_ERR_GGUF, "invalid GGUF file: data section past the end of the file");
        for (const auto& t : tensors_) {
            const uint64_t room = size_ - data_offset_;
            if (t.offset > room || t.bytes() > room - t.offset)
                throw Error(GE_ERR_GGUF, "invalid GGUF file: tensor " + t.name + " extends past the end of the file");
        }
    } catch (...) {
        munmap(base_, size_);
        base_ = nullptr;
        throw;
    }
}

GGUFFile::~GGUFFile() {
    if (base_) munmap(base_, size_);
}

const GGUFValue* GGUFFile::meta(const std::string& key) const {
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

const TensorInfo* GGUFFile::tensor(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

namespace {

std::string shape_str(const std::vector<int64_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); i++) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// ModelWeights.init's tensor() (Weights.swift:93-98): presence, shape and type checks.
const TensorInfo* require(const GGUFFile& f, const std::string& name, std::vector<int64_t> shape, bool f32_only,
                          bool optional = false) {
    const TensorInfo* t = f.tensor(name);
    if (!t) {
        if (optional) return nullptr;
        throw Error(GE_ERR_MODEL, "weight file lacks tensor " + name);
    }
    if (t->shape != shape)
        throw Error(GE_ERR_MODEL, "tensor " + name + " has shape " + shape_str(t->shape) + ", expected " + shape_str(shape));
    if (f32_only && t->type != GE_TYPE_F32)
        throw Error(GE_ERR_MODEL, "tensor " + name + " uses unsupported storage type " + std::to_string(t->type));
    return t;
}

}  // namespace

ModelConfig read_config(const GGUFFile& f) {
    ModelConfig c;
    const GGUFValue* arch = f.meta("general.architecture");
    c.architecture = arch && arch->type == 8 ? arch->s : "";
    if (c.architecture != "gemma-embedding2")
        throw Error(GE_ERR_MODEL, "unsupported architecture '" + c.architecture + "'; GemmaEmbed supports gemma-embedding2");
    const std::string a = c.architecture + ".";
    auto get_int = [&](const std::string& key) -> int {
        const GGUFValue* v = f.meta(a + key);
        if (!v || !v->is_int()) throw Error(GE_ERR_MODEL, "weight file lacks metadata key " + a + key);
        return int(v->i);
    };
    auto get_float = [&](const std::string& key) -> float {
        const GGUFValue* v = f.meta(a + key);
        if (!v || !v->has_float()) throw Error(GE_ERR_MODEL, "weight file lacks metadata key " + a + key);
        return float(v->as_float());
    };
    c.layers = get_int("block_count");
    c.hidden = get_int("embedding_length");
    c.heads = get_int("attention.head_count");
    const GGUFValue* kvh = f.meta(a + "attention.head_count_kv");
    if (!kvh || kvh->type != 9 || int64_t(kvh->ints.size()) != c.layers)
        throw Error(GE_ERR_MODEL, "weight file lacks metadata key " + a + "attention.head_count_kv");
    const GGUFValue* pat = f.meta(a + "attention.sliding_window_pattern");
    if (!pat || pat->type != 9 || pat->arr_type != 7 || int64_t(pat->ints.size()) != c.layers)
        throw Error(GE_ERR_MODEL, "weight file lacks metadata key " + a + "attention.sliding_window_pattern");
    const int hd_global = get_int("attention.key_length");
    const int hd_swa = get_int("attention.key_length_swa");
    if (get_int("attention.value_length") != hd_global || get_int("attention.value_length_swa") != hd_swa)
        throw Error(GE_ERR_GGUF, "invalid GGUF file: key and value head sizes differ");
    const float rope_global = get_float("rope.freq_base");
    const GGUFValue* rs = f.meta(a + "rope.freq_base_swa");
    const float rope_swa = rs && rs->has_float() ? float(rs->as_float()) : rope_global;
    const GGUFValue* toks = f.meta("tokenizer.ggml.tokens");
    if (!toks || toks->type != 9 || toks->arr_type != 8) throw Error(GE_ERR_MODEL, "weight file lacks metadata key tokenizer.ggml.tokens");
    c.vocab = int(toks->arr_len);
    const TensorInfo* q0 = f.tensor("blk.0.attn_q.weight");
    c.quantization = q0 ? type_name(q0->type) : "unknown";
    const GGUFValue* nm = f.meta("general.name");
    c.name = nm && nm->type == 8 ? nm->s : c.architecture;
    c.out_dims = get_int("embedding_length_out");
    c.feed_forward = get_int("feed_forward_length");
    c.sliding_window = get_int("attention.sliding_window");
    c.eps = get_float("attention.layer_norm_rms_epsilon");
    if (auto* b = f.meta("tokenizer.ggml.bos_token_id"); b && b->is_int()) c.bos_id = int(b->i);
    if (auto* e = f.meta("tokenizer.ggml.eos_token_id"); e && e->is_int()) c.eos_id = int(e->i);
    const bool ple = f.tensor("per_layer_model_proj.weight") != nullptr;
    c.per_layer_input = ple ? get_int("embedding_length_per_layer_input") : 0;
    c.embedding_scale = std::sqrt(float(c.hidden));         // ModelConfig.swift:110
    c.per_layer_scale = 1.0f / std::sqrt(float(c.hidden));  // :111

    // ModelWeights.init (Weights.swift:100-131); the per-layer-input tensors only with PLE.
    const int64_t d = c.hidden, ff = c.feed_forward, pl = c.per_layer_input;
    require(f, "token_embd.weight", {d, c.vocab}, false);
    require(f, "output_norm.weight", {d}, true);
    require(f, "output.weight", {d, c.out_dims}, false);
    if (ple) {
        require(f, "per_layer_model_proj.weight", {d, pl * c.layers}, false);
        require(f, "per_layer_proj_norm.weight", {pl}, true);
    }
    for (int i = 0; i < c.layers; i++) {
        LayerConfig L;
        L.index = i;
        L.sliding = pat->ints[i] != 0;
        L.kv_heads = int(kvh->ints[i]);
        L.head_dim = L.sliding ? hd_swa : hd_global;
        L.rope_base = L.sliding ? rope_swa : rope_global;
        if (L.kv_heads <= 0 || c.heads % L.kv_heads != 0)
            throw Error(GE_ERR_MODEL, "layer " + std::to_string(i) + " has " + std::to_string(L.kv_heads) + " KV heads for " +
                                          std::to_string(c.heads) + " query heads");
        const std::string b = "blk." + std::to_string(i) + ".";
        const int64_t qd = int64_t(c.heads) * L.head_dim, kvd = int64_t(L.kv_heads) * L.head_dim, hd = L.head_dim;
        require(f, b + "attn_norm.weight", {d}, true);
        require(f, b + "attn_q.weight", {d, qd}, false);
        require(f, b + "attn_k.weight", {d, kvd}, false);
        require(f, b + "attn_v.weight", {d, kvd}, false);
        require(f, b + "attn_output.weight", {qd, d}, false);
        require(f, b + "attn_q_norm.weight", {hd}, true);
        require(f, b + "attn_k_norm.weight", {hd}, true);
        require(f, b + "post_attention_norm.weight", {d}, true);
        require(f, b + "ffn_norm.weight", {d}, true);
        require(f, b + "ffn_gate.weight", {d, ff}, false);
        require(f, b + "ffn_up.weight", {d, ff}, false);
        require(f, b + "ffn_down.weight", {ff, d}, false);
        require(f, b + "post_ffw_norm.weight", {d}, true);
        if (ple) {
            require(f, b + "inp_gate.weight", {d, pl}, false);
            require(f, b + "proj.weight", {pl, d}, false);
            require(f, b + "post_norm.weight", {d}, true);
        }
        const TensorInfo* os = require(f, b + "layer_output_scale.weight", {1}, true, !ple);
        L.out_scale = 1.0f;
        if (os) std::memcpy(&L.out_scale, f.data(*os), 4);
        c.layer.push_back(L);
    }
    return c;
}

void make_upload_desc(const GGUFFile& f, const ModelConfig& c, UploadDesc* u) {
    u->names.clear();
    u->tensors.clear();
    u->kv_heads.clear();
    u->head_dim.clear();
    u->sliding.clear();
    u->rope_base.clear();
    u->out_scale.clear();
    for (const auto& t : f.tensors()) u->names.push_back(t.name);
    u->tensors.resize(f.tensors().size());
    for (size_t i = 0; i < f.tensors().size(); i++) {
        const TensorInfo& t = f.tensors()[i];
        ge_tensor_desc& d = u->tensors[i];
        d.name = u->names[i].c_str();
        d.offset = f.file_offset(t);
        d.type = t.type;
        d.ndim = int32_t(t.shape.size());
        for (int k = 0; k < 4; k++) d.shape[k] = k < d.ndim ? t.shape[size_t(k)] : 1;
    }
    for (const auto& L : c.layer) {
        u->kv_heads.push_back(L.kv_heads);
        u->head_dim.push_back(L.head_dim);
        u->sliding.push_back(L.sliding ? 1 : 0);
        u->rope_base.push_back(L.rope_base);
        u->out_scale.push_back(L.out_scale);
    }
    ge_model_desc& m = u->desc;
    m.layers = c.layers;
    m.hidden = c.hidden;
    m.heads = c.heads;
    m.feed_forward = c.feed_forward;
    m.out_dims = c.out_dims;
    m.per_layer_input = c.per_layer_input;
    m.vocab = c.vocab;
    m.sliding_window = c.sliding_window;
    m.max_tokens = c.max_tokens;
    m.eps = c.eps;
    m.embedding_scale = c.embedding_scale;
    m.per_layer_scale = c.per_layer_scale;
    m.kv_heads = u->kv_heads.data();
    m.head_dim = u->head_dim.data();
    m.sliding = u->sliding.data();
    m.rope_base = u->rope_base.data();
    m.out_scale = u->out_scale.data();
    m.tensors = u->tensors.data();
    m.n_tensors = int32_t(u->tensors.size());
}

}  // namespace ge
