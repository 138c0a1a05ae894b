// Synthetic gemma-embedding2 GGUF writer for seeded test and bench models.
//
// The file has the reference model's layout: metadata keys read by ModelConfig.init
// (Model/ModelConfig.swift:54-112) and tensors named and shaped as ModelWeights.init expects
// (Model/Weights.swift:100-131), in GGUF v3 with 32-byte alignment (GGUF/GGUFFile.swift:60-62).
// Values follow these rules:
//  - Q8_0 matrices: per 32-block, q ~ U{-127..127}, then an fp16 scale
//    d = fp16(|z| * max|q| / 127) with z ~ N(0, 0.02);
//  - fp32 norm weights and layer_output_scale: 1 + 0.1 N(0, 1);
//  - bf16 per_layer_model_proj: bf16(0.02 N(0, 1));
//  - every tensor draws from its own SplitMix64 stream seeded by (seed, tensor name).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gemmaembed.h"
#include "gguf.hpp"
#include "halfconv.hpp"
#include "prng.hpp"

namespace ge {
namespace {

struct Writer {
    FILE* f = nullptr;
    uint64_t written = 0;
    std::vector<uint8_t> buf;

    explicit Writer(FILE* fp) : f(fp) { buf.reserve(1 << 22); }
    void flush() {
        if (!buf.empty() && std::fwrite(buf.data(), 1, buf.size(), f) != buf.size()) throw Error(GE_ERR_INVALID, "write failed");
        buf.clear();
    }
    void bytes(const void* p, size_t n) {
        const uint8_t* b = static_cast<const uint8_t*>(p);
        buf.insert(buf.end(), b, b + n);
        written += n;
        if (buf.size() >= (1 << 22)) flush();
    }
    template <typename T>
    void put(T v) { bytes(&v, sizeof(T)); }
    void str(const std::string& s) {
        put<uint64_t>(s.size());
        bytes(s.data(), s.size());
    }
    void pad(uint64_t align) {
        static const uint8_t zeros[64] = {0};
        while (written % align) bytes(zeros, size_t(std::min<uint64_t>(align - written % align, 64)));
    }
};

struct KV {
    std::string key;
    int type;
    uint64_t u = 0;
    float f = 0;
    std::string s;
    int arr_type = 0;
    std::vector<int32_t> ints;
    std::vector<uint8_t> bools;
    int64_t nstrings = 0;  // tokenizer tokens: "<t%d>"
};

struct TensorSpec {
    std::string name;
    std::vector<int64_t> shape;
    int type;
    uint64_t offset = 0;
    // value rule: Q8_0 block scales from |N(0, scale)|; F32 offset + scale N(0, 1); F16 and BF16
    // scale N(0, 1)
    double scale = -1, offset_f = 1;
    // F32: this many entries replaced by +-U(outlier / 6, outlier)
    int outliers = 0;
    double outlier = 0;
    size_t bytes() const {
        int64_t n = 1;
        for (auto d : shape) n *= d;
        return size_t(n) / type_block_size(type) * type_block_bytes(type);
    }
};

void write_kv(Writer& w, const KV& kv) {
    w.str(kv.key);
    w.put<uint32_t>(uint32_t(kv.type));
    switch (kv.type) {
    case 4: w.put<uint32_t>(uint32_t(kv.u)); break;
    case 6: w.put<float>(kv.f); break;
    case 8: w.str(kv.s); break;
    case 9:
        w.put<uint32_t>(uint32_t(kv.arr_type));
        if (kv.arr_type == 5) {
            w.put<uint64_t>(kv.ints.size());
            for (auto v : kv.ints) w.put<int32_t>(v);
        } else if (kv.arr_type == 7) {
            w.put<uint64_t>(kv.bools.size());
            for (auto v : kv.bools) w.put<uint8_t>(v ? 1 : 0);
        } else if (kv.arr_type == 8) {
            w.put<uint64_t>(uint64_t(kv.nstrings));
            char name[32];
            for (int64_t i = 0; i < kv.nstrings; i++) {
                int n = std::snprintf(name, sizeof(name), "<t%lld>", (long long)i);
                w.str(std::string(name, size_t(n)));
            }
        }
        break;
    default: throw Error(GE_ERR_INVALID, "internal: kv type");
    }
}

void write_tensor_data(Writer& w, const TensorSpec& t, uint64_t seed) {
    SeededRandom rng(tensor_seed(seed, t.name));
    int64_t n = 1;
    for (auto d : t.shape) n *= d;
    if (t.type == GE_TYPE_Q8_0) {
        uint8_t block[34];
        for (int64_t b = 0; b < n / 32; b++) {
            int maxq = 0;
            for (int j = 0; j < 32; j++) {
                const int q = int(rng.uniform_int(-127, 128));
                block[2 + j] = uint8_t(int8_t(q));
                maxq = std::max(maxq, q < 0 ? -q : q);
            }
            const double z = (t.scale > 0 ? t.scale : 0.02) * rng.gaussian();
            const uint16_t d = float_to_half(float(std::fabs(z) * double(maxq) / 127.0));
            block[0] = uint8_t(d & 0xff);
            block[1] = uint8_t(d >> 8);
            w.bytes(block, 34);
        }
    } else if (t.type == GE_TYPE_F32) {
        const double sc = t.scale >= 0 ? t.scale : 0.1;
        std::vector<float> v(static_cast<size_t>(n));
        for (int64_t i = 0; i < n; i++) v[size_t(i)] = float(t.offset_f + sc * rng.gaussian());
        for (int k = 0; k < t.outliers && n > 0; k++) {
            const int64_t at = int64_t(rng.uniform_int(0, n));
            const double mag = t.outlier * (1.0 / 6.0 + (5.0 / 6.0) * rng.unit());
            v[size_t(at)] = float(rng.unit() < 0.5 ? -mag : mag);
        }
        for (float x : v) w.put<float>(x);
    } else if (t.type == GE_TYPE_BF16) {
        const double sc = t.scale > 0 ? t.scale : 0.02;
        for (int64_t i = 0; i < n; i++) w.put<uint16_t>(float_to_bf16(float(sc * rng.gaussian())));
    } else if (t.type == GE_TYPE_F16) {
        const double sc = t.scale > 0 ? t.scale : 0.02;
        for (int64_t i = 0; i < n; i++) w.put<uint16_t>(float_to_half(float(sc * rng.gaussian())));
    } else {
        throw Error(GE_ERR_INVALID, "internal: tensor type");
    }
}

void write_file(const std::string& path, const std::vector<KV>& kvs, std::vector<TensorSpec>& ts, uint64_t seed);

void synth_write(const std::string& path, const ge_synth_spec& s) {
    if (s.layers <= 0 || s.hidden <= 0 || s.heads <= 0 || s.feed_forward <= 0 || s.out_dims <= 0 || s.vocab <= 2 ||
        s.head_dim_swa <= 0 || s.head_dim_global <= 0 || s.kv_heads_swa <= 0 || s.kv_heads_global <= 0 || !s.pattern)
        throw Error(GE_ERR_INVALID, "synthetic spec has a non-positive size or no pattern");
    if (s.hidden % 32 || s.feed_forward % 32 || s.per_layer_input % 32 || s.head_dim_swa % 32 || s.head_dim_global % 32)
        throw Error(GE_ERR_INVALID, "Q8_0 rows need widths that are multiples of 32");
    const std::string a = "gemma-embedding2.";
    std::vector<KV> kvs;
    auto u32 = [&](const std::string& k, uint64_t v) { KV x; x.key = k; x.type = 4; x.u = v; kvs.push_back(x); };
    auto f32 = [&](const std::string& k, float v) { KV x; x.key = k; x.type = 6; x.f = v; kvs.push_back(x); };
    auto str = [&](const std::string& k, const std::string& v) { KV x; x.key = k; x.type = 8; x.s = v; kvs.push_back(x); };
    str("general.architecture", "gemma-embedding2");
    str("general.name", "synthetic-gemma-embedding2");
    u32("general.alignment", 32);
    u32(a + "block_count", uint64_t(s.layers));
    if (s.context_length < 0 || s.norm_outliers < 0 || s.norm_outlier < 0)
        throw Error(GE_ERR_INVALID, "synthetic spec has a negative context length or outlier setting");
    u32(a + "context_length", uint64_t(s.context_length > 0 ? s.context_length : 8192));
    u32(a + "embedding_length", uint64_t(s.hidden));
    u32(a + "embedding_length_out", uint64_t(s.out_dims));
    if (s.per_layer_input > 0) u32(a + "embedding_length_per_layer_input", uint64_t(s.per_layer_input));
    u32(a + "feed_forward_length", uint64_t(s.feed_forward));
    u32(a + "attention.head_count", uint64_t(s.heads));
    {
        KV x;
        x.key = a + "attention.head_count_kv";
        x.type = 9;
        x.arr_type = 5;
        for (int i = 0; i < s.layers; i++) x.ints.push_back(s.pattern[i] ? s.kv_heads_swa : s.kv_heads_global);
        kvs.push_back(x);
        KV p;
        p.key = a + "attention.sliding_window_pattern";
        p.type = 9;
        p.arr_type = 7;
        for (int i = 0; i < s.layers; i++) p.bools.push_back(s.pattern[i] ? 1 : 0);
        kvs.push_back(p);
    }
    u32(a + "attention.sliding_window", uint64_t(s.sliding_window));
    u32(a + "attention.key_length", uint64_t(s.head_dim_global));
    u32(a + "attention.value_length", uint64_t(s.head_dim_global));
    u32(a + "attention.key_length_swa", uint64_t(s.head_dim_swa));
    u32(a + "attention.value_length_swa", uint64_t(s.head_dim_swa));
    f32(a + "rope.freq_base", s.rope_base);
    f32(a + "rope.freq_base_swa", s.rope_base_swa);
    f32(a + "attention.layer_norm_rms_epsilon", s.eps);
    {
        KV t;
        t.key = "tokenizer.ggml.tokens";
        t.type = 9;
        t.arr_type = 8;
        t.nstrings = s.vocab;
        kvs.push_back(t);
    }
    u32("tokenizer.ggml.bos_token_id", 2);
    u32("tokenizer.ggml.eos_token_id", 1);

    const int64_t d = s.hidden, ff = s.feed_forward, pl = s.per_layer_input;
    std::vector<TensorSpec> ts;
    auto add = [&](const std::string& n, std::vector<int64_t> shape, int type) { ts.push_back({n, shape, type, 0}); };
    // a residual-stream norm weight, with the spec's outliers
    auto add_norm = [&](const std::string& n, int64_t width) {
        add(n, {width}, GE_TYPE_F32);
        ts.back().outliers = s.norm_outliers;
        ts.back().outlier = s.norm_outlier;
    };
    add("output.weight", {d, s.out_dims}, GE_TYPE_Q8_0);
    add_norm("output_norm.weight", d);
    if (pl > 0) {
        add("per_layer_model_proj.weight", {d, pl * s.layers}, GE_TYPE_BF16);
        add("per_layer_proj_norm.weight", {pl}, GE_TYPE_F32);
    }
    add("token_embd.weight", {d, s.vocab}, GE_TYPE_Q8_0);
    for (int i = 0; i < s.layers; i++) {
        const bool sw = s.pattern[i] != 0;
        const int64_t hd = sw ? s.head_dim_swa : s.head_dim_global;
        const int64_t kv = sw ? s.kv_heads_swa : s.kv_heads_global;
        const int64_t qd = s.heads * hd, kvd = kv * hd;
        const std::string b = "blk." + std::to_string(i) + ".";
        add(b + "attn_k.weight", {d, kvd}, GE_TYPE_Q8_0);
        add(b + "attn_k_norm.weight", {hd}, GE_TYPE_F32);
        add_norm(b + "attn_norm.weight", d);
        add(b + "attn_output.weight", {qd, d}, GE_TYPE_Q8_0);
        add(b + "attn_q.weight", {d, qd}, GE_TYPE_Q8_0);
        add(b + "attn_q_norm.weight", {hd}, GE_TYPE_F32);
        add(b + "attn_v.weight", {d, kvd}, GE_TYPE_Q8_0);
        add(b + "ffn_down.weight", {ff, d}, GE_TYPE_Q8_0);
        add(b + "ffn_gate.weight", {d, ff}, GE_TYPE_Q8_0);
        add_norm(b + "ffn_norm.weight", d);
        add(b + "ffn_up.weight", {d, ff}, GE_TYPE_Q8_0);
        if (pl > 0) {
            add(b + "inp_gate.weight", {d, pl}, GE_TYPE_Q8_0);
            add(b + "layer_output_scale.weight", {1}, GE_TYPE_F32);
        }
        add_norm(b + "post_attention_norm.weight", d);
        add_norm(b + "post_ffw_norm.weight", d);
        if (pl > 0) {
            add_norm(b + "post_norm.weight", d);
            add(b + "proj.weight", {pl, d}, GE_TYPE_Q8_0);
        }
    }
    write_file(path, kvs, ts, s.seed);
}

// GGUF v3: header, metadata, tensor directory, then the data section with 32-byte alignment.
void write_file(const std::string& path, const std::vector<KV>& kvs, std::vector<TensorSpec>& ts, uint64_t seed) {
    uint64_t off = 0;
    for (auto& t : ts) {
        t.offset = off;
        off = (off + t.bytes() + 31) / 32 * 32;
    }

    std::unique_ptr<FILE, int (*)(FILE*)> fp(std::fopen(path.c_str(), "wb"), &std::fclose);
    if (!fp) throw Error(GE_ERR_INVALID, "cannot write " + path);
    Writer w(fp.get());
    w.put<uint32_t>(0x46554747u);
    w.put<uint32_t>(3);
    w.put<uint64_t>(ts.size());
    w.put<uint64_t>(kvs.size());
    for (const auto& kv : kvs) write_kv(w, kv);
    for (const auto& t : ts) {
        w.str(t.name);
        w.put<uint32_t>(uint32_t(t.shape.size()));
        for (auto dim : t.shape) w.put<uint64_t>(uint64_t(dim));
        w.put<uint32_t>(uint32_t(t.type));
        w.put<uint64_t>(t.offset);
    }
    w.pad(32);
    const uint64_t data0 = w.written;
    for (const auto& t : ts) {
        while (w.written - data0 < t.offset) w.put<uint8_t>(0);
        write_tensor_data(w, t, seed);
    }
    w.pad(32);
    w.flush();
}


// An image-encoder GGUF ("clip" architecture, projector "gemma3") for BASELINE config 5's tower,
// in the tensor layout ge_upload_vision reads. Values: Q8_0 matrices as the text model's but with
// z ~ N(0, 1 / (64 sqrt(K))) (K: the row width), so each projection keeps its input's scale;
// ffn_down F16 N(0, 1) / sqrt(K); LayerNorm and RMSNorm weights 1 + 0.1 N(0, 1); biases
// 0.1 N(0, 1); position rows 0.5 N(0, 1).
void synth_vision_write(const std::string& path, const ge_synth_vision_spec& s) {
    if (s.layers <= 0 || s.hidden <= 0 || s.heads <= 0 || s.feed_forward <= 0 || s.patch_size <= 0 || s.merge <= 0 ||
        s.proj_dims <= 0 || s.positions <= 0)
        throw Error(GE_ERR_INVALID, "synthetic image encoder spec has a non-positive size");
    const int64_t d = s.hidden, ff = s.feed_forward, area = 3 * int64_t(s.patch_size) * s.patch_size;
    if (d % 32 || area % 32) throw Error(GE_ERR_INVALID, "Q8_0 rows need widths that are multiples of 32");
    const int down_type = s.ffn_down_type ? s.ffn_down_type : GE_TYPE_F16;
    if (down_type == GE_TYPE_Q8_0 && ff % 32) throw Error(GE_ERR_INVALID, "a Q8_0 ffn_down needs feed_forward % 32 == 0");
    if (down_type != GE_TYPE_Q8_0 && down_type != GE_TYPE_F16) throw Error(GE_ERR_INVALID, "ffn_down type must be F16 or Q8_0");
    const std::string a = "clip.vision.";
    std::vector<KV> kvs;
    auto u32 = [&](const std::string& k, uint64_t v) { KV x; x.key = k; x.type = 4; x.u = v; kvs.push_back(x); };
    auto f32 = [&](const std::string& k, float v) { KV x; x.key = k; x.type = 6; x.f = v; kvs.push_back(x); };
    auto str = [&](const std::string& k, const std::string& v) { KV x; x.key = k; x.type = 8; x.s = v; kvs.push_back(x); };
    str("general.architecture", "clip");
    str("general.name", "synthetic-vit");
    u32("general.alignment", 32);
    str(a + "projector_type", "gemma3");
    u32(a + "block_count", uint64_t(s.layers));
    u32(a + "embedding_length", uint64_t(d));
    u32(a + "attention.head_count", uint64_t(s.heads));
    u32(a + "feed_forward_length", uint64_t(ff));
    u32(a + "patch_size", uint64_t(s.patch_size));
    u32(a + "projection_dim", uint64_t(s.proj_dims));
    u32(a + "projector.scale_factor", uint64_t(s.merge));
    f32(a + "attention.layer_norm_epsilon", s.eps);

    std::vector<TensorSpec> ts;
    auto q8 = [&](const std::string& n, int64_t cols, int64_t rows) {
        TensorSpec t{n, {cols, rows}, GE_TYPE_Q8_0, 0};
        t.scale = 1.0 / (64.0 * std::sqrt(double(cols)));
        ts.push_back(t);
    };
    auto vec = [&](const std::string& n, std::vector<int64_t> shape, double offset, double scale) {
        TensorSpec t{n, shape, GE_TYPE_F32, 0};
        t.offset_f = offset;
        t.scale = scale;
        ts.push_back(t);
    };
    q8("v.patch_embd.weight", area, d);
    vec("v.patch_embd.bias", {d}, 0, 0.1);
    vec("v.position_embd.weight", {d, s.positions, 2}, 0, 0.5);
    for (int i = 0; i < s.layers; i++) {
        const std::string b = "v.blk." + std::to_string(i) + ".";
        vec(b + "ln1.weight", {d}, 1, 0.1);
        vec(b + "ln1.bias", {d}, 0, 0.1);
        for (const char* p : {"attn_q", "attn_k", "attn_v", "attn_out"}) {
            q8(b + p + ".weight", d, d);
            vec(b + p + ".bias", {d}, 0, 0.1);
        }
        vec(b + "ln2.weight", {d}, 1, 0.1);
        vec(b + "ln2.bias", {d}, 0, 0.1);
        q8(b + "ffn_up.weight", d, ff);
        vec(b + "ffn_up.bias", {ff}, 0, 0.1);
        if (down_type == GE_TYPE_Q8_0) {
            q8(b + "ffn_down.weight", ff, d);
        } else {
            TensorSpec t{b + "ffn_down.weight", {ff, d}, GE_TYPE_F16, 0};
            t.scale = 1.0 / std::sqrt(double(ff));
            ts.push_back(t);
        }
        vec(b + "ffn_down.bias", {d}, 0, 0.1);
    }
    vec("v.post_ln.weight", {d}, 1, 0.1);
    vec("v.post_ln.bias", {d}, 0, 0.1);
    vec("mm.soft_emb_norm.weight", {d}, 1, 0.1);
    q8("mm.input_projection.weight", d, s.proj_dims);
    write_file(path, kvs, ts, s.seed);
}
}  // namespace
}  // namespace ge

extern "C" int ge_synth_write_gguf(const char* path, const ge_synth_spec* spec, char* err, size_t errlen) {
    try {
        if (!path || !spec) throw ge::Error(GE_ERR_INVALID, "null argument");
        ge::synth_write(path, *spec);
        return GE_OK;
    } catch (const ge::Error& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return e.code;
    } catch (const std::exception& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return GE_ERR_INVALID;
    }
}

extern "C" int ge_synth_tokens(uint64_t seed, int32_t lo, int32_t hi, int32_t count, int32_t* out) {
    if (!out || count < 0 || hi <= lo) return GE_ERR_INVALID;
    ge::SeededRandom rng(seed);
    for (int32_t i = 0; i < count; i++) out[i] = int32_t(rng.uniform_int(lo, hi));
    return GE_OK;
}

extern "C" int ge_synth_write_vision_gguf(const char* path, const ge_synth_vision_spec* spec, char* err, size_t errlen) {
    try {
        if (!path || !spec) throw ge::Error(GE_ERR_INVALID, "null argument");
        ge::synth_vision_write(path, *spec);
        return GE_OK;
    } catch (const ge::Error& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return e.code;
    } catch (const std::exception& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return GE_ERR_INVALID;
    }
}

extern "C" int ge_synth_uniform(uint64_t seed, float lo, float hi, int64_t count, float* out) {
    if (!out || count < 0 || !(hi > lo)) return GE_ERR_INVALID;
    ge::SeededRandom rng(seed);
    for (int64_t i = 0; i < count; i++) out[i] = float(lo + (hi - lo) * rng.unit());
    return GE_OK;
}
