// Image-encoder GGUF loading for the device library: VisionConfig.init's metadata reads
// (Model/VisionConfig.swift:44-81) and the weight directory (Model/VisionWeights.swift), turned
// into the ge_vision_desc that ge_upload_vision takes.
#include <cstdio>
#include <string>
#include <vector>

#include "gemmaembed.h"
#include "gguf.hpp"

namespace ge {
namespace {

int meta_int(const GGUFFile& f, const std::string& key) {
    const GGUFValue* v = f.meta(key);
    if (!v || !v->has_int()) throw Error(GE_ERR_MODEL, "image encoder file lacks metadata key " + key);
    return int(v->i);
}

void load_vision(ge_ctx* ctx, const std::string& path) {
    GGUFFile f(path);
    const GGUFValue* arch = f.meta("general.architecture");
    if (!arch || arch->s != "clip")
        throw Error(GE_ERR_GGUF, "image encoder architecture is '" + (arch ? arch->s : std::string()) + "', expected clip");
    const GGUFValue* proj = f.meta("clip.vision.projector_type");
    if (!proj || proj->s != "gemma3")
        throw Error(GE_ERR_GGUF, "image projector is '" + (proj ? proj->s : std::string()) + "', expected gemma3");
    const std::string a = "clip.vision.";
    ge_vision_desc d{};
    d.layers = meta_int(f, a + "block_count");
    d.hidden = meta_int(f, a + "embedding_length");
    d.heads = meta_int(f, a + "attention.head_count");
    d.feed_forward = meta_int(f, a + "feed_forward_length");
    d.patch_size = meta_int(f, a + "patch_size");
    d.proj_dims = meta_int(f, a + "projection_dim");
    d.merge = meta_int(f, a + "projector.scale_factor");
    const GGUFValue* eps = f.meta(a + "attention.layer_norm_epsilon");
    if (!eps || !eps->has_float()) throw Error(GE_ERR_MODEL, "image encoder file lacks metadata key " + a + "attention.layer_norm_epsilon");
    d.eps = float(eps->as_float());
    const TensorInfo* pos = f.tensor("v.position_embd.weight");
    if (!pos || pos->shape.size() != 3 || pos->shape[2] != 2)
        throw Error(GE_ERR_MODEL, "image encoder file lacks a [hidden, positions, 2] v.position_embd.weight");
    d.positions = int(pos->shape[1]);
    std::vector<ge_tensor_desc> ts;
    for (const TensorInfo& t : f.tensors()) {
        ge_tensor_desc x{};
        x.name = t.name.c_str();
        x.offset = f.file_offset(t);
        x.type = t.type;
        x.ndim = int32_t(t.shape.size());
        for (size_t i = 0; i < t.shape.size() && i < 4; i++) x.shape[i] = t.shape[i];
        ts.push_back(x);
    }
    d.tensors = ts.data();
    d.n_tensors = int32_t(ts.size());
    const int rc = ge_upload_vision(ctx, &d, f.base(), f.size());
    if (rc != GE_OK) throw Error(rc, ge_last_error(ctx));
}

}  // namespace
}  // namespace ge

extern "C" int ge_vision_load(ge_ctx* ctx, const char* path, char* err, size_t errlen) {
    try {
        if (!ctx || !path) throw ge::Error(GE_ERR_INVALID, "null argument");
        ge::load_vision(ctx, path);
        return GE_OK;
    } catch (const ge::Error& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return e.code;
    } catch (const std::exception& e) {
        if (err && errlen) std::snprintf(err, errlen, "%s", e.what());
        return GE_ERR_INVALID;
    }
}
