// The MoE tensors of one GPT-OSS layer inside an MXFP4 safetensors checkpoint:
// names, dtypes and shapes, validated and exposed as views into the file mappings
// (no HIP dependency; gpt_oss_loader.hpp uploads them).
//
// The reference loader (crates/llm-core/src/gpt_oss_loader.rs:57-201) converts every
// tensor from bf16 to f16 (:33-43, :97-104) and looks for per-expert dense weights
// (block_sparse_moe.experts.{e}.w1/w3/w2, :146-157) and the router at
// block_sparse_moe.gate.weight / mlp.router.weight (:139-141). MXFP4 checkpoints
// hold the experts as packed e2m1 blocks with E8M0 scales instead, which that loader
// cannot read. Here the bytes are taken as they are: no f16 round trip, no
// dequantisation, and each expert tensor keeps the layout the layer kernels use.
//
// Two naming conventions are recognised (they are external conventions of the
// published checkpoints; no checkpoint is available offline to confirm them):
//   Hugging Face   model.layers.{i}.mlp.router.{weight,bias}
//                  model.layers.{i}.mlp.experts.{gate_up,down}_proj_{blocks,scales,bias}
//                  model.layers.{i}.post_attention_layernorm.weight
//   original       block.{i}.mlp.gate.{weight,bias}
//                  block.{i}.mlp.mlp1_weight.{blocks,scales}, block.{i}.mlp.mlp1_bias
//                  block.{i}.mlp.mlp2_weight.{blocks,scales}, block.{i}.mlp.mlp2_bias
//                  block.{i}.mlp.norm.scale
// Layouts (R = output rows, C = reduction length):
//   *_blocks  u8 [E, R, C/32, 16] (or the same bytes as [E, R, C/2]); low nibble first
//   *_scales  u8 [E, R, C/32], E8M0
//   gate_up   R = 2I, rows interleaved gate_0, up_0, gate_1, up_1, ...; C = H
//   down      R = H; C = I
//   router    [E, H], bias [E]; biases [E, R]; norm [H]: BF16 (F32 is accepted and
//             rounded to bf16 by the loader)
#pragma once

#include <cstdio>
#include <initializer_list>
#include <string>
#include <vector>

#include "safetensors.hpp"

namespace gpt_oss {

using safetensors::Checkpoint;
using safetensors::Error;
using safetensors::TensorView;

enum class Naming { HuggingFace, Original };

struct LayerNames {
    std::string router_w, router_b, gu_blocks, gu_scales, gu_bias, dn_blocks, dn_scales, dn_bias, norm;
};

inline LayerNames layer_names(Naming n, int i) {
    const std::string k = std::to_string(i);
    if (n == Naming::HuggingFace) {
        const std::string m = "model.layers." + k + ".mlp.";
        return {m + "router.weight",          m + "router.bias",          m + "experts.gate_up_proj_blocks",
                m + "experts.gate_up_proj_scales", m + "experts.gate_up_proj_bias", m + "experts.down_proj_blocks",
                m + "experts.down_proj_scales", m + "experts.down_proj_bias",
                "model.layers." + k + ".post_attention_layernorm.weight"};
    }
    const std::string m = "block." + k + ".mlp.";
    return {m + "gate.weight",         m + "gate.bias", m + "mlp1_weight.blocks", m + "mlp1_weight.scales",
            m + "mlp1_bias",           m + "mlp2_weight.blocks", m + "mlp2_weight.scales", m + "mlp2_bias",
            m + "norm.scale"};
}

// Model-level settings from config.json (either convention's keys), when present.
struct Config {
    int hidden = 0, intermediate = 0, num_experts = 0, experts_per_token = 0, num_layers = 0;
    float rms_norm_eps = 1e-5f;
    float swiglu_limit = 7.0f;
    float swiglu_alpha = 1.702f;  // fixed by the GPT-OSS activation; not a config key
    bool found = false;
};

inline Config read_config(const std::string& dir) {
    Config c;
    std::FILE* f = std::fopen((dir + "/config.json").c_str(), "rb");
    if (!f) return c;
    std::string text;
    char buf[4096];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
    std::fclose(f);
    safetensors::Json j = safetensors::parse_json(text);
    if (j.kind != safetensors::Json::Object) throw Error(dir + "/config.json is not a JSON object");
    auto num = [&](std::initializer_list<const char*> keys, double& out) {
        for (const char* k : keys)
            if (const safetensors::Json* v = j.find(k)) {
                if (v->kind != safetensors::Json::Number) throw Error(std::string("config.json: ") + k + " is not a number");
                out = v->num;
                return true;
            }
        return false;
    };
    double v;
    if (num({"hidden_size"}, v)) c.hidden = (int)v;
    if (num({"intermediate_size"}, v)) c.intermediate = (int)v;
    if (num({"num_local_experts", "num_experts"}, v)) c.num_experts = (int)v;
    if (num({"num_experts_per_tok", "experts_per_token"}, v)) c.experts_per_token = (int)v;
    if (num({"num_hidden_layers"}, v)) c.num_layers = (int)v;
    if (num({"rms_norm_eps"}, v)) c.rms_norm_eps = (float)v;
    if (num({"swiglu_limit"}, v)) c.swiglu_limit = (float)v;
    c.found = true;
    return c;
}

// Views of one layer's MoE tensors, validated against each other.
struct LayerView {
    Naming naming = Naming::HuggingFace;
    int hidden = 0, intermediate = 0, num_experts = 0;
    const TensorView* router_w = nullptr;
    const TensorView* router_b = nullptr;  // optional
    const TensorView* gu_blocks = nullptr;
    const TensorView* gu_scales = nullptr;
    const TensorView* gu_bias = nullptr;  // optional
    const TensorView* dn_blocks = nullptr;
    const TensorView* dn_scales = nullptr;
    const TensorView* dn_bias = nullptr;  // optional
    const TensorView* norm = nullptr;     // optional (the MoE layer alone does not need it)
};

namespace detail {

inline std::string shape_str(const std::vector<int64_t>& s) {
    std::string o = "[";
    for (size_t k = 0; k < s.size(); ++k) o += (k ? ", " : "") + std::to_string(s[k]);
    return o + "]";
}

inline void need(bool ok, const TensorView& t, const std::string& what) {
    if (!ok) throw Error("tensor '" + t.name + "' (" + t.dtype + " " + shape_str(t.shape) + "): " + what);
}

inline void need_16bit(const TensorView& t, std::vector<int64_t> shape) {
    need(t.dtype == "BF16" || t.dtype == "F32", t, "expected BF16 (or F32)");
    need(t.shape == shape, t, "expected shape " + shape_str(shape));
}

// blocks [E, R, C/32, 16] or [E, R, C/2]; scales [E, R, C/32]
inline void need_mx(const TensorView& b, const TensorView& s, int64_t E, int64_t R, int64_t C) {
    need(b.dtype == "U8", b, "MXFP4 blocks must be U8");
    need(s.dtype == "U8", s, "E8M0 scales must be U8");
    const std::vector<int64_t> b4{E, R, C / 32, 16}, b3{E, R, C / 2};
    need(b.shape == b4 || b.shape == b3, b, "expected " + shape_str(b4) + " or " + shape_str(b3));
    need(s.shape == std::vector<int64_t>({E, R, C / 32}), s, "expected " + shape_str({E, R, C / 32}));
}

}  // namespace detail

inline LayerView view_layer(const Checkpoint& ck, int layer) {
    LayerView v;
    const LayerNames hf = layer_names(Naming::HuggingFace, layer), og = layer_names(Naming::Original, layer);
    if (ck.has(hf.router_w)) v.naming = Naming::HuggingFace;
    else if (ck.has(og.router_w)) v.naming = Naming::Original;
    else
        throw Error("layer " + std::to_string(layer) + ": neither '" + hf.router_w + "' nor '" + og.router_w +
                    "' is in the checkpoint at " + ck.dir());
    const LayerNames n = layer_names(v.naming, layer);
    auto opt = [&](const std::string& name) { return ck.has(name) ? &ck.get(name) : nullptr; };
    v.router_w = &ck.get(n.router_w);
    v.router_b = opt(n.router_b);
    v.gu_blocks = &ck.get(n.gu_blocks);
    v.gu_scales = &ck.get(n.gu_scales);
    v.gu_bias = opt(n.gu_bias);
    v.dn_blocks = &ck.get(n.dn_blocks);
    v.dn_scales = &ck.get(n.dn_scales);
    v.dn_bias = opt(n.dn_bias);
    v.norm = opt(n.norm);

    const TensorView& rw = *v.router_w;
    detail::need(rw.shape.size() == 2, rw, "router weight must be [E, H]");
    const int64_t E = rw.shape[0], H = rw.shape[1];
    detail::need(E >= 1 && E <= 1024, rw, "expert count must be in [1, 1024]");
    detail::need(H >= 32 && H % 32 == 0, rw, "hidden size must be a positive multiple of 32");
    detail::need_16bit(rw, {E, H});
    const TensorView& gb = *v.gu_blocks;
    detail::need(gb.shape.size() >= 2 && gb.shape[1] % 2 == 0, gb, "gate_up rows must be 2 x intermediate");
    const int64_t I = gb.shape[1] / 2;
    detail::need(I >= 32 && I % 32 == 0, gb, "intermediate size must be a positive multiple of 32");
    detail::need_mx(gb, *v.gu_scales, E, 2 * I, H);
    detail::need_mx(*v.dn_blocks, *v.dn_scales, E, H, I);
    if (v.router_b) detail::need_16bit(*v.router_b, {E});
    if (v.gu_bias) detail::need_16bit(*v.gu_bias, {E, 2 * I});
    if (v.dn_bias) detail::need_16bit(*v.dn_bias, {E, H});
    if (v.norm) detail::need_16bit(*v.norm, {H});
    v.hidden = (int)H;
    v.intermediate = (int)I;
    v.num_experts = (int)E;
    return v;
}

}  // namespace gpt_oss
