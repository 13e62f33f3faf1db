// Loads one GPT-OSS MoE layer from an MXFP4 safetensors checkpoint straight into
// the device buffers of llm_core::MoELayer: the e2m1 blocks and E8M0 scales are
// copied byte for byte from the file mapping, the 16-bit tensors as bf16 bits.
// This replaces load_gpt_oss_weights (crates/llm-core/src/gpt_oss_loader.rs:57-201)
// for the MoE half of a layer; names, layouts and checks are in gpt_oss_checkpoint.hpp.
#pragma once

#include <cstring>

#include "gpt_oss_checkpoint.hpp"
#include "moe_engine.hpp"

namespace llm_core {

// bf16 bits of a BF16 (copied as is) or F32 (rounded to nearest even) tensor.
inline DeviceTensor<bf16> upload_bf16(const gpt_oss::TensorView& t) {
    std::vector<size_t> shape(t.shape.begin(), t.shape.end());
    if (t.dtype == "BF16") return DeviceTensor<bf16>::from_host((const bf16*)t.data, std::move(shape));
    std::vector<bf16> h((size_t)t.numel());
    for (size_t i = 0; i < h.size(); ++i) {
        uint32_t u;
        std::memcpy(&u, t.data + 4 * i, 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) h[i] = (bf16)((u >> 16) | 0x0040u);
        else h[i] = (bf16)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
    return DeviceTensor<bf16>::from_slice(h, std::move(shape));
}

inline DeviceTensor<uint8_t> upload_u8(const gpt_oss::TensorView& t, std::vector<size_t> shape) {
    return DeviceTensor<uint8_t>::from_host(t.data, std::move(shape));
}

// The MoE sub-layer of one transformer block as loaded: the layer, its RMSNorm
// weight (moe.rs:240-244; empty if the checkpoint has none) and epsilon.
struct GptOssMoEBlock {
    MoELayer layer;
    DeviceTensor<bf16> ffn_norm;
    float rms_norm_eps;
};

// experts_per_token: 0 takes it from config.json.
inline GptOssMoEBlock load_gpt_oss_moe_layer(const gpt_oss::Checkpoint& ck, int layer, int experts_per_token = 0) {
    const gpt_oss::Config cfg = gpt_oss::read_config(ck.dir());
    const gpt_oss::LayerView v = gpt_oss::view_layer(ck, layer);
    const int k = experts_per_token ? experts_per_token : cfg.experts_per_token;
    if (k < 1 || k > v.num_experts)
        throw rocm_backend::BackendError(PHYSLLM_MOE_EINVAL, "gpt-oss layer " + std::to_string(layer) +
                                                                 ": experts per token unknown or out of range");
    auto agree = [&](int from_cfg, int from_tensors, const char* what) {
        if (from_cfg && from_cfg != from_tensors)
            throw rocm_backend::BackendError(PHYSLLM_MOE_EINVAL, std::string("config.json ") + what +
                                                                     " disagrees with the tensor shapes");
    };
    agree(cfg.hidden, v.hidden, "hidden_size");
    agree(cfg.intermediate, v.intermediate, "intermediate_size");
    agree(cfg.num_experts, v.num_experts, "expert count");
    const size_t E = v.num_experts, H = v.hidden, I = v.intermediate;
    MoELayerWeightsMXFP4 w;
    w.router_weight = upload_bf16(*v.router_w);
    if (v.router_b) w.router_bias = upload_bf16(*v.router_b);
    w.gate_up_blocks = upload_u8(*v.gu_blocks, {E, 2 * I, H / 2});
    w.gate_up_scales = upload_u8(*v.gu_scales, {E, 2 * I, H / 32});
    if (v.gu_bias) w.gate_up_bias = upload_bf16(*v.gu_bias);
    w.down_blocks = upload_u8(*v.dn_blocks, {E, H, I / 2});
    w.down_scales = upload_u8(*v.dn_scales, {E, H, I / 32});
    if (v.dn_bias) w.down_bias = upload_bf16(*v.dn_bias);
    MoEShape shape{v.hidden, v.intermediate, v.num_experts, k};
    GptOssMoEBlock b{MoELayer(shape, std::move(w), cfg.swiglu_alpha, cfg.swiglu_limit),
                     v.norm ? upload_bf16(*v.norm) : DeviceTensor<bf16>(), cfg.rms_norm_eps};
    return b;
}

}  // namespace llm_core
