// C++ mirror of the MoE half of PhysLLM's MoEInferenceEngine::forward_moe_layer
// (crates/llm-core/src/moe.rs:237-313) over libphysllm_moe's whole-layer entry
// point. The reference routes on the device, copies the routing to the host and
// runs a host loop over the k experts with per-expert allocations and blocking
// copies (moe.rs:249-299); here the routing, the expert GEMVs/GEMMs and the
// combine stay on the device, in one call, with a workspace allocated once per
// layer. forward_moe_block adds the RMSNorm before (moe.rs:239-244) and the
// residual add after (moe.rs:310-311) in the same single call.
#pragma once

#include "rocm_backend.hpp"

namespace llm_core {

using rocm_backend::bf16;
using rocm_backend::DeviceTensor;
using rocm_backend::GpuDevice;

// Shapes of crates/llm-core/src/config.rs:188-230 (gpt_oss_20b) that the path uses.
struct MoEShape {
    int hidden_dim = 2880;
    int intermediate_dim = 2880;
    int num_experts = 32;
    int experts_per_token = 4;
};

// MXFP4 expert weights of one layer (the role of ExpertWeightsMXFP4, moe.rs:41-51,
// with E8M0 scales and the GPT-OSS fused, row-interleaved gate_up tensor).
struct MoELayerWeightsMXFP4 {
    DeviceTensor<bf16> router_weight;       // [E, H]
    DeviceTensor<bf16> router_bias;         // [E] (may be empty)
    DeviceTensor<uint8_t> gate_up_blocks;   // [E, 2I, H/2]
    DeviceTensor<uint8_t> gate_up_scales;   // [E, 2I, H/32]
    DeviceTensor<bf16> gate_up_bias;        // [E, 2I] (may be empty)
    DeviceTensor<uint8_t> down_blocks;      // [E, H, I/2]
    DeviceTensor<uint8_t> down_scales;      // [E, H, I/32]
    DeviceTensor<bf16> down_bias;           // [E, H] (may be empty)
};

class MoELayer {
  public:
    MoELayer(MoEShape shape, MoELayerWeightsMXFP4&& w, float swiglu_alpha = 1.702f, float swiglu_limit = 7.0f)
        : shape_(shape), w_(std::move(w)) {
        cfg_ = physllm_moe_config{shape.hidden_dim, shape.intermediate_dim, shape.num_experts,
                                  shape.experts_per_token, swiglu_alpha, swiglu_limit};
        ptrs_ = physllm_moe_weights{w_.router_weight.raw_ptr(), w_.router_bias.raw_ptr(),
                                    w_.gate_up_blocks.raw_ptr(), w_.gate_up_scales.raw_ptr(),
                                    w_.gate_up_bias.raw_ptr(),   w_.down_blocks.raw_ptr(),
                                    w_.down_scales.raw_ptr(),    w_.down_bias.raw_ptr()};
    }

    // normed [B, H] -> moe_out [B, H]; optional routing outputs [B, k].
    void forward_moe_layer(const GpuDevice& dev, const DeviceTensor<bf16>& normed, DeviceTensor<bf16>& moe_out,
                           DeviceTensor<int32_t>* expert_indices = nullptr,
                           DeviceTensor<float>* expert_weights = nullptr) {
        const int batch = (int)normed.rows();
        if ((int)normed.cols() != shape_.hidden_dim)
            throw rocm_backend::BackendError(PHYSLLM_MOE_EINVAL, "forward_moe_layer: hidden size mismatch");
        const size_t need = physllm_moe_workspace_bytes(&cfg_, batch);
        if (need == 0 && batch > 0) rocm_backend::moe_check("physllm_moe_workspace_bytes");
        if (workspace_.numel() < need) workspace_ = DeviceTensor<uint8_t>::alloc({need});
        const int rc = physllm_moe_layer_forward(
            &cfg_, &ptrs_, normed.raw_ptr(), batch, moe_out.raw_ptr(),
            expert_indices ? expert_indices->raw_ptr() : nullptr, expert_weights ? expert_weights->raw_ptr() : nullptr,
            workspace_.raw_ptr(), workspace_.numel(), dev.raw_stream());
        if (rc != PHYSLLM_MOE_OK)
            throw rocm_backend::BackendError(rc, std::string("physllm_moe_layer_forward: ") +
                                                     physllm_moe_last_error_message());
        dev.synchronise();
    }

    // The whole MoE sub-layer, moe.rs:238-313 (steps 8-12): residual [B, H] is
    // updated in place to residual + moe(rms_norm(residual, ffn_norm, eps)).
    void forward_moe_block(const GpuDevice& dev, DeviceTensor<bf16>& residual, const DeviceTensor<bf16>& ffn_norm,
                           float eps, DeviceTensor<int32_t>* expert_indices = nullptr,
                           DeviceTensor<float>* expert_weights = nullptr) {
        const int batch = (int)residual.rows();
        if ((int)residual.cols() != shape_.hidden_dim || (int)ffn_norm.numel() != shape_.hidden_dim)
            throw rocm_backend::BackendError(PHYSLLM_MOE_EINVAL, "forward_moe_block: hidden size mismatch");
        const size_t need = physllm_moe_block_workspace_bytes(&cfg_, batch);
        if (need == 0 && batch > 0) rocm_backend::moe_check("physllm_moe_block_workspace_bytes");
        if (workspace_.numel() < need) workspace_ = DeviceTensor<uint8_t>::alloc({need});
        const int rc = physllm_moe_block_forward(
            &cfg_, &ptrs_, residual.raw_ptr(), ffn_norm.raw_ptr(), eps, batch, residual.raw_ptr(),
            expert_indices ? expert_indices->raw_ptr() : nullptr, expert_weights ? expert_weights->raw_ptr() : nullptr,
            workspace_.raw_ptr(), workspace_.numel(), dev.raw_stream());
        if (rc != PHYSLLM_MOE_OK)
            throw rocm_backend::BackendError(rc, std::string("physllm_moe_block_forward: ") +
                                                     physllm_moe_last_error_message());
        dev.synchronise();
    }

    const physllm_moe_config& config() const { return cfg_; }

  private:
    MoEShape shape_;
    MoELayerWeightsMXFP4 w_;
    physllm_moe_config cfg_{};
    physllm_moe_weights ptrs_{};
    DeviceTensor<uint8_t> workspace_;
};

}  // namespace llm_core
