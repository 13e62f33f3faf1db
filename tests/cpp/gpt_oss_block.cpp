// GPU driver: loads MoE layer <i> of a GPT-OSS MXFP4 safetensors checkpoint with
// llm_core::load_gpt_oss_moe_layer and runs the block (rms_norm -> layer -> residual
// add, in place) on B tokens read from a raw bf16 file.
//   gpt_oss_block <ckpt> <i> <x.bin> <B> <out.bin>
// out.bin = out bf16 [B,H], then top-k indices int32 [B,k], then weights fp32 [B,k].
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../physllm_amd/host/gpt_oss_loader.hpp"

int main(int argc, char** argv) {
    if (argc != 6) {
        std::fprintf(stderr, "usage: %s <ckpt> <layer> <x.bin> <B> <out.bin>\n", argv[0]);
        return 2;
    }
    try {
        auto dev = rocm_backend::GpuDevice::open_best();
        gpt_oss::Checkpoint ck(argv[1]);
        llm_core::GptOssMoEBlock blk = llm_core::load_gpt_oss_moe_layer(ck, std::atoi(argv[2]));
        const physllm_moe_config& c = blk.layer.config();
        const size_t B = (size_t)std::atol(argv[4]), H = c.hidden, K = c.top_k;
        std::vector<uint16_t> x(B * H);
        std::FILE* f = std::fopen(argv[3], "rb");
        if (!f || std::fread(x.data(), 2, x.size(), f) != x.size()) throw std::runtime_error("cannot read x");
        std::fclose(f);
        auto resid = rocm_backend::DeviceTensor<uint16_t>::from_slice(x, {B, H});
        auto idx = rocm_backend::DeviceTensor<int32_t>::alloc({B, K});
        auto wts = rocm_backend::DeviceTensor<float>::alloc({B, K});
        blk.layer.forward_moe_block(dev, resid, blk.ffn_norm, blk.rms_norm_eps, &idx, &wts);
        const auto o = resid.copy_to_host();
        const auto i = idx.copy_to_host();
        const auto w = wts.copy_to_host();
        f = std::fopen(argv[5], "wb");
        if (!f) throw std::runtime_error("cannot write output");
        std::fwrite(o.data(), 2, o.size(), f);
        std::fwrite(i.data(), 4, i.size(), f);
        std::fwrite(w.data(), 4, w.size(), f);
        std::fclose(f);
        std::printf("loaded layer %s: H=%d I=%d E=%d k=%d eps=%g; block on %zu tokens done\n", argv[2], c.hidden,
                    c.intermediate, c.num_experts, c.top_k, (double)blk.rms_norm_eps, B);
    } catch (const std::exception& e) {
        std::printf("ERROR: %s\n", e.what());
        return 3;
    }
    return 0;
}
