// CPU driver of the safetensors reader and the GPT-OSS layer view
// (physllm_amd/host/safetensors.hpp, gpt_oss_checkpoint.hpp), built with g++ alone.
//   checkpoint_tool dump <file-or-dir>    one line per tensor: name dtype shape offset nbytes fnv1a64
//   checkpoint_tool layer <dir> <i>       the validated view of layer i and config.json
// Errors print "ERROR: <message>" and exit with status 3.
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../physllm_amd/host/gpt_oss_checkpoint.hpp"

static uint64_t fnv1a(const uint8_t* p, size_t n) {
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}

static void print_view(const char* role, const safetensors::TensorView* t) {
    if (!t) {
        std::printf("%s -\n", role);
        return;
    }
    std::printf("%s %s %s\n", role, t->name.c_str(), t->dtype.c_str());
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s dump <path> | layer <dir> <i>\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    try {
        if (mode == "dump") {
            safetensors::Checkpoint ck(argv[2]);
            std::printf("shards %zu\n", ck.num_shards());
            for (const auto& n : ck.names()) {
                const auto& t = ck.get(n);
                std::string shape;
                for (size_t k = 0; k < t.shape.size(); ++k) shape += (k ? "," : "") + std::to_string(t.shape[k]);
                std::printf("tensor %s %s [%s] %zu %zu %016" PRIx64 "\n", t.name.c_str(), t.dtype.c_str(),
                            shape.c_str(), t.offset, t.nbytes, fnv1a(t.data, t.nbytes));
            }
            for (const auto& m : ck.metadata()) std::printf("meta %s %s\n", m.first.c_str(), m.second.c_str());
        } else if (mode == "layer" && argc >= 4) {
            safetensors::Checkpoint ck(argv[2]);
            const gpt_oss::LayerView v = gpt_oss::view_layer(ck, std::atoi(argv[3]));
            const gpt_oss::Config c = gpt_oss::read_config(ck.dir());
            std::printf("naming %s\n", v.naming == gpt_oss::Naming::HuggingFace ? "huggingface" : "original");
            std::printf("shape %d %d %d\n", v.hidden, v.intermediate, v.num_experts);
            print_view("router_w", v.router_w);
            print_view("router_b", v.router_b);
            print_view("gu_blocks", v.gu_blocks);
            print_view("gu_scales", v.gu_scales);
            print_view("gu_bias", v.gu_bias);
            print_view("dn_blocks", v.dn_blocks);
            print_view("dn_scales", v.dn_scales);
            print_view("dn_bias", v.dn_bias);
            print_view("norm", v.norm);
            std::printf("config %d %d %d %d %d %g %g %d\n", c.hidden, c.intermediate, c.num_experts,
                        c.experts_per_token, c.num_layers, (double)c.rms_norm_eps, (double)c.swiglu_limit,
                        (int)c.found);
        } else {
            std::fprintf(stderr, "bad mode\n");
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("ERROR: %s\n", e.what());
        return 3;
    }
    return 0;
}
