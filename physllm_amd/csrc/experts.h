// Shared declarations of the expert kernels (decode GEMV, prefill GEMM, combine).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace physllm {

enum { kModeGateUp = 0, kModeDown = 1 };

// One grouped-expert pass over routed tokens. The expert of work slot s is
// active[s] (s < *n_active); its tokens are the sorted positions
// offsets[e] .. offsets[e] + counts[e].
struct GemvParams {
    const uint16_t* act;     // gate_up: x [B, Kdim] (row = pair / top_k); down: h [N, Kdim] by sorted position
    const uint8_t* blocks;   // [E, R, Kdim/2] packed e2m1
    const uint8_t* scales;   // [E, R, Kdim/32] E8M0
    const uint16_t* bias;    // [E, R] bf16, nullable
    const int32_t* counts;   // [E]
    const int32_t* offsets;  // [E+1]
    const int32_t* perm;     // [N] sorted position -> pair id
    const int32_t* active;   // [E] touched experts, ascending
    const int32_t* n_active; // [1]
    void* out;               // gate_up: h bf16 [N, R/2]; down: y fp32 [N, R] (by sorted position)
    int Kdim;                // reduction length (H for gate_up, I for down)
    int R;                   // weight rows per expert (2I or H)
    int top_k;
    float alpha, limit;
};

int gemv_launch(int mode, const GemvParams& p, int max_slots, int max_tokens, hipStream_t stream);
int combine_launch(const float* y, const int32_t* pos, const float* wts, uint16_t* out, int B, int H, int K,
                   hipStream_t stream);
int bucket_launch(const void* idx, int N, int E, void* counts, void* offsets, void* perm, void* pos, void* active,
                  void* n_active, hipStream_t stream);

}  // namespace physllm
