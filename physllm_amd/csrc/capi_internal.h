// Host-side helpers shared by the C-ABI translation units (error channel, launch checks).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/physllm_moe.h"

namespace physllm {

// Records (code, message) as the calling thread's last error and returns code.
int set_error(int code, const char* msg);
// Clears the calling thread's last error and returns PHYSLLM_MOE_OK.
int ok();
// Checks hipGetLastError() after a launch; records ELAUNCH with `what` on failure.
int check_launch(const char* what);

int dequant_launch(const void* packed, const void* scales, void* out, int64_t numel, int block_size,
                   hipStream_t stream);
int router_launch(const void* x, const void* w, const void* bias, int B, int H, int E, int K, void* idx,
                  void* wts, hipStream_t stream);
// Batch-1 route: router, top-k, softmax and bucketing in one launch (E <= 256); with
// norm_w, the token is first RMS-normalised into h_out and routed from there.
int route1_launch(const void* x, const void* w, const void* bias, int H, int E, int K, void* idx, void* wts,
                  void* counts, void* offsets, void* perm, void* pos, void* slots, void* n_slots, void* passes,
                  void* n_passes, hipStream_t stream, const void* norm_w = nullptr, float eps = 0.f,
                  void* h_out = nullptr);
// Largest hidden size whose normalised row the batch-1 route keeps in LDS.
constexpr int kRoute1NormMaxH = 16384;

}  // namespace physllm
