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
// lg_ws (nullable): B * E doubles of workspace; mid-size batches then take the
// two-launch router (logits, then selection), which needs it.
int router_launch(const void* x, const void* w, const void* bias, int B, int H, int E, int K, void* idx,
                  void* wts, hipStream_t stream, void* lg_ws = nullptr);
// Whether router_launch takes the two-launch form for (B, E) when given lg_ws and
// 16-byte-aligned rows with H % 8 == 0, outside the two-pass range.
bool router_two_launch(int B, int E);
// Whether the layer's router takes the tiled two-pass form (bounds, then selection) for
// (B, E), which needs lg_ws as well (B * E float2 bounds).
bool rmx_tiled(int B, int E);
// Batch-1 route: router, top-k, softmax and bucketing in one launch (E <= 256); with
// norm_w, the token is first RMS-normalised into h_out and routed from there.
int route1_launch(const void* x, const void* w, const void* bias, int H, int E, int K, void* idx, void* wts,
                  void* counts, void* offsets, void* perm, void* pos, void* slots, void* n_slots, void* passes,
                  void* n_passes, hipStream_t stream, const void* norm_w = nullptr, float eps = 0.f,
                  void* h_out = nullptr);
// Largest hidden size whose normalised row the batch-1 route keeps in LDS.
constexpr int kRoute1NormMaxH = 16384;

}  // namespace physllm
