// RMSNorm of one bf16 row in the summation order of kernels/rms_norm_gpu.hip:11-24
// (shared by the norm kernel and the batch-1 route kernel, which fuses the norm).
// Threads 0..255 of the workgroup take part in the sum: thread j accumulates v*v
// over i = j, j + 256, ... with one fma per element (hipcc contracts the
// reference's `tsum += v * v`); the 256 partials are added by the tree
// s = 128, 64, ..., 1 (p[j] += p[j + s]): the first two levels through LDS, the
// last six inside wave 0 with lane shuffles, which add the same operands in the
// same order. Contraction is off and `/` and sqrtf are correctly rounded (HIP's
// default), so the result is bit-identical to that order evaluated in fp32.
#pragma once

#include "common.h"

namespace physllm {

// Every thread of the workgroup calls this (it contains barriers). part: 128 floats
// of LDS; rms_slot: one float of LDS. Returns rms = sqrtf(sum / H + eps) to all.
__device__ __forceinline__ float rms_of_row(const uint16_t* xr, int H, float eps, float* part, float* rms_slot) {
#pragma clang fp contract(off)
    const int j = threadIdx.x;
    float t = 0.f;
    if (j < 256)
        for (int i = j; i < H; i += 256) {
            const float v = bf16_to_f32(xr[i]);
            t = __builtin_fmaf(v, v, t);
        }
    if (j >= 128 && j < 256) part[j - 128] = t;  // level s = 128
    __syncthreads();
    if (j < 128) t = t + part[j];
    __syncthreads();
    if (j >= 64 && j < 128) part[j - 64] = t;  // level s = 64
    __syncthreads();
    if (j < 64) {
        t = t + part[j];
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) {  // levels s = 32 .. 1 in wave 0
            const float o = __shfl_down(t, s, 64);
            t = t + o;
        }
        if (j == 0) *rms_slot = __builtin_sqrtf(t / (float)H + eps);
    }
    __syncthreads();
    return *rms_slot;
}

// bf16((v / rms) * w) for one element, and for 8 packed elements.
__device__ __forceinline__ uint32_t rms_apply1(uint32_t xb, uint32_t wb, float rms) {
#pragma clang fp contract(off)
    return f32_to_bf16((bf16_to_f32(xb) / rms) * bf16_to_f32(wb));
}

__device__ __forceinline__ uint4 rms_apply8(uint4 a, uint4 w, float rms) {
#pragma clang fp contract(off)
    const uint32_t* ap = (const uint32_t*)&a;
    const uint32_t* wp = (const uint32_t*)&w;
    uint4 r;
    uint32_t* rp = (uint32_t*)&r;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const float lo = (bf16_lo(ap[u]) / rms) * bf16_lo(wp[u]);
        const float hi = (bf16_hi(ap[u]) / rms) * bf16_hi(wp[u]);
        rp[u] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
    }
    return r;
}

}  // namespace physllm
