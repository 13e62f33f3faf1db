// The steps either side of the MoE layer in one transformer block
// (crates/llm-core/src/moe.rs:238-313): RMSNorm of the hidden state before the
// router (:239-244) and the residual add after the combine (:310-311), plus the
// legacy launchers kernels/rms_norm_gpu.hip:36-45 and kernels/residual_add.hip:12-19
// with bf16 data.
//
// RMSNorm keeps the reference's summation order exactly (rmsnorm.h), so that its
// output is bit-identical.
#include "capi_internal.h"
#include "common.h"
#include "experts.h"
#include "rmsnorm.h"

namespace physllm {

constexpr int kNormThreads = 256;

// One workgroup per row. VEC: H % 8 == 0 and x, w, out 16-byte aligned, so the
// output pass moves 8 elements per 16-byte access. x may equal out: every element
// is read by the thread that writes it, after the barrier that ends the sum.
template <bool VEC>
__global__ __launch_bounds__(kNormThreads) void k_rms_norm(const uint16_t* x, const uint16_t* __restrict__ wt,
                                                           uint16_t* out, int H, float eps) {
    __shared__ float part[128];
    __shared__ float rms_s;
    const int j = threadIdx.x;
    const size_t base = (size_t)blockIdx.x * H;
    const uint16_t* xr = x + base;
    const float rms = rms_of_row(xr, H, eps, part, &rms_s);
    if (VEC) {
        const uint4* xv = (const uint4*)xr;
        const uint4* wv = (const uint4*)wt;
        uint4* ov = (uint4*)(out + base);
        for (int c = j; c < (H >> 3); c += kNormThreads) ov[c] = rms_apply8(xv[c], wv[c], rms);
    } else {
        for (int i = j; i < H; i += kNormThreads) out[base + i] = (uint16_t)rms_apply1(xr[i], wt[i], rms);
    }
}

// out[i] = bf16(out[i] + res[i]) in fp32; 8 elements per thread.
__global__ __launch_bounds__(256) void k_residual_add(uint16_t* out, const uint16_t* res, int64_t n, int vec) {
#pragma clang fp contract(off)
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i0 = c * 8;
    if (i0 >= n) return;
    if (vec && i0 + 8 <= n) {
        uint4 a = ((const uint4*)out)[c];
        const uint4 b = ((const uint4*)res)[c];
        uint32_t* ap = (uint32_t*)&a;
        const uint32_t* bp = (const uint32_t*)&b;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            ap[u] = f32_to_bf16(bf16_lo(ap[u]) + bf16_lo(bp[u])) |
                    (f32_to_bf16(bf16_hi(ap[u]) + bf16_hi(bp[u])) << 16);
        ((uint4*)out)[c] = a;
    } else {
        const int64_t i1 = i0 + 8 < n ? i0 + 8 : n;
        for (int64_t i = i0; i < i1; ++i) out[i] = (uint16_t)f32_to_bf16(bf16_to_f32(out[i]) + bf16_to_f32(res[i]));
    }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int rms_norm_launch(const void* x, const void* w, void* out, int B, int H, float eps, hipStream_t stream) {
    if (B < 0 || H < 1) return set_error(PHYSLLM_MOE_EINVAL, "rms_norm: batch < 0 or hidden < 1");
    if (B == 0) return ok();
    if (!x || !w || !out) return set_error(PHYSLLM_MOE_EINVAL, "rms_norm: null pointer");
    const bool vec = H % 8 == 0 && aligned16(x) && aligned16(w) && aligned16(out);
    if (vec)
        hipLaunchKernelGGL(k_rms_norm<true>, dim3(B), dim3(kNormThreads), 0, stream, (const uint16_t*)x,
                           (const uint16_t*)w, (uint16_t*)out, H, eps);
    else
        hipLaunchKernelGGL(k_rms_norm<false>, dim3(B), dim3(kNormThreads), 0, stream, (const uint16_t*)x,
                           (const uint16_t*)w, (uint16_t*)out, H, eps);
    return check_launch("rms_norm");
}

int residual_add_launch(void* out, const void* res, int64_t n, hipStream_t stream) {
    if (n < 0) return set_error(PHYSLLM_MOE_EINVAL, "residual_add: size < 0");
    if (n == 0) return ok();
    if (!out || !res) return set_error(PHYSLLM_MOE_EINVAL, "residual_add: null pointer");
    const int vec = aligned16(out) && aligned16(res);
    const int64_t chunks = (n + 7) / 8;
    hipLaunchKernelGGL(k_residual_add, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, (uint16_t*)out,
                       (const uint16_t*)res, n, vec);
    return check_launch("residual_add");
}

}  // namespace physllm

using namespace physllm;

extern "C" void launch_rms_norm(const void* input, const void* weight, void* output, int batch_size, int hidden_dim,
                                float eps, void* stream) {
    rms_norm_launch(input, weight, output, batch_size, hidden_dim, eps, (hipStream_t)stream);
}

extern "C" void launch_residual_add(void* output, const void* residual, int size, void* stream) {
    residual_add_launch(output, residual, size, (hipStream_t)stream);
}
