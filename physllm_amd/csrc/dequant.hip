// MXFP4 (e2m1 codes + E8M0 block scales) -> bf16 dequantization for gfx950.
//
// Semantics follow kernels/mxfp4_dequant.hip:19-51 of the reference (e2m1 table,
// low nibble = even element, scale index = element / block_size over the flat
// tensor, the scale of element 2i also serving 2i+1) with E8M0 scales and bf16
// output: out = bf16(e2m1(code) * 2^(s-127)), exact, s = 255 -> NaN 0x7FC0.
//
// Fast path (block_size 32, numel % 32 == 0, aligned pointers): each lane turns
// one 4-byte word of codes (8 elements, a quarter of a scale block) into one
// 16-byte store, so a wave reads 256 contiguous code bytes and writes 1 KiB
// contiguous output per step. A byte is decoded through a 256-entry LDS table
// holding its two bf16 values at unit scale plus a "which halves are nonzero"
// multiplier; the scale is applied by adding (s-127) << 7 to each nonzero
// half's exponent field with one 24-bit multiply-add. That is exact whenever the
// result stays a normal bf16, i.e. for s in [2, 252]; other scales take the
// integer closed form (mx_bits_exact), so every (code, scale) pair is exact.
#include "common.h"
#include "capi_internal.h"

namespace physllm {

// {pair of bf16 at unit scale, nonzero multiplier} for byte b.
__device__ __forceinline__ uint2 dq_table_entry(uint32_t b) {
    const uint32_t lo = b & 15u, hi = b >> 4;
    uint2 r;
    r.x = mx_bits_exact(lo, 127u) | (mx_bits_exact(hi, 127u) << 16);
    r.y = ((lo & 7u) ? 1u : 0u) + ((hi & 7u) ? 65536u : 0u);
    return r;
}

__device__ __forceinline__ uint32_t dq_pair_fast(const uint2* tab, uint32_t byte, int delta128) {
    const uint2 t = tab[byte];
    return (uint32_t)__mul24((int)t.y, delta128) + t.x;
}

__device__ __forceinline__ uint32_t dq_pair_exact(uint32_t byte, uint32_t s) {
    return mx_bits_exact(byte & 15u, s) | (mx_bits_exact(byte >> 4, s) << 16);
}

constexpr int kDqThreads = 256;
constexpr int kDqUnroll = 4;  // 4-byte words per lane per step

// Fast path: numel % 32 == 0, block size 32. n_words = numel / 8.
__global__ __launch_bounds__(kDqThreads) void k_mxfp4_dequant32(const uint32_t* __restrict__ packed,
                                                                const uint8_t* __restrict__ scales,
                                                                u32x4_t* __restrict__ out,
                                                                int64_t n_words) {
    __shared__ uint2 tab[256];
    tab[threadIdx.x] = dq_table_entry(threadIdx.x);
    __syncthreads();

    const int64_t base = (int64_t)blockIdx.x * (kDqThreads * kDqUnroll) + threadIdx.x;
    uint32_t v[kDqUnroll];
    uint32_t s[kDqUnroll];
#pragma unroll
    for (int i = 0; i < kDqUnroll; ++i) {
        const int64_t w = base + (int64_t)i * kDqThreads;
        v[i] = 0u;
        s[i] = 127u;
        if (w < n_words) {
            v[i] = __builtin_nontemporal_load(packed + w);
            s[i] = scales[w >> 2];
        }
    }
#pragma unroll
    for (int i = 0; i < kDqUnroll; ++i) {
        const int64_t w = base + (int64_t)i * kDqThreads;
        if (w >= n_words) continue;
        u32x4_t o;
        if (s[i] - 2u <= 250u) {
            const int d = ((int)s[i] - 127) * 128;
            o[0] = dq_pair_fast(tab, v[i] & 0xffu, d);
            o[1] = dq_pair_fast(tab, (v[i] >> 8) & 0xffu, d);
            o[2] = dq_pair_fast(tab, (v[i] >> 16) & 0xffu, d);
            o[3] = dq_pair_fast(tab, v[i] >> 24, d);
        } else {
            o[0] = dq_pair_exact(v[i] & 0xffu, s[i]);
            o[1] = dq_pair_exact((v[i] >> 8) & 0xffu, s[i]);
            o[2] = dq_pair_exact((v[i] >> 16) & 0xffu, s[i]);
            o[3] = dq_pair_exact(v[i] >> 24, s[i]);
        }
        __builtin_nontemporal_store(o, out + w);
    }
}

// Generic path: any block size >= 1, any numel; one byte (two elements) per lane.
__global__ __launch_bounds__(kDqThreads) void k_mxfp4_dequant_generic(const uint8_t* __restrict__ packed,
                                                                      const uint8_t* __restrict__ scales,
                                                                      uint16_t* __restrict__ out,
                                                                      int64_t numel, int block_size) {
    const int64_t i = (int64_t)blockIdx.x * kDqThreads + threadIdx.x;
    const int64_t v = 2 * i;
    if (v >= numel) return;
    const uint32_t b = packed[i];
    const uint32_t s = scales[v / block_size];
    out[v] = (uint16_t)mx_bits_exact(b & 15u, s);
    if (v + 1 < numel) out[v + 1] = (uint16_t)mx_bits_exact(b >> 4, s);
}

int dequant_launch(const void* packed, const void* scales, void* out, int64_t numel, int block_size,
                   hipStream_t stream) {
    if (numel < 0) return set_error(PHYSLLM_MOE_EINVAL, "mxfp4_dequant: numel < 0");
    if (block_size < 1) return set_error(PHYSLLM_MOE_EINVAL, "mxfp4_dequant: block_size < 1");
    if (numel == 0) return ok();
    if (!packed || !scales || !out) return set_error(PHYSLLM_MOE_EINVAL, "mxfp4_dequant: null pointer");
    const bool aligned = ((uintptr_t)packed % 4 == 0) && ((uintptr_t)out % 16 == 0);
    if (block_size == 32 && numel % 32 == 0 && aligned) {
        const int64_t n_words = numel / 8;
        const int64_t per_block = (int64_t)kDqThreads * kDqUnroll;
        const int64_t grid = (n_words + per_block - 1) / per_block;
        if (grid > 0x7fffffffLL) return set_error(PHYSLLM_MOE_EINVAL, "mxfp4_dequant: tensor too large");
        hipLaunchKernelGGL(k_mxfp4_dequant32, dim3((unsigned)grid), dim3(kDqThreads), 0, stream,
                           (const uint32_t*)packed, (const uint8_t*)scales, (u32x4_t*)out, n_words);
    } else {
        const int64_t npairs = (numel + 1) / 2;
        const int64_t grid = (npairs + kDqThreads - 1) / kDqThreads;
        if (grid > 0x7fffffffLL) return set_error(PHYSLLM_MOE_EINVAL, "mxfp4_dequant: tensor too large");
        hipLaunchKernelGGL(k_mxfp4_dequant_generic, dim3((unsigned)grid), dim3(kDqThreads), 0, stream,
                           (const uint8_t*)packed, (const uint8_t*)scales, (uint16_t*)out, numel, block_size);
    }
    return check_launch("mxfp4_dequant");
}

}  // namespace physllm

extern "C" void launch_mxfp4_dequant(const void* packed_data, const void* scales, void* output, int numel,
                                     int block_size, void* stream) {
    physllm::dequant_launch(packed_data, scales, output, (int64_t)numel, block_size, (hipStream_t)stream);
}

extern "C" int physllm_moe_mxfp4_dequant(const void* packed, const void* scales, void* out, int64_t numel,
                                         void* stream) {
    return physllm::dequant_launch(packed, scales, out, numel, 32, (hipStream_t)stream);
}
