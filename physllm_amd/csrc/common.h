// Device-side helpers shared by the gfx950 kernels of the MXFP4 MoE path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define PHYSLLM_WAVE 64

namespace physllm {

// ---- bf16 ----------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16; NaN -> quiet NaN with the sign kept.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x0040u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// ---- MXFP4 -----------------------------------------------------------------
// Exact bf16 bits of e2m1(code) * 2^(s-127) for any code and any E8M0 byte s,
// in integer arithmetic only (no dependence on the denormal mode).
// Magnitude codes 1..7 are (1 + mant/128) * 2^(eo) with (eo, mant) below.
__device__ __forceinline__ uint32_t mx_bits_exact(uint32_t code, uint32_t s) {
    if (s == 255u) return 0x7fc0u;
    const uint32_t sign = (code & 8u) << 12;
    const uint32_t mag = code & 7u;
    if (mag == 0u) return sign;
    // eo+1 for mag 1..7: 0.5->0, 1->1, 1.5->1, 2->2, 3->2, 4->3, 6->3
    const int eo1 = (int)((0x33221100u >> (mag * 4u)) & 0xfu);
    const uint32_t mant = (mag >= 3u && (mag & 1u)) ? 0x40u : 0u;
    const int E = eo1 - 1 + (int)s;  // biased exponent of the result
    if (E >= 255) return sign | 0x7f80u;   // overflow -> inf (round-to-nearest-even)
    if (E >= 1) return sign | ((uint32_t)E << 7) | mant;
    // subnormal: (128 + mant) * 2^(E-1) units of 2^-133, E in {0, -1}, exact
    return sign | ((128u + mant) >> (1 - E));
}

// E8M0 byte as the f32 scale operand of v_cvt_scalef32_pk_bf16_fp4.
__device__ __forceinline__ float e8m0_scale_operand(uint32_t s) { return __uint_as_float(s << 23); }

// 4 packed bytes (8 e2m1 codes, lower element in the low nibble) -> 8 bf16 with
// the hardware scaled conversion; used in the GEMV/GEMM fragments.
__device__ __forceinline__ bf16x8_t mx_cvt8(uint32_t v, float scale) {
    bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 0);
    bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 1);
    bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 2);
    bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, scale, 3);
    bf16x8_t r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
    return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---- activation -------------------------------------------------------------
// Clamped SwiGLU of GPT-OSS: g = min(g, limit), u = clamp(u, -limit, limit),
// g * sigmoid(alpha g) * (u + 1); comparisons keep NaN.
__device__ __forceinline__ float swiglu(float g, float u, float alpha, float limit) {
    g = (g > limit) ? limit : g;
    u = (u > limit) ? limit : ((u < -limit) ? -limit : u);
    const float sig = 1.0f / (1.0f + expf(-alpha * g));
    return (g * sig) * (u + 1.0f);
}

// ---- wave reductions ----------------------------------------------------------
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace physllm
