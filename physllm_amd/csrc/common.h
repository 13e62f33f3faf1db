// Device-side helpers shared by the gfx950 kernels of the MXFP4 MoE path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

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

// The k-steps of one 16-row MXFP4 tile against the B columns staged in LDS (the
// decode GEMVs' pass): wq = the tile's stripes (step j: 16 bytes of codes of block
// 4j + g per lane), sl = this lane's scale row in LDS at block g, xl = its
// activation row in LDS at block g, xz = 64 zero bytes in LDS. The scale byte of
// step j is read two steps ahead (its LDS latency would stall every step). A lane
// whose block is past the K range takes the scale operand 0.0 (its codes decode to
// zeros) and reads its activations from xz, so it adds exactly 0 without a per-step
// branch. Four accumulators, summed in a fixed order.
template <int NIT>
__device__ __forceinline__ f32x4_t mx_tile_steps(const u32x4_t (&wq)[NIT], const uint8_t* sl, const uint4* xl,
                                                 const uint4* xz, int nblk, int g) {
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;
    uint32_t sp0 = sl[0], sp1 = sl[4];
#pragma unroll
    for (int j = 0; j < NIT; ++j) {
        if (4 * j < nblk) {  // wave-uniform
            uint32_t sj = (j & 1) ? sp1 : sp0;
            if (4 * j + 8 < nblk) {  // wave-uniform: the read for step j + 2
                if (j & 1) sp1 = sl[4 * j + 8];
                else sp0 = sl[4 * j + 8];
            }
            const bool bv = 4 * j + g < nblk;
            sj = bv ? sj : 0u;
            // an opaque no-op on the scale keeps the compiler from hoisting all the
            // converted fragments ahead of the MFMAs
            asm volatile("" : "+v"(sj));
            const float sf = e8m0_scale_operand(sj);
            const u32x4_t q = wq[j];
            const uint4* xp = bv ? xl + 16 * j : xz;
            const uint4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
            acc0 = mfma16x16x32(mx_cvt8(q[0], sf), as_bf16x8(x0), acc0);
            acc1 = mfma16x16x32(mx_cvt8(q[1], sf), as_bf16x8(x1), acc1);
            acc2 = mfma16x16x32(mx_cvt8(q[2], sf), as_bf16x8(x2), acc2);
            acc3 = mfma16x16x32(mx_cvt8(q[3], sf), as_bf16x8(x3), acc3);
        }
    }
    return (acc0 + acc1) + (acc2 + acc3);
}

// ---- buffer loads -----------------------------------------------------------
// A raw buffer over [base, base + bytes): loads past the range read zeros and
// make no memory access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

constexpr uint32_t kRsrcPast = 0xfffff000u;  // an offset past any buffer range used here (a load there reads zeros)

__device__ __forceinline__ u32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, int imm) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff + (uint32_t)imm, 0, 0);
}

// ---- activation -------------------------------------------------------------
// Clamped SwiGLU of GPT-OSS: g = min(g, limit), u = clamp(u, -limit, limit),
// g * sigmoid(alpha g) * (u + 1); comparisons keep NaN.
// The sigmoid uses the hardware base-2 exponential (v_exp_f32) and reciprocal
// (v_rcp_f32), each within about one fp32 ulp: the result is rounded to bf16
// (8 significant bits), so this is indistinguishable from a correctly rounded
// sigmoid except at bf16 rounding ties, and it costs 4 instructions instead of an
// accurate expf and an IEEE division (about 35), which matters in the GEMM
// epilogue where the matrix cores idle. Limits match expf: exp2 overflows to +inf
// (sigmoid 0) and underflows to 0 (sigmoid 1).
__device__ __forceinline__ float swiglu(float g, float u, float alpha, float limit) {
    g = (g > limit) ? limit : g;
    u = (u > limit) ? limit : ((u < -limit) ? -limit : u);
    const float e = __builtin_amdgcn_exp2f(g * (-alpha * 1.4426950408889634f));
    const float sig = __builtin_amdgcn_rcpf(1.0f + e);
    return (g * sig) * (u + 1.0f);
}

// ---- wave reductions ----------------------------------------------------------
// Sums over the 64 lanes without LDS round trips: DPP quad swaps and row
// mirrors inside each 16-lane row, then the gfx950 cross-row swaps
// (v_permlane16_swap, v_permlane32_swap). Every lane ends with the same value;
// the pairing order is fixed, so the result is deterministic.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint32_t lo = __builtin_amdgcn_update_dpp(0u, (uint32_t)__double2loint(v), CTRL, 0xf, 0xf, false);
    const uint32_t hi = __builtin_amdgcn_update_dpp(0u, (uint32_t)__double2hiint(v), CTRL, 0xf, 0xf, false);
    return __hiloint2double((int)hi, (int)lo);
}
// Pair sums across 16-lane rows: v_permlane16_swap(v, v) returns the rows
// paired (0,1) and (2,3) in its two results, one from each row of a pair in
// every lane, so their sum is the pair's sum in every lane (v_permlane32_swap:
// rows (0,2) and (1,3)); the operands arrive in the same order everywhere.
__device__ __forceinline__ float rowpair16_sum_f32(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float rowpair32_sum_f32(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ double rowpair16_sum_f64(double v) {
    const uint32_t lo = (uint32_t)__double2loint(v), hi = (uint32_t)__double2hiint(v);
    const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return __hiloint2double((int)rh[0], (int)rl[0]) + __hiloint2double((int)rh[1], (int)rl[1]);
}
__device__ __forceinline__ double rowpair32_sum_f64(double v) {
    const uint32_t lo = (uint32_t)__double2loint(v), hi = (uint32_t)__double2hiint(v);
    const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return __hiloint2double((int)rh[0], (int)rl[0]) + __hiloint2double((int)rh[1], (int)rl[1]);
}

constexpr int kDppXor1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within each 16

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    v += dpp_f32<kDppMirror>(v);
    v = rowpair16_sum_f32(v);
    return rowpair32_sum_f32(v);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<kDppXor1>(v);
    v += dpp_f64<kDppXor2>(v);
    v += dpp_f64<kDppHalfMirror>(v);
    v += dpp_f64<kDppMirror>(v);
    v = rowpair16_sum_f64(v);
    return rowpair32_sum_f64(v);
}

// ---- LDS pointers and direct copies into LDS ----------------------------------
// LDS addresses as 32-bit local pointers
typedef __attribute__((address_space(3))) uint8_t lds_u8;
template <class T>
__device__ __forceinline__ T lds_ld(const lds_u8* q) {
    return *(const __attribute__((address_space(3))) T*)q;
}
template <class T>
__device__ __forceinline__ void lds_st(lds_u8* q, T v) {
    *(__attribute__((address_space(3))) T*)q = v;
}

// The four words of a raw buffer descriptor over [base, base + bytes) (stride 0, the
// flags word of make_rsrc above), in scalar registers.
__device__ __forceinline__ u32x4_t rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return u32x4_t{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                   (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                   (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}

// Every lane copies the 16 (dma16) or 4 (dma4) bytes at buffer offset voff to LDS at
// lds_window + 16 * lane (+ 4 * lane); loads past the range write zeros. The
// wave-uniform window is an M0-bound input operand, so the compiler itself sets M0
// before the statement and knows its value afterwards (M0 is never clobbered). The
// s_nop covers the M0-write to LDS-DMA hazard, which the compiler does not see
// inside the statement.
__device__ __forceinline__ void dma16(const u32x4_t& r, const lds_u8* lds_window, uint32_t voff) {
    const uint32_t w = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_window);
    asm volatile(
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, 0 offen lds"
        :
        : "v"(voff), "s"(r), "{m0}"(w)
        : "memory");
}
__device__ __forceinline__ void dma4(const u32x4_t& r, const lds_u8* lds_window, uint32_t voff) {
    const uint32_t w = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_window);
    asm volatile(
        "s_nop 0\n\t"
        "buffer_load_dword %0, %1, 0 offen lds"
        :
        : "v"(voff), "s"(r), "{m0}"(w)
        : "memory");
}

// Waits for every vector-memory load of this wave, the LDS copies included.
__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace physllm
