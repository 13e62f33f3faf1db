// Decode-regime expert kernels for gfx950: grouped MXFP4 GEMV on bf16 MFMA.
//
// Decode streams each touched expert's weights once (HBM-bound). At 8 TB/s a
// 4.25-bit format delivers ~15 T elements/s, while the whole chip issues ~39 T
// VALU lane-ops/s: ~2.6 vector ops per element, too few to decode AND multiply
// on the vector ALUs. So the reduction runs on the matrix cores even for one token: weights are the A
// operand of v_mfma_f32_16x16x32_bf16 (16 rows x one 32-element MX block), the
// tokens routed to the expert are the B operand's 16 columns (zero-padded), and
// the VALU only converts codes with v_cvt_scalef32_pk_bf16_fp4 (one instruction
// per 2 elements, the E8M0 scale applied in the conversion).
//
// Operand mapping (lane l, m = l % 16, g = l / 16):
//   A: lane holds row m, block (b0 + g): one 16-byte load = 32 codes = 4 MFMA
//      fragments of 8 bf16 (fragment i = elements 8i..8i+7 of the block);
//   B: lane holds token column m, the same 8 elements of block (b0 + g), read from
//      the activation rows staged in LDS;
//   C: lane holds rows 4g..4g+3 of its 16-row tile for token column m.
// The K index each lane supplies is the same for A and B, so the sum covers every
// element exactly once. A wave owns 16 consecutive weight rows of one expert and
// walks the whole K range, so a row's 90 blocks arrive as 16-row x 64-byte stripes
// (one 1 KiB load per wave per step), prefetched a chunk ahead.
//
// gate_up rows are interleaved (2i = gate_i, 2i+1 = up_i), so each lane's four C
// rows are two (gate, up) pairs of the same token: bias + clamped SwiGLU happen in
// registers and the lane stores two adjacent bf16 of h.
#include "common.h"
#include "capi_internal.h"
#include "experts.h"

namespace physllm {

constexpr int kGemvChunk = 8;  // k-steps (4 MX blocks each) prefetched per chunk

template <int MODE>
__global__ __launch_bounds__(512) void k_mx_gemv(GemvParams p) {
    extern __shared__ uint4 lds_act[];  // [16][Kdim + 8] bf16, in 16-byte units
    const int slot = blockIdx.y;
    if (slot >= *p.n_active) return;
    const int e = p.active[slot];
    const int ne = p.counts[e];
    const int p0 = p.offsets[e];
    const int nwaves = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * nwaves + wave) * 16;
    const bool wave_active = r0 < p.R;
    const int m = lane & 15, g = lane >> 4;
    const int NB = p.Kdim >> 5;
    const int nit = (NB + 3) >> 2;
    const int ldsu = (p.Kdim >> 3) + 1;  // LDS row stride in uint4 (16 B pad per row)
    const size_t row = (size_t)e * p.R + (wave_active ? r0 + m : 0);
    const uint4* wrow = (const uint4*)(p.blocks + row * (size_t)(p.Kdim >> 1));
    const uint8_t* srow = p.scales + row * (size_t)NB;
    const int u4_row = p.Kdim >> 3;

    for (int tb = 0; tb < ne; tb += 16) {
        const int ntok = min(16, ne - tb);
        __syncthreads();
        for (int i = threadIdx.x; i < ntok * u4_row; i += blockDim.x) {
            const int r = i / u4_row, c = i - r * u4_row;
            const uint16_t* src;
            if (MODE == kModeGateUp) {
                const int pair = p.perm[p0 + tb + r];
                src = p.act + (size_t)(pair / p.top_k) * p.Kdim;
            } else {
                src = p.act + (size_t)(p0 + tb + r) * p.Kdim;
            }
            lds_act[r * ldsu + c] = ((const uint4*)src)[c];
        }
        __syncthreads();
        if (!wave_active) continue;

        const bool tv = m < ntok;
        const uint4* xl = lds_act + m * ldsu;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};

        // Ping-pong chunk buffers: chunk c+1's loads are in flight while chunk c computes.
        uint4 qa[kGemvChunk], qb[kGemvChunk];
        uint32_t sa[kGemvChunk], sb[kGemvChunk];
        auto load_chunk = [&](uint4 (&q)[kGemvChunk], uint32_t (&s)[kGemvChunk], int c0) {
#pragma unroll
            for (int j = 0; j < kGemvChunk; ++j) {
                const int blk = (c0 + j) * 4 + g;
                const bool bv = blk < NB;
                q[j] = bv ? wrow[blk] : make_uint4(0, 0, 0, 0);
                s[j] = bv ? (uint32_t)srow[blk] : 127u;
            }
        };
        auto compute_chunk = [&](const uint4 (&q)[kGemvChunk], const uint32_t (&s)[kGemvChunk], int c0) {
#pragma unroll
            for (int j = 0; j < kGemvChunk; ++j) {
                if (c0 + j >= nit) break;
                const int blk = (c0 + j) * 4 + g;
                const float sf = e8m0_scale_operand(s[j]);
                const bf16x8_t a0 = mx_cvt8(q[j].x, sf);
                const bf16x8_t a1 = mx_cvt8(q[j].y, sf);
                const bf16x8_t a2 = mx_cvt8(q[j].z, sf);
                const bf16x8_t a3 = mx_cvt8(q[j].w, sf);
                uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0, x2 = x0, x3 = x0;
                if (tv && blk < NB) {
                    x0 = xl[blk * 4 + 0];
                    x1 = xl[blk * 4 + 1];
                    x2 = xl[blk * 4 + 2];
                    x3 = xl[blk * 4 + 3];
                }
                acc = mfma16x16x32(a0, as_bf16x8(x0), acc);
                acc = mfma16x16x32(a1, as_bf16x8(x1), acc);
                acc = mfma16x16x32(a2, as_bf16x8(x2), acc);
                acc = mfma16x16x32(a3, as_bf16x8(x3), acc);
            }
        };
        load_chunk(qa, sa, 0);
        for (int c0 = 0; c0 < nit; c0 += 2 * kGemvChunk) {
            load_chunk(qb, sb, c0 + kGemvChunk);
            compute_chunk(qa, sa, c0);
            load_chunk(qa, sa, c0 + 2 * kGemvChunk);
            compute_chunk(qb, sb, c0 + kGemvChunk);
        }

        if (!tv) continue;
        const int pp = p0 + tb + m;  // sorted position of this lane's token
        const int rr = r0 + 4 * g;
        float bsum[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias) {
            const uint2 bb = *(const uint2*)(p.bias + (size_t)e * p.R + rr);
            bsum[0] = bf16_lo(bb.x);
            bsum[1] = bf16_hi(bb.x);
            bsum[2] = bf16_lo(bb.y);
            bsum[3] = bf16_hi(bb.y);
        }
        if (MODE == kModeGateUp) {
            const float h0 = swiglu(acc[0] + bsum[0], acc[1] + bsum[1], p.alpha, p.limit);
            const float h1 = swiglu(acc[2] + bsum[2], acc[3] + bsum[3], p.alpha, p.limit);
            const int I = p.R >> 1;
            uint32_t* hout = (uint32_t*)((uint16_t*)p.out + (size_t)pp * I + (rr >> 1));
            *hout = f32_to_bf16(h0) | (f32_to_bf16(h1) << 16);
        } else {
            float4 y;
            y.x = acc[0] + bsum[0];
            y.y = acc[1] + bsum[1];
            y.z = acc[2] + bsum[2];
            y.w = acc[3] + bsum[3];
            *(float4*)((float*)p.out + (size_t)pp * p.R + rr) = y;
        }
    }
}

// out[t, d] = bf16( sum_j w[t,j] * y[pos[t*k+j], d] ), fp32 fma in k order
// (kernels/moe_combine.hip:16-20, batched). Each lane handles 4 consecutive d.
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ y, const int32_t* __restrict__ pos,
                                                 const float* __restrict__ wts, uint16_t* __restrict__ out, int H,
                                                 int K) {
    const int t = blockIdx.y;
    const int d4 = blockIdx.x * 256 + threadIdx.x;
    if (d4 * 4 >= H) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < K; ++j) {
        const int q = pos[(size_t)t * K + j];
        const float w = wts[(size_t)t * K + j];
        const float4 v = ((const float4*)(y + (size_t)q * H))[d4];
        acc.x = __builtin_fmaf(w, v.x, acc.x);
        acc.y = __builtin_fmaf(w, v.y, acc.y);
        acc.z = __builtin_fmaf(w, v.z, acc.z);
        acc.w = __builtin_fmaf(w, v.w, acc.w);
    }
    uint2 o;
    o.x = f32_to_bf16(acc.x) | (f32_to_bf16(acc.y) << 16);
    o.y = f32_to_bf16(acc.z) | (f32_to_bf16(acc.w) << 16);
    ((uint2*)(out + (size_t)t * H))[d4] = o;
}

static size_t gemv_lds_bytes(int kdim, int max_tokens) {
    return (size_t)max_tokens * ((size_t)(kdim >> 3) + 1) * 16;
}

int gemv_launch(int mode, const GemvParams& p, int max_slots, int max_tokens, hipStream_t stream) {
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)k_mx_gemv<kModeGateUp>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024);
        (void)hipFuncSetAttribute((const void*)k_mx_gemv<kModeDown>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024);
        attr_set = true;
    }
    const int ntok = max_tokens < 16 ? max_tokens : 16;
    const size_t lds = gemv_lds_bytes(p.Kdim, ntok);
    if (lds > 160 * 1024) return set_error(PHYSLLM_MOE_EINVAL, "gemv: reduction dimension too large for LDS");
    // One token: many small groups (4 waves) so every CU gets work; more tokens: 8
    // waves share the staged activations.
    const int waves = ntok <= 4 ? 4 : 8;
    const int rows_per_group = waves * 16;
    dim3 grid((p.R + rows_per_group - 1) / rows_per_group, max_slots);
    if (mode == kModeGateUp)
        hipLaunchKernelGGL(k_mx_gemv<kModeGateUp>, grid, dim3(waves * 64), lds, stream, p);
    else
        hipLaunchKernelGGL(k_mx_gemv<kModeDown>, grid, dim3(waves * 64), lds, stream, p);
    return check_launch(mode == kModeGateUp ? "gate_up gemv" : "down gemv");
}

int combine_launch(const float* y, const int32_t* pos, const float* wts, uint16_t* out, int B, int H, int K,
                   hipStream_t stream) {
    dim3 grid((H / 4 + 255) / 256, B);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, stream, y, pos, wts, out, H, K);
    return check_launch("combine");
}

// ---------------------------------------------------------------------------
// Legacy single-token kernels (dense bf16 weights).
// kernels/moe_expert_forward.hip:8-52 computes one output row per thread with a
// serial 2880-long dot, so neighbouring threads read addresses a full row apart.
// Here a wave owns a row: lanes read consecutive 16-byte chunks (coalesced), sum
// in fp32 and reduce with a butterfly.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dot_bf16_row(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int n,
                                              int lane, bool vec) {
    float s = 0.f;
    if (vec) {
        for (int c = lane; c < (n >> 3); c += 64) {
            const uint4 av = ((const uint4*)a)[c], bv = ((const uint4*)b)[c];
            s = __builtin_fmaf(bf16_lo(av.x), bf16_lo(bv.x), s);
            s = __builtin_fmaf(bf16_hi(av.x), bf16_hi(bv.x), s);
            s = __builtin_fmaf(bf16_lo(av.y), bf16_lo(bv.y), s);
            s = __builtin_fmaf(bf16_hi(av.y), bf16_hi(bv.y), s);
            s = __builtin_fmaf(bf16_lo(av.z), bf16_lo(bv.z), s);
            s = __builtin_fmaf(bf16_hi(av.z), bf16_hi(bv.z), s);
            s = __builtin_fmaf(bf16_lo(av.w), bf16_lo(bv.w), s);
            s = __builtin_fmaf(bf16_hi(av.w), bf16_hi(bv.w), s);
        }
    } else {
        for (int d = lane; d < n; d += 64) s = __builtin_fmaf(bf16_to_f32(a[d]), bf16_to_f32(b[d]), s);
    }
    return wave_sum_f32(s);
}

__global__ __launch_bounds__(256) void k_legacy_silu(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
                                                     const uint16_t* __restrict__ wu, uint16_t* __restrict__ out,
                                                     int H, int I, int vec) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= I) return;
    const float gsum = dot_bf16_row(x, wg + (size_t)row * H, H, lane, vec);
    const float usum = dot_bf16_row(x, wu + (size_t)row * H, H, lane, vec);
    if (lane == 0) {
        const float silu = gsum / (1.0f + expf(-gsum));
        out[row] = (uint16_t)f32_to_bf16(silu * usum);
    }
}

__global__ __launch_bounds__(256) void k_legacy_down(const uint16_t* __restrict__ inter,
                                                     const uint16_t* __restrict__ wd, uint16_t* __restrict__ out,
                                                     int H, int I, int vec) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= H) return;
    const float s = dot_bf16_row(inter, wd + (size_t)row * I, I, lane, vec);
    if (lane == 0) out[row] = (uint16_t)f32_to_bf16(s);
}

__global__ __launch_bounds__(256) void k_legacy_combine(const uint16_t* __restrict__ y, const float* __restrict__ w,
                                                        uint16_t* __restrict__ out, int H, int K) {
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= H) return;
    float s = 0.f;
    for (int k = 0; k < K; ++k) s = __builtin_fmaf(w[k], bf16_to_f32(y[(size_t)k * H + d]), s);
    out[d] = (uint16_t)f32_to_bf16(s);
}

}  // namespace physllm

using namespace physllm;

extern "C" void launch_moe_expert_silu(const void* input, const void* w_gate, const void* w_up, void* output,
                                       int hidden_dim, int intermediate_dim, void* stream) {
    if (hidden_dim < 1 || intermediate_dim < 1) { set_error(PHYSLLM_MOE_EINVAL, "expert_silu: bad sizes"); return; }
    if (!input || !w_gate || !w_up || !output) { set_error(PHYSLLM_MOE_EINVAL, "expert_silu: null pointer"); return; }
    const int vec = (hidden_dim % 8 == 0) && ((uintptr_t)input % 16 == 0) && ((uintptr_t)w_gate % 16 == 0) &&
                    ((uintptr_t)w_up % 16 == 0);
    hipLaunchKernelGGL(k_legacy_silu, dim3((intermediate_dim + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)input, (const uint16_t*)w_gate, (const uint16_t*)w_up, (uint16_t*)output,
                       hidden_dim, intermediate_dim, vec);
    check_launch("expert_silu");
}

extern "C" void launch_moe_expert_down(const void* input, const void* w_down, void* output, int hidden_dim,
                                       int intermediate_dim, void* stream) {
    if (hidden_dim < 1 || intermediate_dim < 1) { set_error(PHYSLLM_MOE_EINVAL, "expert_down: bad sizes"); return; }
    if (!input || !w_down || !output) { set_error(PHYSLLM_MOE_EINVAL, "expert_down: null pointer"); return; }
    const int vec = (intermediate_dim % 8 == 0) && ((uintptr_t)input % 16 == 0) && ((uintptr_t)w_down % 16 == 0);
    hipLaunchKernelGGL(k_legacy_down, dim3((hidden_dim + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)input, (const uint16_t*)w_down, (uint16_t*)output, hidden_dim,
                       intermediate_dim, vec);
    check_launch("expert_down");
}

extern "C" void launch_moe_combine(const void* expert_outputs, const void* expert_weights, void* output,
                                   int hidden_dim, int top_k, void* stream) {
    if (hidden_dim < 1 || top_k < 1) { set_error(PHYSLLM_MOE_EINVAL, "combine: bad sizes"); return; }
    if (!expert_outputs || !expert_weights || !output) { set_error(PHYSLLM_MOE_EINVAL, "combine: null pointer"); return; }
    hipLaunchKernelGGL(k_legacy_combine, dim3((hidden_dim + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)expert_outputs, (const float*)expert_weights, (uint16_t*)output,
                       hidden_dim, top_k);
    check_launch("combine");
}
