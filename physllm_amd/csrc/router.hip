// Router (GEMV + top-k + softmax) and token bucketing for gfx950.
//
// Router semantics (kernels/moe_router.hip:24-78 of the reference, with a bias):
//   logits[b,e] = sum_d fl32(x[b,d] * W[e,d]) accumulated in fp64, + bias[e] —
//   each product formed in fp32 as the reference does (exact for bf16 operands in
//   the fp32 normal range); top-k by repeated selection of the largest unused
//   logit (strict '>', so ties go to the lowest index; NaN ranks lowest); softmax
//   over the k selected, in fp64, rounded to fp32.
// The GPU sums the products in another order than the CPU oracle's serial loop
// (lane partials, then a wave reduction), so the fp64 logits may differ in their
// last bits: by at most 2 (H - 1) 2^-53 sum_d |x[d] W[e,d]| (about 6e-13 of that
// sum at H = 2880). The indices equal the oracle's unless two of a token's logits
// that the selection compares lie within that bound of each other; below it the
// order is fixed by rounding, not by the data (the tests' one-ulp-apart bf16
// logits are about 2^-8 apart, nine orders of magnitude above it).
//
// Layout: one workgroup of 8 waves handles TB tokens. Wave w computes experts
// w*EPI.., with every lane's 16-byte chunks of all EPI router rows and TB token
// rows loaded up front (a wave reads contiguous 1 KiB slices of each row), then a
// DPP/permlane reduction per dot. Logits go to LDS; then every wave ranks a share
// of each token's experts (ballot_select: one ballot per expert instead of k
// dependent arg-max rounds) and one wave per token writes the selection and its
// softmax.
#include "common.h"
#include "rmsnorm.h"
#include "route_math.h"
#include "capi_internal.h"
#include "experts.h"

namespace physllm {

constexpr int kRouterThreads = 512;  // 8 waves
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;

template <int TB, int EPI, int U>
__global__ __launch_bounds__(kRouterThreads) void k_router(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ bias, int B, int H,
                                                           int E, int K, int32_t* __restrict__ idx,
                                                           float* __restrict__ wts, int vec) {
    extern __shared__ double lg[];  // [TB][E]
    constexpr int NW = kRouterThreads / 64;
    const int t0 = blockIdx.x * TB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ntb = min(TB, B - t0);

    for (int e0 = wave * EPI; e0 < E; e0 += NW * EPI) {
        double acc[EPI][TB];
        if (vec) {
            router_dots<TB, EPI, U>(x, w, t0, ntb, e0, E, H, lane, acc);
        } else {
#pragma unroll
            for (int ei = 0; ei < EPI; ++ei)
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) acc[ei][tb] = 0.0;
            for (int d = lane; d < H; d += 64) {
#pragma unroll
                for (int ei = 0; ei < EPI; ++ei) {
                    if (e0 + ei >= E) continue;
                    const float wv = bf16_to_f32(w[(size_t)(e0 + ei) * H + d]);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
                        if (tb < ntb)
                            acc[ei][tb] = acc_prod(acc[ei][tb], bf16_to_f32(x[(size_t)(t0 + tb) * H + d]), wv);
                }
            }
        }
#pragma unroll
        for (int ei = 0; ei < EPI; ++ei) {
            const int e = e0 + ei;
            const double b = (bias && e < E) ? (double)bf16_to_f32(bias[e]) : 0.0;
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                const double sum = wave_sum_f64(acc[ei][tb]);
                if (lane == 0 && e < E) lg[tb * E + e] = sum + b;
            }
        }
    }
    __syncthreads();

    if (E <= kRankMax) {
        // every wave ranks a share of each token's experts, then one wave per token
        // takes the softmax of its selection
        double* selv = lg + TB * E;               // [TB][32]
        int32_t* seli = (int32_t*)(selv + TB * 32);  // [TB][32]
        for (int tb = 0; tb < ntb; ++tb)
            ballot_select(lg + tb * E, E, K, wave, NW, lane, seli + tb * 32, selv + tb * 32);
        __syncthreads();
        for (int tb = wave; tb < ntb; tb += NW) {
            const int t = t0 + tb;
            softmax_selected(seli + tb * 32, selv + tb * 32, K, lane, idx + (size_t)t * K, wts + (size_t)t * K);
        }
    } else {
        for (int tb = wave; tb < ntb; tb += NW) {
            const int t = t0 + tb;
            select_topk(lg + tb * E, E, K, lane, idx + (size_t)t * K, wts + (size_t)t * K);
        }
    }
}

// ---------------------------------------------------------------------------
// One-token route (decode at batch 1): router logits, top-k, softmax and the
// bucketing of the k pairs in one workgroup of 16 waves, one launch instead of
// two. Wave w computes the logits of experts w * EPI.. (every 16-byte chunk of
// its rows loaded up front, as k_router does); all waves then rank them
// (ballot_select, the order of rank_beats) and wave 0 takes the softmax. Since a
// token's k experts are distinct, the stable counting sort of its k pairs by
// expert is the ascending order of the selected ids: pair j goes to sorted
// position #{i : e_i < e_j}. E <= 256.
// ---------------------------------------------------------------------------
constexpr int kRoute1Threads = 1024;

// LDS of k_route1 (bytes): logits [E] f64 | selected values [32] f64 | selected ids
// [32] i32 | (NORM) norm partials [128] f32 + rms | the normalised row [H] bf16
__host__ __device__ inline uint32_t route1_norm_off(int E) { return (uint32_t)E * 8u + 32u * 8u + 32u * 4u; }
__host__ __device__ inline uint32_t route1_row_off(int E) { return (route1_norm_off(E) + 129u * 4u + 15u) & ~15u; }

// NORM: the route of the block's token (crates/llm-core/src/moe.rs:239-259) with the
// RMSNorm in front: h = bf16((x / rms) * norm_w) in the reference's order
// (rmsnorm.h), written to h_out for the expert projections and kept in LDS as the
// router's input, so the norm costs no launch of its own.
template <int EPI, bool NORM>
__global__ __launch_bounds__(kRoute1Threads) void k_route1(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias, int H, int E,
    int K, int32_t* __restrict__ idx, float* __restrict__ wts, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ pos, int4* __restrict__ slots,
    int32_t* __restrict__ n_slots, int4* __restrict__ passes, int32_t* __restrict__ n_passes, int vec,
    const uint16_t* __restrict__ norm_w, float eps, uint16_t* __restrict__ h_out) {
    extern __shared__ double lg[];  // layout: route1_norm_off / route1_row_off
    constexpr int NW = kRoute1Threads / 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint16_t* xin = x;
    if (NORM) {
        float* part = (float*)((char*)lg + route1_norm_off(E));
        uint16_t* hrow = (uint16_t*)((char*)lg + route1_row_off(E));
        const float rms = rms_of_row(x, H, eps, part, part + 128);
        if (vec) {
            for (int c = threadIdx.x; c < (H >> 3); c += kRoute1Threads) {
                const uint4 hv = rms_apply8(((const uint4*)x)[c], ((const uint4*)norm_w)[c], rms);
                ((uint4*)hrow)[c] = hv;
                ((uint4*)h_out)[c] = hv;
            }
        } else {
            for (int i = threadIdx.x; i < H; i += kRoute1Threads) {
                const uint16_t hv = (uint16_t)rms_apply1(x[i], norm_w[i], rms);
                hrow[i] = hv;
                h_out[i] = hv;
            }
        }
        __syncthreads();
        xin = hrow;
    }
    for (int e0 = wave * EPI; e0 < E; e0 += NW * EPI) {
        double acc[EPI][1];
        if (vec) {
            router_dots<1, EPI, 6>(xin, w, 0, 1, e0, E, H, lane, acc);
        } else {
#pragma unroll
            for (int ei = 0; ei < EPI; ++ei) acc[ei][0] = 0.0;
            for (int d = lane; d < H; d += 64) {
                const float xv = bf16_to_f32(xin[d]);
#pragma unroll
                for (int ei = 0; ei < EPI; ++ei)
                    if (e0 + ei < E) acc[ei][0] = acc_prod(acc[ei][0], xv, bf16_to_f32(w[(size_t)(e0 + ei) * H + d]));
            }
        }
#pragma unroll
        for (int ei = 0; ei < EPI; ++ei) {
            const int e = e0 + ei;
            const double b = (bias && e < E) ? (double)bf16_to_f32(bias[e]) : 0.0;
            const double sum = wave_sum_f64(acc[ei][0]);
            if (lane == 0 && e < E) lg[e] = sum + b;
        }
    }
    __syncthreads();
    double* selval = lg + E;                      // [32]
    int32_t* selid = (int32_t*)(selval + 32);     // [32]
    ballot_select(lg, E, K, wave, NW, lane, selid, selval);
    __syncthreads();
    if (wave != 0) return;
    const int ej = lane < K ? selid[lane] : 0x7fffffff;  // pair j = lane (token 0, slot j)
    const double vj = lane < K ? selval[lane] : 0.0;
    // softmax over the k selected in selection order (the first pick is the maximum)
    const double ex = lane < K ? exp(vj - selval[0]) : 0.0;
    double sum = 0.0;
    for (int j = 0; j < K; ++j) sum += __shfl(ex, j, 64);
    // sorted position of pair j: the number of selected experts below e_j
    int pj = 0;
    for (int i = 0; i < K; ++i) pj += (__shfl(ej, i, 64) < ej) ? 1 : 0;
    if (lane < K) {
        idx[lane] = ej;
        wts[lane] = (float)(ex / sum);
        pos[lane] = pj;
        perm[pj] = lane;
        slots[pj] = make_int4(ej, 1, pj, 0);
        passes[pj] = make_int4(ej, 1, pj, 1 << 16);
    }
    if (lane == 0) {
        *n_slots = K;
        n_passes[0] = K;
        n_passes[1] = 0;
        offsets[E] = K;
    }
    // counts[e] = 1 for the selected experts, offsets[e] = #{selected < e}; later slots cleared
    for (int e = lane; e < E; e += 64) {
        int c = 0, below = 0;
        for (int i = 0; i < K; ++i) {
            const int ei = __shfl(ej, i, 64);
            c += (ei == e) ? 1 : 0;
            below += (ei < e) ? 1 : 0;
        }
        counts[e] = c;
        offsets[e] = below;
        if (e >= K) slots[e] = make_int4(0, 0, 0, 0);
    }
}

int route1_launch(const void* x, const void* w, const void* bias, int H, int E, int K, void* idx, void* wts,
                  void* counts, void* offsets, void* perm, void* pos, void* slots, void* n_slots, void* passes,
                  void* n_passes, hipStream_t stream, const void* norm_w, float eps, void* h_out) {
    if (E > kRankMax || K > E || K > kMaxTopK) return set_error(PHYSLLM_MOE_EINVAL, "route1: sizes out of range");
    if (norm_w && (!h_out || H > kRoute1NormMaxH)) return set_error(PHYSLLM_MOE_EINVAL, "route1: bad norm arguments");
    const int vec = (H % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0) &&
                    (!norm_w || ((uintptr_t)norm_w % 16 == 0 && (uintptr_t)h_out % 16 == 0));
    const size_t lds = norm_w ? (size_t)route1_row_off(E) + (size_t)H * 2 : (size_t)E * sizeof(double) + 32 * 8 + 32 * 4;
    if (norm_w)
        hipLaunchKernelGGL((k_route1<2, true>), dim3(1), dim3(kRoute1Threads), lds, stream, (const uint16_t*)x,
                           (const uint16_t*)w, (const uint16_t*)bias, H, E, K, (int32_t*)idx, (float*)wts,
                           (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm, (int32_t*)pos, (int4*)slots,
                           (int32_t*)n_slots, (int4*)passes, (int32_t*)n_passes, vec, (const uint16_t*)norm_w, eps,
                           (uint16_t*)h_out);
    else
        hipLaunchKernelGGL((k_route1<2, false>), dim3(1), dim3(kRoute1Threads), lds, stream, (const uint16_t*)x,
                           (const uint16_t*)w, (const uint16_t*)bias, H, E, K, (int32_t*)idx, (float*)wts,
                           (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm, (int32_t*)pos, (int4*)slots,
                           (int32_t*)n_slots, (int4*)passes, (int32_t*)n_passes, vec, nullptr, 0.f, nullptr);
    return check_launch("route1");
}

// ---------------------------------------------------------------------------
// Two-pass router for batches of kRmxMinBatch tokens or more (E <= 128,
// H % 32 == 0, H <= kRmxMaxH): one workgroup of 8 waves per 16 tokens, the
// tokens' rows staged once in LDS.
//  1. Approximate logits on the matrix cores (bf16 MFMA, fp32 accumulation):
//     a[t][e] = sum x*w, with S = sum |x||w|, W1[e] = sum |w| and X1[t] = sum |x|
//     from three more MFMAs on sign-cleared operands and ones. Each 32-term MFMA
//     adds at most 33 roundings to a chain of H/32 of them, so
//     |a + b - exact| <= eps = g/(1-g) (S + c) + c + 2^-126 (W1 + X1)(1 + 2g) + u|a + b|
//     with u = 2^-23 (covers truncating as well as rounding adders), g = m u / (1 - m u)
//     for m = 33 H/32 + 16 roundings, c bounding products and partial sums the
//     hardware may flush below 2^-126, and the W1/X1 term the products of an
//     input it may flush as subnormal.
//  2. Candidates: expert e can be among the k largest exact logits only if
//     a + b + eps >= T, the k-th largest a + b - eps (k experts have exact logits
//     >= T). A token with any non-finite approximate sum (overflow, inf, NaN) makes
//     all its experts candidates.
//  3. Exact logits of the candidates only, as k_router computes them (fp32
//     products, fp64 sums in the same lane order and wave reduction, + bias), then
//     the selection (ballot_select) and softmax among the candidates: the same
//     indices and weights as ranking every exact logit.
// ---------------------------------------------------------------------------
constexpr int kRmxTok = 16;
constexpr int kRmxThreads = 512;
constexpr int kRmxWaves = kRmxThreads / 64;
constexpr int kRmxMaxE = 128;  // experts per token the LDS layout holds (taken above 64 only for large batches:
                               // a workgroup streams all E rows, and few workgroups stream slowly)
constexpr int kRmxMaxH = 3072;  // the LDS layout of k_router_mx fits 160 KiB up to here
constexpr int kRmxMinBatch = 128;

// LDS layout of k_router_mx (bytes): token rows | partial sums | W1/X1 partials |
// bounds | candidate ids | candidate counts + flags | exact logits | selections
struct RmxLayout {
    uint32_t xstride, red, wx, lohi, cand, cnt, exact, sel, total;
};

__host__ __device__ inline RmxLayout rmx_layout(int H) {
    RmxLayout L;
    L.xstride = (uint32_t)H * 2u + 16u;                    // odd multiple of 16 bytes per row
    L.red = kRmxTok * L.xstride;                           // [8 waves][8][64] f32: a (4), S (4)
    L.wx = L.red + kRmxWaves * 8 * 64 * 4;                 // [8 waves][32] f32: W1 (16), X1 (16)
    L.lohi = L.wx + kRmxWaves * 32 * 4;                    // [16][kRmxMaxE][2] f32: lower, upper bound
    L.cand = L.lohi + kRmxTok * kRmxMaxE * 8;              // [16][kRmxMaxE] i32 candidate expert ids
    L.cnt = L.cand + kRmxTok * kRmxMaxE * 4;               // [16] counts, [16] all-candidate flags
    L.exact = L.cnt + 2 * kRmxTok * 4;                     // [16][kRmxMaxE] f64 exact logits
    L.sel = L.exact + kRmxTok * kRmxMaxE * 8;              // [16][32] f64 values, [16][32] i32 ids
    L.total = L.sel + kRmxTok * 32 * 12;
    return L;
}

// |v| of 8 packed bf16 (sign bits cleared)
__device__ __forceinline__ uint4 bf16x8_abs(uint4 v) {
    return make_uint4(v.x & 0x7fff7fffu, v.y & 0x7fff7fffu, v.z & 0x7fff7fffu, v.w & 0x7fff7fffu);
}

__global__ __launch_bounds__(kRmxThreads) void k_router_mx(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ bias, int B, int H,
                                                           int E, int K, int32_t* __restrict__ idx,
                                                           float* __restrict__ wts) {
    extern __shared__ uint4 lds4[];
    char* lds = (char*)lds4;
    const RmxLayout L = rmx_layout(H);
    const int t0 = blockIdx.x * kRmxTok;
    const int ntok = min(kRmxTok, B - t0);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m = lane & 15, g = lane >> 4;
    const int nc = H >> 5;   // 32-element chunks
    const int nch = H >> 3;  // 8-element chunks (exact pass)

    // ---- stage the tokens' rows (rows past B are zero): every load of a thread is
    // issued before its first store, so the rows arrive in one memory round trip ----
    {
        const uint32_t units = (uint32_t)nch;  // 16-byte units per row
        const uint32_t total = kRmxTok * units;
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)t0 * H, (uint32_t)ntok * (uint32_t)H * 2u);
        constexpr int SU = (kRmxTok * (kRmxMaxH / 8) + kRmxThreads - 1) / kRmxThreads;  // 12 units per thread at most
        u32x4_t v[SU];
#pragma unroll
        for (int k2 = 0; k2 < SU; ++k2) {
            const uint32_t i = tid + k2 * kRmxThreads;  // unit i = row * units + column; past the tile: no load
            const uint32_t r = i / units, c = i - r * units;
            v[k2] = buf_load16(rx, i < total ? (r * (uint32_t)H + c * 8u) * 2u : kRsrcPast, 0);
        }
#pragma unroll
        for (int k2 = 0; k2 < SU; ++k2) {
            const uint32_t i = tid + k2 * kRmxThreads;
            const uint32_t r = i / units, c = i - r * units;
            if (i < total) *(u32x4_t*)(lds + r * L.xstride + c * 16u) = v[k2];
        }
    }
    int* cnt = (int*)(lds + L.cnt);
    if (tid < 2 * kRmxTok) cnt[tid] = 0;
    __syncthreads();

    // ---- 1. approximate sums: wave = (expert tile, K part) ----
    const int nt = (E + 15) >> 4;
    const int nt8 = nt <= 1 ? 1 : nt <= 2 ? 2 : nt <= 4 ? 4 : 8;
    const int nk = kRmxWaves / nt8;
    const int tile = wave % nt8, kp = wave / nt8;
    const int cb = kp * nc / nk, ce = (kp + 1) * nc / nk;
    {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)E * (uint32_t)H * 2u);
        const uint32_t wrow = (uint32_t)(tile * 16 + m) * (uint32_t)H * 2u + (uint32_t)g * 16u;
        const char* xrow = lds + m * L.xstride + g * 16;
        const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, accS = acc, accW = acc, accX = acc;
        constexpr int D = 8;  // weight chunks in flight per wave
        u32x4_t wb[D];
#pragma unroll
        for (int i = 0; i < D; ++i) wb[i] = buf_load16(rw, cb + i < ce ? wrow + (uint32_t)(cb + i) * 64u : kRsrcPast, 0);
        for (int c0 = cb; c0 < ce; c0 += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                const int c = c0 + i;
                if (c < ce) {  // wave-uniform
                    const uint4 xv = *(const uint4*)(xrow + c * 64);
                    const u32x4_t q = wb[i];
                    const uint4 wv = make_uint4(q[0], q[1], q[2], q[3]);
                    const uint4 wa = bf16x8_abs(wv), xa = bf16x8_abs(xv);
                    acc = mfma16x16x32(as_bf16x8(wv), as_bf16x8(xv), acc);
                    accS = mfma16x16x32(as_bf16x8(wa), as_bf16x8(xa), accS);
                    accW = mfma16x16x32(as_bf16x8(wa), as_bf16x8(ones), accW);
                    accX = mfma16x16x32(as_bf16x8(ones), as_bf16x8(xa), accX);
                }
                wb[i] = buf_load16(rw, c + D < ce ? wrow + (uint32_t)(c + D) * 64u : kRsrcPast, 0);
            }
        }
        // partials: lane holds rows (experts) 4g + i of the tile, column (token) m
        float* red = (float*)(lds + L.red) + wave * 8 * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            red[i * 64 + lane] = acc[i];
            red[(4 + i) * 64 + lane] = accS[i];
        }
        float* wx = (float*)(lds + L.wx) + wave * 32;
        if (m == 0)
#pragma unroll
            for (int i = 0; i < 4; ++i) wx[4 * g + i] = accW[i];  // sum |w| of row 4g + i
        if (g == 0) wx[16 + m] = accX[0];                         // sum |x| of token m
    }
    __syncthreads();

    // ---- bounds: the waves of K part 0 sum the parts in order ----
    const float u = 0x1p-23f;
    if (kp == 0) {
        const double mr = 33.0 * nc + 16.0;
        const double gm = mr * (double)u / (1.0 - mr * (double)u);
        const double cab = (33.0 * nc + H + 16.0) * 0x1p-125;
        float a[4] = {0.f, 0.f, 0.f, 0.f}, S[4] = {0.f, 0.f, 0.f, 0.f}, W1[4] = {0.f, 0.f, 0.f, 0.f}, X1 = 0.f;
        for (int p2 = 0; p2 < nk; ++p2) {
            const int w2 = p2 * nt8 + tile;
            const float* red = (const float*)(lds + L.red) + w2 * 8 * 64;
            const float* wx = (const float*)(lds + L.wx) + w2 * 32;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] += red[i * 64 + lane];
                S[i] += red[(4 + i) * 64 + lane];
                W1[i] += wx[4 * g + i];
            }
            X1 += wx[16 + m];
        }
        float2* lohi = (float2*)(lds + L.lohi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tile * 16 + 4 * g + i;
            if (e < E && m < ntok) {
                const float bb = bias ? bf16_to_f32(bias[e]) : 0.f;
                const float ab = a[i] + bb;
                const double eps = gm / (1.0 - gm) * ((double)S[i] + cab) + cab +
                                   0x1p-126 * ((double)W1[i] + (double)X1) * (1.0 + 2.0 * gm) +
                                   (double)u * fabs((double)ab);
                const bool fin = __builtin_isfinite(ab) && __builtin_isfinite(S[i]) && __builtin_isfinite(W1[i]) &&
                                 __builtin_isfinite(X1) && __builtin_isfinite(eps);
                if (!fin) atomicOr(&cnt[kRmxTok + m], 1);
                const double e2 = eps * (1.0 + 0x1p-20);
                lohi[m * kRmxMaxE + e] = make_float2(__double2float_rd((double)ab - e2), __double2float_ru((double)ab + e2));
            }
        }
    }
    __syncthreads();

    // ---- 2. candidates of token t: wave t % 8 ----
    int32_t* cand = (int32_t*)(lds + L.cand);
    for (int t = wave; t < ntok; t += kRmxWaves) {
        const float2* lh = (const float2*)(lds + L.lohi) + t * kRmxMaxE;
        const bool all = cnt[kRmxTok + t] != 0;
        const bool v0 = lane < E, v1 = lane + 64 < E;
        const float2 q0 = v0 ? lh[lane] : make_float2(0.f, 0.f);
        const float2 q1 = v1 ? lh[lane + 64] : make_float2(0.f, 0.f);
        bool c0 = v0, c1 = v1;
        if (!all) {
            // T = k-th largest lower bound: k rounds, each removing one largest
            float l0 = v0 ? q0.x : -INFINITY, l1 = v1 ? q1.x : -INFINITY;
            bool r0 = !v0, r1 = !v1;  // removed
            float T = -INFINITY;
            for (int j = 0; j < K; ++j) {
                float mx = fmaxf(r0 ? -INFINITY : l0, r1 ? -INFINITY : l1);
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
                T = mx;
                // remove one element equal to the maximum (the lowest slot)
                const uint64_t b0 = __ballot(!r0 && l0 == mx), b1 = __ballot(!r1 && l1 == mx);
                if (b0) {
                    if (lane == __builtin_ctzll(b0)) r0 = true;
                } else if (b1) {
                    if (lane == __builtin_ctzll(b1)) r1 = true;
                }
            }
            c0 = v0 && q0.y >= T;
            c1 = v1 && q1.y >= T;
        }
        const uint64_t m0 = __ballot(c0), m1 = __ballot(c1);
        const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        const int n0 = __popcll(m0);
        if (c0) cand[t * kRmxMaxE + __popcll(m0 & lt)] = lane;
        if (c1) cand[t * kRmxMaxE + n0 + __popcll(m1 & lt)] = lane + 64;
        if (lane == 0) cnt[t] = n0 + __popcll(m1);
    }
    __syncthreads();

    // ---- 3. exact logits of the candidates: pairs (t, j) over all waves, two at a time ----
    int poff[kRmxTok + 1];
    poff[0] = 0;
#pragma unroll
    for (int t = 0; t < kRmxTok; ++t) poff[t + 1] = poff[t] + (t < ntok ? cnt[t] : 0);
    const int npairs = poff[kRmxTok];
    double* exact = (double*)(lds + L.exact);
    auto pair_at = [&](int p, int& t, int& j) {
        t = 0;
#pragma unroll
        for (int i = 1; i < kRmxTok; ++i) t += (p >= poff[i]) ? 1 : 0;
        j = p - poff[t];
    };
    const int nu = (nch + 63) >> 6;  // 8-element chunks per lane
    for (int p = wave * 2; p < npairs; p += kRmxWaves * 2) {
        int ta, ja, tb2, jb;
        pair_at(p, ta, ja);
        const bool hb = p + 1 < npairs;
        pair_at(hb ? p + 1 : p, tb2, jb);
        const int ea = cand[ta * kRmxMaxE + ja], eb = cand[tb2 * kRmxMaxE + jb];
        const uint4* wa = (const uint4*)(w + (size_t)ea * H);
        const uint4* wbp = (const uint4*)(w + (size_t)eb * H);
        const char* xa = lds + ta * L.xstride;
        const char* xb = lds + tb2 * L.xstride;
        double sa = 0.0, sb = 0.0;
        for (int u0 = 0; u0 < nu; u0 += 6) {
            uint4 qa[6], qb[6];
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const int c = lane + 64 * (u0 + i);
                qa[i] = c < nch ? wa[c] : make_uint4(0, 0, 0, 0);
                qb[i] = c < nch ? wbp[c] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const int c = lane + 64 * (u0 + i);
                if (u0 + i < nu) {
                    const uint4 va = c < nch ? *(const uint4*)(xa + c * 16) : make_uint4(0, 0, 0, 0);
                    const uint4 vb = c < nch ? *(const uint4*)(xb + c * 16) : make_uint4(0, 0, 0, 0);
                    float xf[8], wf[8];
                    bf16x8_to_f32(va, xf);
                    bf16x8_to_f32(qa[i], wf);
#pragma unroll
                    for (int k2 = 0; k2 < 8; ++k2) sa = acc_prod(sa, xf[k2], wf[k2]);
                    bf16x8_to_f32(vb, xf);
                    bf16x8_to_f32(qb[i], wf);
#pragma unroll
                    for (int k2 = 0; k2 < 8; ++k2) sb = acc_prod(sb, xf[k2], wf[k2]);
                }
            }
        }
        const double ra = wave_sum_f64(sa), rb = wave_sum_f64(sb);
        if (lane == 0) {
            exact[ta * kRmxMaxE + ja] = ra + (bias ? (double)bf16_to_f32(bias[ea]) : 0.0);
            if (hb) exact[tb2 * kRmxMaxE + jb] = rb + (bias ? (double)bf16_to_f32(bias[eb]) : 0.0);
        }
    }
    __syncthreads();

    // ---- selection among the candidates, in candidate (= expert id) order ----
    double* selv = (double*)(lds + L.sel);
    int32_t* seli = (int32_t*)(selv + kRmxTok * 32);
    for (int t = wave; t < ntok; t += kRmxWaves) {
        ballot_select(exact + t * kRmxMaxE, cnt[t], K, 0, 1, lane, seli + t * 32, selv + t * 32);
        __builtin_amdgcn_wave_barrier();
        if (lane < K) seli[t * 32 + lane] = cand[t * kRmxMaxE + seli[t * 32 + lane]];
        __builtin_amdgcn_wave_barrier();
        softmax_selected(seli + t * 32, selv + t * 32, K, lane, idx + (size_t)(t0 + t) * K,
                         wts + (size_t)(t0 + t) * K);
    }
}

// logits [TB][E] (fp64), then the selections [TB][32] (fp64 values, int ids)
static size_t router_smem_bytes(int TB, int E) { return (size_t)TB * E * sizeof(double) + (size_t)TB * 32 * 12; }

// ---------------------------------------------------------------------------
// Router for mid-size batches (B * E >= kRl2MinWork, outside the two-pass path) in
// two launches, so that no workgroup streams every router row (k_router's
// one-token groups each read all E rows: 737 KB per token at E = 128):
//   k_router_logits: a workgroup computes the logits of 8 tokens x 16 experts
//     exactly as k_router does (router_dots: fp32 products summed in fp64 in the
//     same lane order, the same wave reduction, + bias) into a [B][E] fp64 buffer;
//   k_router_select: one workgroup per token ranks its logits (ballot_select,
//     or arg-max rounds for E > 256) and takes the softmax.
// The logits are bit-identical to k_router's (a lane visits its chunks
// c = lane, lane + 64, ... in the same order for any unroll), so are the
// selection and the weights.
// ---------------------------------------------------------------------------
constexpr int kRlTok = 8;                           // tokens per logits workgroup
constexpr int kRlExp = 2 * (kRouterThreads / 64);   // experts per logits workgroup (2 per wave)
constexpr int64_t kRl2MinWork = 8192;               // B * E from which the two launches pay

__global__ __launch_bounds__(kRouterThreads) void k_router_logits(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ bias, int B, int H,
                                                                  int E, double* __restrict__ lg) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * kRlTok;
    const int ntb = min(kRlTok, B - t0);
    const int e0 = blockIdx.y * kRlExp + wave * 2;
    if (e0 >= E) return;
    double acc[2][kRlTok];
    router_dots<kRlTok, 2, 2>(x, w, t0, ntb, e0, E, H, lane, acc);
#pragma unroll
    for (int ei = 0; ei < 2; ++ei) {
        const int e = e0 + ei;
        const double b = (bias && e < E) ? (double)bf16_to_f32(bias[e]) : 0.0;
#pragma unroll
        for (int tb = 0; tb < kRlTok; ++tb) {
            const double sum = wave_sum_f64(acc[ei][tb]);
            if (lane == 0 && e < E && tb < ntb) lg[(size_t)(t0 + tb) * E + e] = sum + b;
        }
    }
}

constexpr int kRsThreads = 256;

__global__ __launch_bounds__(kRsThreads) void k_router_select(const double* __restrict__ lg, int E, int K,
                                                              int32_t* __restrict__ idx, float* __restrict__ wts) {
    extern __shared__ double ls[];  // [E] logits | selected values [32] | selected ids [32]
    constexpr int NW = kRsThreads / 64;
    const int t = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int e = threadIdx.x; e < E; e += kRsThreads) ls[e] = lg[(size_t)t * E + e];
    __syncthreads();
    if (E <= kRankMax) {
        double* selv = ls + E;
        int32_t* seli = (int32_t*)(selv + 32);
        ballot_select(ls, E, K, wave, NW, lane, seli, selv);
        __syncthreads();
        if (wave == 0) softmax_selected(seli, selv, K, lane, idx + (size_t)t * K, wts + (size_t)t * K);
    } else if (wave == 0) {
        select_topk(ls, E, K, lane, idx + (size_t)t * K, wts + (size_t)t * K);
    }
}

bool router_two_launch(int B, int E) { return B >= kRlTok * 2 && (int64_t)B * E >= kRl2MinWork; }

bool rmx_tiled(int B, int E) { return B >= kRmxMinBatch && E > 64 && E <= kRmxMaxE; }

// ---------------------------------------------------------------------------
// Tiled two-pass router (inside the layer, where the workspace holds the bounds):
// the same bounds, candidate rule and exact arithmetic as k_router_mx, in two
// launches so that no workgroup streams every router row or computes every
// candidate of 16 tokens alone.
//   k_rmx_bounds: workgroup (16 tokens, 16 experts); its 8 waves split K and load
//     their weight and activation fragments straight from memory (no staging),
//     wave 0 adds the parts in order and writes each (token, expert)'s [lo, hi] to
//     a [B][E] buffer, or (-inf, +inf) where an approximate sum is not finite
//     (16 waves, every chunk of a wave in flight at once, measured slower: route
//     stage 25 against 20 us at config 4);
//   k_rmx_select: one 4-wave workgroup per token: threshold T (k-th largest lo),
//     candidates hi >= T (every expert when any bound is (-inf, +inf)), their exact
//     logits (fp32 products summed in fp64 in k_router's lane order, + bias), the
//     selection among them (ballot_select) and the softmax.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRmxThreads) void k_rmx_bounds(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias, int B, int H, int E,
                                                            float2* __restrict__ lohi) {
    __shared__ float red[kRmxWaves][8][64];
    __shared__ float wxs[kRmxWaves][32];
    const int t0 = blockIdx.x * kRmxTok;
    const int ntok = min(kRmxTok, B - t0);
    const int tile = blockIdx.y;  // experts 16 * tile ..
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int nc = H >> 5;
    const int cb = wave * nc / kRmxWaves, ce = (wave + 1) * nc / kRmxWaves;
    {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)E * (uint32_t)H * 2u);
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)t0 * H, (uint32_t)ntok * (uint32_t)H * 2u);
        const uint32_t wrow = (uint32_t)(tile * 16 + m) * (uint32_t)H * 2u + (uint32_t)g * 16u;
        const uint32_t xrow = (uint32_t)m * (uint32_t)H * 2u + (uint32_t)g * 16u;
        const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, accS = acc, accW = acc, accX = acc;
        constexpr int D = 6;  // chunks in flight per wave
        u32x4_t wb[D], xb[D];
#pragma unroll
        for (int i = 0; i < D; ++i) {
            wb[i] = buf_load16(rw, cb + i < ce ? wrow + (uint32_t)(cb + i) * 64u : kRsrcPast, 0);
            xb[i] = buf_load16(rx, cb + i < ce ? xrow + (uint32_t)(cb + i) * 64u : kRsrcPast, 0);
        }
        for (int c0 = cb; c0 < ce; c0 += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                const int c = c0 + i;
                if (c < ce) {  // wave-uniform
                    const u32x4_t q = wb[i], r = xb[i];
                    const uint4 wv = make_uint4(q[0], q[1], q[2], q[3]);
                    const uint4 xv = make_uint4(r[0], r[1], r[2], r[3]);
                    const uint4 wa = bf16x8_abs(wv), xa = bf16x8_abs(xv);
                    acc = mfma16x16x32(as_bf16x8(wv), as_bf16x8(xv), acc);
                    accS = mfma16x16x32(as_bf16x8(wa), as_bf16x8(xa), accS);
                    accW = mfma16x16x32(as_bf16x8(wa), as_bf16x8(ones), accW);
                    accX = mfma16x16x32(as_bf16x8(ones), as_bf16x8(xa), accX);
                }
                wb[i] = buf_load16(rw, c + D < ce ? wrow + (uint32_t)(c + D) * 64u : kRsrcPast, 0);
                xb[i] = buf_load16(rx, c + D < ce ? xrow + (uint32_t)(c + D) * 64u : kRsrcPast, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            red[wave][i][lane] = acc[i];
            red[wave][4 + i][lane] = accS[i];
        }
        if (m == 0)
#pragma unroll
            for (int i = 0; i < 4; ++i) wxs[wave][4 * g + i] = accW[i];
        if (g == 0) wxs[wave][16 + m] = accX[0];
    }
    __syncthreads();
    if (wave != 0) return;
    const float u = 0x1p-23f;
    const double mr = 33.0 * nc + 16.0;
    const double gm = mr * (double)u / (1.0 - mr * (double)u);
    const double cab = (33.0 * nc + H + 16.0) * 0x1p-125;
    float a[4] = {0.f, 0.f, 0.f, 0.f}, S[4] = {0.f, 0.f, 0.f, 0.f}, W1[4] = {0.f, 0.f, 0.f, 0.f}, X1 = 0.f;
    for (int p2 = 0; p2 < kRmxWaves; ++p2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] += red[p2][i][lane];
            S[i] += red[p2][4 + i][lane];
            W1[i] += wxs[p2][4 * g + i];
        }
        X1 += wxs[p2][16 + m];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = tile * 16 + 4 * g + i;
        if (e < E && m < ntok) {
            const float bb = bias ? bf16_to_f32(bias[e]) : 0.f;
            const float ab = a[i] + bb;
            const double eps = gm / (1.0 - gm) * ((double)S[i] + cab) + cab +
                               0x1p-126 * ((double)W1[i] + (double)X1) * (1.0 + 2.0 * gm) +
                               (double)u * fabs((double)ab);
            const bool fin = __builtin_isfinite(ab) && __builtin_isfinite(S[i]) && __builtin_isfinite(W1[i]) &&
                             __builtin_isfinite(X1) && __builtin_isfinite(eps);
            const double e2 = eps * (1.0 + 0x1p-20);
            lohi[(size_t)(t0 + m) * E + e] =
                fin ? make_float2(__double2float_rd((double)ab - e2), __double2float_ru((double)ab + e2))
                    : make_float2(-INFINITY, INFINITY);
        }
    }
}

// waves per token in the tiled router's selection: each computes the threshold and the
// candidate list, then the exact logits of its share of the candidate pairs (a token's
// 5-10 candidates in one round of loads instead of 3-5 in a row)
constexpr int kRsSplit = 4;

__global__ __launch_bounds__(64 * kRsSplit) void k_rmx_select(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias, int B, int H, int E,
                                                            int K, const float2* __restrict__ lohi,
                                                            int32_t* __restrict__ idx, float* __restrict__ wts) {
    __shared__ double exact[kRmxMaxE];
    __shared__ int32_t cand[kRsSplit][kRmxMaxE];  // the same list from every wave
    __shared__ double selv[32];
    __shared__ int32_t seli[32];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int t = blockIdx.x;  // one workgroup per token (grid = B)
    const float2* lh = lohi + (size_t)t * E;
    const bool v0 = lane < E, v1 = lane + 64 < E;
    const float2 q0 = v0 ? lh[lane] : make_float2(0.f, 0.f);
    const float2 q1 = v1 ? lh[lane + 64] : make_float2(0.f, 0.f);
    const bool all = __ballot((v0 && q0.x == -INFINITY && q0.y == INFINITY) ||
                              (v1 && q1.x == -INFINITY && q1.y == INFINITY)) != 0ull;
    bool c0 = v0, c1 = v1;
    if (!all) {
        // T = k-th largest lower bound: k rounds, each removing one largest
        float l0 = v0 ? q0.x : -INFINITY, l1 = v1 ? q1.x : -INFINITY;
        bool r0 = !v0, r1 = !v1;
        float T = -INFINITY;
        for (int j = 0; j < K; ++j) {
            float mx = fmaxf(r0 ? -INFINITY : l0, r1 ? -INFINITY : l1);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            T = mx;
            const uint64_t b0 = __ballot(!r0 && l0 == mx), b1 = __ballot(!r1 && l1 == mx);
            if (b0) {
                if (lane == __builtin_ctzll(b0)) r0 = true;
            } else if (b1) {
                if (lane == __builtin_ctzll(b1)) r1 = true;
            }
        }
        c0 = v0 && q0.y >= T;
        c1 = v1 && q1.y >= T;
    }
    const uint64_t m0 = __ballot(c0), m1 = __ballot(c1);
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int n0 = __popcll(m0);
    const int nc = n0 + __popcll(m1);
    if (c0) cand[wave][__popcll(m0 & lt)] = lane;
    if (c1) cand[wave][n0 + __popcll(m1 & lt)] = lane + 64;
    __builtin_amdgcn_wave_barrier();
    // exact logits of the candidates, two at a time (k_router's lane order): wave w takes
    // pairs 2w, 2w + 2 * kRsSplit, ...
    const int nch = H >> 3;
    const uint4* xr = (const uint4*)(x + (size_t)t * H);
    uint4 xv[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int c = lane + 64 * i;
        xv[i] = c < nch ? xr[c] : make_uint4(0, 0, 0, 0);
    }
    for (int j = 2 * wave; j < nc; j += 2 * kRsSplit) {
        const bool hb = j + 1 < nc;
        const int ea = cand[wave][j], eb = cand[wave][hb ? j + 1 : j];
        const uint4* wa = (const uint4*)(w + (size_t)ea * H);
        const uint4* wbp = (const uint4*)(w + (size_t)eb * H);
        uint4 qa[6], qb[6];
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            const int c = lane + 64 * i;
            qa[i] = c < nch ? wa[c] : make_uint4(0, 0, 0, 0);
            qb[i] = c < nch ? wbp[c] : make_uint4(0, 0, 0, 0);
        }
        double sa = 0.0, sb = 0.0;
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            float xf[8], wf[8];
            bf16x8_to_f32(xv[i], xf);
            bf16x8_to_f32(qa[i], wf);
#pragma unroll
            for (int k2 = 0; k2 < 8; ++k2) sa = acc_prod(sa, xf[k2], wf[k2]);
            bf16x8_to_f32(qb[i], wf);
#pragma unroll
            for (int k2 = 0; k2 < 8; ++k2) sb = acc_prod(sb, xf[k2], wf[k2]);
        }
        const double ra = wave_sum_f64(sa), rb = wave_sum_f64(sb);
        if (lane == 0) {
            exact[j] = ra + (bias ? (double)bf16_to_f32(bias[ea]) : 0.0);
            if (hb) exact[j + 1] = rb + (bias ? (double)bf16_to_f32(bias[eb]) : 0.0);
        }
    }
    __syncthreads();  // every candidate's exact logit is in LDS
    if (wave != 0) return;
    ballot_select(exact, nc, K, 0, 1, lane, seli, selv);
    __builtin_amdgcn_wave_barrier();
    if (lane < K) seli[lane] = cand[0][seli[lane]];
    __builtin_amdgcn_wave_barrier();
    softmax_selected(seli, selv, K, lane, idx + (size_t)t * K, wts + (size_t)t * K);
}

int router_launch(const void* x, const void* w, const void* bias, int B, int H, int E, int K, void* idx,
                  void* wts, hipStream_t stream, void* lg_ws) {
    if (B < 0 || H < 1 || E < 1 || K < 1) return set_error(PHYSLLM_MOE_EINVAL, "router: bad sizes");
    if (E > kMaxExperts) return set_error(PHYSLLM_MOE_EINVAL, "router: num_experts > 1024");
    if (K > E || K > kMaxTopK) return set_error(PHYSLLM_MOE_EINVAL, "router: top_k > min(num_experts, 32)");
    if (B == 0) return ok();
    if (!x || !w || !idx || !wts) return set_error(PHYSLLM_MOE_EINVAL, "router: null pointer");
    const int vec = (H % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0);
    if (lg_ws && rmx_tiled(B, E) && H % 32 == 0 && H <= kRmxMaxH && vec) {
        // inside the layer, E > 64: the tiled two-pass router (bounds into the workspace);
        // at config 4 the route stage takes 20 us against 30 for the two-launch exact
        // router, while with E <= 64 (config 3) k_router_mx is as fast in one launch
        hipLaunchKernelGGL(k_rmx_bounds, dim3((B + kRmxTok - 1) / kRmxTok, (E + 15) / 16), dim3(kRmxThreads), 0,
                           stream, (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, B, H, E,
                           (float2*)lg_ws);
        if (int rc = check_launch("router bounds")) return rc;
        hipLaunchKernelGGL(k_rmx_select, dim3(B), dim3(64 * kRsSplit), 0, stream,
                           (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, B, H, E, K,
                           (const float2*)lg_ws, (int32_t*)idx, (float*)wts);
    } else if (B >= kRmxMinBatch && E <= kRmxMaxE && H % 32 == 0 && H <= kRmxMaxH && vec &&
        (E <= 64 || (int64_t)B * E >= 64 * 4096)) {
        // two passes: matrix-core bounds, exact fp64 logits of the candidates only
        const RmxLayout Lr = rmx_layout(H);
        static std::once_flag attr_once[kMaxDevices];
        once_per_device(attr_once, [] {
            (void)hipFuncSetAttribute((const void*)k_router_mx, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)rmx_layout(kRmxMaxH).total);
        });
        hipLaunchKernelGGL(k_router_mx, dim3((B + kRmxTok - 1) / kRmxTok), dim3(kRmxThreads), (size_t)Lr.total, stream,
                           (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, B, H, E, K, (int32_t*)idx,
                           (float*)wts);
    } else if (lg_ws && vec && router_two_launch(B, E)) {
        hipLaunchKernelGGL(k_router_logits, dim3((B + kRlTok - 1) / kRlTok, (E + kRlExp - 1) / kRlExp),
                           dim3(kRouterThreads), 0, stream, (const uint16_t*)x, (const uint16_t*)w,
                           (const uint16_t*)bias, B, H, E, (double*)lg_ws);
        if (int rc = check_launch("router logits")) return rc;
        hipLaunchKernelGGL(k_router_select, dim3(B), dim3(kRsThreads), (size_t)E * 8 + 32 * 12, stream,
                           (const double*)lg_ws, E, K, (int32_t*)idx, (float*)wts);
    } else if (B > 1024) {
        // prefill: 4 tokens per group share every loaded router row
        constexpr int TB = 4;
        hipLaunchKernelGGL((k_router<TB, 1, 4>), dim3((B + TB - 1) / TB), dim3(kRouterThreads),
                           router_smem_bytes(TB, E), stream, (const uint16_t*)x, (const uint16_t*)w,
                           (const uint16_t*)bias, B, H, E, K, (int32_t*)idx, (float*)wts, vec);
    } else {
        // decode: one token per group, 4 experts' rows in flight per wave
        hipLaunchKernelGGL((k_router<1, 4, 6>), dim3(B), dim3(kRouterThreads),
                           router_smem_bytes(1, E), stream,
                           (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, B, H, E, K,
                           (int32_t*)idx, (float*)wts, vec);
    }
    return check_launch("router");
}

// ---------------------------------------------------------------------------
// Bucketing: counting sort of the B*k (token, slot) pairs by expert, stable in
// pair id p = t*k + j, by one workgroup of 1024 threads in one of two ways (both
// give the same tables; each is the faster one where the launcher uses it).
//
// k_bucket_chunked (N <= 1024):
//   1. histogram with LDS integer atomics (order-free, so deterministic);
//   2. exclusive scans -> offsets[E+1] and the compact list of touched experts;
//   3. pairs in chunks of 1024, in order: a lane's rank among equal keys of its
//      wave comes from a ballot-based match, the wave's base from per-wave counts
//      of the chunk; running per-expert totals carry across chunks.
//
// k_bucket_waves (larger N, where k_bucket_chunked spends four barriers per
// chunk): wave w owns the contiguous pair range [w N / 16, (w + 1) N / 16),
// walked in groups of 64:
//   1. per-wave counts: in each group a lane finds the lanes with its key by
//      ballots over the key bits, and the lowest of them adds their number to the
//      wave's row of counts (no atomics, no barrier);
//   2. counts summed over the waves, exclusive scans -> offsets[E+1], the
//      compact list of touched experts and each wave's start within every
//      expert (the counts of the waves before it);
//   3. the same walk again: pair p goes to offsets[e] + the wave's start in e +
//      the pairs of e the wave has placed so far + its rank among its group's
//      lanes with key e.
// Outputs perm (sorted position -> pair id), pos (pair id -> sorted position),
// counts, offsets and the work-slot table slots[E]: slot a < #touched holds
// {expert, tokens, first sorted position, 0} for the a-th touched expert
// (ascending id), later slots hold zeros.
// Pairs whose expert id is outside [0, E) are dropped.
// ---------------------------------------------------------------------------
constexpr int kBucketThreads = 1024;
constexpr int kBucketChunkedMaxN = 1024;  // k_bucket_chunked up to this N, k_bucket_waves (or the blocks) above
constexpr int kBucketBlk = 16;  // groups of 64 pairs whose keys a wave loads at once
static_assert(kBucketThreads / 64 == 16, "the bucketing scans assume 16 waves");

// Exclusive prefix over the first n <= 1024 threads' values (later threads
// contribute 0): shuffle scans inside each wave, then the wave totals; two
// barriers. sbuf holds 16 ints.
__device__ __forceinline__ int block_excl_scan(int v, int* sbuf, int n) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int mine = (tid < n) ? v : 0;
    int x = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) sbuf[wave] = x;
    __syncthreads();
    int base = 0;
    for (int w2 = 0; w2 < wave; ++w2) base += sbuf[w2];
    __syncthreads();  // sbuf may be reused by the next scan
    return base + x - mine;
}

// The pass table (decode GEMV work list): each touched expert's sorted positions in
// chunks of kPassRows, {expert, tokens, first position, chunk index | chunk count
// << 16}. Entries of experts with two or more chunks come first, then those of the
// single-chunk experts, each group in expert order; n_passes = {entries, entries of
// multi-chunk experts}. Called by every thread of the workgroup: thread tid < E owns
// expert tid, with c pairs from sorted position ex (chunk counts stay below 2^16: the
// GEMV path has fewer than 64 E pairs).
__device__ __forceinline__ void write_pass_table(int c, int ex, int E, int* sbuf, int4* __restrict__ passes,
                                                 int32_t* __restrict__ n_passes) {
    const int tid = threadIdx.x;
    const int np = (c + kPassRows - 1) / kPassRows;
    const int mex = block_excl_scan(np > 1 ? np : 0, sbuf, E);
    const int sex = block_excl_scan(np == 1 ? 1 : 0, sbuf, E);
    if (tid == E - 1) {
        sbuf[0] = mex + (np > 1 ? np : 0);
        sbuf[1] = sex + (np == 1 ? 1 : 0);
    }
    __syncthreads();
    const int nmulti = sbuf[0], nsingle = sbuf[1];
    if (tid < E) {
        const int base = np > 1 ? mex : nmulti + sex;
        for (int t = 0; t < np; ++t)
            passes[base + t] = make_int4(tid, min(kPassRows, c - t * kPassRows), ex + t * kPassRows, t | (np << 16));
    }
    if (tid == 0 && n_passes) {
        n_passes[0] = nmulti + nsingle;
        n_passes[1] = nmulti;
    }
    __syncthreads();  // sbuf may be reused
}

// The body of k_bucket_chunked, called by the whole workgroup: idx (global or
// LDS) holds the N pairs' experts; smem is the scratch of bucket_smem_bytes(E).
__device__ __forceinline__ void bucket_chunked_block(const int32_t* idx, int N, int E, int* smem,
                                                     int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                     int32_t* __restrict__ perm, int32_t* __restrict__ pos,
                                                     int4* __restrict__ slots, int32_t* __restrict__ n_slots,
                                                     int32_t* __restrict__ tprefix, int tile_n,
                                                     int4* __restrict__ passes, int32_t* __restrict__ n_passes) {
    int* cnt = smem;                   // [E]
    int* off = cnt + E;                // [E]
    int* run = off + E;                // [E]
    int* scan = run + E;               // [16] wave totals of the block scans
    int* wcnt = scan + 16;             // [16][E]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = kBucketThreads / 64;

    for (int i = tid; i < E; i += kBucketThreads) { cnt[i] = 0; run[i] = 0; }
    for (int i = tid; i < nwaves * E; i += kBucketThreads) wcnt[i] = 0;
    __syncthreads();
    for (int p = tid; p < N; p += kBucketThreads) {
        const int e = idx[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();

    // offsets and the touched-expert list (E <= 1024: one expert per thread)
    {
        const int c = (tid < E) ? cnt[tid] : 0;
        const int ex = block_excl_scan(c, scan, E);
        const int na = block_excl_scan(c > 0 ? 1 : 0, scan, E);
        if (tid < E) {
            off[tid] = ex;
            counts[tid] = c;
            offsets[tid] = ex;
            if (tid == E - 1) offsets[E] = ex + c;
        }
        if (slots) {
            // touched experts take slots 0..#touched-1; the rest are cleared
            const int ntouched = __syncthreads_count(tid < E && c > 0);
            if (tid == 0 && n_slots) *n_slots = ntouched;
            if (tid < E && c > 0) slots[na] = make_int4(tid, c, ex, 0);
            if (tid >= ntouched && tid < E) slots[tid] = make_int4(0, 0, 0, 0);
            if (tprefix) {
                // exclusive prefix of token tiles over the slots (GEMM tile scheduling)
                const int nt = (c + tile_n - 1) / tile_n;
                const int tex = block_excl_scan(nt, scan, E);
                if (tid < E && c > 0) tprefix[na] = tex;
                if (tid == E - 1) tprefix[ntouched] = tex + nt;
            }
            if (passes) write_pass_table(c, ex, E, scan, passes, n_passes);
        }
    }
    __syncthreads();

    int nbits = 1;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int c0 = 0; c0 < N; c0 += kBucketThreads) {
        const int p = c0 + tid;
        int key = (p < N) ? idx[p] : -1;
        const bool valid = key >= 0 && key < E;
        uint64_t peers = __ballot(valid);
        if (!valid) peers = 0;
        for (int b = 0; b < nbits; ++b) {
            const bool bit = (key >> b) & 1;
            const uint64_t bb = __ballot(bit);
            peers &= bit ? bb : ~bb;
        }
        const int rank_w = __popcll(peers & lt);
        const bool leader = valid && (peers & lt) == 0;
        if (leader) wcnt[wave * E + key] = __popcll(peers);
        __syncthreads();
        if (valid) {
            int before = 0;
            for (int w2 = 0; w2 < wave; ++w2) before += wcnt[w2 * E + key];
            const int q = off[key] + run[key] + before + rank_w;
            perm[q] = p;
            if (pos) pos[p] = q;
        }
        __syncthreads();
        if (leader) atomicAdd(&run[key], wcnt[wave * E + key]);
        __syncthreads();
        if (leader) wcnt[wave * E + key] = 0;
        __syncthreads();
    }
}

__global__ __launch_bounds__(kBucketThreads) void k_bucket_chunked(const int32_t* __restrict__ idx, int N, int E,
                                                           int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ perm, int32_t* __restrict__ pos,
                                                           int4* __restrict__ slots, int32_t* __restrict__ n_slots,
                                                           int32_t* __restrict__ tprefix, int tile_n,
                                                           int4* __restrict__ passes, int32_t* __restrict__ n_passes) {
    extern __shared__ int smem[];
    bucket_chunked_block(idx, N, E, smem, counts, offsets, perm, pos, slots, n_slots, tprefix, tile_n, passes,
                         n_passes);
}

__global__ __launch_bounds__(kBucketThreads) void k_bucket_waves(const int32_t* __restrict__ idx, int N, int E,
                                                           int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ perm, int32_t* __restrict__ pos,
                                                           int4* __restrict__ slots, int32_t* __restrict__ n_slots,
                                                           int32_t* __restrict__ tprefix, int tile_n,
                                                           int4* __restrict__ passes, int32_t* __restrict__ n_passes) {
    extern __shared__ int smem[];
    int* cnt = smem;                   // [E] totals
    int* off = cnt + E;                // [E] offsets
    int* scan = off + E;               // [16] wave totals of the block scans
    int* wcnt = scan + 16;             // [16][E] per-wave counts, then the waves' running starts
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = kBucketThreads / 64;

    for (int i = tid; i < nwaves * E; i += kBucketThreads) wcnt[i] = 0;
    __syncthreads();

    int nbits = 1;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int pb = (int)((int64_t)wave * N / nwaves), pe = (int)((int64_t)(wave + 1) * N / nwaves);
    int* mycnt = wcnt + wave * E;
    // lanes of one group with the same valid key: `peers`; the lowest one leads
    auto match = [&](int key) {
        const bool valid = key >= 0 && key < E;
        uint64_t peers = __ballot(valid);
        if (!valid) peers = 0;
        for (int bb = 0; bb < nbits; ++bb) {
            const bool bit = (key >> bb) & 1;
            const uint64_t m2 = __ballot(bit);
            peers &= bit ? m2 : ~m2;
        }
        return peers;
    };
    // the keys of kBucketBlk groups at a time, all loads issued before the first use
    int kk[kBucketBlk];
    auto load_keys = [&](int base) {
#pragma unroll
        for (int i = 0; i < kBucketBlk; ++i) {
            const int p = base + 64 * i + lane;
            kk[i] = (p < pe) ? idx[p] : -1;
        }
    };
    // ---- 1. per-wave counts ----
    for (int base = pb; base < pe; base += 64 * kBucketBlk) {
        load_keys(base);
#pragma unroll
        for (int i = 0; i < kBucketBlk; ++i) {
            if (base + 64 * i >= pe) break;  // wave-uniform
            const uint64_t peers = match(kk[i]);
            if (peers && (peers & lt) == 0) mycnt[kk[i]] += __popcll(peers);
        }
    }
    __syncthreads();
    // counts -> starts of the waves within each expert, and the totals
    if (E <= 64) {
        // wave w, lane e: the rows before w read at once
        int st = 0, tot = 0;
        if (lane < E) {
#pragma unroll
            for (int w2 = 0; w2 < 16; ++w2) {
                const int c = wcnt[w2 * E + lane];
                st += (w2 < wave) ? c : 0;
                tot += c;
            }
        }
        __syncthreads();
        if (lane < E) {
            wcnt[wave * E + lane] = st;
            if (wave == 0) cnt[lane] = tot;
        }
    } else {
        for (int e = tid; e < E; e += kBucketThreads) {
            int run = 0;
            for (int w0 = 0; w0 < nwaves; w0 += 8) {  // eight counts read per LDS wait
                int v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = wcnt[min(w0 + i, nwaves - 1) * E + e];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (w0 + i < nwaves) {
                        wcnt[(w0 + i) * E + e] = run;
                        run += v[i];
                    }
                }
            }
            cnt[e] = run;
        }
    }
    __syncthreads();

    // offsets and the touched-expert list (E <= 1024: one expert per thread)
    {
        const int c = (tid < E) ? cnt[tid] : 0;  // E <= 1024
        const int ex = block_excl_scan(c, scan, E);
        const int na = block_excl_scan(c > 0 ? 1 : 0, scan, E);
        if (tid < E) {
            off[tid] = ex;
            counts[tid] = c;
            offsets[tid] = ex;
            if (tid == E - 1) offsets[E] = ex + c;
        }
        if (slots) {
            // touched experts take slots 0..#touched-1; the rest are cleared
            const int ntouched = __syncthreads_count(tid < E && c > 0);
            if (tid == 0 && n_slots) *n_slots = ntouched;
            if (tid < E && c > 0) slots[na] = make_int4(tid, c, ex, 0);
            if (tid >= ntouched && tid < E) slots[tid] = make_int4(0, 0, 0, 0);
            if (tprefix) {
                // exclusive prefix of token tiles over the slots (GEMM tile scheduling)
                const int nt = (c + tile_n - 1) / tile_n;
                const int tex = block_excl_scan(nt, scan, E);
                if (tid < E && c > 0) tprefix[na] = tex;
                if (tid == E - 1) tprefix[ntouched] = tex + nt;
            }
            if (passes) write_pass_table(c, ex, E, scan, passes, n_passes);
        }
    }
    __syncthreads();

    // ---- 3. scatter, in the order of step 1 (one block of keys stays loaded) ----
    for (int base = pb; base < pe; base += 64 * kBucketBlk) {
        if (base != pb || pe - pb > 64 * kBucketBlk) load_keys(base);
#pragma unroll
        for (int i = 0; i < kBucketBlk; ++i) {
            if (base + 64 * i >= pe) break;  // wave-uniform
            const int key = kk[i], p = base + 64 * i + lane;
            const uint64_t peers = match(key);
            if (peers) {
                const int q = off[key] + mycnt[key] + __popcll(peers & lt);
                perm[q] = p;
                if (pos) pos[p] = q;
            }
            __builtin_amdgcn_wave_barrier();  // every lane has read mycnt before the leaders advance it
            if (peers && (peers & lt) == 0) mycnt[key] += __popcll(peers);
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// ---------------------------------------------------------------------------
// Multi-workgroup bucketing (the layer, N > 1024 pairs, with a workspace for the
// block histograms). k_bucket_waves runs in one workgroup at about 1 ns per pair
// (20 us at 16k pairs, 250 us at 262k), so the pairs are cut into nblk contiguous
// blocks of C pairs (C = bucket_block_pairs(N): at least 1024, at most 256 blocks):
//   k_bucket_hist    one workgroup per block: the block's count of each expert
//                    (per-wave rows from ballot matches, no atomics) -> hist[b][e];
//   k_bucket_scan    one workgroup: expert totals and offsets, the slot / tile /
//                    pass tables, and hist[b][e] rewritten as block b's first sorted
//                    position in expert e;
//   k_bucket_scatter one workgroup per block: the block's walk again; pair p goes to
//                    its block's start in e + the pairs of e of the earlier waves of
//                    the block + those its wave placed before + its rank in its group.
// The order is k_bucket_waves': by expert, then by pair index.
// ---------------------------------------------------------------------------
constexpr int kBkThreads = 256;  // 4 waves
constexpr int kBkMaxBlocks = 256;

int bucket_block_pairs(int N) {
    const int per = (N + kBkMaxBlocks - 1) / kBkMaxBlocks;
    return std::max(1024, (per + 255) / 256 * 256);
}
size_t bucket_hist_bytes(int N, int E) {
    if (N <= kBucketChunkedMaxN) return 0;
    const int C = bucket_block_pairs(N);
    return (size_t)((N + C - 1) / C) * (size_t)E * 4;
}

// lanes of this wave with the same valid key as this lane (empty for invalid keys)
__device__ __forceinline__ uint64_t bucket_match(int key, int E, int nbits) {
    const bool valid = key >= 0 && key < E;
    uint64_t peers = __ballot(valid);
    if (!valid) peers = 0;
    for (int bb = 0; bb < nbits; ++bb) {
        const bool bit = (key >> bb) & 1;
        const uint64_t m2 = __ballot(bit);
        peers &= bit ? m2 : ~m2;
    }
    return peers;
}

// The counts of this wave's share of block b into wcnt[wave][e] (zeroed by the caller).
__device__ __forceinline__ void bucket_block_counts(const int32_t* __restrict__ idx, int N, int E, int C, int b,
                                                    int* wcnt) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int nbits = 1;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int wp = C / 4;  // pairs per wave (a multiple of 64)
    const int pb = b * C + wave * wp, pe = min(N, pb + wp);
    int* mycnt = wcnt + wave * E;
    for (int base = pb; base < pe; base += 256) {
        int kk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = base + 64 * i + lane;
            kk[i] = (p < pe) ? idx[p] : -1;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t peers = bucket_match(kk[i], E, nbits);
            if (peers && (peers & lt) == 0) mycnt[kk[i]] += __popcll(peers);
        }
    }
}

__global__ __launch_bounds__(kBkThreads) void k_bucket_hist(const int32_t* __restrict__ idx, int N, int E, int C,
                                                            int32_t* __restrict__ hist) {
    extern __shared__ int smem[];
    int* wcnt = smem;  // [4][E]
    const int b = blockIdx.x;
    for (int i = threadIdx.x; i < 4 * E; i += kBkThreads) wcnt[i] = 0;
    __syncthreads();
    bucket_block_counts(idx, N, E, C, b, wcnt);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kBkThreads)
        hist[(size_t)b * E + e] = wcnt[e] + wcnt[E + e] + wcnt[2 * E + e] + wcnt[3 * E + e];
}

// One workgroup of kBucketThreads (E <= 1024). Thread t serves expert t % E over the
// blocks of chunk t / E (T = kBucketThreads / E chunks per expert).
__global__ __launch_bounds__(kBucketThreads) void k_bucket_scan(int32_t* __restrict__ hist, int nblk, int E,
                                                                 int32_t* __restrict__ counts,
                                                                 int32_t* __restrict__ offsets,
                                                                 int4* __restrict__ slots,
                                                                 int32_t* __restrict__ n_slots,
                                                                 int32_t* __restrict__ tprefix, int tile_n,
                                                                 int4* __restrict__ passes,
                                                                 int32_t* __restrict__ n_passes) {
    extern __shared__ int smem[];
    int* part = smem;                      // [T][E] chunk sums, then their exclusive prefixes
    int* tot = part + kBucketThreads;      // [E]
    int* offs = tot + E;                   // [E]
    int* scan = offs + E;                  // [16]
    const int tid = threadIdx.x;
    const int T = kBucketThreads / E;      // >= 1
    const int e = tid % E, j = tid / E;
    const int per = (nblk + T - 1) / T;
    const int b0 = min(nblk, j * per), b1 = min(nblk, b0 + per);
    int sum = 0;
    if (j < T)
        for (int b = b0; b < b1; ++b) sum += hist[(size_t)b * E + e];
    if (j < T) part[j * E + e] = sum;
    __syncthreads();
    if (tid < E) {
        // eight part sums read before their prefixes are written back (one LDS wait
        // per eight, not one per part)
        int run = 0;
        for (int j0 = 0; j0 < T; j0 += 8) {
            int v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = part[min(j0 + i, T - 1) * E + tid];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (j0 + i < T) {
                    part[(j0 + i) * E + tid] = run;
                    run += v[i];
                }
            }
        }
        tot[tid] = run;
    }
    __syncthreads();

    // offsets and the tables of the touched experts (as k_bucket_waves)
    const int c = (tid < E) ? tot[tid] : 0;
    const int ex = block_excl_scan(c, scan, E);
    const int na = block_excl_scan(c > 0 ? 1 : 0, scan, E);
    if (tid < E) {
        offs[tid] = ex;
        counts[tid] = c;
        offsets[tid] = ex;
        if (tid == E - 1) offsets[E] = ex + c;
    }
    if (slots) {
        const int ntouched = __syncthreads_count(tid < E && c > 0);
        if (tid == 0 && n_slots) *n_slots = ntouched;
        if (tid < E && c > 0) slots[na] = make_int4(tid, c, ex, 0);
        if (tid >= ntouched && tid < E) slots[tid] = make_int4(0, 0, 0, 0);
        if (tprefix) {
            const int nt = (c + tile_n - 1) / tile_n;
            const int tex = block_excl_scan(nt, scan, E);
            if (tid < E && c > 0) tprefix[na] = tex;
            if (tid == E - 1) tprefix[ntouched] = tex + nt;
        }
        if (passes) write_pass_table(c, ex, E, scan, passes, n_passes);
    }
    __syncthreads();

    // hist[b][e] -> the first sorted position of block b's pairs of expert e
    if (j < T) {
        int run = offs[e] + part[j * E + e];
        for (int b = b0; b < b1; ++b) {
            const int v = hist[(size_t)b * E + e];
            hist[(size_t)b * E + e] = run;
            run += v;
        }
    }
}

__global__ __launch_bounds__(kBkThreads) void k_bucket_scatter(const int32_t* __restrict__ idx, int N, int E,
                                                               int C, const int32_t* __restrict__ hist,
                                                               int32_t* __restrict__ perm,
                                                               int32_t* __restrict__ pos) {
    extern __shared__ int smem[];
    int* wcnt = smem;  // [4][E] counts, then the waves' running positions
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * E; i += kBkThreads) wcnt[i] = 0;
    __syncthreads();
    bucket_block_counts(idx, N, E, C, b, wcnt);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kBkThreads) {
        int run = hist[(size_t)b * E + e];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int c = wcnt[w * E + e];
            wcnt[w * E + e] = run;
            run += c;
        }
    }
    __syncthreads();
    int nbits = 1;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int wp = C / 4;
    const int pb = b * C + wave * wp, pe = min(N, pb + wp);
    int* mypos = wcnt + wave * E;
    for (int base = pb; base < pe; base += 64) {
        const int p = base + lane;
        const int key = (p < pe) ? idx[p] : -1;
        const uint64_t peers = bucket_match(key, E, nbits);
        if (peers) {
            const int q = mypos[key] + __popcll(peers & lt);
            perm[q] = p;
            if (pos) pos[p] = q;
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read mypos before the leaders advance it
        if (peers && (peers & lt) == 0) mypos[key] += __popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
}

// LDS of either bucketing kernel (k_bucket_chunked's is the larger)
size_t bucket_smem_bytes(int E) { return sizeof(int) * ((size_t)3 * E + 16 + 16 * (size_t)E); }

// ---------------------------------------------------------------------------
// Small bucketing (N <= 1024 pairs, E <= 256, no GEMM tile prefix): the outputs of
// k_bucket_chunked in one pass with two barriers. Pair p = thread p; its rank
// among the lanes of its wave with the same expert comes from ballots over the
// key bits; wave 0's lane l then sums the per-wave counts of experts
// l*EPL .. l*EPL + EPL - 1 (EPL = ceil(E / 64) <= 4 consecutive experts, keeping each
// wave's start within each expert), and three wave scans over the lanes' totals give
// the sorted offsets, the slot index and the pass-table index; every pair is then
// placed at offset + its wave's start + its rank: by expert, then by pair index.
// ---------------------------------------------------------------------------
constexpr int kBucketSmallMaxE = 256;
constexpr int kBucketSmallEpl = kBucketSmallMaxE / 64;  // experts per lane of wave 0, at most

// Exclusive prefix of v over a wave's lanes; *total = the sum over all 64.
__device__ __forceinline__ int wave_excl_scan(int v, int lane, int* total) {
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    *total = __shfl(x, 63, 64);
    return x - v;
}

__global__ __launch_bounds__(kBucketThreads) void k_bucket_small(const int32_t* __restrict__ idx, int N, int E,
                                                                 int32_t* __restrict__ counts,
                                                                 int32_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ perm, int32_t* __restrict__ pos,
                                                                 int4* __restrict__ slots, int32_t* __restrict__ n_slots,
                                                                 int4* __restrict__ passes,
                                                                 int32_t* __restrict__ n_passes) {
    __shared__ int wcnt[16 * kBucketSmallMaxE];  // pairs per wave and expert, then the waves' starts
    __shared__ int eoff[kBucketSmallMaxE];       // first sorted position of each expert
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int kp = tid < N ? idx[tid] : -1;
    if (kp >= E) kp = -1;  // pairs outside [0, E) are dropped
    for (int i = tid; i < 16 * E; i += kBucketThreads) wcnt[i] = 0;
    int nbits = 1;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint64_t peers = __ballot(kp >= 0);
    if (kp < 0) peers = 0;
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (kp >> b) & 1;
        const uint64_t bb = __ballot(bit);
        peers &= bit ? bb : ~bb;
    }
    const int rank_w = __popcll(peers & lt);
    __syncthreads();
    if (kp >= 0 && (peers & lt) == 0) wcnt[wave * E + kp] = __popcll(peers);
    __syncthreads();
    if (wave == 0) {
        const int epl = (E + 63) >> 6;  // experts per lane
        constexpr int kW = kBucketThreads / 64;
        // every wave's count of this lane's experts first (one LDS wait, not one per
        // wave), then the waves' starts in their place
        int v[kBucketSmallEpl][kW];
#pragma unroll
        for (int k = 0; k < kBucketSmallEpl; ++k) {
            const int e = lane * epl + k;
            const int ec = (k < epl && e < E) ? e : 0;  // unconditional reads (the sums below skip the rest)
#pragma unroll
            for (int w2 = 0; w2 < kW; ++w2) v[k][w2] = wcnt[w2 * E + ec];
        }
        int c[kBucketSmallEpl];
        int csum = 0, tsum = 0, msum = 0, ssum = 0;
#pragma unroll
        for (int k = 0; k < kBucketSmallEpl; ++k) {
            const int e = lane * epl + k;
            c[k] = 0;
            if (k < epl && e < E) {
#pragma unroll
                for (int w2 = 0; w2 < kW; ++w2) {
                    wcnt[w2 * E + e] = c[k];
                    c[k] += v[k][w2];
                }
            }
            csum += c[k];
            tsum += c[k] > 0 ? 1 : 0;
            const int np = (c[k] + kPassRows - 1) / kPassRows;
            msum += np > 1 ? np : 0;
            ssum += np == 1 ? 1 : 0;
        }
        // pass table order (write_pass_table): multi-chunk experts' entries first
        int ntot, ntouched, nmulti, nsingle;
        int ex = wave_excl_scan(csum, lane, &ntot);
        int na = wave_excl_scan(tsum, lane, &ntouched);
        int mex = wave_excl_scan(msum, lane, &nmulti);
        int sex = wave_excl_scan(ssum, lane, &nsingle);
#pragma unroll
        for (int k = 0; k < kBucketSmallEpl; ++k) {
            const int e = lane * epl + k;
            if (k < epl && e < E) {
                const int ce = c[k];
                const int np = (ce + kPassRows - 1) / kPassRows;
                eoff[e] = ex;
                counts[e] = ce;
                offsets[e] = ex;
                if (e == E - 1) offsets[E] = ex + ce;
                if (slots) {
                    if (ce > 0) slots[na] = make_int4(e, ce, ex, 0);
                    if (e >= ntouched) slots[e] = make_int4(0, 0, 0, 0);
                }
                if (passes) {
                    const int base = np > 1 ? mex : nmulti + sex;
                    for (int t = 0; t < np; ++t)
                        passes[base + t] =
                            make_int4(e, min(kPassRows, ce - t * kPassRows), ex + t * kPassRows, t | (np << 16));
                }
                ex += ce;
                na += ce > 0 ? 1 : 0;
                mex += np > 1 ? np : 0;
                sex += np == 1 ? 1 : 0;
            }
        }
        if (lane == 0) {
            if (n_slots) *n_slots = ntouched;
            if (n_passes) {
                n_passes[0] = nmulti + nsingle;
                n_passes[1] = nmulti;
            }
        }
    }
    __syncthreads();
    if (kp >= 0) {
        const int q = eoff[kp] + wcnt[wave * E + kp] + rank_w;
        perm[q] = tid;
        if (pos) pos[tid] = q;
    }
}

// ---------------------------------------------------------------------------
// Decode route for small B * E (the layer at decode batch, E <= 64): k_router
// computes a token's E logits on one CU, where the fp64 sums of 2880-long dots
// take several microseconds; here
//   k_dec_logits: each wave computes one (token, expert) logit exactly as k_router
//     does (router_dots + the wave reduction + bias: the same bits) into a [B][E]
//     fp64 buffer, B * E waves over the whole chip;
//   k_router_select: one workgroup per token ranks its logits (ballot_select) and
//     takes the softmax (softmax_selected), as in the two-launch router;
//   k_bucket_small: the bucketing.
// ---------------------------------------------------------------------------
constexpr int kDecMaxE = 64;  // (E = 128 measured slower than the two-pass route: 36.7 against 26.8 us)

__global__ __launch_bounds__(256) void k_dec_logits(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                    const uint16_t* __restrict__ bias, int B, int H, int E,
                                                    double* __restrict__ lg) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.y * 4 + wave;
    if (t >= B) return;
    const int e = blockIdx.x;
    double acc[1][1];
    router_dots<1, 1, 6>(x, w, t, 1, e, E, H, lane, acc);
    const double b = bias ? (double)bf16_to_f32(bias[e]) : 0.0;
    const double sum = wave_sum_f64(acc[0][0]);
    if (lane == 0) lg[(size_t)t * E + e] = sum + b;
}

bool dec_route_ok(int B, int E, int K) { return B >= 2 && E <= kDecMaxE && (int64_t)B * K <= kBucketChunkedMaxN; }

int dec_route_launch(const void* x, const void* w, const void* bias, int B, int H, int E, int K, void* lg,
                     void* idx, void* wts, void* counts, void* offsets, void* perm, void* pos, void* slots,
                     void* n_slots, void* passes, void* n_passes, hipStream_t stream) {
    if (!dec_route_ok(B, E, K) || K > E || K > kMaxTopK || H % 8 || ((uintptr_t)x | (uintptr_t)w) % 16)
        return set_error(PHYSLLM_MOE_EINVAL, "decode route: sizes or alignment out of range");
    hipLaunchKernelGGL(k_dec_logits, dim3(E, (B + 3) / 4), dim3(256), 0, stream, (const uint16_t*)x,
                       (const uint16_t*)w, (const uint16_t*)bias, B, H, E, (double*)lg);
    if (int rc = check_launch("decode logits")) return rc;
    hipLaunchKernelGGL(k_router_select, dim3(B), dim3(kRsThreads), (size_t)E * 8 + 32 * 12, stream,
                       (const double*)lg, E, K, (int32_t*)idx, (float*)wts);
    if (int rc = check_launch("decode select")) return rc;
    hipLaunchKernelGGL(k_bucket_small, dim3(1), dim3(kBucketThreads), 0, stream, (const int32_t*)idx, B * K, E,
                       (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm, (int32_t*)pos, (int4*)slots,
                       (int32_t*)n_slots, (int4*)passes, (int32_t*)n_passes);
    return check_launch("decode bucket");
}

int bucket_launch(const void* idx, int N, int E, void* counts, void* offsets, void* perm, void* pos, void* slots,
                  void* n_slots, void* tprefix, int tile_n, void* passes, void* n_passes, hipStream_t stream,
                  void* hist) {
    static std::once_flag attr_once[kMaxDevices];
    const size_t smem = bucket_smem_bytes(E);
    once_per_device(attr_once, [] {
        for (const void* k : {(const void*)k_bucket_chunked, (const void*)k_bucket_waves})
            (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bucket_smem_bytes(kMaxExperts));
    });
    if (N <= kBucketChunkedMaxN && E <= kBucketSmallMaxE && !tprefix) {
        hipLaunchKernelGGL(k_bucket_small, dim3(1), dim3(kBucketThreads), 0, stream, (const int32_t*)idx, N, E,
                           (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm, (int32_t*)pos, (int4*)slots,
                           (int32_t*)n_slots, (int4*)passes, (int32_t*)n_passes);
        return check_launch("bucket");
    }
    if (hist && N > kBucketChunkedMaxN && E <= kBucketThreads) {
        const int C = bucket_block_pairs(N);
        const int nblk = (N + C - 1) / C;
        const size_t sm_b = (size_t)4 * E * 4;
        hipLaunchKernelGGL(k_bucket_hist, dim3(nblk), dim3(kBkThreads), sm_b, stream, (const int32_t*)idx, N, E, C,
                           (int32_t*)hist);
        if (int rc = check_launch("bucket hist")) return rc;
        hipLaunchKernelGGL(k_bucket_scan, dim3(1), dim3(kBucketThreads), (size_t)(kBucketThreads + 2 * E + 16) * 4,
                           stream, (int32_t*)hist, nblk, E, (int32_t*)counts, (int32_t*)offsets, (int4*)slots,
                           (int32_t*)n_slots, (int32_t*)tprefix, tile_n, (int4*)passes, (int32_t*)n_passes);
        if (int rc = check_launch("bucket scan")) return rc;
        hipLaunchKernelGGL(k_bucket_scatter, dim3(nblk), dim3(kBkThreads), sm_b, stream, (const int32_t*)idx, N, E,
                           C, (const int32_t*)hist, (int32_t*)perm, (int32_t*)pos);
        return check_launch("bucket scatter");
    }
    hipLaunchKernelGGL(N <= kBucketChunkedMaxN ? k_bucket_chunked : k_bucket_waves, dim3(1), dim3(kBucketThreads), smem,
                       stream, (const int32_t*)idx, N, E, (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm,
                       (int32_t*)pos, (int4*)slots, (int32_t*)n_slots, (int32_t*)tprefix, tile_n, (int4*)passes,
                       (int32_t*)n_passes);
    return check_launch("bucket");
}

}  // namespace physllm

extern "C" void launch_moe_router(const void* hidden, const void* router_weight, void* expert_indices,
                                  void* expert_weights, int batch_size, int hidden_dim, int num_experts, int top_k,
                                  void* stream) {
    physllm::router_launch(hidden, router_weight, nullptr, batch_size, hidden_dim, num_experts, top_k,
                           expert_indices, expert_weights, (hipStream_t)stream);
}

extern "C" int physllm_moe_bucket(const void* idx, int batch, int top_k, int num_experts, void* counts,
                                  void* offsets, void* perm, void* pos, void* stream) {
    using namespace physllm;
    if (batch < 0 || top_k < 1 || num_experts < 1 || num_experts > kMaxExperts)
        return set_error(PHYSLLM_MOE_EINVAL, "bucket: bad sizes");
    if ((int64_t)batch * top_k > 0x7fffffffLL) return set_error(PHYSLLM_MOE_EINVAL, "bucket: batch*top_k too large");
    if (!idx || !counts || !offsets || !perm || !pos) return set_error(PHYSLLM_MOE_EINVAL, "bucket: null pointer");
    return bucket_launch(idx, batch * top_k, num_experts, counts, offsets, perm, pos, nullptr, nullptr, nullptr, 1,
                         nullptr, nullptr, (hipStream_t)stream);
}

extern "C" int physllm_moe_route_topk(const void* x, const void* router_w, const void* router_b, int batch,
                                      int hidden, int num_experts, int top_k, void* idx, void* w, void* stream) {
    return physllm::router_launch(x, router_w, router_b, batch, hidden, num_experts, top_k, idx, w,
                                  (hipStream_t)stream);
}
