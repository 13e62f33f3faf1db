// Router (GEMV + top-k + softmax) and token bucketing for gfx950.
//
// Router semantics (kernels/moe_router.hip:24-78 of the reference, with a bias):
//   logits[b,e] = sum_d x[b,d] * W[e,d]  — every bf16*bf16 product is exact in
//   fp32 and is accumulated in fp64, then + bias[e]; top-k by repeated selection of
//   the largest unused logit (strict '>', so ties go to the lowest index; NaN ranks
//   lowest); softmax over the k selected, in fp64, rounded to fp32.
// fp64 accumulation makes the logits independent of the summation order to far
// below any realistic top-k gap, so this kernel's indices equal the CPU oracle's
// serial sums bit for bit.
//
// Layout: one workgroup of 4 waves handles TB tokens. Wave w computes experts
// w, w+4, ... : each lane accumulates 8-element chunks (16-byte loads, so a wave
// reads one contiguous 1 KiB slice of the expert row per step) and a butterfly
// reduction finishes the dot. Logits go to LDS; then one wave per token runs the
// selection with a wave-wide arg-max per round.
#include "common.h"
#include "capi_internal.h"
#include "experts.h"

namespace physllm {

constexpr int kRouterThreads = 256;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;

// a ranks above b in the selection order (value descending, NaN lowest, index ascending).
__device__ __forceinline__ bool rank_beats(double av, int ae, double bv, int be) {
    if (ae < 0) return false;
    if (be < 0) return true;
    const bool an = __builtin_isnan(av), bn = __builtin_isnan(bv);
    if (!an && (bn || av > bv)) return true;
    if (!bn && (an || bv > av)) return false;
    return ae < be;
}

template <int TB>
__global__ __launch_bounds__(kRouterThreads) void k_router(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ bias, int B, int H,
                                                           int E, int K, int32_t* __restrict__ idx,
                                                           float* __restrict__ wts, int vec) {
    extern __shared__ double lg[];  // [TB][E]
    const int t0 = blockIdx.x * TB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ntb = min(TB, B - t0);

    for (int e = wave; e < E; e += kRouterThreads / 64) {
        double acc[TB];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[tb] = 0.0;
        const uint16_t* wr = w + (size_t)e * H;
        if (vec) {
            const int nch = H >> 3;
            for (int c = lane; c < nch; c += 64) {
                const uint4 wv = ((const uint4*)wr)[c];
                const uint32_t wa[4] = {wv.x, wv.y, wv.z, wv.w};
                double wd[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    wd[2 * j] = (double)bf16_lo(wa[j]);
                    wd[2 * j + 1] = (double)bf16_hi(wa[j]);
                }
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
                    if (tb < ntb) {
                        const uint4 xv = ((const uint4*)(x + (size_t)(t0 + tb) * H))[c];
                        const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            acc[tb] = __builtin_fma((double)bf16_lo(xa[j]), wd[2 * j], acc[tb]);
                            acc[tb] = __builtin_fma((double)bf16_hi(xa[j]), wd[2 * j + 1], acc[tb]);
                        }
                    }
                }
            }
        } else {
            for (int d = lane; d < H; d += 64) {
                const double wv = (double)bf16_to_f32(wr[d]);
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
                    if (tb < ntb) acc[tb] = __builtin_fma((double)bf16_to_f32(x[(size_t)(t0 + tb) * H + d]), wv, acc[tb]);
            }
        }
        const double b = bias ? (double)bf16_to_f32(bias[e]) : 0.0;
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const double s = wave_sum_f64(acc[tb]);
            if (lane == 0) lg[tb * E + e] = s + b;
        }
    }
    __syncthreads();

    for (int tb = wave; tb < ntb; tb += kRouterThreads / 64) {
        const int t = t0 + tb;
        const double* L = lg + tb * E;
        uint32_t used = 0;  // bit i: expert lane + 64 i taken
        double my_sel = 0.0;
        int my_idx = 0;
        for (int j = 0; j < K; ++j) {
            double bv = 0.0;
            int be = -1;
            for (int i = 0; lane + 64 * i < E; ++i) {
                const int e = lane + 64 * i;
                if (used & (1u << i)) continue;
                const double v = L[e];
                if (rank_beats(v, e, bv, be)) { bv = v; be = e; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const double ov = __shfl_xor(bv, o, 64);
                const int oe = __shfl_xor(be, o, 64);
                if (rank_beats(ov, oe, bv, be)) { bv = ov; be = oe; }
            }
            if (be >= 0 && (be & 63) == lane) used |= 1u << (be >> 6);
            if (lane == j) { my_sel = bv; my_idx = be; }
        }
        // softmax over the k selected, in selection order (moe_router.hip:61-78)
        double m = __shfl(my_sel, 0, 64);
        for (int j = 1; j < K; ++j) m = fmax(m, __shfl(my_sel, j, 64));
        const double ex = (lane < K) ? exp(my_sel - m) : 0.0;
        double sum = 0.0;
        for (int j = 0; j < K; ++j) sum += __shfl(ex, j, 64);
        if (lane < K) {
            idx[(size_t)t * K + lane] = my_idx;
            wts[(size_t)t * K + lane] = (float)(ex / sum);
        }
    }
}

int router_launch(const void* x, const void* w, const void* bias, int B, int H, int E, int K, void* idx,
                  void* wts, hipStream_t stream) {
    if (B < 0 || H < 1 || E < 1 || K < 1) return set_error(PHYSLLM_MOE_EINVAL, "router: bad sizes");
    if (E > kMaxExperts) return set_error(PHYSLLM_MOE_EINVAL, "router: num_experts > 1024");
    if (K > E || K > kMaxTopK) return set_error(PHYSLLM_MOE_EINVAL, "router: top_k > min(num_experts, 32)");
    if (B == 0) return ok();
    if (!x || !w || !idx || !wts) return set_error(PHYSLLM_MOE_EINVAL, "router: null pointer");
    const int vec = (H % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0);
    if (B >= 64) {
        constexpr int TB = 4;
        hipLaunchKernelGGL(k_router<TB>, dim3((B + TB - 1) / TB), dim3(kRouterThreads),
                           (size_t)TB * E * sizeof(double), stream, (const uint16_t*)x, (const uint16_t*)w,
                           (const uint16_t*)bias, B, H, E, K, (int32_t*)idx, (float*)wts, vec);
    } else {
        hipLaunchKernelGGL(k_router<1>, dim3(B), dim3(kRouterThreads), (size_t)E * sizeof(double), stream,
                           (const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)bias, B, H, E, K,
                           (int32_t*)idx, (float*)wts, vec);
    }
    return check_launch("router");
}

// ---------------------------------------------------------------------------
// Bucketing: counting sort of the B*k (token, slot) pairs by expert, stable in
// pair id p = t*k + j. One workgroup of 1024 threads:
//   1. histogram with LDS integer atomics (order-free, so deterministic);
//   2. exclusive scans -> offsets[E+1] and the compact list of touched experts;
//   3. pairs in chunks of 1024, in order: a lane's rank among equal keys of its
//      wave comes from a ballot-based match, the wave's base from per-wave counts
//      of the chunk; running per-expert totals carry across chunks.
// Outputs perm (sorted position -> pair id), pos (pair id -> sorted position),
// counts, offsets, active[n_active] (touched experts, ascending) and n_active.
// Pairs whose expert id is outside [0, E) are dropped.
// ---------------------------------------------------------------------------
constexpr int kBucketThreads = 1024;

__device__ __forceinline__ int block_excl_scan(int v, int* sbuf, int n) {
    // Hillis-Steele over n <= 1024 entries held one per thread; returns exclusive prefix.
    const int tid = threadIdx.x;
    if (tid < n) sbuf[tid] = v;
    __syncthreads();
    for (int off = 1; off < n; off <<= 1) {
        int add = 0;
        if (tid < n && tid >= off) add = sbuf[tid - off];
        __syncthreads();
        if (tid < n) sbuf[tid] += add;
        __syncthreads();
    }
    const int incl = (tid < n) ? sbuf[tid] : 0;
    __syncthreads();
    return incl - ((tid < n) ? v : 0);
}

__global__ __launch_bounds__(kBucketThreads) void k_bucket(const int32_t* __restrict__ idx, int N, int E,
                                                           int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ perm, int32_t* __restrict__ pos,
                                                           int32_t* __restrict__ active,
                                                           int32_t* __restrict__ n_active) {
    extern __shared__ int smem[];
    int* cnt = smem;                   // [E]
    int* off = cnt + E;                // [E]
    int* run = off + E;                // [E]
    int* scan = run + E;               // [1024]
    int* wcnt = scan + kBucketThreads; // [16][E]
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
            if (active && c > 0) active[na] = tid;
            if (tid == E - 1) {
                offsets[E] = ex + c;
                if (n_active) *n_active = na + (c > 0 ? 1 : 0);
            }
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

size_t bucket_smem_bytes(int E) { return sizeof(int) * ((size_t)3 * E + kBucketThreads + 16 * (size_t)E); }

int bucket_launch(const void* idx, int N, int E, void* counts, void* offsets, void* perm, void* pos, void* active,
                  void* n_active, hipStream_t stream) {
    static bool attr_set = false;
    const size_t smem = bucket_smem_bytes(E);
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)k_bucket, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)bucket_smem_bytes(kMaxExperts));
        attr_set = true;
    }
    hipLaunchKernelGGL(k_bucket, dim3(1), dim3(kBucketThreads), smem, stream, (const int32_t*)idx, N, E,
                       (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm, (int32_t*)pos, (int32_t*)active,
                       (int32_t*)n_active);
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
    return bucket_launch(idx, batch * top_k, num_experts, counts, offsets, perm, pos, nullptr, nullptr,
                         (hipStream_t)stream);
}

extern "C" int physllm_moe_route_topk(const void* x, const void* router_w, const void* router_b, int batch,
                                      int hidden, int num_experts, int top_k, void* idx, void* w, void* stream) {
    return physllm::router_launch(x, router_w, router_b, batch, hidden, num_experts, top_k, idx, w,
                                  (hipStream_t)stream);
}
