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
// Layout: one workgroup of 8 waves handles TB tokens. Wave w computes experts
// w*EPI.., with every lane's 16-byte chunks of all EPI router rows and TB token
// rows loaded up front (a wave reads contiguous 1 KiB slices of each row), then a
// butterfly reduction per dot. Logits go to LDS; then one wave per token runs
// the selection with a wave-wide arg-max per round.
#include "common.h"
#include "capi_internal.h"
#include "experts.h"

namespace physllm {

constexpr int kRouterThreads = 512;  // 8 waves
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

__device__ __forceinline__ void bf16x8_to_f64(uint4 v, double (&d)[8]) {
    d[0] = (double)bf16_lo(v.x);
    d[1] = (double)bf16_hi(v.x);
    d[2] = (double)bf16_lo(v.y);
    d[3] = (double)bf16_hi(v.y);
    d[4] = (double)bf16_lo(v.z);
    d[5] = (double)bf16_hi(v.z);
    d[6] = (double)bf16_lo(v.w);
    d[7] = (double)bf16_hi(v.w);
}

// Logits of TB tokens x EPI experts for one wave: each lane owns 8-element chunks
// c = lane + 64 u; all U chunks of every operand are loaded before any is used, so
// a wave has (EPI + TB) * U 16-byte loads in flight instead of one round trip per
// chunk. bf16 products are exact in fp64 and summed in fp64.
template <int TB, int EPI, int U>
__device__ __forceinline__ void router_dots(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int t0,
                                            int ntb, int e0, int E, int H, int lane, double (&acc)[EPI][TB]) {
#pragma unroll
    for (int ei = 0; ei < EPI; ++ei)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[ei][tb] = 0.0;
    const int nch = H >> 3;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        uint4 wv[EPI][U], xv[TB][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
#pragma unroll
            for (int ei = 0; ei < EPI; ++ei)
                wv[ei][u] = (c < nch && e0 + ei < E) ? ((const uint4*)(w + (size_t)(e0 + ei) * H))[c]
                                                     : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
                xv[tb][u] = (c < nch && tb < ntb) ? ((const uint4*)(x + (size_t)(t0 + tb) * H))[c]
                                                  : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            double xd[TB][8];
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) bf16x8_to_f64(xv[tb][u], xd[tb]);
#pragma unroll
            for (int ei = 0; ei < EPI; ++ei) {
                double wd[8];
                bf16x8_to_f64(wv[ei][u], wd);
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[ei][tb] = __builtin_fma(xd[tb][i], wd[i], acc[ei][tb]);
            }
        }
    }
}

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
                    const double wv = (double)bf16_to_f32(w[(size_t)(e0 + ei) * H + d]);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
                        if (tb < ntb)
                            acc[ei][tb] = __builtin_fma((double)bf16_to_f32(x[(size_t)(t0 + tb) * H + d]), wv, acc[ei][tb]);
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

    for (int tb = wave; tb < ntb; tb += NW) {
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
    if (B > 1024) {
        // prefill: 4 tokens per group share every loaded router row
        constexpr int TB = 4;
        hipLaunchKernelGGL((k_router<TB, 1, 4>), dim3((B + TB - 1) / TB), dim3(kRouterThreads),
                           (size_t)TB * E * sizeof(double), stream, (const uint16_t*)x, (const uint16_t*)w,
                           (const uint16_t*)bias, B, H, E, K, (int32_t*)idx, (float*)wts, vec);
    } else {
        // decode: one token per group, 4 experts' rows in flight per wave
        hipLaunchKernelGGL((k_router<1, 4, 6>), dim3(B), dim3(kRouterThreads), (size_t)E * sizeof(double), stream,
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
// counts, offsets and the work-slot table slots[E]: slot a < #touched holds
// {expert, tokens, first sorted position, 0} for the a-th touched expert
// (ascending id), later slots hold zeros.
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
                                                           int4* __restrict__ slots, int32_t* __restrict__ n_slots,
                                                           int32_t* __restrict__ tprefix, int tile_n) {
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

int bucket_launch(const void* idx, int N, int E, void* counts, void* offsets, void* perm, void* pos, void* slots,
                  void* n_slots, void* tprefix, int tile_n, hipStream_t stream) {
    static bool attr_set = false;
    const size_t smem = bucket_smem_bytes(E);
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)k_bucket, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)bucket_smem_bytes(kMaxExperts));
        attr_set = true;
    }
    hipLaunchKernelGGL(k_bucket, dim3(1), dim3(kBucketThreads), smem, stream, (const int32_t*)idx, N, E,
                       (int32_t*)counts, (int32_t*)offsets, (int32_t*)perm, (int32_t*)pos, (int4*)slots,
                       (int32_t*)n_slots, (int32_t*)tprefix, tile_n);
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
                         (hipStream_t)stream);
}

extern "C" int physllm_moe_route_topk(const void* x, const void* router_w, const void* router_b, int batch,
                                      int hidden, int num_experts, int top_k, void* idx, void* w, void* stream) {
    return physllm::router_launch(x, router_w, router_b, batch, hidden, num_experts, top_k, idx, w,
                                  (hipStream_t)stream);
}
