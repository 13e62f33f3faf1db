// Batch-1 MoE layer (one decode token) in three short launches.
//
// The per-stage path at one token runs a one-workgroup route launch (router
// logits, top-k, softmax, bucketing), the gate_up GEMV and the down projection +
// combine. Its route launch computes all E logits on one CU, where the fp64 sums
// take most of its ~7 us, and each expert launch starts its weight reads only
// after a dependent load of the bucketing tables. Here:
//   1. k_b1_logits: one workgroup per expert computes that expert's logit (wave
//      0, router_dots: the route launch's arithmetic, so the same bits) and, for
//      the transformer block, the RMSNorm of the token in front of it;
//   2. k_b1_gate_up: every workgroup reads the E logits, selects the top k itself
//      (ballot_select: the same selection in every workgroup, and the route
//      launch's), and computes one 64-row gate_up tile of pair j's expert
//      (+ bias, SwiGLU) into h[j]; workgroup 0 also writes the selection and its
//      softmax weights;
//   3. k_b1_down: one workgroup per 16 output rows, wave s = pair s: the down
//      projection of the k experts for those rows, then the weighted combine
//      (+ residual) of the k results through LDS.
// The same three launches serve 2 tokens (B * k <= 16 pairs): the logits of
// each (token, expert) (one wave per token), gate_up workgroups that select every
// token's top k and each compute one 64-row tile of one distinct selected expert
// for all of its tokens (the MFMA columns), and down workgroups with one wave per
// pair (pair p = token p / k, slot p % k; h and y rows by pair) whose combine sums
// each token's k slots.
// No workgroup waits for another: the launch boundaries order the phases.
// The tiles, k-steps, accumulators and epilogues are those of the per-stage
// kernels (k_mx_gemv, k_mx_down1, k_combine's order; MFMA columns are independent,
// so a token's column does not depend on the others), so the layer output is the
// same bits as the per-stage path's wherever that path does not split the down
// projection's K (it splits at small shapes to fill the chip).
#include "common.h"
#include "capi_internal.h"
#include "experts.h"
#include "rmsnorm.h"
#include "route_math.h"

namespace physllm {

constexpr int kB1Threads = 256;    // 4 waves
constexpr int kB1Nit = 23;         // k-steps per tile (16 bytes of codes per lane each): K range <= 92 MX blocks
constexpr int kB1MaxNB = 92;
constexpr int kB1MaxK = 4;         // k_b1_down's waves are the k pairs
constexpr int kB1MaxE = kRankMax;  // ballot_select's limit (logits kept in LDS)
constexpr int kB1Slice = 128 * 16; // a wave's scale slice: 16 rows x NB <= 1472 bytes, then unread padding
constexpr int kB1MaxPairs = 16;    // batch * k of the generalised path
constexpr int kB1DownWaves = 8;    // its down workgroups: 8 / k whole tokens each
constexpr int kB1MaxB = 2;         // tokens (one wave each in k_b1_logits and the selection)
// k_b1_gate_up's LDS header: logits [B][E] (8 KiB), per-token selection values [B][32]
// and ids [B][32], softmax scratch, the pairs' experts, the distinct experts
constexpr int kB1HdrLg = 0, kB1HdrSelv = 8192, kB1HdrSeli = 9216, kB1HdrSidx = 9728, kB1HdrWl = 9856,
              kB1HdrPe = 9984, kB1HdrDist = 10048, kB1HdrNd = 10112;
constexpr int kB1HdrZero = 10176;  // 64 zero bytes: the activations of lanes past K
constexpr int kB1Hdr = 10240;

struct B1Params {
    const uint8_t* blocks;  // gate_up [E, 2I, H/2] or down [E, H, I/2]
    const uint8_t* scales;  // gate_up [E, 2I, H/32] or down [E, H, I/32]
    const uint16_t* bias;   // [E, 2I] or [E, H], nullable
    const uint16_t* act;    // gate_up: [B, H] the tokens (normalised for the block); down: h [B*k, I]
    const double* logits;   // [B, E] from k_b1_logits (gate_up)
    uint16_t* h;            // [B*k, I] SwiGLU output, row p = token p / k, selection slot p % k (gate_up)
    int32_t* idx;           // [B, k] selected experts, selection order (written by gate_up, read by down)
    float* wts;             // [B, k] their routing weights (same)
    uint16_t* out;          // [B, H] (down)
    const uint16_t* res;    // [B, H] residual added to the output, nullable, may equal out (down)
    int H, I, E, K, B;
    int gu_sets;            // 64-row gate_up tiles per expert: ceil(2I / 64)
    float alpha, limit;
};

// Logits of expert blockIdx.x for the B tokens (wave t: token t; router_dots<1, 1, 6>
// + bias, the route launch's order). NORM (4 waves): every workgroup normalises the
// tokens into LDS first (rms_of_row, the norm kernel's order, one row after the
// other) and workgroup 0 writes them to h_out for the expert launches; otherwise B
// waves.
template <bool NORM, bool MULTI>
__global__ __launch_bounds__(kB1Threads) void k_b1_logits(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ bias, int H, int E, int B,
                                                          double* __restrict__ logits,
                                                          const uint16_t* __restrict__ norm_w, float eps,
                                                          uint16_t* __restrict__ h_out) {
    extern __shared__ uint4 lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = blockIdx.x;
    const uint16_t* xin = x;
    if (NORM) {
        float* part = (float*)lds;                        // [128] + rms
        uint16_t* hrow = (uint16_t*)((char*)lds + 1024);  // [B][H]
        for (int t = 0; t < (MULTI ? B : 1); ++t) {
            const uint16_t* xr = x + (size_t)t * H;
            const float rms = rms_of_row(xr, H, eps, part, part + 128);
            for (int c = threadIdx.x; c < (H >> 3); c += kB1Threads) {
                const uint4 hv = rms_apply8(((const uint4*)xr)[c], ((const uint4*)norm_w)[c], rms);
                ((uint4*)(hrow + (size_t)t * H))[c] = hv;
                if (e == 0) ((uint4*)(h_out + (size_t)t * H))[c] = hv;
            }
        }
        __syncthreads();
        xin = hrow;
    }
    // token t = wave
    if (MULTI ? wave >= B : wave != 0) return;
    const int t = MULTI ? wave : 0;
    double acc[1][1];
    router_dots<1, 1, 6>(xin, w, t, 1, e, E, H, lane, acc);
    const double b = bias ? (double)bf16_to_f32(bias[e]) : 0.0;
    const double sum = wave_sum_f64(acc[0][0]);
    if (lane == 0) logits[(size_t)t * E + e] = sum + b;
}

// Loads of one 16-row tile (rows r0.., all K blocks) of expert e: the scales
// (two 16-byte loads per lane: 16 rows x NB bytes are contiguous), this lane's
// four biases, then the 23 stripes. live = false loads nothing (empty ranges).
struct B1Tile {
    u32x4_t sv0, sv1;
    u32x2_t b2;
    u32x4_t wq[kB1Nit];
};

__device__ __forceinline__ void b1_tile_load(B1Tile& t, const B1Params& p, int e, int R, int Kdim, int r0,
                                             int lane, bool live) {
    const int NB = Kdim >> 5;
    const int m = lane & 15, g = lane >> 4;
    const uint32_t row_bytes = (uint32_t)(Kdim >> 1);
    const uint32_t exp_w = (uint32_t)R * row_bytes;
    const uint32_t exp_s = (uint32_t)R * (uint32_t)NB;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales + (size_t)e * exp_s, live ? exp_s : 0u);
    const uint32_t soff = (uint32_t)r0 * NB + lane * 16u;
    t.sv0 = buf_load16(rs, soff, 0);
    t.sv1 = buf_load16(rs, soff, 1024);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.bias + (size_t)e * R, (live && p.bias) ? (uint32_t)R * 2u : 0u);
    t.b2 = __builtin_amdgcn_raw_buffer_load_b64(rb, (uint32_t)(r0 + 4 * g) * 2u, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.blocks + (size_t)e * exp_w, live ? exp_w : 0u);
    const uint32_t woff = (uint32_t)(r0 + m) * row_bytes + (uint32_t)g * 16u;
#pragma unroll
    for (int j = 0; j < kB1Nit; ++j) t.wq[j] = buf_load16(rw, 4 * j < NB ? woff : kRsrcPast, 64 * j);
    __builtin_amdgcn_sched_barrier(0);
}

// Workgroup t: gate_up rows (t % gu_sets) * 64 + 16 w .. of distinct expert
// u = t / gu_sets (the selected experts in order of first selection: token 0's
// slots, then token 1's new ones, ...), for every token that selected it: lane
// column m < n_u holds the m-th such pair.
template <int MAXB>
__global__ __launch_bounds__(kB1Threads) void k_b1_gate_up(B1Params p) {
    extern __shared__ uint4 lds[];
    char* L = (char*)lds;
    double* lg = (double*)(L + kB1HdrLg);      // [B][E]
    double* selv = (double*)(L + kB1HdrSelv);  // [B][32]
    int32_t* seli = (int32_t*)(L + kB1HdrSeli);  // [B][32]
    int32_t* sidx = (int32_t*)(L + kB1HdrSidx);  // [32]
    float* wl = (float*)(L + kB1HdrWl);          // [32]
    int32_t* pe = (int32_t*)(L + kB1HdrPe);      // [B*k] expert of pair p
    int32_t* dist = (int32_t*)(L + kB1HdrDist);  // [<= 16] distinct experts
    int32_t* nd = (int32_t*)(L + kB1HdrNd);      // [1] their count
    // wave-uniform values are read into scalar registers, so buffer resources built
    // from them need no per-lane (waterfall) loop
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    uint8_t* scl = (uint8_t*)(L + kB1Hdr) + wave * kB1Slice;  // this wave's tile scales [16][NB]
    uint4* xs = (uint4*)(L + kB1Hdr + 4 * kB1Slice);         // the tokens' rows [B][su]
    const int H = p.H, I = p.I, R = 2 * I, NB = H >> 5, K = p.K, B = p.B, N = B * K;
    if (threadIdx.x < 4) ((uint4*)(L + kB1HdrZero))[threadIdx.x] = make_uint4(0, 0, 0, 0);  // (barriers below)
    const int cu = H >> 3, su = MAXB == 1 ? cu : cu + 1;  // 16-byte units per row, LDS row stride

    // the tokens' rows are loaded before the routing, so their latency overlaps the
    // logits' (units past B rows read zeros)
    constexpr int kXv = 2 * MAXB;  // 16-byte units per thread: B * H / 8 <= MAXB * 368 <= 2 * MAXB * 256
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.act, (uint32_t)B * (uint32_t)H * 2u);
    u32x4_t xv[kXv];
#pragma unroll
    for (int u = 0; u < kXv; ++u) xv[u] = buf_load16(rx, (uint32_t)(threadIdx.x + kB1Threads * u) * 16u, 0);
    for (int i = threadIdx.x; i < B * p.E; i += kB1Threads) lg[i] = p.logits[i];
    __syncthreads();
    if (MAXB == 1) {
        ballot_select(lg, p.E, K, wave, kB1Threads / 64, lane, seli, selv);
    } else if (wave < B) {
        ballot_select(lg + wave * p.E, p.E, K, 0, 1, lane, seli + wave * 32, selv + wave * 32);
    }
    __syncthreads();
    if (MAXB > 1 && wave == 0) {
        // pair lane p: its expert; the distinct experts in order of first selection
        const int e_p = lane < N ? seli[(lane / K) * 32 + lane % K] : -1;
        bool first = lane < N;
        for (int q = 0; q < N; ++q) {
            const int eq = __shfl(e_p, q, 64);
            if (q < lane && eq == e_p) first = false;
        }
        const uint64_t fb = __ballot(first);
        const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        if (lane < N) pe[lane] = e_p;
        if (first) dist[__popcll(fb & lt)] = e_p;
        if (lane == 0) *nd = __popcll(fb);
    }
    const int u = blockIdx.x / p.gu_sets;
    int e, pm = u, nu = 1;  // one token: distinct expert u is selection slot u, its one pair
    if (MAXB == 1) {
        e = __builtin_amdgcn_readfirstlane(seli[u]);
    } else {
        __syncthreads();
        if (u >= *nd) return;  // fewer distinct experts than the grid's upper bound
        e = __builtin_amdgcn_readfirstlane(dist[u]);
        // this lane's column: the m-th pair that selected e (columns past them repeat the last)
        nu = 0;
        for (int q = 0; q < N; ++q) {
            if (pe[q] == e) {
                if (nu <= m) pm = q;
                ++nu;
            }
        }
    }
    const int r0 = (blockIdx.x - u * p.gu_sets) * 64 + wave * 16;
    B1Tile tl;
    b1_tile_load(tl, p, e, R, H, r0, lane, true);
    if (blockIdx.x == 0 && wave < B) {
        softmax_selected(seli + wave * 32, selv + wave * 32, K, lane, sidx + wave * 8, wl + wave * 8);
        if (lane < K) {
            p.idx[wave * K + lane] = seli[wave * 32 + lane];
            p.wts[wave * K + lane] = wl[wave * 8 + lane];
        }
    }
    ((u32x4_t*)scl)[lane] = tl.sv0;
    ((u32x4_t*)scl)[lane + 64] = tl.sv1;
#pragma unroll
    for (int v = 0; v < kXv; ++v) {
        const int i = threadIdx.x + kB1Threads * v;
        if (MAXB == 1) {
            if (i < cu) ((u32x4_t*)xs)[i] = xv[v];
        } else {
            const int t = i / cu;
            if (t < B) ((u32x4_t*)xs)[t * su + (i - t * cu)] = xv[v];
        }
    }
    __syncthreads();
    const f32x4_t acc = mx_tile_steps<kB1Nit>(tl.wq, scl + m * NB + g, xs + (MAXB == 1 ? 0 : (pm / K) * su) + 4 * g,
                                 (const uint4*)(L + kB1HdrZero), NB, g);
    if (m < nu && r0 < R) {
        const int rr = r0 + 4 * g;
        const float h0 = swiglu(acc[0] + bf16_lo(tl.b2[0]), acc[1] + bf16_hi(tl.b2[0]), p.alpha, p.limit);
        const float h1 = swiglu(acc[2] + bf16_lo(tl.b2[1]), acc[3] + bf16_hi(tl.b2[1]), p.alpha, p.limit);
        *(uint32_t*)(p.h + (size_t)pm * I + (rr >> 1)) = f32_to_bf16(h0) | (f32_to_bf16(h1) << 16);
    }
}

// Workgroup (b, c): output rows 16 b .. 16 b + 15 of tokens c T .. c T + T - 1
// (T = NW / k whole tokens); wave s < T k: pair c T k + s's expert over those rows
// (k_mx_down1's tile), then per token the combine over its k pairs in LDS.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_b1_down(B1Params p) {
    extern __shared__ uint4 lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int H = p.H, I = p.I, NB = I >> 5, cu = I >> 3, su = cu + 1, N = p.B * p.K;
    // this workgroup's tokens and first pair (the 4-wave instance: one token)
    const int T = NW == kB1MaxK ? 1 : NW / p.K, t0 = NW == kB1MaxK ? 0 : blockIdx.y * T, pb = t0 * p.K;
    uint8_t* scl = (uint8_t*)lds + wave * kB1Slice;      // this wave's tile scales [16][NB]
    uint4* xs = (uint4*)((uint8_t*)lds + NW * kB1Slice);  // h rows [N][su]
    float* ys = (float*)(xs + NW * su);                   // y [N][16]
    uint4* xz = (uint4*)(ys + NW * 16);                    // 64 zero bytes
    if (threadIdx.x < 4) xz[threadIdx.x] = make_uint4(0, 0, 0, 0);  // (the barrier below orders it)
    const int r0 = blockIdx.x * 16;
    const int s = wave;
    const bool live = s < T * p.K && pb + s < N;
    // h row of pair pb + s (independent of the routing tables, so issued first), then the expert
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.act + (size_t)(pb + s) * I, live ? (uint32_t)I * 2u : 0u);
    u32x4_t hv[6];
#pragma unroll
    for (int u = 0; u < 6; ++u) hv[u] = buf_load16(ra, (uint32_t)(lane + 64 * u) * 16u, 0);
    const int e = __builtin_amdgcn_readfirstlane(p.idx[live ? pb + s : 0]);
    B1Tile tl;
    b1_tile_load(tl, p, e, H, I, r0, lane, live);
    ((u32x4_t*)scl)[lane] = tl.sv0;
    ((u32x4_t*)scl)[lane + 64] = tl.sv1;
#pragma unroll
    for (int u = 0; u < 6; ++u)
        if (live && lane + 64 * u < cu) ((u32x4_t*)xs)[s * su + lane + 64 * u] = hv[u];
    __syncthreads();
    if (live) {
        const f32x4_t acc = mx_tile_steps<kB1Nit>(tl.wq, scl + m * NB + g, xs + s * su + 4 * g, xz, NB, g);
        if (m == 0) {
            float* yr = ys + s * 16 + 4 * g;
            yr[0] = acc[0] + bf16_lo(tl.b2[0]);
            yr[1] = acc[1] + bf16_hi(tl.b2[0]);
            yr[2] = acc[2] + bf16_lo(tl.b2[1]);
            yr[3] = acc[3] + bf16_hi(tl.b2[1]);
        }
    }
    __syncthreads();
    // combine (k_combine's order: fmaf over a token's k pairs in selection order, one
    // rounding); thread i: token t0 + i / 16, row r0 + i % 16
    const int i = threadIdx.x;
    const int tw = i >> 4, t = t0 + tw, r = r0 + (i & 15);
    if (tw < T && t < p.B && r < H) {
        float a = 0.f;
        for (int jj = 0; jj < p.K; ++jj)
            a = __builtin_fmaf(p.wts[t * p.K + jj], ys[(tw * p.K + jj) * 16 + (i & 15)], a);
        uint32_t o = f32_to_bf16(a);
        if (p.res) o = f32_to_bf16(bf16_to_f32(o) + bf16_to_f32(p.res[(size_t)t * H + r]));
        p.out[(size_t)t * H + r] = (uint16_t)o;
    }
}

bool b1_ok(int H, int I, int E, int K, int B) {
    return K >= 1 && K <= kB1MaxK && E <= kB1MaxE && (H >> 5) <= kB1MaxNB && (I >> 5) <= kB1MaxNB &&
           H <= kRoute1NormMaxH && B >= 1 && B <= kB1MaxB && B * K <= kB1MaxPairs;
}

int b1_layer_launch(const B1Layer& a, hipStream_t stream, int only) {
    if (!b1_ok(a.H, a.I, a.E, a.K, a.B))
        return set_error(PHYSLLM_MOE_EINVAL, "batch-1 layer: sizes out of range");
    if (only < -1 || only > 2) return set_error(PHYSLLM_MOE_EINVAL, "batch-1 layer: launch must be 0, 1 or 2");
    static std::once_flag attr_once[kMaxDevices];
    once_per_device(attr_once, [] {
        (void)hipFuncSetAttribute((const void*)k_b1_down<kB1DownWaves>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024);
        (void)hipFuncSetAttribute((const void*)k_b1_logits<true, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024);
    });
    const uint16_t* rx = (const uint16_t*)(a.norm_w ? a.norm_x : a.x);
    const uint16_t* rw = (const uint16_t*)a.router_w;
    const uint16_t* rb = (const uint16_t*)a.router_b;
    const uint16_t* nw = (const uint16_t*)a.norm_w;
    if (only == 0 || only == -1) {
        if (a.norm_w) {
            const size_t lds = 1024 + (size_t)a.B * a.H * 2;
            if (a.B == 1)
                hipLaunchKernelGGL((k_b1_logits<true, false>), dim3(a.E), dim3(kB1Threads), lds, stream, rx, rw, rb, a.H,
                                   a.E, 1, a.logits, nw, a.eps, (uint16_t*)a.x);
            else
                hipLaunchKernelGGL((k_b1_logits<true, true>), dim3(a.E), dim3(kB1Threads), lds, stream, rx, rw, rb, a.H,
                                   a.E, a.B, a.logits, nw, a.eps, (uint16_t*)a.x);
        } else {
            if (a.B == 1)
                hipLaunchKernelGGL((k_b1_logits<false, false>), dim3(a.E), dim3(64), 0, stream, rx, rw, rb, a.H, a.E, 1,
                                   a.logits, nullptr, 0.f, nullptr);
            else
                hipLaunchKernelGGL((k_b1_logits<false, true>), dim3(a.E), dim3(64 * a.B), 0, stream, rx, rw, rb, a.H, a.E,
                                   a.B, a.logits, nullptr, 0.f, nullptr);
        }
        if (int rc = check_launch("batch-1 logits")) return rc;
    }
    B1Params p{};
    p.blocks = (const uint8_t*)a.gu_blocks;
    p.scales = (const uint8_t*)a.gu_scales;
    p.bias = (const uint16_t*)a.gu_bias;
    p.act = (const uint16_t*)a.x;
    p.logits = a.logits;
    p.h = a.h;
    p.idx = a.idx;
    p.wts = a.wts;
    p.H = a.H;
    p.I = a.I;
    p.E = a.E;
    p.K = a.K;
    p.B = a.B;
    p.gu_sets = (2 * a.I + 63) / 64;
    p.alpha = a.alpha;
    p.limit = a.limit;
    // + 256: the k-steps' edge lanes read (and discard) up to 15 units past the last row
    const int cu = a.H >> 3;
    const int n_dist = std::min(a.B * a.K, a.E);  // distinct selected experts, at most
    if (only == 1 || only == -1) {
        if (a.B == 1) {
            const size_t lds_gu = (size_t)kB1Hdr + 4 * kB1Slice + (size_t)cu * 16 + 256;
            hipLaunchKernelGGL(k_b1_gate_up<1>, dim3(n_dist * p.gu_sets), dim3(kB1Threads), lds_gu, stream, p);
        } else {
            const size_t lds_gu = (size_t)kB1Hdr + 4 * kB1Slice + (size_t)a.B * (cu + 1) * 16 + 256;
            hipLaunchKernelGGL(k_b1_gate_up<kB1MaxB>, dim3(n_dist * p.gu_sets), dim3(kB1Threads), lds_gu, stream, p);
        }
        if (int rc = check_launch("batch-1 gate_up")) return rc;
    }
    if (only != 2 && only != -1) return PHYSLLM_MOE_OK;
    p.blocks = (const uint8_t*)a.dn_blocks;
    p.scales = (const uint8_t*)a.dn_scales;
    p.bias = (const uint16_t*)a.dn_bias;
    p.act = a.h;
    p.out = (uint16_t*)a.out;
    p.res = (const uint16_t*)a.res;
    const int su_dn = (a.I >> 3) + 1;
    if (a.B == 1) {
        const size_t lds_dn =
            (size_t)kB1MaxK * kB1Slice + (size_t)kB1MaxK * su_dn * 16 + (size_t)kB1MaxK * 16 * 4 + 64;
        hipLaunchKernelGGL(k_b1_down<kB1MaxK>, dim3((a.H + 15) / 16), dim3(64 * kB1MaxK), lds_dn, stream, p);
    } else {
        const int T = kB1DownWaves / a.K;  // >= 2 (k <= 4)
        const size_t lds_dn =
            (size_t)kB1DownWaves * kB1Slice + (size_t)kB1DownWaves * su_dn * 16 + (size_t)kB1DownWaves * 16 * 4 + 64;
        hipLaunchKernelGGL(k_b1_down<kB1DownWaves>, dim3((a.H + 15) / 16, (a.B + T - 1) / T),
                           dim3(64 * kB1DownWaves), lds_dn, stream, p);
    }
    return check_launch("batch-1 down");
}

}  // namespace physllm
