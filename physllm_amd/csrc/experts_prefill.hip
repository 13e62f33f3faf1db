// Prefill-regime expert kernels for gfx950: grouped MXFP4 x bf16 GEMM on MFMA.
//
// With hundreds of tokens per expert the expert projections are GEMMs
// (2 * tokens * rows * K flops against rows * K / 2 code bytes): MFMA-bound. One
// workgroup (4 waves, 2 x 2) computes a 128-row x 128-token tile of one expert:
//   A = weights, MXFP4: each wave keeps its 64 rows' stripes of the current
//       k-step in registers (one 16-byte buffer load per lane per 16-row tile =
//       one full MX block of one row) and decodes them with
//       v_cvt_scalef32_pk_bf16_fp4 right before the MFMA;
//   B = activations, bf16: the tile's 128 token rows (gathered through the
//       bucketing permutation for gate_up, contiguous for down) are staged in
//       LDS, double-buffered across k-steps, rows padded by 16 bytes so the 16
//       token columns of a fragment read hit distinct banks.
// A k-step covers 4 MX blocks (128 elements); lane group g supplies block g of
// the step to both operands (the same K-permutation on A and B), so one MFMA
// (v_mfma_f32_16x16x32_bf16) consumes 8 elements of each of 4 blocks.
// Epilogues: gate_up adds the bias and applies the clamped SwiGLU to each lane's
// (gate, up) row pairs (rows are interleaved) -> h bf16; down adds the bias ->
// y fp32. Tiles are scheduled from a device-side per-expert prefix of token
// tiles, and consecutive token tiles of one weight row tile are mapped to the
// same XCD so they share its L2.
// Two forms: k_mx_gemm2 (256 x 128 tiles, 8 waves, loads two k-steps ahead,
// the tile's scales staged in LDS) for K up to 96 MX blocks, and k_mx_gemm
// (128 x 128, 4 waves) for longer K.
#include "common.h"
#include "capi_internal.h"
#include "experts.h"

namespace physllm {

constexpr int kGemmThreads = 256;
constexpr int kTM = 128;          // weight rows per tile
constexpr int kTN = 128;          // tokens per tile
constexpr int kKS = 128;          // elements per k-step (4 MX blocks)
constexpr int kBRowU = kKS * 2 / 16 + 1;  // LDS row stride of the B tile in 16-byte units (16 + pad)
constexpr int kBUnitsPerThread = kTN * (kKS * 2 / 16) / kGemmThreads;  // 8

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4_t gemm_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
}

template <int MODE>
__global__ __launch_bounds__(kGemmThreads, 2) void k_mx_gemm(GemvParams p, const int32_t* __restrict__ tprefix) {
    extern __shared__ uint4 lds[];
    // ---- tile id -> (expert slot, row tile, token tile), XCD-aware ----
    const int G = gridDim.x;  // a multiple of 8
    const int bid = blockIdx.x;
    const int t = (bid & 7) * (G >> 3) + (bid >> 3);
    const int n_slots = *p.n_slots;
    const int row_tiles = (p.R + kTM - 1) / kTM;
    if (t >= row_tiles * tprefix[n_slots]) return;
    int lo = 0, hi = n_slots;  // largest s with row_tiles * tprefix[s] <= t
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (row_tiles * tprefix[mid] <= t) lo = mid; else hi = mid;
    }
    const int slot = lo;
    const int4 si = p.slots[slot];
    const int e = si.x, ne = si.y, p0 = si.z;
    const int ntt = (ne + kTN - 1) / kTN;
    const int local = t - row_tiles * tprefix[slot];
    const int rtile = local / ntt;
    const int ttile = local - rtile * ntt;
    const int row0 = rtile * kTM;
    const int tok0 = ttile * kTN;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;  // wave quadrant: rows 64*wm.., tokens 64*wn..
    const int NB = p.Kdim >> 5;
    const int nks = (NB + 3) >> 2;
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;
    const uint32_t exp_s = (uint32_t)p.R * (uint32_t)NB;
    const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(p.blocks + (size_t)e * exp_w, exp_w);
    const uint8_t* sbase = p.scales + (size_t)e * exp_s;
    const __amdgpu_buffer_rsrc_t ract = gemm_rsrc(p.act, (uint32_t)p.act_rows * (uint32_t)p.Kdim * 2u);

    // A: this lane's rows (4 tiles of 16) and its block within each k-step
    uint32_t aoff[4];
    int arow[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        arow[mt] = row0 + wm * 64 + mt * 16 + m;
        aoff[mt] = (uint32_t)arow[mt] * row_bytes + (uint32_t)g * 16u;
    }
    // B: this thread's staging units: token rows r = tid/16 + 16u (u < 8), chunk c = tid%16
    const int bc = threadIdx.x & 15;
    uint32_t boff[kBUnitsPerThread];
#pragma unroll
    for (int u = 0; u < kBUnitsPerThread; ++u) {
        const int r = (threadIdx.x >> 4) + 16 * u;
        const int q = min(tok0 + r, ne - 1);  // rows past the expert's tokens: any valid row
        const uint32_t arow_act = (MODE == kModeGateUp) ? (uint32_t)(p.perm[p0 + q] / p.top_k) : (uint32_t)(p0 + q);
        boff[u] = arow_act * (uint32_t)(p.Kdim * 2) + (uint32_t)bc * 16u;
    }

    u32x4_t aq[4];
    uint32_t as[4];
    u32x4_t bv[kBUnitsPerThread];
    auto load_step = [&](int ks) {
        const int blk = ks * 4 + g;
        const bool in = blk < NB;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            aq[mt] = gemm_load16(rw, aoff[mt] + (uint32_t)ks * 64u);
            as[mt] = (in && arow[mt] < p.R) ? (uint32_t)sbase[(size_t)arow[mt] * NB + blk] : 0u;
        }
        const int kel = ks * kKS + bc * 8;  // first element of this thread's B chunk
#pragma unroll
        for (int u = 0; u < kBUnitsPerThread; ++u)
            bv[u] = kel < p.Kdim ? gemm_load16(ract, boff[u] + (uint32_t)ks * (kKS * 2)) : u32x4_t{0u, 0u, 0u, 0u};
    };
    auto store_b = [&](int buf) {
        u32x4_t* bs = (u32x4_t*)lds + buf * (kTN * kBRowU);
#pragma unroll
        for (int u = 0; u < kBUnitsPerThread; ++u) {
            const int r = (threadIdx.x >> 4) + 16 * u;
            bs[r * kBRowU + bc] = bv[u];
        }
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    load_step(0);
    store_b(0);
    __syncthreads();
    for (int ks = 0; ks < nks; ++ks) {
        // this step's A (registers) and scales; the next step's loads go out first
        u32x4_t a_cur[4];
        uint32_t s_cur[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            a_cur[mt] = aq[mt];
            s_cur[mt] = as[mt];
        }
        const bool more = ks + 1 < nks;
        if (more) load_step(ks + 1);
        const bool in = ks * 4 + g < NB;
        const uint4* bs = lds + (ks & 1) * (kTN * kBRowU);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // B fragments: token column m of each 16-token tile, 8 elements of block g
            uint4 b[4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const int r = wn * 64 + nt * 16 + m;
                const uint4* src = bs + r * kBRowU + g * 4 + i;
                b[nt] = *src;
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const uint32_t code = in ? a_cur[mt][i] : 0u;
                const bf16x8_t a = mx_cvt8(code, e8m0_scale_operand(s_cur[mt]));
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mfma16x16x32(a, as_bf16x8(b[nt]), acc[mt][nt]);
            }
        }
        if (more) {
            store_b((ks + 1) & 1);
        }
        __syncthreads();
    }

    // ---- epilogue ----
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int q = tok0 + wn * 64 + nt * 16 + m;  // token column of this lane
        if (q >= ne) continue;
        const int pp = p0 + q;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int rr = row0 + wm * 64 + mt * 16 + 4 * g;
            if (rr >= p.R) continue;
            float bsum[4] = {0.f, 0.f, 0.f, 0.f};
            if (p.bias) {
                const uint2 bb = *(const uint2*)(p.bias + (size_t)e * p.R + rr);
                bsum[0] = bf16_lo(bb.x);
                bsum[1] = bf16_hi(bb.x);
                bsum[2] = bf16_lo(bb.y);
                bsum[3] = bf16_hi(bb.y);
            }
            const f32x4_t c = acc[mt][nt];
            if (MODE == kModeGateUp) {
                const float h0 = swiglu(c[0] + bsum[0], c[1] + bsum[1], p.alpha, p.limit);
                const float h1 = swiglu(c[2] + bsum[2], c[3] + bsum[3], p.alpha, p.limit);
                const int I = p.R >> 1;
                uint32_t* hout = (uint32_t*)((uint16_t*)p.out + (size_t)pp * I + (rr >> 1));
                *hout = f32_to_bf16(h0) | (f32_to_bf16(h1) << 16);
            } else {
                float4 y;
                y.x = c[0] + bsum[0];
                y.y = c[1] + bsum[1];
                y.z = c[2] + bsum[2];
                y.w = c[3] + bsum[3];
                *(float4*)((float*)p.out + (size_t)pp * p.R + rr) = y;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Wide-tile form: one workgroup of 8 waves (4 x 2, 64 x 64 each) computes 256
// weight rows x 128 tokens, halving the activation re-reads per flop of the
// 128 x 128 form. Loads run kGemmPD k-steps ahead of the MFMAs:
//   A (weights): each lane's 4 stripes of a k-step in a register ring;
//   B (activations): staged through registers into a double-buffered LDS tile
//     (the registers of step ks + 1 were filled during step ks - 1);
//   scales: the tile's 256 rows x NB bytes, staged into LDS once.
// Waves whose 64 rows all lie past R skip their MFMAs.
// ---------------------------------------------------------------------------
constexpr int kG2Threads = 512;
constexpr int kG2TM = 256;
constexpr int kG2BUnits = kTN * (kKS * 2 / 16) / kG2Threads;  // 4 B units per thread per k-step
constexpr int kG2MaxNB = 96;                                   // scale row bytes staged per tile row
constexpr int kG2BRow = kKS * 2 / 16;  // B tile row (one token's k-step): 16 units of 16 bytes, XOR-swizzled

// Tile t of the wide-tile GEMM (expert slot, row tile, token tile), decoded from the
// slot table and token-tile prefix staged in LDS: slot = the number of s in
// [1, n_slots] with row_tiles * tp[s] <= t (the prefix is strictly increasing).
struct G2Tile {
    int e, ne, p0, row0, tok0;
};

__device__ __forceinline__ G2Tile g2_decode(int t, int row_tiles, int n_slots, const int32_t* tp, const int4* st,
                                           int lane) {
    int slot = 0;
    for (int s0 = 1; s0 <= n_slots; s0 += 64) {
        const int s = s0 + lane;
        slot += __popcll(__ballot(s <= n_slots && row_tiles * tp[s] <= t));
    }
    slot = __builtin_amdgcn_readfirstlane(slot);
    const int4 si = st[slot];
    G2Tile d;
    d.e = __builtin_amdgcn_readfirstlane(si.x);
    d.ne = __builtin_amdgcn_readfirstlane(si.y);
    d.p0 = __builtin_amdgcn_readfirstlane(si.z);
    const int ntt = (d.ne + kTN - 1) / kTN;
    const int local = t - row_tiles * tp[slot];
    const int rtile = local / ntt;
    d.row0 = rtile * kG2TM;
    d.tok0 = (local - rtile * ntt) * kTN;
    return d;
}

// Persistent: the tiles (expert slot, row tile, token tile in that order) are split
// into 8 contiguous ranges, one per XCD (workgroup b runs on XCD b % 8), so every
// XCD gets the same number of tiles and works on few experts at a time. The next
// tile's first loads (biases, scales, gathered activation rows, weights of its
// first two k-steps) are issued before the current tile's epilogue, so its
// prologue latency hides behind the SwiGLU and the stores.
template <int MODE>
__global__ __launch_bounds__(kG2Threads, 1) void k_mx_gemm2(GemvParams p, const int32_t* __restrict__ tprefix,
                                                            int max_slots) {
    extern __shared__ uint4 lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;  // rows 64*wm.., tokens 64*wn..
    const int NB = p.Kdim >> 5;
    const int nks = (NB + 3) >> 2;
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;
    const uint32_t act_bytes = (uint32_t)p.act_rows * (uint32_t)p.Kdim * 2u;
    const int bc = threadIdx.x & 15;  // this thread's 16-byte chunk of a staged token row

    // LDS: B tile [2][kTN][16 units] (unit c of token row r at r * 16 + (c ^ (r & 15)), so the 16
    // token rows of a fragment read cover all 64 banks) | the tile's scales [256][NB] as in memory
    // (rows past R: zeros) | slot table [max_slots] | token-tile prefix [max_slots + 1]
    uint4* bsm = lds;
    uint8_t* ssm = (uint8_t*)(lds + 2 * kTN * kG2BRow);
    int4* stl = (int4*)(ssm + kG2TM * kG2MaxNB);
    int32_t* tpl = (int32_t*)(stl + max_slots);
    const int n_slots = *p.n_slots;
    for (int i = threadIdx.x; i < n_slots; i += kG2Threads) stl[i] = p.slots[i];
    for (int i = threadIdx.x; i <= n_slots; i += kG2Threads) tpl[i] = tprefix[i];
    __syncthreads();
    const int row_tiles = (p.R + kG2TM - 1) / kG2TM;
    const int T = row_tiles * tpl[n_slots];
    const int xcd = blockIdx.x & 7, per_xcd = gridDim.x >> 3;
    const int t_end = (int)(((int64_t)(xcd + 1) * T) >> 3);
    int t = (int)(((int64_t)xcd * T) >> 3) + (int)(blockIdx.x >> 3);
    if (t >= t_end) return;

    constexpr uint32_t kPast = 0x80000000u;  // offset past every range: zeros
    constexpr int kScUnits = (kG2TM * kG2MaxNB / 16 + kG2Threads - 1) / kG2Threads;  // 3
    // per-tile state: weights base, A lane offsets, B lane offsets, biases
    const uint8_t* wexp;
    uint32_t aoff[4], boff[kG2BUnits];
    uint2 bias[4];
    u32x4_t scv[kScUnits];
    u32x4_t A[3][4];
    u32x4_t Bv[2][kG2BUnits];

    // A: this lane's 4 rows (one per 16-row tile) at block g of a k-step; rows past
    // R lie past the buffer range and read zeros. The buffer base advances by one
    // k-step (64 bytes of every row) per step in scalar registers, so the lane
    // offsets never change. ks >= nks: an empty range (no traffic).
    auto load_a = [&](int ks, u32x4_t (&a)[4]) {
        const uint32_t adv = (uint32_t)ks * 64u;
        const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(wexp + adv, ks < nks ? exp_w - adv : 0u);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) a[mt] = gemm_load16(rw, aoff[mt]);
    };
    // B: token rows r = tid/16 + 32u (u < 4) of the tile; chunks past K read zeros
    // (the next row's elements must not enter the sums)
    auto load_b = [&](int ks, u32x4_t (&b)[kG2BUnits]) {
        const uint32_t adv = (uint32_t)ks * (kKS * 2);
        const __amdgpu_buffer_rsrc_t ra = gemm_rsrc(p.act + adv / 2, ks < nks ? act_bytes - adv : 0u);
        const bool ok = ks * kKS + bc * 8 < p.Kdim;
#pragma unroll
        for (int u = 0; u < kG2BUnits; ++u) b[u] = gemm_load16(ra, ok ? boff[u] : kPast);
    };
    auto store_b = [&](int buf, const u32x4_t (&b)[kG2BUnits]) {
        u32x4_t* bs = (u32x4_t*)bsm + buf * (kTN * kG2BRow);
#pragma unroll
        for (int u = 0; u < kG2BUnits; ++u) {
            const int r = (threadIdx.x >> 4) + 32 * u;
            bs[r * kG2BRow + (bc ^ (r & 15))] = b[u];
        }
    };
    // first loads of tile d: biases, scales, activation row ids, A of steps 0 and 1,
    // then (after the row ids arrive) B of steps 0 and 1
    int32_t rowid[kG2BUnits];
    auto prologue_issue = [&](const G2Tile& d) {
        wexp = p.blocks + (size_t)d.e * exp_w;
        // no biases: an empty range (reads zeros) on a valid pointer
        const __amdgpu_buffer_rsrc_t rb = p.bias ? gemm_rsrc(p.bias + (size_t)d.e * p.R, (uint32_t)p.R * 2u)
                                                 : gemm_rsrc(p.blocks, 0u);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const u32x2_t b2 = __builtin_amdgcn_raw_buffer_load_b64(
                rb, (uint32_t)(d.row0 + wm * 64 + mt * 16 + 4 * g) * 2u, 0, 0);
            bias[mt] = make_uint2(b2[0], b2[1]);
        }
        const int rows = min(kG2TM, p.R - d.row0);
        const __amdgpu_buffer_rsrc_t rsc =
            gemm_rsrc(p.scales + ((size_t)d.e * p.R + d.row0) * NB, (uint32_t)rows * (uint32_t)NB);
#pragma unroll
        for (int u = 0; u < kScUnits; ++u) scv[u] = gemm_load16(rsc, 16u * (uint32_t)(threadIdx.x + u * kG2Threads));
#pragma unroll
        for (int u = 0; u < kG2BUnits; ++u) {
            const int q = min(d.tok0 + (int)(threadIdx.x >> 4) + 32 * u, d.ne - 1);  // past the tokens: a valid row
            rowid[u] = (MODE == kModeGateUp) ? p.perm[d.p0 + q] : d.p0 + q;
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            aoff[mt] = (uint32_t)(d.row0 + wm * 64 + mt * 16 + m) * row_bytes + (uint32_t)g * 16u;
        load_a(0, A[0]);
        load_a(1, A[1]);
    };
    auto prologue_finish = [&]() {
#pragma unroll
        for (int u = 0; u < kG2BUnits; ++u) {
            const uint32_t arow = (MODE == kModeGateUp) ? (uint32_t)(rowid[u] / p.top_k) : (uint32_t)rowid[u];
            boff[u] = arow * (uint32_t)(p.Kdim * 2) + (uint32_t)bc * 16u;
        }
        load_b(0, Bv[0]);
        load_b(1, Bv[1]);
#pragma unroll
        for (int u = 0; u < kScUnits; ++u) {
            const int i = threadIdx.x + u * kG2Threads;
            if (i < ((kG2TM * NB) >> 4)) ((u32x4_t*)ssm)[i] = scv[u];
        }
        store_b(0, Bv[0]);
    };

    G2Tile cur = g2_decode(t, row_tiles, n_slots, tpl, stl, lane);
    prologue_issue(cur);
    prologue_finish();
    // this lane's scale bytes: row (wm*64 + mt*16 + m), block 4ks + g; B fragment rows: r & 15 == m
    const uint8_t* sl = ssm + (wm * 64 + m) * NB + g;
    const uint4* bl = lds + (wn * 64 + m) * kG2BRow;

    for (;;) {
        __syncthreads();  // B(0) and the scales are in LDS
        const bool wave_rows = cur.row0 + wm * 64 < p.R;  // wave-uniform
        f32x4_t acc[4][4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        // Rings: A[ks % 3] holds step ks, Bv[ks % 2] step ks (before it is stored)
        // or ks + 2 (after). Six steps are unrolled so that every ring index is a
        // constant: no register copies, whose sources would have to be waited for.
        for (int kb = 0; kb < nks; kb += 6) {
#pragma unroll
            for (int u = 0; u < 6; ++u) {
                const int ks = kb + u;
                // loads for step ks + 2 go out first (past K: zeros, no traffic), always,
                // so that the rings never hold either-or values
                load_a(ks + 2, A[(u + 2) % 3]);
                load_b(ks + 2, Bv[u % 2]);
                if (ks < nks) {  // block-uniform
                    if (wave_rows) {
                        // blocks past NB (last step): scale 0, so the (finite) codes read
                        // there cannot make a NaN against the zero activations; the reads
                        // are unconditional (in LDS bounds for every step) and the mask is
                        // opaque, so they do not become masked reads waited for one by one
                        uint32_t keep = (4 * ks + g < NB) ? 0xffu : 0u;
                        asm volatile("" : "+v"(keep));
                        uint32_t sc[4];
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) sc[mt] = (uint32_t)sl[mt * 16 * NB + 4 * ks];
                        // all four reads in flight together, then one wait (a shared
                        // destination register would serialise them)
                        asm volatile("" : "+v"(sc[0]), "+v"(sc[1]), "+v"(sc[2]), "+v"(sc[3]));
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) sc[mt] &= keep;
                        const uint4* bs = bl + (ks & 1) * (kTN * kG2BRow);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            uint4 b[4];
#pragma unroll
                            for (int nt = 0; nt < 4; ++nt) b[nt] = bs[nt * 16 * kG2BRow + ((g * 4 + i) ^ m)];
#pragma unroll
                            for (int mt = 0; mt < 4; ++mt) {
                                const bf16x8_t a = mx_cvt8(A[u % 3][mt][i], e8m0_scale_operand(sc[mt]));
#pragma unroll
                                for (int nt = 0; nt < 4; ++nt)
                                    acc[mt][nt] = mfma16x16x32(a, as_bf16x8(b[nt]), acc[mt][nt]);
                            }
                        }
                    }
                    // B of step ks + 1 (loaded during step ks - 1) into the other buffer
                    if (ks + 1 < nks) store_b((ks + 1) & 1, Bv[(u + 1) % 2]);
                    __syncthreads();
                }
            }
        }

        // every wave is past its last LDS read of this tile: the next tile's first
        // loads go out now, ahead of this tile's epilogue
        const G2Tile d = cur;
        const uint2 bias_cur[4] = {bias[0], bias[1], bias[2], bias[3]};
        t += per_xcd;
        const bool more = t < t_end;
        if (more) {
            cur = g2_decode(t, row_tiles, n_slots, tpl, stl, lane);
            prologue_issue(cur);
        }

        // ---- epilogue of tile d ----
        if (MODE == kModeGateUp) {
            // h of the tile (128 tokens x 128 columns, bf16) goes through B buffer 1,
            // free until the next tile's first k-step stores into it (after the
            // barrier at the top of the loop): 16-byte chunk c of token row r at
            // chunk c ^ (r & 15), so the fragment-order writes (16 token rows per
            // instruction) are bank-conflict-free; then every 1 KiB store instruction
            // writes 4 tokens' 256 contiguous bytes instead of 16 tokens' 16 bytes
            uint32_t* ht = (uint32_t*)(bsm + kTN * kG2BRow);
            if (wave_rows) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const int tl = wn * 64 + nt * 16 + m;  // token row of the tile
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        const float b0 = bf16_lo(bias_cur[mt].x), b1 = bf16_hi(bias_cur[mt].x);
                        const float b2 = bf16_lo(bias_cur[mt].y), b3 = bf16_hi(bias_cur[mt].y);
                        const f32x4_t c = acc[mt][nt];
                        const float h0 = swiglu(c[0] + b0, c[1] + b1, p.alpha, p.limit);
                        const float h1 = swiglu(c[2] + b2, c[3] + b3, p.alpha, p.limit);
                        // h columns wm*32 + mt*8 + 2g, +1: word g of chunk wm*4 + mt
                        ht[tl * 64 + (((wm * 4 + mt) ^ m) << 2) + g] = f32_to_bf16(h0) | (f32_to_bf16(h1) << 16);
                    }
                }
            }
            __syncthreads();
            const int I = p.R >> 1;
            const int hc0 = d.row0 >> 1;  // the tile's first h column
#pragma unroll
            for (int u = 0; u < (kTN * 16) / kG2Threads; ++u) {
                const int i = threadIdx.x + u * kG2Threads;
                const int r = i >> 4, c = i & 15;  // token row, 16-byte chunk (8 h columns)
                const int q = d.tok0 + r;
                const int col = hc0 + c * 8;
                // rows past R leave whole chunks past I (R and the tile rows are multiples of 16)
                if (q < d.ne && col < I) {
                    const uint4 v = ((const uint4*)ht)[r * 16 + (c ^ (r & 15))];
                    *(uint4*)((uint16_t*)p.out + (size_t)(d.p0 + q) * I + col) = v;
                }
            }
        } else if (wave_rows) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const int q = d.tok0 + wn * 64 + nt * 16 + m;  // token column of this lane
                if (q >= d.ne) continue;
                const int pp = d.p0 + q;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    const int rr = d.row0 + wm * 64 + mt * 16 + 4 * g;
                    if (rr >= p.R) continue;
                    const float b0 = bf16_lo(bias_cur[mt].x), b1 = bf16_hi(bias_cur[mt].x);
                    const float b2 = bf16_lo(bias_cur[mt].y), b3 = bf16_hi(bias_cur[mt].y);
                    const f32x4_t c = acc[mt][nt];
                    float4 y;
                    y.x = c[0] + b0;
                    y.y = c[1] + b1;
                    y.z = c[2] + b2;
                    y.w = c[3] + b3;
                    *(float4*)((float*)p.out + (size_t)pp * p.R + rr) = y;
                }
            }
        }
        if (!more) break;
        prologue_finish();
    }
}

int gemm_launch(int mode, const GemvParams& p, const int32_t* tprefix, int max_slots, int n_pairs,
                hipStream_t stream) {
    static bool attr_set = false;
    if (!attr_set) {
        const void* ks[] = {(const void*)k_mx_gemm<kModeGateUp>, (const void*)k_mx_gemm<kModeDown>,
                            (const void*)k_mx_gemm2<kModeGateUp>, (const void*)k_mx_gemm2<kModeDown>};
        for (const void* k : ks) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr_set = true;
    }
    if (p.split != 1) return set_error(PHYSLLM_MOE_EINVAL, "gemm: split must be 1");
    const long token_tiles_ub = (long)(n_pairs + kTN - 1) / kTN + max_slots;
    if ((p.Kdim >> 5) <= kG2MaxNB) {
        // wide tiles, persistent: one workgroup per CU (a multiple of 8, one range of
        // tiles per XCD); the tile count is only known on the device
        const long tiles_ub = (long)((p.R + kG2TM - 1) / kG2TM) * token_tiles_ub;
        if (tiles_ub > 0x7fffffffL) return set_error(PHYSLLM_MOE_EINVAL, "gemm: too many tiles");
        static int n_cu = 0;
        if (n_cu == 0) {
            int dev = 0;
            (void)hipGetDevice(&dev);
            if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
                n_cu = 256;
        }
        const long tiles = (n_cu + 7) & ~7;
        // B tiles, scales, slot table, token-tile prefix
        const size_t lds = (size_t)2 * kTN * kG2BRow * 16 + (size_t)kG2TM * kG2MaxNB + (size_t)max_slots * 16 +
                           (size_t)(max_slots + 1) * 4;
        if (mode == kModeGateUp)
            hipLaunchKernelGGL(k_mx_gemm2<kModeGateUp>, dim3((unsigned)tiles), dim3(kG2Threads), lds, stream, p,
                               tprefix, max_slots);
        else
            hipLaunchKernelGGL(k_mx_gemm2<kModeDown>, dim3((unsigned)tiles), dim3(kG2Threads), lds, stream, p,
                               tprefix, max_slots);
        return check_launch(mode == kModeGateUp ? "gate_up gemm" : "down gemm");
    }
    const int row_tiles = (p.R + kTM - 1) / kTM;
    // upper bound on token tiles: every touched expert may add one partial tile
    const long token_tiles = (long)(n_pairs + kTN - 1) / kTN + max_slots;
    long tiles = row_tiles * token_tiles;
    tiles = (tiles + 7) & ~7L;
    if (tiles > 0x7fffffffL) return set_error(PHYSLLM_MOE_EINVAL, "gemm: too many tiles");
    const size_t lds = (size_t)2 * kTN * kBRowU * 16;
    if (mode == kModeGateUp)
        hipLaunchKernelGGL(k_mx_gemm<kModeGateUp>, dim3((unsigned)tiles), dim3(kGemmThreads), lds, stream, p, tprefix);
    else
        hipLaunchKernelGGL(k_mx_gemm<kModeDown>, dim3((unsigned)tiles), dim3(kGemmThreads), lds, stream, p, tprefix);
    return check_launch(mode == kModeGateUp ? "gate_up gemm" : "down gemm");
}

}  // namespace physllm
