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
// Three forms: k_mx_gemm3 (384- or 320-row x 128-token tiles, 8 waves, every
// operand copied straight into LDS; the default), k_mx_gemm2 (256 x 128 tiles,
// weights loaded into registers, activations staged through registers; for scale
// or bias arrays that are not 16-byte aligned, and K of 4 blocks) for K up to 96
// MX blocks, and k_mx_gemm (128 x 128, 4 waves) for longer K.
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

// ---------------------------------------------------------------------------
// LDS-staged form (k_mx_gemm3): 8 waves compute a tile of MT*64 weight rows x 128
// tokens; wave (wm, wn) owns rows wm*16*MT.. (MT 16-row tiles) and tokens wn*64..
// (4 16-token tiles), i.e. 1.5-2x the rows per wave of k_mx_gemm2, so fewer LDS
// bytes per flop for B. Every operand reaches LDS by direct copies from memory
// (buffer_load ... lds: no register staging, no per-lane byte loads):
//   A: per 128-element k-step, the tile's codes, 64 bytes per row; one copy
//      instruction covers 16 rows with 4 consecutive lanes per row (each row read
//      once per tile, coalesced); unit g of row r is stored at
//      r*64 + 16*(g ^ ((r >> 2) & 3)), so the 16 rows of a fragment read fall in
//      16 different bank groups;
//   B: per k-step, the 128 gathered token rows, unit c of row r at
//      r*256 + 16*(c ^ (r & 15));
//   per tile: its E8M0 scales (MT*64 rows x NB bytes, one contiguous block in
//      memory), its biases, and (gate_up) the next tile's 128 sorted pair ids, from
//      which the next tile's activation rows are found without a global load.
// A and B use a two-stage ring, one k-step ahead; the steps of consecutive tiles
// form one sequence, so the next tile's first step is copied during the current
// tile's last. The scales of the next tile are copied at the start of the
// current tile's epilogue (one scale buffer; the epilogue hides the copy) and the
// biases into a two-slot buffer. The kernel issues no other vector-memory load
// inside its steps: the compiler would make a use of such a load wait for the
// copies issued before it, and the copies are issued as inline assembly, so the
// compiler does not wait for them before LDS reads of the other stage. One
// barrier per step, after a vmcnt(0): the step's copies are complete and the
// other stage is free.
// ---------------------------------------------------------------------------
constexpr int kG3MaxNB = 96;
constexpr int kG3Waves = 8;     // two waves per SIMD
constexpr int kG3MtGateUp = 6;  // 16-row tiles per wave: 384-row tiles (2I = 5760 = 15 of them)
constexpr int kG3MtDown = 5;    // 320-row tiles (H = 2880 = 9 of them)

// LDS layout of k_mx_gemm3 for tiles of `tm` rows and `nb` scale blocks per row (bytes)
struct G3Layout {
    int a_stage, b_stage, stage, ring, scales, bias, perm, tables;
};
__host__ __device__ constexpr G3Layout g3_layout(int tm, int nb) {
    G3Layout L{};
    L.a_stage = tm * 64;
    L.b_stage = kTN * 256;
    L.stage = L.a_stage + L.b_stage;
    L.ring = 0;
    L.scales = 2 * L.stage;
    // the last copy of the scale block may run up to one 1 KiB window past it
    L.bias = L.scales + ((tm * nb + 1023) / 1024) * 1024;
    L.perm = L.bias + 2 * 1024;  // two slots of up to 512 biases (bf16), each a 1 KiB copy window
    L.tables = L.perm + 512;     // 128 pair ids
    return L;
}

template <int MT>
__device__ __forceinline__ G2Tile g3_decode(int t, int row_tiles, int n_slots, const int32_t* tp, const int4* st,
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
    d.row0 = rtile * (MT * 64);
    d.tok0 = (local - rtile * ntt) * kTN;
    return d;
}

template <int MODE, int MT, int NW>
__global__ __launch_bounds__(64 * NW, 1) void k_mx_gemm3(GemvParams p, const int32_t* __restrict__ tprefix,
                                                         int max_slots) {
    extern __shared__ uint4 lds[];
    constexpr int kThreads = 64 * NW;
    constexpr int TM = MT * 16 * (NW / 2);  // tile rows: NW/2 row groups of MT 16-row tiles
    constexpr int kBWin = 32 / NW;          // B copy windows (4 token rows each) per wave
    // (& (NW - 1): lets the compiler see wave < NW, so whole-tile copy windows need no test)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & (NW - 1), lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int NB = p.Kdim >> 5;
    const int nks = (NB + 3) >> 2;  // >= 2 (launcher)
    const G3Layout L = g3_layout(TM, NB);
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;
    const uint32_t exp_s = (uint32_t)p.R * (uint32_t)NB;
    const uint32_t act_bytes = (uint32_t)p.act_rows * (uint32_t)p.Kdim * 2u;
    constexpr uint32_t kPast = 0x80000000u;  // an offset past every range: zeros

    lds_u8* base = (lds_u8*)lds;
    int4* stl = (int4*)((uint8_t*)lds + L.tables);  // slot table
    int32_t* tpl = (int32_t*)(stl + max_slots);       // token-tile prefix
    const int n_slots = *p.n_slots;
    for (int i = threadIdx.x; i < n_slots; i += kThreads) stl[i] = p.slots[i];
    for (int i = threadIdx.x; i <= n_slots; i += kThreads) tpl[i] = tprefix[i];
    __syncthreads();
    const int row_tiles = (p.R + TM - 1) / TM;
    const int T = row_tiles * tpl[n_slots];
    const int xcd = blockIdx.x & 7, per_xcd = gridDim.x >> 3;
    const int t_end = (int)(((int64_t)(xcd + 1) * T) >> 3);
    int t = (int)(((int64_t)xcd * T) >> 3) + (int)(blockIdx.x >> 3);
    if (t >= t_end) return;

    // A copy lane map: window w (rows 16w..16w+15), lane l -> row 16w + l/4, unit (l & 3) ^ (l >> 4)
    const uint32_t a_dma = (uint32_t)(lane >> 2) * row_bytes + (uint32_t)(((lane & 3) ^ (lane >> 4)) << 4);
    // B copy lane map: window b = wave + NW*u (token rows 4b..4b+3), lane l -> row 4b + l/16,
    // unit (l & 15) ^ ((4b + l/16) & 15); per tile: the gathered row's byte offset plus the unit's
    uint32_t b_dma[kBWin];
    auto b_rows = [&](const G2Tile& d, int id_src) {  // id_src: 0 = global perm, 1 = the LDS copy
#pragma unroll
        for (int u = 0; u < kBWin; ++u) {
            const int r = (wave + NW * u) * 4 + (lane >> 4);  // token row of the tile
            const int q = min(d.tok0 + r, d.ne - 1);         // past the tokens: a valid row
            uint32_t row;
            if (MODE == kModeGateUp)
                row = (uint32_t)((id_src ? lds_ld<int32_t>(base + L.perm + 4 * (q - d.tok0)) : p.perm[d.p0 + q]) /
                                 p.top_k);
            else
                row = (uint32_t)(d.p0 + q);
            b_dma[u] = row * (uint32_t)(p.Kdim * 2) + (uint32_t)(((lane & 15) ^ (r & 15)) << 4);
            // rows past the tokens are never used: copy zeros from past the range (no
            // memory request; the step offsets added below keep it under 2^32)
            if (d.tok0 + r >= d.ne) b_dma[u] = kPast;
        }
    };
    // copies of a step: this wave's A windows wave + NW*u (16 rows each) for the bits u set
    // in amask and its B windows wave + NW*u (4 token rows each) for the bits set in bmask
    constexpr int kAWin = (TM / 16 + NW - 1) / NW;  // A windows per wave (at most)
    static_assert(kAWin <= 4 && kBWin <= 4, "the copy masks hold 4 windows");
    // live = false: empty ranges (zeros into the stage, no memory requests), so the
    // caller selects what to copy without a branch
    auto copy_sel = [&](const G2Tile& d, int ks, int st, int amask, int bmask, bool live) {
        const lds_u8* sb = base + st * L.stage;
        const u32x4_t rw = rsrc_words(p.blocks + (size_t)d.e * exp_w, live ? exp_w : 0u);
        const u32x4_t rb = rsrc_words(p.act, live ? act_bytes : 0u);
#pragma unroll
        for (int u = 0; u < kAWin; ++u) {
            const int w = wave + NW * u;
            if (((amask >> u) & 1) && w * 16 < TM)  // wave-uniform
                dma16(rw, sb + w * 1024, a_dma + (uint32_t)(d.row0 + 16 * w) * row_bytes + (uint32_t)ks * 64u);
        }
        const int kvalid = p.Kdim - ks * kKS;  // elements of this step inside K; units past it read zeros
#pragma unroll
        for (int u = 0; u < kBWin; ++u) {
            if (!((bmask >> u) & 1)) continue;
            const int b = wave + NW * u;
            const int c = (lane & 15) ^ ((4 * b + (lane >> 4)) & 15);
            dma16(rb, sb + L.a_stage + b * 1024, c * 8 < kvalid ? b_dma[u] + (uint32_t)ks * 256u : kPast);
        }
    };
    // the windows fragment group i (0..3) of a step issues for the next step: gate_up one A
    // and one B window per group; down, whose groups hold fewer MFMAs, all of them in groups
    // 0 and 1 (config 3: down 300 -> 290 us; the same split for gate_up measured slower)
    auto group_amask = [](int i) { return MODE == kModeGateUp ? 1 << i : (i == 0 ? 3 : i == 1 ? 4 : 0); };
    auto group_bmask = [](int i) { return MODE == kModeGateUp ? 1 << i : (i == 0 ? 3 : i == 1 ? 12 : 0); };
    auto copy_step = [&](const G2Tile& d, int ks, int st, bool live) { copy_sel(d, ks, st, 15, 15, live); };
    // the tile's scale block (rows row0.. of expert e: TM*NB contiguous bytes, 16-byte aligned)
    // and biases (TM bf16) into bias slot `bs`
    auto copy_tile = [&](const G2Tile& d, int bs) {
        const uint32_t sbytes = (uint32_t)TM * (uint32_t)NB;
        const u32x4_t rs = rsrc_words(p.scales + ((size_t)d.e * p.R + d.row0) * NB,
                                      min(sbytes, exp_s - (uint32_t)d.row0 * (uint32_t)NB));
        const int windows = (int)((sbytes + 1023) / 1024);
        for (int w = wave; w < windows; w += NW) dma16(rs, base + L.scales + w * 1024, (uint32_t)(w * 1024 + lane * 16));
        if (wave == 0) {
            const u32x4_t rb = rsrc_words(p.bias ? p.bias + (size_t)d.e * p.R + d.row0 : (const uint16_t*)p.blocks,
                                          p.bias ? (uint32_t)min(TM, p.R - d.row0) * 2u : 0u);
            dma16(rb, base + L.bias + bs * 1024, (uint32_t)lane * 16u);
        }
    };
    // the pair ids of a tile's 128 token rows (gate_up), as 4-byte copies
    auto copy_ids = [&](const G2Tile& d) {
        if (wave == 0) {
            const u32x4_t rp = rsrc_words(p.perm, (uint32_t)p.n_pairs * 4u);
            dma4(rp, base + L.perm, (uint32_t)(d.p0 + d.tok0 + lane) * 4u);
            dma4(rp, base + L.perm + 256, (uint32_t)(d.p0 + d.tok0 + 64 + lane) * 4u);
        }
    };

    G2Tile cur = g3_decode<MT>(t, row_tiles, n_slots, tpl, stl, lane);
    int bslot = 0;
    b_rows(cur, 0);
    copy_tile(cur, bslot);
    copy_step(cur, 0, 0, true);
    int buf = 0;
    // lane-constant LDS offsets of the fragment reads
    const int a_lane = (wm * 16 * MT + m) * 64 + ((g ^ ((m >> 2) & 3)) << 4);
    const int b_lane = L.a_stage + (wn * 64 + m) * 256;
    const int s_lane = L.scales + (wm * 16 * MT + m) * NB + g;

    for (;;) {
        // wave-uniform: this wave's rows and token half hold work. A tile whose upper 64
        // tokens are all past the expert's (the last, partial token tile of about half
        // the experts) leaves those waves only their copies: gate_up 636 -> 619 us at
        // config 3 (remapping the token halves so each SIMD holds one of each measured 628)
        const bool wave_rows = cur.row0 + wm * 16 * MT < p.R && cur.tok0 + wn * 64 < cur.ne;
        f32x4_t acc[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const int t_next = t + per_xcd;
        const bool more_tiles = t_next < t_end;
        G2Tile nxt = cur;
        if (more_tiles) nxt = g3_decode<MT>(t_next, row_tiles, n_slots, tpl, stl, lane);
        uint32_t sc_next[MT];
        for (int ks = 0; ks < nks; ++ks) {
            wait_vmem_all();  // this wave's copies of step ks
            __syncthreads();  // every wave's: step ks is in stage `buf`; the other stage is free
            if (ks == 0 && MODE == kModeGateUp && more_tiles) copy_ids(nxt);  // read at step nks - 1
            // the next step's copies (of this tile, or the first of the next tile), issued in
            // parts between the fragment groups (group_amask, group_bmask): issued together
            // right after the barrier, the 8 waves' 56 one-KiB copies hold every wave at issue
            // for ~1000 cycles (the memory pipeline takes ~1 KiB per 18 cycles) before its
            // first MFMA
            const bool copy_cur = ks + 1 < nks;
            const bool copy_nxt = !copy_cur && more_tiles;
            if (copy_nxt) b_rows(nxt, 1);
            // what this step copies: selected, not branched on (one scheduling region per part)
            G2Tile cd;
            cd.e = copy_cur ? cur.e : nxt.e;
            cd.ne = copy_cur ? cur.ne : nxt.ne;
            cd.p0 = copy_cur ? cur.p0 : nxt.p0;
            cd.row0 = copy_cur ? cur.row0 : nxt.row0;
            cd.tok0 = copy_cur ? cur.tok0 : nxt.tok0;
            const int cks = copy_cur ? ks + 1 : 0;
            const bool clive = copy_cur || copy_nxt;
            if (!wave_rows) copy_step(cd, cks, buf ^ 1, clive);
            if (wave_rows) {
                const lds_u8* sb = base + buf * L.stage;
                u32x4_t au[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) au[mt] = lds_ld<u32x4_t>(sb + a_lane + mt * 16 * 64);
                // the step's scale bytes: read during the previous step (the tile's scales stay
                // in LDS for the whole tile), at the tile's first step here
                if (ks == 0) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) sc_next[mt] = lds_ld<uint8_t>(base + s_lane + mt * 16 * NB);
                }
                float sf[MT];
                const bool blk_in = 4 * ks + g < NB;  // blocks past K: scale 0 (their codes are the next row's)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) sf[mt] = e8m0_scale_operand(blk_in ? sc_next[mt] : 0u);
                if (ks + 1 < nks) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        sc_next[mt] = lds_ld<uint8_t>(base + s_lane + mt * 16 * NB + 4 * (ks + 1));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    u32x4_t bf[4];
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt)
                        bf[nt] = lds_ld<u32x4_t>(sb + b_lane + nt * 16 * 256 + (((4 * g + i) ^ m) << 4));
                    copy_sel(cd, cks, buf ^ 1, group_amask(i), group_bmask(i), clive);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const bf16x8_t a = mx_cvt8(au[mt][i], sf[mt]);
#pragma unroll
                        for (int nt = 0; nt < 4; ++nt)
                            acc[mt][nt] = mfma16x16x32(a, __builtin_bit_cast(bf16x8_t, bf[nt]), acc[mt][nt]);
                    }
                    // issue order: two MFMAs, then two VALU (the next row tile's conversions),
                    // so the conversions run under the MFMAs (gate_up 611 -> 603 us at config 3)
#pragma unroll
                    for (int k = 0; k < MT * 2; ++k) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
                    }
                }
            }
            buf ^= 1;
        }

        // ---- epilogue of tile cur; its last stage (buf ^ 1) and the scale buffer are free
        // once every wave is here ----
        __syncthreads();
        if (more_tiles) copy_tile(nxt, bslot ^ 1);
        uint2 bias[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const u32x2_t b2 = lds_ld<u32x2_t>(base + L.bias + bslot * 1024 + (wm * 16 * MT + mt * 16 + 4 * g) * 2);
            bias[mt] = make_uint2(b2[0], b2[1]);
        }
        if (MODE == kModeGateUp) {
            // h of the tile: 128 tokens x TM/2 columns bf16, through the finished stage:
            // 16-byte chunk c of token row r at c ^ (r & SW) (rows of TM bytes)
            lds_u8* ht = base + (buf ^ 1) * L.stage;
            constexpr int HC = TM / 16;  // 16-byte chunks per token row (8 h columns each)
            // SW + 1 divides HC, so the XOR stays in the row
            constexpr int SW = HC % 16 == 0 ? 15 : (HC % 8 == 0 ? 7 : 3);
            static_assert(HC % 4 == 0, "the chunk swizzle needs a multiple of 4 chunks");
            // an opaque lane index: keeps the epilogue's lane-constant addresses from being
            // hoisted out of the tile loop (they would stay live through the k-steps)
            int mm = m;
            asm volatile("" : "+v"(mm));
            if (wave_rows) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const int tl = wn * 64 + nt * 16 + mm;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const float b0 = bf16_lo(bias[mt].x), b1 = bf16_hi(bias[mt].x);
                        const float b2 = bf16_lo(bias[mt].y), b3 = bf16_hi(bias[mt].y);
                        const f32x4_t c = acc[mt][nt];
                        const float h0 = swiglu(c[0] + b0, c[1] + b1, p.alpha, p.limit);
                        const float h1 = swiglu(c[2] + b2, c[3] + b3, p.alpha, p.limit);
                        // h columns (wm*16*MT + mt*16)/2 + 2g, +1: word g of chunk wm*MT + mt
                        const int chunk = wm * MT + mt;
                        lds_st<uint32_t>(ht + tl * TM + ((chunk ^ (tl & SW)) << 4) + 4 * g,
                                         f32_to_bf16(h0) | (f32_to_bf16(h1) << 16));
                    }
                }
            }
            __syncthreads();
            const int I = p.R >> 1;
            const int hc0 = cur.row0 >> 1;
            int tid = threadIdx.x;
            asm volatile("" : "+v"(tid));
#pragma unroll
            for (int u = 0; u < (kTN * HC + kThreads - 1) / kThreads; ++u) {
                const int i = tid + u * kThreads;
                if (i >= kTN * HC) break;
                const int r = i / HC, c = i % HC;
                const int q = cur.tok0 + r;
                const int col = hc0 + c * 8;
                if (q < cur.ne && col < I) {
                    const u32x4_t v = lds_ld<u32x4_t>(ht + r * TM + ((c ^ (r & SW)) << 4));
                    *(u32x4_t*)((uint16_t*)p.out + (size_t)(cur.p0 + q) * I + col) = v;
                }
            }
        } else if (wave_rows) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const int q = cur.tok0 + wn * 64 + nt * 16 + m;
                if (q >= cur.ne) continue;
                const int pp = cur.p0 + q;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int rr = cur.row0 + wm * 16 * MT + mt * 16 + 4 * g;
                    if (rr >= p.R) continue;
                    const float b0 = bf16_lo(bias[mt].x), b1 = bf16_hi(bias[mt].x);
                    const float b2 = bf16_lo(bias[mt].y), b3 = bf16_hi(bias[mt].y);
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
        if (!more_tiles) break;
        t = t_next;
        cur = nxt;
        bslot ^= 1;
    }
}

int gemm_launch(int mode, const GemvParams& p, const int32_t* tprefix, int max_slots, int n_pairs,
                hipStream_t stream) {
    static std::once_flag attr_once[kMaxDevices];
    once_per_device(attr_once, [] {
        const void* ks[] = {(const void*)k_mx_gemm<kModeGateUp>, (const void*)k_mx_gemm<kModeDown>,
                            (const void*)k_mx_gemm2<kModeGateUp>, (const void*)k_mx_gemm2<kModeDown>,
                            (const void*)k_mx_gemm3<kModeGateUp, kG3MtGateUp, kG3Waves>,
                            (const void*)k_mx_gemm3<kModeDown, kG3MtDown, kG3Waves>};
        for (const void* k : ks) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    if (p.split != 1) return set_error(PHYSLLM_MOE_EINVAL, "gemm: split must be 1");
    const long token_tiles_ub = (long)(n_pairs + kTN - 1) / kTN + max_slots;
    const int NB = p.Kdim >> 5;
    const int tm3 = 16 * (kG3Waves / 2) * (mode == kModeGateUp ? kG3MtGateUp : kG3MtDown);
    const size_t lds3 = (size_t)g3_layout(tm3, NB).tables + (size_t)max_slots * 16 + (size_t)(max_slots + 1) * 4;
    // k_mx_gemm3 copies activations, code blocks, scales and biases straight into LDS
    // in 16-byte units: all four must be 16-byte aligned
    const uintptr_t align = (uintptr_t)p.scales | (uintptr_t)p.bias | (uintptr_t)p.act | (uintptr_t)p.blocks;
    if (NB > 4 && NB <= kG3MaxNB && lds3 <= 160 * 1024 && (align & 15) == 0) {
        // LDS-staged form: at least two k-steps; the scale and bias blocks copied in 16-byte units
        // tile heights: 384 rows for gate_up (2I = 5760 = 15 tiles at GPT-OSS shape), 320 for
        // down (H = 2880 = 9 tiles)
        const long tiles_ub = (long)((p.R + tm3 - 1) / tm3) * token_tiles_ub;
        if (tiles_ub > 0x7fffffffL) return set_error(PHYSLLM_MOE_EINVAL, "gemm: too many tiles");
        const unsigned grid = (unsigned)((device_cu_count() + 7) & ~7);
        if (mode == kModeGateUp)
            hipLaunchKernelGGL((k_mx_gemm3<kModeGateUp, kG3MtGateUp, kG3Waves>), dim3(grid), dim3(64 * kG3Waves), lds3,
                               stream, p, tprefix, max_slots);
        else
            hipLaunchKernelGGL((k_mx_gemm3<kModeDown, kG3MtDown, kG3Waves>), dim3(grid), dim3(64 * kG3Waves), lds3,
                               stream, p, tprefix, max_slots);
        return check_launch(mode == kModeGateUp ? "gate_up gemm" : "down gemm");
    }
    if ((p.Kdim >> 5) <= kG2MaxNB) {
        // wide tiles, persistent: one workgroup per CU (a multiple of 8, one range of
        // tiles per XCD); the tile count is only known on the device
        const long tiles_ub = (long)((p.R + kG2TM - 1) / kG2TM) * token_tiles_ub;
        if (tiles_ub > 0x7fffffffL) return set_error(PHYSLLM_MOE_EINVAL, "gemm: too many tiles");
        const int n_cu = device_cu_count();
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
