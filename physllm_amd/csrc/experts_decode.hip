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

constexpr int kGemvThreads = 256;  // 4 waves, each one 16-row weight tile at a time
constexpr int kGemvNit = 23;       // k-steps of 4 MX blocks held in registers: 92 blocks = 2944 elements
constexpr int kPassTok = 8;        // tokens staged in LDS per pass
constexpr int kGemvSclSlice = 128 * 16;  // bytes of a wave's scale slice: 16 x NB <= 1472, then unread padding
constexpr int kStageU = 4;         // 16-byte activation loads in flight per thread while staging
constexpr int kMaxScaleBlocks = 256;  // K <= 8192: a tile's scales (16 x NB bytes) fit a wave's LDS slice

// Stages activation rows for tokens [tb, tb + ntok) and MX blocks [sb0, sb1) into
// LDS as xs[r][c] (c in 16-byte units, row stride su = 4 * (sb1 - sb0) + 1: the
// one-unit pad spreads the 16 token rows of a B-fragment read over the banks).
template <int MODE>
__device__ __forceinline__ void gemv_stage(const GemvParams& p, uint4* xs, int p0, int tb, int ntok, int sb0,
                                           int sb1, int su) {
    const int cu = (sb1 - sb0) * 4;  // 16-byte units per row in this segment
    const int units = ntok * cu;
    for (int i0 = threadIdx.x; i0 < units; i0 += kGemvThreads * kStageU) {
        uint4 v[kStageU];
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
            const int i = i0 + u * kGemvThreads;
            v[u] = make_uint4(0, 0, 0, 0);
            if (i < units) {
                const int r = i / cu, c = i - r * cu;
                const int q = tb + r;
                const size_t arow = (MODE == kModeGateUp) ? (size_t)(p.perm[p0 + q] / p.top_k) : (size_t)(p0 + q);
                v[u] = ((const uint4*)(p.act + arow * (size_t)p.Kdim))[sb0 * 4 + c];
            }
        }
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
            const int i = i0 + u * kGemvThreads;
            if (i < units) {
                const int r = i / cu, c = i - r * cu;
                xs[r * su + c] = v[u];
            }
        }
    }
}

// Generic form (any K up to 8192, several row-tile sets per group). Grid: x =
// groups of `rt` row-tile sets (a set = 4 waves x 16 rows), y = expert work slot,
// z = K split. Per row tile, a wave
//   1. fetches the tile's 16 x NB scale bytes with at most 4 wide loads into its
//      own LDS slice (one 16-byte load per lane, not one byte load per k-step:
//      the memory pipeline is bound by load instructions, not bytes);
//   2. loads its 16 rows over the split's K range into registers (up to 23
//      k-steps, 16 bytes per lane each = 16 rows x 64 contiguous bytes per wave;
//      longer K ranges run in segments);
//   3. runs every 8-token pass of the expert's tokens against the registers:
//      heavy experts cost extra activation reads and MFMA issue, not extra HBM
//      traffic.
// The activations of a pass are staged once per group in LDS and reused by all
// of the group's row tiles when the expert has at most 8 tokens. Four
// accumulators break the MFMA dependency chain; they are summed in a fixed order.
template <int MODE>
__global__ __launch_bounds__(kGemvThreads) void k_mx_gemv_generic(GemvParams p) {
    extern __shared__ uint4 lds[];
    const int4 si = p.slots[blockIdx.y];  // {expert, tokens, first sorted position, 0}
    const int e = si.x, ne = si.y, p0 = si.z;
    if (ne <= 0) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int NB = p.Kdim >> 5;
    const int split = blockIdx.z;
    const int per = (NB + p.split - 1) / p.split;
    const int kb0 = min(NB, split * per);
    const int kb1 = min(NB, kb0 + per);
    const int seg_blocks = 4 * kGemvNit;
    const int nseg = (kb1 - kb0 + seg_blocks - 1) / seg_blocks;
    const int su = 4 * min(kb1 - kb0, seg_blocks) + 1;
    const int npass = (ne + kPassTok - 1) / kPassTok;
    const bool restage = npass > 1 || nseg > 1;  // else: one staging serves every tile

    uint8_t* scl = (uint8_t*)lds + wave * 16 * NB;           // this wave's tile scales [16][NB]
    uint4* xs = lds + (4 * 16 * NB) / 16;                     // activations [kPassTok][su]
    const int sc_units = NB;  // 16 * NB bytes = NB 16-byte units

    uint4 wq[kGemvNit];
    for (int it = 0; it < p.rt; ++it) {
        const int r0 = ((blockIdx.x * p.rt + it) * (kGemvThreads / 64) + wave) * 16;
        // the group stops together (its first tile past the end: the later ones are
        // too); a wave whose own tile is past R (R not a multiple of 64) keeps staging
        // its share of the activations and meeting the barriers, on tile 0's rows,
        // and stores nothing
        if (r0 - 16 * wave >= p.R) break;
        const bool live = r0 < p.R;  // wave-uniform
        const size_t row0 = (size_t)e * p.R + (live ? r0 : 0);
        const uint4* wrow = (const uint4*)(p.blocks + (row0 + m) * (size_t)(p.Kdim >> 1));
        const uint4* scg = (const uint4*)(p.scales + row0 * (size_t)NB);
        uint4 sv[kMaxScaleBlocks / 64];
#pragma unroll
        for (int u = 0; u < kMaxScaleBlocks / 64; ++u)
            sv[u] = (lane + 64 * u < sc_units) ? scg[lane + 64 * u] : make_uint4(0, 0, 0, 0);
        auto load_w = [&](int sb0, int sb1) {
#pragma unroll
            for (int j = 0; j < kGemvNit; ++j) {
                const int blk = sb0 + 4 * j + g;
                wq[j] = blk < sb1 ? wrow[blk] : make_uint4(0, 0, 0, 0);
            }
        };
        if (nseg == 1) load_w(kb0, kb1);
#pragma unroll
        for (int u = 0; u < kMaxScaleBlocks / 64; ++u)
            if (lane + 64 * u < sc_units) ((uint4*)scl)[lane + 64 * u] = sv[u];

        for (int tb = 0; tb < ne; tb += kPassTok) {
            const int ntok = min(kPassTok, ne - tb);
            const bool tv = m < ntok;
            f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;
            for (int sg = 0; sg < nseg; ++sg) {
                const int sb0 = kb0 + sg * seg_blocks;
                const int sb1 = min(kb1, sb0 + seg_blocks);
                if (nseg > 1) load_w(sb0, sb1);
                if (restage || it == 0) {
                    // every wave of the group reaches this point together (those whose
                    // tile is past R as well): the staging below is shared by all four
                    __syncthreads();  // previous pass/segment finished reading xs
                    gemv_stage<MODE>(p, xs, p0, tb, ntok, sb0, sb1, su);
                    __syncthreads();
                }
                const uint4* xl = xs + m * su;
                const uint8_t* sl = scl + m * NB;
#pragma unroll
                for (int j = 0; j < kGemvNit; ++j) {
                    const int lb = 4 * j + g;  // block index within the segment
                    if (sb0 + 4 * j < sb1) {   // wave-uniform
                        const bool bv = sb0 + lb < sb1;
                        uint32_t sj = sl[sb0 + (bv ? lb : 0)];
                        // decode inside the pass loop: an opaque no-op on the scale keeps the
                        // compiler from hoisting 23 x 16 VGPRs of converted fragments
                        asm volatile("" : "+v"(sj));
                        const float sf = e8m0_scale_operand(sj);
                        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0, x2 = x0, x3 = x0;
                        if (tv && bv) {
                            x0 = xl[lb * 4 + 0];
                            x1 = xl[lb * 4 + 1];
                            x2 = xl[lb * 4 + 2];
                            x3 = xl[lb * 4 + 3];
                        }
                        acc0 = mfma16x16x32(mx_cvt8(wq[j].x, sf), as_bf16x8(x0), acc0);
                        acc1 = mfma16x16x32(mx_cvt8(wq[j].y, sf), as_bf16x8(x1), acc1);
                        acc2 = mfma16x16x32(mx_cvt8(wq[j].z, sf), as_bf16x8(x2), acc2);
                        acc3 = mfma16x16x32(mx_cvt8(wq[j].w, sf), as_bf16x8(x3), acc3);
                    }
                }
            }
            if (!tv || !live) continue;
            const f32x4_t acc = (acc0 + acc1) + (acc2 + acc3);
            const int pp = p0 + tb + m;  // sorted position of this lane's token
            const int rr = r0 + 4 * g;
            float bsum[4] = {0.f, 0.f, 0.f, 0.f};
            if (p.bias && split == 0) {
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
                float* ybase = (float*)p.out + (size_t)split * p.n_pairs * p.R;
                *(float4*)(ybase + (size_t)pp * p.R + rr) = y;
            }
        }
    }
}

// Buffer resource (V#) for raw buffer loads on gfx9-family GPUs: `bytes` of
// range-checked memory from `base`; loads past the range return zeros, so tile
// edges need no clamped (per-load) addresses and the k-step of a load is an
// immediate offset.
// Fast form for K ranges of at most 92 MX blocks (2944 elements: GPT-OSS H = I =
// 2880 = 90 blocks), one 16-row tile per wave, loads in this order:
//   1. the expert slot and the first pass's token rows (scalar loads of the
//      sorted pair ids; none at batch 1, where every pair reads row 0);
//   2. the activation units this thread stages (NS 16-byte loads) and the tile's
//      scales (two 16-byte loads per lane);
//   3. the wave's 23 weight stripes (16 bytes per lane each: 16 rows x 64
//      contiguous bytes per wave).
// Vector loads retire in issue order, so staging the small loads to LDS (one
// barrier) waits only for them, and the 23 k-steps then run as the stripes
// arrive instead of after the last one. The pair ids come in as a restrict
// kernel argument, so they are read with scalar loads, which do not wait behind
// the vector loads. Experts with more than 8 tokens run further passes against
// the same registers.
template <int MODE, int NS>
__global__ __launch_bounds__(kGemvThreads) void k_mx_gemv(GemvParams p, const int32_t* __restrict__ perm) {
    extern __shared__ uint4 lds[];
    const int4 si = p.slots[blockIdx.y];  // {expert, tokens, first sorted position, 0}
    const int e = si.x, ne = si.y, p0 = si.z;
    if (ne <= 0) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int NB = p.Kdim >> 5;
    const int split = blockIdx.z;
    const int per = (NB + p.split - 1) / p.split;
    const int kb0 = min(NB, split * per);
    const int nblk = min(NB, kb0 + per) - kb0;  // <= 92
    const int cu = nblk * 4;                    // 16-byte activation units per token row
    const int su = cu + 1;                      // LDS row stride (one-unit pad)
    const int r0 = (blockIdx.x * (kGemvThreads / 64) + wave) * 16;
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;   // one expert's codes
    const uint32_t exp_s = (uint32_t)p.R * (uint32_t)NB;  // one expert's scales

    uint8_t* scl = (uint8_t*)lds + wave * kGemvSclSlice;  // this wave's tile scales [16][NB <= 92]
    uint4* xs = lds + (kGemvThreads / 64) * kGemvSclSlice / 16;  // activations [kPassTok][su]
    uint4* xz = xs + kPassTok * (4 * per + 1);                   // 64 zero bytes (after the launch's rows)
    if (threadIdx.x < 4) xz[threadIdx.x] = make_uint4(0, 0, 0, 0);  // (ordered by the barrier below)

    const __amdgpu_buffer_rsrc_t ract = make_rsrc(p.act, (uint32_t)p.act_rows * (uint32_t)p.Kdim * 2u);
    auto stage_load = [&](int tb, u32x4_t (&v)[NS]) {
        // lane r < kPassTok holds the activation row of pass row r (scalar loads of
        // the sorted pair ids, then one register); units fetch theirs by shuffle
        int rowid = 0;
#pragma unroll
        for (int r = 0; r < kPassTok; ++r) {
            const int q = min(tb + r, ne - 1);
            const int id = (MODE == kModeGateUp) ? (p.act_rows == 1 ? 0 : perm[p0 + q] / p.top_k) : p0 + q;
            rowid = (lane == r) ? id : rowid;
        }
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int i = threadIdx.x + u * kGemvThreads;
            const int r = i / cu, c = i - r * cu;
            const int row = __shfl(rowid, r & (kPassTok - 1), 64);
            const uint32_t off = (uint32_t)row * (uint32_t)(p.Kdim * 2) + (uint32_t)(kb0 * 4 + c) * 16u;
            v[u] = buf_load16(ract, off, 0);
        }
    };
    auto stage_store = [&](int ntok, const u32x4_t (&v)[NS]) {
        const int units = ntok * cu;
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int i = threadIdx.x + u * kGemvThreads;
            if (i < units) {
                const int r = i / cu, c = i - r * cu;
                ((u32x4_t*)xs)[r * su + c] = v[u];
            }
        }
    };
    int ntok = min(kPassTok, ne);
    u32x4_t wq[kGemvNit];
    {
        // ---- activations of pass 0 and the tile's scales, then the weights (rows past R read zeros)
        u32x4_t xv[NS];
        stage_load(0, xv);
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales + (size_t)e * exp_s, exp_s);
        const uint32_t soff = (uint32_t)r0 * NB + lane * 16u;  // 16 rows x NB bytes, contiguous
        const u32x4_t sv0 = buf_load16(rs, soff, 0);
        const u32x4_t sv1 = buf_load16(rs, soff, 1024);
        __builtin_amdgcn_sched_barrier(0);
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.blocks + (size_t)e * exp_w, exp_w);
        const uint32_t woff = (uint32_t)(r0 + m) * row_bytes + (uint32_t)(kb0 + g) * 16u;
        // k-steps past this split's K range load from past the buffer's end (zeros,
        // no memory traffic): straight-line loads, no branch for a load to sink into
#pragma unroll
        for (int j = 0; j < kGemvNit; ++j) wq[j] = buf_load16(rw, 4 * j < nblk ? woff : kRsrcPast, 64 * j);
        __builtin_amdgcn_sched_barrier(0);
        // every lane stores both scale units (the slice holds 128; units past the
        // tile's 16 x NB bytes are never read): a store under `lane < NB` would let
        // the compiler sink its load into the branch, behind the weight stripes
        ((u32x4_t*)scl)[lane] = sv0;
        ((u32x4_t*)scl)[lane + 64] = sv1;
        stage_store(ntok, xv);
    }
    __syncthreads();

    const bool row_ok = r0 < p.R;
    // one pass: the 23 k-steps against the staged tokens tb..tb+ntok-1, then the epilogue
    auto run_pass = [&](int tb) {
        // lane's column of the B fragment at block 4j+g; lanes past the pass's tokens
        // read a valid row (an MFMA output column depends only on its own B column,
        // and those columns are not stored)
        const uint4* xl = xs + min(m, ntok - 1) * su + 4 * g;
        const f32x4_t acc = mx_tile_steps<kGemvNit>(wq, scl + m * NB + kb0 + g, xl, xz, nblk, g);
        const bool tv = m < ntok;
        if (!row_ok || !tv) return;
        const int pp = p0 + tb + m;  // sorted position of this lane's token
        const int rr = r0 + 4 * g;
        float bsum[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias && split == 0) {
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
            float* ybase = (float*)p.out + (size_t)split * p.n_pairs * p.R;
            *(float4*)(ybase + (size_t)pp * p.R + rr) = y;
        }
    };
    // the first pass outside the loop: its k-steps wait for each stripe as it
    // arrives (inside a loop the first use of the stripes waits for all of them)
    run_pass(0);
    for (int tb = kPassTok; tb < ne; tb += kPassTok) {
        ntok = min(kPassTok, ne - tb);
        u32x4_t xn[NS];
        stage_load(tb, xn);
        __syncthreads();  // every wave finished reading the previous pass
        stage_store(ntok, xn);
        __syncthreads();
        run_pass(tb);
    }
}

// ---------------------------------------------------------------------------
// Streaming form (decode with many touched experts): persistent, one 4-wave
// workgroup per CU, so each SIMD runs a single wave.
//
// A read-only model of this loop (persistent groups, a 23-stripe register ring
// per wave, the k-steps' LDS reads, conversions and MFMAs) streams 1.1 GB at
// 6.2 TB/s with 4 waves per CU, 5.75 with 8 and 5.1-5.3 with 12 or 16: a second
// wave on a SIMD does not hide the k-step latency, it competes with the first
// for issue slots, LDS and the load-return path.
//
// Work items are (pass entry, 64-row set) in entry-major order, so the row sets of
// one 16-token chunk of one expert are consecutive. Workgroup b takes one
// contiguous range of items (all ranges within one item of each other), and the
// ranges of the workgroups of one XCD (b % 8) are consecutive: the chunks of one
// expert run on one XCD at about the same time and meet in its L2.
//  - The 16 activation rows of the current entry stay in LDS. A workgroup copies
//    them in (direct copies into LDS, no registers) at its start and again only
//    when its range crosses into the next entry, about once per workgroup. Unit c
//    of staged row q sits at unit c ^ q, so the 16 token rows of an MFMA fragment
//    read hit 16 different bank groups.
//  - Each wave keeps its 16 rows x 23 k-steps in a circular register buffer:
//    right after k-step j of the current item is decoded, register j is
//    reloaded with k-step j of the next item (23 loads in flight per wave).
//  - The next item's scales and biases load at the start of the current item,
//    ahead of its refills; the scales go to a wave-private LDS slice.
//  - Outputs go to a wave-private LDS ring, written to memory in bursts (ring
//    full, and at the start of the workgroup's last item). A store sits in the
//    in-order vector-memory counter: every load issued after it counts as
//    complete only once the store is acknowledged, which under the read stream
//    takes longer than an item. Per-item stores cost 12% at the GPT-OSS-120B
//    shape (decode batch 256).
// ---------------------------------------------------------------------------
constexpr int kStreamWaves = 4;
constexpr int kStreamThreads = 64 * kStreamWaves;
constexpr int kStreamSetRows = 16 * kStreamWaves;                  // weight rows per item
constexpr int kStreamMaxNB = 4 * kGemvNit;                         // K <= 2944: the 23 k-steps of a tile
constexpr int kStreamActUnits = 384;                               // 16-byte units per staged row (>= K/8)
constexpr int kStreamActBytes = kPassRows * kStreamActUnits * 16;  // 96 KiB
constexpr int kStreamSlice = 2048;                                 // a wave's scale slice: 16 x NB bytes
constexpr int kStreamOutWave = 12 * 1024;                          // a wave's output ring
constexpr int kStreamLds = kStreamActBytes + 2 * kStreamWaves * kStreamSlice + kStreamWaves * kStreamOutWave;
static_assert(kStreamLds <= 160 * 1024, "streaming GEMV LDS");
static_assert(4 * kStreamMaxNB <= kStreamActUnits && 16 * kStreamMaxNB <= kStreamSlice, "streaming GEMV tiles");

// The streaming kernel's work split: workgroup rix (of G, XCD-grouped) takes items
// f in [f0, f1) of entries ebase + f / sets (row set f % sets), given the pass table's
// entry count npass and its nm multi-chunk entries. Returns {ebase, f0, f1}.
__device__ __forceinline__ int3 stream_range(int npass, int nm, int G, int rix, int sets) {
    int ebase, f0, f1;
    // an entry of an expert with several chunks gets P workgroups of its own, each
    // a 1/P share of its row sets; rix = part * nm + entry, so the chunks of one
    // expert (adjacent entries) run on one XCD, start together and read the same
    // rows at the same time (one HBM read, the rest L2 hits). The single-chunk
    // entries share the other workgroups in contiguous ranges.
    int P = (nm > 0 && npass <= G) ? max(1, (G + npass / 2) / npass) : 0;
    if (P > 0) P = min(min(P, G / nm), sets);
    if (P > 0 && npass > nm && G - P * nm < 1) P = (G - 1) / nm;
    const int M = P * nm;
    if (rix < M) {
        const int part = rix / nm;
        ebase = rix - part * nm;
        f0 = part * sets / P;
        f1 = (part + 1) * sets / P;
    } else {
        const int e0 = P > 0 ? nm : 0;
        const int total = (npass - e0) * sets, g = G - M, r = rix - M;
        ebase = e0;
        f0 = (int)((int64_t)total * r / g);
        f1 = (int)((int64_t)total * (r + 1) / g);
    }
    return make_int3(ebase, f0, f1);
}

template <int MODE>
__global__ __launch_bounds__(kStreamThreads) void k_mx_gemv_stream(GemvParams p, const int4* __restrict__ passes,
                                                                   const int32_t* __restrict__ perm,
                                                                   const int32_t* __restrict__ n_passes,
                                                                   void* __restrict__ out) {
    extern __shared__ uint4 lds[];
    const int NB = p.Kdim >> 5;       // <= kStreamMaxNB (launcher)
    const int ku = p.Kdim >> 3;       // 16-byte activation units per row, <= kStreamActUnits
    const int sets = (p.R + kStreamSetRows - 1) / kStreamSetRows;
    const int G = (int)gridDim.x;     // a multiple of 8
    const int rix = (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3);
    // this workgroup's items f in [f0, f1): entry ebase + f / sets, row set f % sets
    const int npass = n_passes[0], nm = n_passes[1];
    const int3 rg = stream_range(npass, nm, G, rix, sets);
    const int ebase = rg.x, f0 = rg.y, f1 = rg.z;
    if (f0 >= f1) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & (kStreamWaves - 1);
    const int lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;
    const uint32_t exp_s = (uint32_t)p.R * (uint32_t)NB;
    const uint32_t exp_b = p.bias ? (uint32_t)p.R * 2u : 0u;  // empty range: the bias reads as zero
    const uint32_t act_bytes = (uint32_t)p.act_rows * (uint32_t)p.Kdim * 2u;
    constexpr uint32_t kPast = 0x80000000u;  // an offset past every range: zeros
    lds_u8* act = (lds_u8*)lds;
    uint8_t* slice0 = (uint8_t*)lds + kStreamActBytes + wave * kStreamSlice;  // [2 buffers][4 waves][kStreamSlice]
    // the refills of the last item: the down launch's first item for this workgroup index
    // (stream_range with the down launch's row sets), or nothing (an empty range)
    __amdgpu_buffer_rsrc_t pf_rs = make_rsrc(p.blocks, 0u);
    uint32_t pf_off = 0;
    if (MODE == kModeGateUp && p.pf_blocks) {
        const int sets_d = (p.pf_R + kStreamSetRows - 1) / kStreamSetRows;
        const int3 rd = stream_range(npass, nm, G, rix, sets_d);
        if (rd.y < rd.z) {
            const int u = rd.x + rd.y / sets_d, sd = rd.y - (rd.y / sets_d) * sets_d;
            const int xd = __builtin_amdgcn_readfirstlane(passes[u].x);
            const uint32_t rb_d = (uint32_t)(p.pf_Kdim >> 1);
            const uint32_t ew_d = (uint32_t)p.pf_R * rb_d;
            pf_rs = make_rsrc(p.pf_blocks + (size_t)xd * ew_d, ew_d);
            pf_off = (uint32_t)(sd * kStreamSetRows + 16 * wave + m) * rb_d + (uint32_t)g * 16u;
        }
    }
    constexpr int kSliceBuf = kStreamWaves * kStreamSlice;

    // the 16 activation rows of pass entry pe into LDS: wave w copies rows 4w..4w+3,
    // 6 copies of 64 units per row (units past K and rows past the entry's tokens
    // read zeros)
    auto stage_act = [&](int4 pe) {
        const u32x4_t ra = rsrc_words(p.act, act_bytes);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int q = 4 * wave + rr;
            const int row = q < pe.y ? ((MODE == kModeGateUp) ? perm[pe.z + q] / p.top_k : pe.z + q) : -1;
#pragma unroll
            for (int k = 0; k < kStreamActUnits / 64; ++k) {
                const int c = (64 * k + lane) ^ q;  // source unit of destination unit 64k + lane
                const uint32_t voff =
                    (row >= 0 && c < ku) ? (uint32_t)row * (uint32_t)(p.Kdim * 2) + (uint32_t)c * 16u : kPast;
                dma16(ra, act + (q * kStreamActUnits + 64 * k) * 16, voff);
            }
        }
    };
    u32x4_t sv0, sv1;
    uint2 bnx;
    auto side_load = [&](int e, int r0, bool live) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales + (size_t)e * exp_s, live ? exp_s : 0u);
        sv0 = buf_load16(rs, (uint32_t)r0 * NB + lane * 16u, 0);
        sv1 = buf_load16(rs, (uint32_t)r0 * NB + lane * 16u, 1024);
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.bias + (size_t)e * p.R, live ? exp_b : 0u);
        const u32x2_t b2 = __builtin_amdgcn_raw_buffer_load_b64(rb, (uint32_t)(r0 + 4 * g) * 2u, 0, 0);
        bnx = make_uint2(b2[0], b2[1]);
    };
    // wave-private slice, no barrier. Every lane stores both units (units past the
    // tile's 16 x NB bytes are never read): a store under a lane test lets the
    // compiler sink the scale load into that branch, behind the item's stripes,
    // and wait for all of them.
    auto scale_store = [&](int b) {
        uint8_t* sb = slice0 + b * kSliceBuf;
        ((u32x4_t*)sb)[lane] = sv0;
        ((u32x4_t*)sb)[lane + 64] = sv1;
    };

    // a pass-table entry, wave-uniform
    auto entry = [&](int u) -> int4 {
        const int4 v = passes[u];
        return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                         __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
    };
    auto item_at = [&](int f) -> int2 {  // {entry, set}
        const int u = f / sets;
        return make_int2(ebase + u, f - u * sets);
    };
    // this wave's output ring: per item and lane 4 bytes (two bf16 of h) or 16 (four
    // fp32 of y), from item fa on; flush(fb) writes items fa .. fb - 1 to memory
    constexpr int kOutLane = (MODE == kModeGateUp) ? 4 : 16;
    constexpr int kOutCap = kStreamOutWave / (64 * kOutLane);
    uint8_t* oring =
        (uint8_t*)lds + kStreamActBytes + 2 * kStreamWaves * kStreamSlice + wave * kStreamOutWave + lane * kOutLane;
    int fa = f0;  // first staged item
    auto flush = [&](int fb) {
        for (int ff = fa; ff < fb; ++ff) {
            const int2 it2 = item_at(ff);
            const int e2 = it2.x, s2 = it2.y;
            const int4 q2 = entry(e2);
            const int r2 = s2 * kStreamSetRows + 16 * wave;
            const uint8_t* src = oring + (ff - fa) * (64 * kOutLane);
            if (r2 < p.R && m < q2.y) {
                const int pp = q2.z + m;
                const int rr = r2 + 4 * g;
                if (MODE == kModeGateUp) {
                    uint32_t* hout = (uint32_t*)((uint16_t*)out + (size_t)pp * (p.R >> 1) + (rr >> 1));
                    *hout = *(const uint32_t*)src;
                } else {
                    *(float4*)((float*)out + (size_t)pp * p.R + rr) = *(const float4*)src;
                }
            }
        }
        fa = fb;
    };
    const int2 it0 = item_at(f0);
    int en = it0.x, s = it0.y;
    int4 pe = entry(en);
    stage_act(pe);
    side_load(pe.x, s * kStreamSetRows + 16 * wave, true);
    u32x4_t wq[kGemvNit];
    {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.blocks + (size_t)pe.x * exp_w, exp_w);
        const uint32_t voff = (uint32_t)(s * kStreamSetRows + 16 * wave + m) * row_bytes + (uint32_t)g * 16u;
#pragma unroll
        for (int j = 0; j < kGemvNit; ++j) wq[j] = buf_load16(rw, voff, 64 * j);
    }
    uint2 bcur = bnx;
    scale_store(0);
    // the activation copies (issued first, and not counted by the compiler's waits):
    // at most the 2 scale loads, the bias load and the 23 stripes may still be in flight
    asm volatile("s_waitcnt vmcnt(26)" ::: "memory");
    __syncthreads();
    int buf = 0;
    // this lane's activation fragment i of k-step j: unit 16j + ((4g + i) ^ m) of row m
    const uint4* xrow = (const uint4*)lds + m * kStreamActUnits;
    const int xo0 = (4 * g + 0) ^ m, xo1 = (4 * g + 1) ^ m, xo2 = (4 * g + 2) ^ m, xo3 = (4 * g + 3) ^ m;

    for (int f = f0; f < f1; ++f) {
        const bool has_next = f + 1 < f1;
        if (!has_next) flush(f);  // the staged outputs go out while the last item computes
        const int2 itn = has_next ? item_at(f + 1) : make_int2(en, s);
        const int en_n = itn.x, s_n = itn.y;
        const int4 pe_n = (has_next && en_n != en) ? entry(en_n) : pe;
        const int r0 = s * kStreamSetRows + 16 * wave;
        const int r0_n = s_n * kStreamSetRows + 16 * wave;
        side_load(pe_n.x, r0_n, has_next);
        const __amdgpu_buffer_rsrc_t rsrc = has_next ? make_rsrc(p.blocks + (size_t)pe_n.x * exp_w, exp_w) : pf_rs;
        const uint32_t svoff = has_next ? (uint32_t)(r0_n + m) * row_bytes + (uint32_t)g * 16u : pf_off;
        const uint8_t* sl = slice0 + buf * kSliceBuf + m * NB + g;
        f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;
        // the scale byte of k-step j is read two steps ahead (its LDS latency would
        // otherwise stall every step). A lane whose block is past K (the last step of
        // a K that is not a multiple of 128) takes the scale operand 0.0: its codes
        // (the next row's) decode to zeros, and its staged activations past K are
        // zeros too, so it adds exactly 0 without a per-step branch
        uint32_t sp0 = sl[0], sp1 = sl[4];
#pragma unroll
        for (int j = 0; j < kGemvNit; ++j) {
            if (4 * j < NB) {  // wave-uniform
                uint32_t sj = (j & 1) ? sp1 : sp0;
                if (4 * j + 8 < NB) {  // wave-uniform: the read for step j + 2
                    if (j & 1) sp1 = sl[4 * j + 8];
                    else sp0 = sl[4 * j + 8];
                }
                sj = 4 * j + g < NB ? sj : 0u;
                asm volatile("" : "+v"(sj));
                const float sf = e8m0_scale_operand(sj);
                const u32x4_t q = wq[j];
                const uint4 x0 = xrow[16 * j + xo0], x1 = xrow[16 * j + xo1], x2 = xrow[16 * j + xo2],
                            x3 = xrow[16 * j + xo3];
                acc0 = mfma16x16x32(mx_cvt8(q[0], sf), as_bf16x8(x0), acc0);
                acc1 = mfma16x16x32(mx_cvt8(q[1], sf), as_bf16x8(x1), acc1);
                acc2 = mfma16x16x32(mx_cvt8(q[2], sf), as_bf16x8(x2), acc2);
                acc3 = mfma16x16x32(mx_cvt8(q[3], sf), as_bf16x8(x3), acc3);
            }
            wq[j] = buf_load16(rsrc, svoff, 64 * j);
            __builtin_amdgcn_sched_barrier(0);  // one refill per k-step
        }
        {
            const f32x4_t acc = (acc0 + acc1) + (acc2 + acc3);
            const float b0 = bf16_lo(bcur.x), b1 = bf16_hi(bcur.x), b2 = bf16_lo(bcur.y), b3 = bf16_hi(bcur.y);
            uint32_t hv = 0;
            float4 y;
            if (MODE == kModeGateUp) {
                const float h0 = swiglu(acc[0] + b0, acc[1] + b1, p.alpha, p.limit);
                const float h1 = swiglu(acc[2] + b2, acc[3] + b3, p.alpha, p.limit);
                hv = f32_to_bf16(h0) | (f32_to_bf16(h1) << 16);
            } else {
                y.x = acc[0] + b0;
                y.y = acc[1] + b1;
                y.z = acc[2] + b2;
                y.w = acc[3] + b3;
            }
            if (has_next) {
                uint8_t* dst = oring + (f - fa) * (64 * kOutLane);
                if (MODE == kModeGateUp) *(uint32_t*)dst = hv;
                else *(float4*)dst = y;
            } else if (r0 < p.R && m < pe.y) {
                const int pp = pe.z + m;
                const int rr = r0 + 4 * g;
                if (MODE == kModeGateUp) *(uint32_t*)((uint16_t*)out + (size_t)pp * (p.R >> 1) + (rr >> 1)) = hv;
                else *(float4*)((float*)out + (size_t)pp * p.R + rr) = y;
            }
        }
        if (!has_next) break;
        if (f + 1 - fa == kOutCap) flush(f + 1);
        buf ^= 1;
        scale_store(buf);
        bcur = bnx;
        if (en_n != en) {
            // the next item starts a new pass entry: its activation rows replace these
            __syncthreads();  // every wave has finished reading the current rows
            stage_act(pe_n);
            wait_vmem_all();
            __syncthreads();
        }
        en = en_n;
        s = s_n;
        pe = pe_n;
    }
}

// out[t, d] = bf16( sum_j w[t,j] * y[pos[t*k+j], d] ), fp32 fma in k order
// (kernels/moe_combine.hip:16-20, batched). With a K-split down projection, y is
// the sum of the split partials, added in split order first. Each lane handles 4
// consecutive d.
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ y, const int32_t* __restrict__ pos,
                                                 const float* __restrict__ wts, uint16_t* out, const uint16_t* res,
                                                 int H, int K, int nsplit, size_t split_stride) {
    const int t = blockIdx.y;
    const int d4 = blockIdx.x * 256 + threadIdx.x;
    if (d4 * 4 >= H) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < K; ++j) {
        const int q = pos[(size_t)t * K + j];
        const float w = wts[(size_t)t * K + j];
        float4 v = ((const float4*)(y + (size_t)q * H))[d4];
        for (int sp = 1; sp < nsplit; ++sp) {
            const float4 u = ((const float4*)(y + sp * split_stride + (size_t)q * H))[d4];
            v.x += u.x;
            v.y += u.y;
            v.z += u.z;
            v.w += u.w;
        }
        acc.x = __builtin_fmaf(w, v.x, acc.x);
        acc.y = __builtin_fmaf(w, v.y, acc.y);
        acc.z = __builtin_fmaf(w, v.z, acc.z);
        acc.w = __builtin_fmaf(w, v.w, acc.w);
    }
    uint2 o;
    o.x = f32_to_bf16(acc.x) | (f32_to_bf16(acc.y) << 16);
    o.y = f32_to_bf16(acc.z) | (f32_to_bf16(acc.w) << 16);
    if (res) {
        // the layer's output is a bf16 tensor first, then the residual add
        // (crates/llm-core/src/moe.rs:310-311, kernels/residual_add.hip:9)
        const uint2 r = ((const uint2*)(res + (size_t)t * H))[d4];
        o.x = f32_to_bf16(bf16_lo(o.x) + bf16_lo(r.x)) | (f32_to_bf16(bf16_hi(o.x) + bf16_hi(r.x)) << 16);
        o.y = f32_to_bf16(bf16_lo(o.y) + bf16_lo(r.y)) | (f32_to_bf16(bf16_hi(o.y) + bf16_hi(r.y)) << 16);
    }
    ((uint2*)(out + (size_t)t * H))[d4] = o;
}

// ---------------------------------------------------------------------------
// Batch 1: the down projection of all k selected experts and the weighted
// combine in one launch. Workgroup b owns output rows 16 * kD1Rt * b ..; wave
// w = s * kD1Rt + t computes the 16-row tile t of slot s exactly as k_mx_gemv
// does (the same stripes, k-steps, four accumulators and their sum, + bias), and
// the workgroup then combines its rows over the k slots in k order through LDS
// (out = bf16(sum_j w_j * y_j), then + residual): the combine launch and the
// round trip of y through HBM disappear. K <= kD1MaxK, K range <= 92 MX blocks.
// ---------------------------------------------------------------------------
constexpr int kD1Rt = 1;     // 16-row tiles per slot per workgroup
constexpr int kD1MaxK = 4;   // slots (selected experts) the workgroup holds (8 waves at most)
constexpr int kD1MaxNB = 92;

__global__ __launch_bounds__(64 * kD1Rt * kD1MaxK) void k_mx_down1(GemvParams p, const float* __restrict__ wts,
                                                                  const int32_t* __restrict__ pos,
                                                                  uint16_t* out, const uint16_t* res, int K) {
    extern __shared__ uint4 lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int s = wave / kD1Rt, t = wave - s * kD1Rt;
    const int NB = p.Kdim >> 5;
    const int cu = NB * 4, su = cu + 1;  // activation units per row, LDS row stride
    uint8_t* scl = (uint8_t*)lds + wave * kGemvSclSlice;          // this wave's tile scales [16][NB]
    uint4* xs = lds + (K * kD1Rt) * kGemvSclSlice / 16;          // activation rows [K][su]
    float* ys = (float*)(xs + K * su);                           // y [K][16 * kD1Rt]
    uint4* xz = (uint4*)(ys + K * 16 * kD1Rt);                   // 64 zero bytes
    if (threadIdx.x < 4) xz[threadIdx.x] = make_uint4(0, 0, 0, 0);  // (ordered by the barrier below)
    const int rb0 = blockIdx.x * 16 * kD1Rt;                     // first output row of the workgroup
    const int r0 = rb0 + t * 16;                                 // this wave's tile
    const int4 si = p.slots[s];                                  // {expert, 1, sorted position, 0}
    const int e = si.x;
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;
    const uint32_t exp_s = (uint32_t)p.R * (uint32_t)NB;
    // activation row of slot s (h at sorted position si.z): the wave's lanes stage it
    const __amdgpu_buffer_rsrc_t ract = make_rsrc(p.act + (size_t)si.z * p.Kdim, (uint32_t)p.Kdim * 2u);
    u32x4_t xv[6];
#pragma unroll
    for (int u = 0; u < 6; ++u) xv[u] = buf_load16(ract, (uint32_t)(lane + 64 * u) * 16u, 0);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales + (size_t)e * exp_s, exp_s);
    const uint32_t soff = (uint32_t)r0 * NB + lane * 16u;
    const u32x4_t sv0 = buf_load16(rs, soff, 0);
    const u32x4_t sv1 = buf_load16(rs, soff, 1024);
    __builtin_amdgcn_sched_barrier(0);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.blocks + (size_t)e * exp_w, exp_w);
    const uint32_t woff = (uint32_t)(r0 + m) * row_bytes + (uint32_t)g * 16u;
    u32x4_t wq[kGemvNit];
#pragma unroll
    for (int j = 0; j < kGemvNit; ++j) wq[j] = buf_load16(rw, 4 * j < NB ? woff : kRsrcPast, 64 * j);
    __builtin_amdgcn_sched_barrier(0);
    ((u32x4_t*)scl)[lane] = sv0;
    ((u32x4_t*)scl)[lane + 64] = sv1;
    if (t == 0) {
#pragma unroll
        for (int u = 0; u < 6; ++u)
            if (lane + 64 * u < cu) ((u32x4_t*)xs)[s * su + lane + 64 * u] = xv[u];
    }
    __syncthreads();
    // k_mx_gemv's pass for one token (every B column reads the token's row)
    const f32x4_t acc = mx_tile_steps<kGemvNit>(wq, scl + m * NB + g, xs + s * su + 4 * g, xz, NB, g);
    // column 0 holds the token: y of rows r0 + 4g .. + 3 (+ bias), into LDS
    if (m == 0) {
        const int rr = r0 + 4 * g;
        float bsum[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias && rr < p.R) {
            const uint2 bb = *(const uint2*)(p.bias + (size_t)e * p.R + rr);
            bsum[0] = bf16_lo(bb.x);
            bsum[1] = bf16_hi(bb.x);
            bsum[2] = bf16_lo(bb.y);
            bsum[3] = bf16_hi(bb.y);
        }
        float* yr = ys + s * (16 * kD1Rt) + t * 16 + 4 * g;
        yr[0] = acc[0] + bsum[0];
        yr[1] = acc[1] + bsum[1];
        yr[2] = acc[2] + bsum[2];
        yr[3] = acc[3] + bsum[3];
    }
    __syncthreads();
    // combine (k_combine's order: fmaf over the k pairs in k order, one rounding)
    const int i = threadIdx.x;
    const int r = rb0 + i;
    if (i < 16 * kD1Rt && r < p.R) {
        float a = 0.f;
        for (int j = 0; j < K; ++j) a = __builtin_fmaf(wts[j], ys[pos[j] * (16 * kD1Rt) + i], a);
        uint32_t o = f32_to_bf16(a);
        if (res) o = f32_to_bf16(bf16_to_f32(o) + bf16_to_f32(res[r]));
        out[r] = (uint16_t)o;
    }
}

bool down1_ok(int K, int Kdim) { return K >= 1 && K <= kD1MaxK && (Kdim >> 5) <= kD1MaxNB; }

// ---------------------------------------------------------------------------
// Small decode batches (N = B * k <= 24 routed pairs): the down projection of every
// touched expert and the weighted combine in one launch, as k_mx_down1 does for one
// token. Workgroup b owns output rows 16b..16b+15; wave s computes that 16-row tile of
// slot s's expert for the slot's tokens (the MFMA columns; k_mx_gemv's tile, so the
// same bits as the per-stage down projection without a K split); the workgroup
// stages the N rows of h (by sorted position) once, keeps y in LDS, and each token's
// row is combined over its k pairs in k order (k_combine's arithmetic).
// ---------------------------------------------------------------------------
constexpr int kDsMaxPairs = 24;  // the h rows in LDS: 24 x 5.9 KB at K = 2944
constexpr int kDsWaves = 8;      // wave w takes slots w, w + 8, w + 16
constexpr int kDsSlotsPerWave = 3;

__global__ __launch_bounds__(64 * kDsWaves) void k_mx_downs(GemvParams p, const float* __restrict__ wts,
                                                            const int32_t* __restrict__ pos, uint16_t* out,
                                                            const uint16_t* res, int B, int K) {
    extern __shared__ uint4 lds[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & (kDsWaves - 1);
    const int lane = threadIdx.x & 63;
    const int m = lane & 15, g = lane >> 4;
    const int N = p.n_pairs;
    const int NB = p.Kdim >> 5;
    const int cu = NB * 4, su = cu + 1;  // activation units per row, LDS row stride
    uint8_t* scl = (uint8_t*)lds + wave * kGemvSclSlice;          // this wave's tile scales [16][NB]
    uint4* xs = lds + kDsWaves * kGemvSclSlice / 16;              // h rows [N][su] by sorted position
    const int ncopy = (N * su + 63) / 64;                         // 1 KiB copies covering them
    float* ys = (float*)(xs + 64 * ncopy);                        // y [N][16]
    uint4* xz = (uint4*)(ys + N * 16);                            // 64 zero bytes
    const int r0 = blockIdx.x * 16;
    const int ns = *p.n_slots;
    const uint32_t row_bytes = (uint32_t)(p.Kdim >> 1);
    const uint32_t exp_w = (uint32_t)p.R * row_bytes;
    const uint32_t exp_s = (uint32_t)p.R * (uint32_t)NB;
    constexpr uint32_t kPast = 0x80000000u;  // an offset past every range: zeros
    // this wave's slots (wave, wave + 8, ...): {expert, tokens, first sorted position}, read
    // before anything else is in flight (a vector load waited on behind the copies or
    // the stripes would wait for all of them)
    int4 sl[kDsSlotsPerWave];
#pragma unroll
    for (int k = 0; k < kDsSlotsPerWave; ++k) {
        const int sk = wave + k * kDsWaves;
        const int4 v = sk < ns ? p.slots[sk] : make_int4(0, 0, 0, 0);
        sl[k] = make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                          __builtin_amdgcn_readfirstlane(v.z), 0);
    }
    // the N rows of h into LDS by direct copies (no registers): unit d of the flattened
    // [N][su] array from row d / su, unit d % su (the pad unit and the last copy's tail
    // read zeros)
    {
        const u32x4_t ra = rsrc_words(p.act, (uint32_t)N * (uint32_t)p.Kdim * 2u);
        for (int k = wave; k < ncopy; k += kDsWaves) {
            const int d = 64 * k + lane;
            const int q = d / su, c = d - q * su;
            const uint32_t voff = (q < N && c < cu) ? (uint32_t)q * (uint32_t)(p.Kdim * 2) + (uint32_t)c * 16u : kPast;
            dma16(ra, (const lds_u8*)(xs + 64 * k), voff);
        }
    }
    if (threadIdx.x < 4) xz[threadIdx.x] = make_uint4(0, 0, 0, 0);  // (ordered by the barrier below)
    // slot s's tile: scales into this wave's slice, then the 23 stripes
    u32x4_t sv0, sv1, wq[kGemvNit];
    auto tile_loads = [&](int k) {
        const bool live = wave + k * kDsWaves < ns;
        const int e = sl[k].x;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales + (size_t)e * exp_s, live ? exp_s : 0u);
        const uint32_t soff = (uint32_t)r0 * NB + lane * 16u;
        sv0 = buf_load16(rs, soff, 0);
        sv1 = buf_load16(rs, soff, 1024);
        __builtin_amdgcn_sched_barrier(0);
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.blocks + (size_t)e * exp_w, live ? exp_w : 0u);
        const uint32_t woff = (uint32_t)(r0 + m) * row_bytes + (uint32_t)g * 16u;
#pragma unroll
        for (int j = 0; j < kGemvNit; ++j) wq[j] = buf_load16(rw, 4 * j < NB ? woff : kRsrcPast, 64 * j);
        __builtin_amdgcn_sched_barrier(0);
    };
    tile_loads(0);
    // the activation copies (issued first, not counted by the compiler's waits): at most
    // the 2 scale loads and the 23 stripes may still be in flight
    asm volatile("s_waitcnt vmcnt(25)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kDsSlotsPerWave; ++k) {
        if (wave + k * kDsWaves >= ns) break;  // wave-uniform
        ((u32x4_t*)scl)[lane] = sv0;
        ((u32x4_t*)scl)[lane + 64] = sv1;
        const int e = sl[k].x, nt = sl[k].y, z = sl[k].z;
        // k_mx_gemv's pass: column m is the slot's token m (columns past its tokens
        // compute on its first row and are not stored)
        const uint4* xl = xs + (z + (m < nt ? m : 0)) * su + 4 * g;
        const f32x4_t acc = mx_tile_steps<kGemvNit>(wq, scl + m * NB + g, xl, xz, NB, g);
        if (m < nt) {
            const int rr = r0 + 4 * g;
            float bsum[4] = {0.f, 0.f, 0.f, 0.f};
            if (p.bias && rr < p.R) {
                const uint2 bb = *(const uint2*)(p.bias + (size_t)e * p.R + rr);
                bsum[0] = bf16_lo(bb.x);
                bsum[1] = bf16_hi(bb.x);
                bsum[2] = bf16_lo(bb.y);
                bsum[3] = bf16_hi(bb.y);
            }
            float* yr = ys + (z + m) * 16 + 4 * g;
            yr[0] = acc[0] + bsum[0];
            yr[1] = acc[1] + bsum[1];
            yr[2] = acc[2] + bsum[2];
            yr[3] = acc[3] + bsum[3];
        }
        if (k + 1 < kDsSlotsPerWave && wave + (k + 1) * kDsWaves < ns) tile_loads(k + 1);  // wave-uniform
    }
    __syncthreads();
    // combine (k_combine's order: fmaf over the k pairs in k order, one rounding)
    for (int i = threadIdx.x; i < B * 16; i += 64 * kDsWaves) {
        const int t = i >> 4, rr = i & 15;
        const int r = r0 + rr;
        if (r < p.R) {
            float a = 0.f;
            for (int j = 0; j < K; ++j) a = __builtin_fmaf(wts[t * K + j], ys[pos[t * K + j] * 16 + rr], a);
            uint32_t o = f32_to_bf16(a);
            if (res) o = f32_to_bf16(bf16_to_f32(o) + bf16_to_f32(res[(size_t)t * p.R + r]));
            out[(size_t)t * p.R + r] = (uint16_t)o;
        }
    }
}

bool downs_ok(int N, int E, int Kdim, int R) {
    const int slots = N < E ? N : E;
    const size_t lds = (size_t)kDsWaves * kGemvSclSlice + ((size_t)N * (4 * (Kdim >> 5) + 1) + 63) / 64 * 1024 +
                       (size_t)N * 64 + 64;
    return N >= 1 && N <= kDsMaxPairs && slots <= kDsSlotsPerWave * kDsWaves && (Kdim >> 5) <= kStreamMaxNB &&
           R % 16 == 0 && lds <= 160 * 1024;
}

int downs_launch(const GemvParams& p, const float* wts, const int32_t* pos, uint16_t* out, const uint16_t* res,
                 int B, int K, int max_slots, hipStream_t stream) {
    if (!downs_ok(p.n_pairs, max_slots, p.Kdim, p.R)) return set_error(PHYSLLM_MOE_EINVAL, "downs: sizes out of range");
    static std::once_flag attr_once[kMaxDevices];
    once_per_device(attr_once, [] {
        (void)hipFuncSetAttribute((const void*)k_mx_downs, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    const int NB = p.Kdim >> 5;
    const size_t ncopy = ((size_t)p.n_pairs * (4 * NB + 1) + 63) / 64;
    const size_t lds = (size_t)kDsWaves * kGemvSclSlice + ncopy * 64 * 16 + (size_t)p.n_pairs * 16 * sizeof(float) + 64;
    const unsigned grid = (unsigned)((p.R + 15) / 16);
    hipLaunchKernelGGL(k_mx_downs, dim3(grid), dim3(64 * kDsWaves), lds, stream, p, wts, pos, out, res, B, K);
    return check_launch("downs");
}



int down1_launch(const GemvParams& p, const float* wts, const int32_t* pos, uint16_t* out, const uint16_t* res,
                 int K, hipStream_t stream) {
    if (!down1_ok(K, p.Kdim)) return set_error(PHYSLLM_MOE_EINVAL, "down1: sizes out of range");
    static std::once_flag attr_once[kMaxDevices];
    once_per_device(attr_once, [] {
        (void)hipFuncSetAttribute((const void*)k_mx_down1, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    const int NB = p.Kdim >> 5;
    const size_t lds = (size_t)K * kD1Rt * kGemvSclSlice + (size_t)K * (4 * NB + 1) * 16 +
                       (size_t)K * 16 * kD1Rt * sizeof(float) + 64;
    const unsigned grid = (unsigned)((p.R + 16 * kD1Rt - 1) / (16 * kD1Rt));
    hipLaunchKernelGGL(k_mx_down1, dim3(grid), dim3(64 * kD1Rt * K), lds, stream, p, wts, pos, out, res, K);
    return check_launch("down1");
}

// The streaming kernel takes whole K rows (no split: it loads the 23 k-steps of a tile
// as one row segment) of experts below 2 GiB (32-bit buffer offsets), copies
// activation rows straight into LDS in 16-byte units (16-byte aligned), and pays once
// the items cover the chip twice.
bool gemv_streams(const GemvParams& p, int max_slots, int max_tokens) {
    const int NB = p.Kdim >> 5;
    const int per = (NB + p.split - 1) / p.split;
    const bool fast = per <= 4 * kGemvNit && NB <= kStreamMaxNB;
    const bool stream_ok =
        p.split == 1 && (int64_t)p.R * (p.Kdim / 2) < 0x80000000LL && ((uintptr_t)p.act & 15) == 0;
    const long stream_items = (long)((p.R + kStreamSetRows - 1) / kStreamSetRows) * max_slots * p.split;
    return fast && stream_ok && p.passes && max_tokens > 1 && stream_items >= 2L * device_cu_count();
}

int gemv_launch(int mode, const GemvParams& p0, int max_slots, int max_tokens, hipStream_t stream) {
    GemvParams p = p0;
    if (p.split < 1 || p.split > kMaxSplit) return set_error(PHYSLLM_MOE_EINVAL, "gemv: bad split");
    const int NB = p.Kdim >> 5;
    if (NB > kMaxScaleBlocks) return set_error(PHYSLLM_MOE_EINVAL, "gemv: reduction dimension > 8192");
    static std::once_flag attr_once[kMaxDevices];
    once_per_device(attr_once, [] {
        const void* ks[] = {(const void*)k_mx_gemv_stream<kModeGateUp>, (const void*)k_mx_gemv_stream<kModeDown>,
                            (const void*)k_mx_gemv<kModeGateUp, 2>, (const void*)k_mx_gemv<kModeGateUp, 12>,
                            (const void*)k_mx_gemv<kModeDown, 2>, (const void*)k_mx_gemv<kModeDown, 12>,
                            (const void*)k_mx_gemv_generic<kModeGateUp>, (const void*)k_mx_gemv_generic<kModeDown>};
        for (const void* k : ks) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    const int per = (NB + p.split - 1) / p.split;
    const int ntok = max_tokens < kPassTok ? max_tokens : kPassTok;
    const int rows_per_set = (kGemvThreads / 64) * 16;
    const int sets = (p.R + rows_per_set - 1) / rows_per_set;
    const int n_cu = device_cu_count();
    const bool fast = per <= 4 * kGemvNit && NB <= kStreamMaxNB;
    if (gemv_streams(p, max_slots, max_tokens)) {
        // many touched experts: persistent streaming kernel, one 4-wave group per CU
        // (a multiple of 8 groups: the item order is XCD-aware)
        const unsigned grid = (unsigned)((n_cu + 7) & ~7);
        p.rt = 1;
        if (mode == kModeGateUp)
            hipLaunchKernelGGL(k_mx_gemv_stream<kModeGateUp>, dim3(grid), dim3(kStreamThreads), kStreamLds, stream, p,
                               p.passes, p.perm, p.n_passes, p.out);
        else
            hipLaunchKernelGGL(k_mx_gemv_stream<kModeDown>, dim3(grid), dim3(kStreamThreads), kStreamLds, stream, p,
                               p.passes, p.perm, p.n_passes, p.out);
    } else if (fast) {
        // activation units one thread stages per pass: ntok rows x 4*per 16-byte units
        const int units = ntok * 4 * per;
        const int ns = (units + kGemvThreads - 1) / kGemvThreads;
        const size_t lds = (size_t)(kGemvThreads / 64) * kGemvSclSlice + (size_t)kPassTok * (4 * per + 1) * 16 + 64;
        dim3 grid(sets, max_slots, p.split);
        p.rt = 1;
        if (ns <= 2) {
            if (mode == kModeGateUp) hipLaunchKernelGGL((k_mx_gemv<kModeGateUp, 2>), grid, dim3(kGemvThreads), lds, stream, p, p.perm);
            else hipLaunchKernelGGL((k_mx_gemv<kModeDown, 2>), grid, dim3(kGemvThreads), lds, stream, p, p.perm);
        } else {
            if (mode == kModeGateUp) hipLaunchKernelGGL((k_mx_gemv<kModeGateUp, 12>), grid, dim3(kGemvThreads), lds, stream, p, p.perm);
            else hipLaunchKernelGGL((k_mx_gemv<kModeDown, 12>), grid, dim3(kGemvThreads), lds, stream, p, p.perm);
        }
    } else {
        const int seg = 4 * kGemvNit;
        const size_t lds = (size_t)4 * 16 * NB + (size_t)ntok * (4 * seg + 1) * 16;
        const long total = (long)sets * max_slots * p.split;
        int rt = (int)(total / 1024);
        rt = rt < 1 ? 1 : (rt > 8 ? 8 : rt);
        p.rt = rt;
        dim3 grid((sets + rt - 1) / rt, max_slots, p.split);
        if (mode == kModeGateUp)
            hipLaunchKernelGGL(k_mx_gemv_generic<kModeGateUp>, grid, dim3(kGemvThreads), lds, stream, p);
        else
            hipLaunchKernelGGL(k_mx_gemv_generic<kModeDown>, grid, dim3(kGemvThreads), lds, stream, p);
    }
    return check_launch(mode == kModeGateUp ? "gate_up gemv" : "down gemv");
}

int combine_launch(const float* y, int nsplit, size_t split_stride, const int32_t* pos, const float* wts,
                   uint16_t* out, const uint16_t* res, int B, int H, int K, hipStream_t stream) {
    dim3 grid((H / 4 + 255) / 256, B);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, stream, y, pos, wts, out, res, H, K, nsplit, split_stride);
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
