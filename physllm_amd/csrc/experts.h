// Shared declarations of the expert kernels (decode GEMV, prefill GEMM, combine).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace physllm {

enum { kModeGateUp = 0, kModeDown = 1 };

// One grouped-expert pass over routed tokens. Work slot s covers the s-th touched
// expert (ascending id); its tokens are the sorted positions
// slots[s].z .. slots[s].z + slots[s].y.
struct GemvParams {
    const uint16_t* act;     // gate_up: x [B, Kdim] (row = pair / top_k); down: h [N, Kdim] by sorted position
    const uint8_t* blocks;   // [E, R, Kdim/2] packed e2m1
    const uint8_t* scales;   // [E, R, Kdim/32] E8M0
    const uint16_t* bias;    // [E, R] bf16, nullable
    const int32_t* perm;     // [N] sorted position -> pair id
    const int4* slots;       // [E] {expert, tokens, first sorted position, 0}; tokens = 0 past the touched ones
    const int32_t* n_slots;  // [1] number of touched experts
    const int4* passes;      // [<= N/16 + E] {expert, tokens <= 16, first sorted position, chunk | chunks << 16}:
                             // each touched expert's tokens in chunks of kPassRows (decode only); the entries
                             // of experts with two or more chunks first, then the others, each in expert order
    const int32_t* n_passes; // [2] {entries, entries of multi-chunk experts}
    void* out;               // gate_up: h bf16 [N, R/2]; down: y fp32 [N, R] (by sorted position)
    int act_rows;            // rows of act (gate_up: batch; down: N)
    int Kdim;                // reduction length (H for gate_up, I for down)
    int R;                   // weight rows per expert (2I or H)
    int top_k;
    int split;               // K splits (down only; partials at out + s * n_pairs * R)
    int n_pairs;             // N = batch * top_k
    int rt;                  // row-tile sets per workgroup (set by the launcher)
    float alpha, limit;
    // streaming gate_up only (nullable): the down projection's codes [E, pf_R, pf_Kdim/2].
    // The refills of a workgroup's last item then load the down launch's first item of
    // the same workgroup index (the same XCD) into L2 instead of nothing.
    const uint8_t* pf_blocks;
    int pf_R, pf_Kdim;
};

constexpr int kMaxSplit = 4;
constexpr int kPassRows = 16;  // tokens per pass-table entry (the MFMA's N)

// Whether gemv_launch runs p on the streaming kernel (the layer's gate_up launch then
// prefetches the down launch's first items when both stream).
bool gemv_streams(const GemvParams& p, int max_slots, int max_tokens);
int gemv_launch(int mode, const GemvParams& p, int max_slots, int max_tokens, hipStream_t stream);
// out [B,H] = bf16(sum over k of w * y), then, when res is not null,
// out = bf16(out + res) (the residual add after the layer; res may equal out).
int combine_launch(const float* y, int nsplit, size_t split_stride, const int32_t* pos, const float* wts,
                   uint16_t* out, const uint16_t* res, int B, int H, int K, hipStream_t stream);
// Batch 1: down projection of the k slots and the weighted combine in one launch
// (out = bf16(sum_j w_j * y_j) [+ res]); down1_ok says whether (K, Kdim) fit it.
bool down1_ok(int K, int Kdim);
// Small decode batches (N = B * k <= 24 pairs over at most 24 experts): the down
// projection of every touched expert and the combine in one launch; downs_ok says
// whether (pairs, slots, K, rows) fit it.
bool downs_ok(int N, int E, int Kdim, int R);
int downs_launch(const GemvParams& p, const float* wts, const int32_t* pos, uint16_t* out, const uint16_t* res,
                 int B, int K, int max_slots, hipStream_t stream);
int down1_launch(const GemvParams& p, const float* wts, const int32_t* pos, uint16_t* out, const uint16_t* res,
                 int K, hipStream_t stream);
// Batch 1 (and 2 tokens with batch * k <= 16) in three launches: the router
// logits (one workgroup per expert; with norm_w, batch 1 only, after the RMSNorm of
// norm_x into x), then selection + gate_up, then down + combine.
struct B1Layer {
    int H, I, E, K, B;
    void* x;             // [B, H] the tokens; with norm_w, where its normalised row is written
    const void* norm_x;  // with norm_w: the token before the norm
    const void* norm_w;  // nullable
    float eps;
    const void* router_w;
    const void* router_b;
    const void* gu_blocks;
    const void* gu_scales;
    const void* gu_bias;
    const void* dn_blocks;
    const void* dn_scales;
    const void* dn_bias;
    double* logits;   // [B, E]
    uint16_t* h;      // [B*K, I]
    int32_t* idx;     // [B, K]
    float* wts;       // [B, K]
    void* out;        // [B, H]
    const void* res;  // [B, H] nullable
    float alpha, limit;
};
bool b1_ok(int H, int I, int E, int K, int B);
// The three launches of the batch-1 layer (logits, gate_up with the selection,
// down with the combine); only = 0, 1 or 2 runs that launch alone on the state the
// earlier ones left in the workspace, -1 runs all three.
int b1_layer_launch(const B1Layer& a, hipStream_t stream, int only = -1);
// RMSNorm of B rows of H bf16 values (out may equal x) and the bf16 residual add.
int rms_norm_launch(const void* x, const void* w, void* out, int B, int H, float eps, hipStream_t stream);
int residual_add_launch(void* out, const void* res, int64_t n, hipStream_t stream);
// Counting sort of the routed pairs by expert. Optional outputs (nullable): the
// slot table and its count, the per-slot prefix of tile_n-token tiles, and the
// pass table (chunks of kPassRows tokens) with its count.
// hist (nullable): bucket_hist_bytes(N, E) of workspace; with it, N > 1024 pairs are
// bucketed by many workgroups (three launches) instead of one.
int bucket_launch(const void* idx, int N, int E, void* counts, void* offsets, void* perm, void* pos, void* slots,
                  void* n_slots, void* tprefix, int tile_n, void* passes, void* n_passes, hipStream_t stream,
                  void* hist = nullptr);
size_t bucket_hist_bytes(int N, int E);
// Grouped GEMM for many tokens per expert; tprefix = per-slot exclusive prefix of
// kGemmTileN-token tiles (from bucketing).
constexpr int kGemmTileN = 128;
int gemm_launch(int mode, const GemvParams& p, const int32_t* tprefix, int max_slots, int n_pairs,
                hipStream_t stream);

}  // namespace physllm
