// Host side of the C ABI: error channel, workspace carving and the whole-layer
// entry point (the MoE half of crates/llm-core/src/moe.rs:246-307 without the
// host round trips of :261-299 — routing stays on the device, so one layer is a
// fixed sequence of asynchronous launches on the caller's stream).
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "capi_internal.h"
#include "experts.h"

namespace physllm {

static thread_local int t_err_code = 0;
static thread_local char t_err_msg[256] = {0};

int set_error(int code, const char* msg) {
    t_err_code = code;
    snprintf(t_err_msg, sizeof(t_err_msg), "%s", msg ? msg : "");
    return code;
}

int ok() {
    t_err_code = 0;
    t_err_msg[0] = 0;
    return PHYSLLM_MOE_OK;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        char buf[256];
        snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(e));
        return set_error(PHYSLLM_MOE_ELAUNCH, buf);
    }
    return ok();
}

static int current_device() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess ? dev : 0;
}

static int query_cu_count(int dev) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    return n;
}

int device_cu_count() {
    static std::once_flag flags[kMaxDevices];
    static int n_cu[kMaxDevices];
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return query_cu_count(dev);
    std::call_once(flags[dev], [dev] { n_cu[dev] = query_cu_count(dev); });
    return n_cu[dev];
}

void once_per_device(std::once_flag (&flags)[kMaxDevices], void (*init)()) {
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) {
        init();
        return;
    }
    std::call_once(flags[dev], init);
}

// Workspace regions, each 256-byte aligned.
struct Workspace {
    int32_t* idx;
    float* wts;
    int32_t* counts;
    int32_t* offsets;
    int4* slots;
    int32_t* n_slots;
    int32_t* tprefix;  // [E+1] token-tile prefix over slots
    int4* passes;      // [N/16 + E] pass table (decode)
    int32_t* n_passes;
    int32_t* perm;
    int32_t* pos;
    int32_t* bhist;  // [blocks][E] the multi-workgroup bucketing's block counts (N > 1024)
    double* lg;   // [B][E] router logits (two-launch router, batch-1 layer)
    uint16_t* h;
    float* y;     // [split][N][H]
    int split;
    size_t bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Many tokens per touched expert (prefill): grouped GEMM; otherwise the GEMV.
static bool use_gemm(const physllm_moe_config& c, int B) {
    const int64_t N = (int64_t)B * c.top_k;
    const int64_t slots = std::min<int64_t>(N, c.num_experts);
    return N >= 64 * slots;
}

// K splits of the down projection: enough 16-row work tiles (one per wave) to
// cover the chip when very few rows are touched (small layers at small batch).
// Measured at GPT-OSS shape, batch 1 (720 tiles): splitting K 3 ways ends the
// down projection at 10.2 us, 2 ways at 8.3 us, unsplit at 7.8 us: a split
// multiplies the workgroups whose first loads all wait on the same routing
// tables and, past ~512 of them, leaves some to start in a second round.
static int down_split(const physllm_moe_config& c, int B) {
    if (use_gemm(c, B)) return 1;
    const int64_t slots = std::min<int64_t>((int64_t)B * c.top_k, c.num_experts);
    const int64_t tiles = slots * ((c.hidden + 15) / 16);
    const int64_t want = 512;
    int split = (int)std::min<int64_t>(kMaxSplit, (want + tiles - 1) / std::max<int64_t>(tiles, 1));
    split = std::max(1, std::min(split, c.intermediate / 32));
    return split;
}

// Batches the three-launch batch-1 layer takes (batch1.hip): up to 2 tokens,
// decode-shaped, E <= 256. With 3 or 4 tokens its down waves (one per routed pair)
// re-stream experts that pairs share and it measured no faster than the per-stage path.
static bool b1_batch(const physllm_moe_config& c, int B) {
    return B >= 1 && B <= 2 && (int64_t)B * c.top_k <= 16 && !use_gemm(c, B) && c.num_experts <= 256;
}

static Workspace carve(const physllm_moe_config& c, int B, char* base) {
    const size_t N = (size_t)B * c.top_k;
    const size_t E = (size_t)c.num_experts;
    Workspace w;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        char* p = base ? base + o : nullptr;
        o += align256(bytes);
        return p;
    };
    w.idx = (int32_t*)take(N * 4);
    w.wts = (float*)take(N * 4);
    w.counts = (int32_t*)take(E * 4);
    w.offsets = (int32_t*)take((E + 1) * 4);
    w.slots = (int4*)take(E * 16);
    w.n_slots = (int32_t*)take(4);
    w.tprefix = (int32_t*)take((E + 1) * 4);
    const bool decode = !use_gemm(c, B);
    w.passes = (int4*)take(decode ? (N / kPassRows + std::min(N, E)) * 16 : 0);
    w.n_passes = (int32_t*)take(8);  // {entries, entries of multi-chunk experts}
    w.perm = (int32_t*)take(N * 4);
    w.pos = (int32_t*)take(N * 4);
    w.bhist = (int32_t*)take(bucket_hist_bytes((int)N, (int)E));
    // router logits (two-launch router) or bounds (tiled two-pass router), B x E x 8
    // bytes; null when neither router form can run, so no router writes an empty region
    const bool need_lg = router_two_launch(B, c.num_experts) || rmx_tiled(B, c.num_experts) || b1_batch(c, B) ||
                         (decode && dec_route_ok(B, c.num_experts, c.top_k));
    w.lg = need_lg ? (double*)take((size_t)B * E * 8) : nullptr;
    w.h = (uint16_t*)take(N * (size_t)c.intermediate * 2);
    w.split = down_split(c, B);
    w.y = (float*)take((size_t)w.split * N * (size_t)c.hidden * 4);
    w.bytes = o;
    return w;
}

// Every expert kernel reads its activations and weights through 32-bit buffer
// resources (a range of bytes from a base), and loads that must read zeros use
// offsets at or past 2^31. So no range one launch reads may reach 2^31 bytes:
// one expert's codes, the router rows, x [b, H] and h [b*k, I] (bf16). y and the
// outputs are addressed with 64-bit offsets.
constexpr int64_t kMaxRangeBytes = (1LL << 31) - (1LL << 20);

static int validate(const physllm_moe_config* c, int B) {
    if (!c) return set_error(PHYSLLM_MOE_EINVAL, "layer: null config");
    if (c->hidden < 32 || c->hidden % 32) return set_error(PHYSLLM_MOE_EINVAL, "layer: hidden must be a positive multiple of 32");
    if (c->intermediate < 32 || c->intermediate % 32)
        return set_error(PHYSLLM_MOE_EINVAL, "layer: intermediate must be a positive multiple of 32");
    if (c->num_experts < 1 || c->num_experts > 1024) return set_error(PHYSLLM_MOE_EINVAL, "layer: num_experts must be in [1, 1024]");
    if (c->top_k < 1 || c->top_k > c->num_experts || c->top_k > 32)
        return set_error(PHYSLLM_MOE_EINVAL, "layer: top_k must be in [1, min(num_experts, 32)]");
    if (c->max_chunk_tokens < 0) return set_error(PHYSLLM_MOE_EINVAL, "layer: max_chunk_tokens < 0");
    // one expert's gate_up codes [2I, H/2] (the down codes [H, I/2] are half of that)
    if ((int64_t)c->intermediate * c->hidden > kMaxRangeBytes)
        return set_error(PHYSLLM_MOE_EINVAL, "layer: one expert's weights exceed 2^31 bytes");
    if ((int64_t)c->num_experts * c->hidden * 2 > kMaxRangeBytes)
        return set_error(PHYSLLM_MOE_EINVAL, "layer: router weights exceed 2^31 bytes");
    if (B < 0) return set_error(PHYSLLM_MOE_EINVAL, "layer: batch < 0");
    return PHYSLLM_MOE_OK;
}

// Tokens per chunk: the layer runs larger batches as consecutive chunks over one
// workspace, each a whole layer call (routing is per token and every output
// element's sums run in a fixed order, so chunking does not change the results
// as long as every chunk takes the kernels the whole batch would). The limit keeps
// x [b, H] and h [b*k, I] below kMaxRangeBytes; a nonzero max_chunk_tokens lowers it
// (and with it the workspace).
static int chunk_limit(const physllm_moe_config& c) {
    int64_t lim = kMaxRangeBytes / ((int64_t)c.hidden * 2);
    lim = std::min(lim, kMaxRangeBytes / ((int64_t)c.top_k * c.intermediate * 2));
    if (c.max_chunk_tokens > 0) lim = std::min<int64_t>(lim, c.max_chunk_tokens);
    return (int)std::max<int64_t>(1, lim);
}

// B tokens in n chunks of near-equal size: chunk i has base + (i < rem) tokens.
struct Chunks {
    int n, base, rem;
    int size(int i) const { return base + (i < rem ? 1 : 0); }
    int64_t first(int i) const { return (int64_t)i * base + std::min(i, rem); }
};

static Chunks chunks(const physllm_moe_config& c, int B) {
    const int lim = chunk_limit(c);
    const int n = B > 0 ? (int)(((int64_t)B + lim - 1) / lim) : 1;
    return Chunks{n, B / n, B % n};
}

// Workspace of a call on B tokens: the larger of its (at most two) chunk sizes'.
static size_t layer_ws_bytes(const physllm_moe_config& c, int B) {
    const Chunks ch = chunks(c, B);
    size_t b = carve(c, ch.size(0), nullptr).bytes;
    if (ch.rem > 0) b = std::max(b, carve(c, ch.base, nullptr).bytes);
    return b;
}

}  // namespace physllm

using namespace physllm;

extern "C" int physllm_moe_last_error(void) { return t_err_code; }
extern "C" const char* physllm_moe_last_error_message(void) { return t_err_msg; }

extern "C" size_t physllm_moe_workspace_bytes(const physllm_moe_config* cfg, int batch) {
    if (validate(cfg, batch) != PHYSLLM_MOE_OK) return 0;
    ok();
    return layer_ws_bytes(*cfg, batch);
}

// Stages of one layer over a shared workspace. Bit i of `stages` runs stage i:
// 0 route (router + bucketing), 1 gate_up (+ SwiGLU), 2 down, 3 combine.
enum { kStageRoute = 1, kStageGateUp = 2, kStageDown = 4, kStageCombine = 8, kStageAll = 15 };

// `residual` (nullable) is added to the combined output: out = bf16(out + residual).
// `norm_w` (nullable, batch-1 route only): the route stage normalises `norm_x` into
// x (RMSNorm with eps) before routing it, in the same launch.
static bool route1_path(const physllm_moe_config& c, int batch) {
    return batch == 1 && !use_gemm(c, batch) && c.num_experts <= 256;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// One or two tokens through every stage: the three-launch batch-1 layer (batch1.hip)
// when the shape fits it and the rows it loads 16 bytes at a time are 16-byte
// aligned.
static bool b1_layer_path(const physllm_moe_config& c, int batch, int stages, const void* x,
                          const physllm_moe_weights* w, const void* norm_w, const void* norm_x) {
    if (stages != kStageAll || !b1_batch(c, batch)) return false;
    if (!b1_ok(c.hidden, c.intermediate, c.num_experts, c.top_k, batch)) return false;
    if (!aligned16(x) || !aligned16(w->router_w)) return false;
    return !norm_w || (aligned16(norm_w) && aligned16(norm_x));
}

// The batch-1 layer's arguments over the workspace ws.
static B1Layer b1_layer(const physllm_moe_config& c, const physllm_moe_weights* w, const void* x, int batch,
                        void* out, int32_t* idx, float* wts, const Workspace& ws, const void* residual,
                        const void* norm_w, float eps, const void* norm_x) {
    B1Layer a{};
    a.H = c.hidden;
    a.I = c.intermediate;
    a.E = c.num_experts;
    a.K = c.top_k;
    a.B = batch;
    a.x = (void*)x;
    a.norm_x = norm_x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.router_w = w->router_w;
    a.router_b = w->router_b;
    a.gu_blocks = w->gate_up_blocks;
    a.gu_scales = w->gate_up_scales;
    a.gu_bias = w->gate_up_bias;
    a.dn_blocks = w->down_blocks;
    a.dn_scales = w->down_scales;
    a.dn_bias = w->down_bias;
    a.logits = ws.lg;
    a.h = ws.h;
    a.idx = idx;
    a.wts = wts;
    a.out = out;
    a.res = residual;
    a.alpha = c.swiglu_alpha;
    a.limit = c.swiglu_limit;
    return a;
}

static int run_stages(const physllm_moe_config* cfg, const physllm_moe_weights* w, const void* x, int batch,
                      void* out, void* topk_idx, void* topk_w, void* workspace, size_t workspace_bytes,
                      hipStream_t s, int stages, const void* residual = nullptr, const void* norm_w = nullptr,
                      float eps = 0.f, const void* norm_x = nullptr) {
    int rc = validate(cfg, batch);
    if (rc) return rc;
    if (batch == 0) return ok();
    const physllm_moe_config& c = *cfg;
    if ((stages & (kStageRoute | kStageGateUp | kStageDown)) &&
        (!w || !w->router_w || !w->gate_up_blocks || !w->gate_up_scales || !w->down_blocks || !w->down_scales))
        return set_error(PHYSLLM_MOE_EINVAL, "layer: null weight pointer");
    if ((stages & (kStageRoute | kStageGateUp)) && !x) return set_error(PHYSLLM_MOE_EINVAL, "layer: null x");
    if ((stages & kStageCombine) && !out) return set_error(PHYSLLM_MOE_EINVAL, "layer: null out");
    const size_t need = carve(c, batch, nullptr).bytes;
    if (!workspace || workspace_bytes < need) return set_error(PHYSLLM_MOE_EWORKSPACE, "layer: workspace too small");
    Workspace ws = carve(c, batch, (char*)workspace);
    const int N = batch * c.top_k;
    int32_t* idx = topk_idx ? (int32_t*)topk_idx : ws.idx;
    float* wts = topk_w ? (float*)topk_w : ws.wts;

    if (b1_layer_path(c, batch, stages, x, w, norm_w, norm_x)) {
        const B1Layer a = b1_layer(c, w, x, batch, out, idx, wts, ws, residual, norm_w, eps, norm_x);
        if ((rc = b1_layer_launch(a, s))) return rc;
        return ok();
    }

    if (stages & kStageRoute) {
        const bool gemm = use_gemm(c, batch);
        if (route1_path(c, batch)) {
            // one token: the whole route (and the bucketing of its k pairs) in one launch
            rc = route1_launch(norm_w ? norm_x : x, w->router_w, w->router_b, c.hidden, c.num_experts, c.top_k, idx,
                               wts, ws.counts, ws.offsets, ws.perm, ws.pos, ws.slots, ws.n_slots, ws.passes,
                               ws.n_passes, s, norm_w, eps, norm_w ? (void*)x : nullptr);
        } else if (!gemm && dec_route_ok(batch, c.num_experts, c.top_k) && c.hidden % 8 == 0 && aligned16(x) &&
                   aligned16(w->router_w)) {
            // decode at small B * E: logits over many waves, one selection workgroup per
            // token, then the one-workgroup bucketing
            rc = dec_route_launch(x, w->router_w, w->router_b, batch, c.hidden, c.num_experts, c.top_k, ws.lg, idx,
                                  wts, ws.counts, ws.offsets, ws.perm, ws.pos, ws.slots, ws.n_slots, ws.passes,
                                  ws.n_passes, s);
        } else {
            rc = router_launch(x, w->router_w, w->router_b, batch, c.hidden, c.num_experts, c.top_k, idx, wts, s,
                               ws.lg);
            // prefill: the GEMM's token-tile prefix; decode: the GEMV's pass table
            if (!rc)
                rc = bucket_launch(idx, N, c.num_experts, ws.counts, ws.offsets, ws.perm, ws.pos, ws.slots,
                                   ws.n_slots, gemm ? ws.tprefix : nullptr, kGemmTileN, gemm ? nullptr : ws.passes,
                                   ws.n_passes, s, ws.bhist);
        }
        if (rc) return rc;
    }
    const int max_slots = N < c.num_experts ? N : c.num_experts;
    GemvParams p{};
    p.perm = ws.perm;
    p.slots = ws.slots;
    p.n_slots = ws.n_slots;
    p.passes = ws.passes;
    p.n_passes = ws.n_passes;
    p.top_k = c.top_k;
    p.split = 1;
    p.n_pairs = N;
    p.alpha = c.swiglu_alpha;
    p.limit = c.swiglu_limit;
    if (stages & kStageGateUp) {
        p.act = (const uint16_t*)x;
        p.act_rows = batch;
        p.blocks = (const uint8_t*)w->gate_up_blocks;
        p.scales = (const uint8_t*)w->gate_up_scales;
        p.bias = (const uint16_t*)w->gate_up_bias;
        p.out = ws.h;
        p.Kdim = c.hidden;
        p.R = 2 * c.intermediate;
        if (!use_gemm(c, batch) && (stages & kStageDown)) {
            // when the down projection streams too, the gate_up launch's last refills
            // prefetch its first items
            GemvParams pd = p;
            pd.act = ws.h;
            pd.act_rows = N;
            pd.Kdim = c.intermediate;
            pd.R = c.hidden;
            pd.split = ws.split;
            if (gemv_streams(pd, max_slots, batch)) {
                p.pf_blocks = (const uint8_t*)w->down_blocks;
                p.pf_R = c.hidden;
                p.pf_Kdim = c.intermediate;
            }
        }
        rc = use_gemm(c, batch) ? gemm_launch(kModeGateUp, p, ws.tprefix, max_slots, N, s)
                                : gemv_launch(kModeGateUp, p, max_slots, batch, s);
        p.pf_blocks = nullptr;
        if (rc) return rc;
    }
    // one token, and small batches (at most 24 routed pairs): the down projection and
    // the combine run as one launch
    const bool fuse = (stages & kStageDown) && (stages & kStageCombine) && !use_gemm(c, batch);
    const bool down1 = fuse && batch == 1 && down1_ok(c.top_k, c.intermediate);
    const bool downs = fuse && batch >= 2 && downs_ok(N, max_slots, c.intermediate, c.hidden);
    if (stages & kStageDown) {
        p.act = ws.h;
        p.act_rows = N;
        p.blocks = (const uint8_t*)w->down_blocks;
        p.scales = (const uint8_t*)w->down_scales;
        p.bias = (const uint16_t*)w->down_bias;
        p.out = ws.y;
        p.Kdim = c.intermediate;
        p.R = c.hidden;
        p.split = ws.split;
        if (down1) {
            p.split = 1;
            rc = down1_launch(p, wts, ws.pos, (uint16_t*)out, (const uint16_t*)residual, c.top_k, s);
        } else if (downs) {
            p.split = 1;
            rc = downs_launch(p, wts, ws.pos, (uint16_t*)out, (const uint16_t*)residual, batch, c.top_k, max_slots, s);
        } else {
            rc = use_gemm(c, batch) ? gemm_launch(kModeDown, p, ws.tprefix, max_slots, N, s)
                                    : gemv_launch(kModeDown, p, max_slots, batch, s);
        }
        if (rc) return rc;
    }
    if ((stages & kStageCombine) && !down1 && !downs) {
        if ((rc = combine_launch(ws.y, ws.split, (size_t)N * c.hidden, ws.pos, wts, (uint16_t*)out,
                                 (const uint16_t*)residual, batch, c.hidden, c.top_k, s)))
            return rc;
    }
    return ok();
}

static const char* at(const void* p, int64_t bytes) { return p ? (const char*)p + bytes : nullptr; }
static char* at(void* p, int64_t bytes) { return p ? (char*)p + bytes : nullptr; }

extern "C" int physllm_moe_layer_forward(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                                         const void* x, int batch, void* out, void* topk_idx, void* topk_w,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    int rc = validate(cfg, batch);
    if (rc) return rc;
    if (batch == 0) return ok();
    if (!w || !w->router_w || !w->gate_up_blocks || !w->gate_up_scales || !w->down_blocks || !w->down_scales)
        return set_error(PHYSLLM_MOE_EINVAL, "layer: null weight pointer");
    if (!x || !out) return set_error(PHYSLLM_MOE_EINVAL, "layer: null x or out");
    if (!workspace || workspace_bytes < layer_ws_bytes(*cfg, batch))
        return set_error(PHYSLLM_MOE_EWORKSPACE, "layer: workspace too small");
    const Chunks ch = chunks(*cfg, batch);
    const int64_t row = (int64_t)cfg->hidden * 2, krow = (int64_t)cfg->top_k * 4;
    for (int i = 0; i < ch.n && !rc; ++i) {
        const int64_t t0 = ch.first(i);
        rc = run_stages(cfg, w, at(x, t0 * row), ch.size(i), at(out, t0 * row), at(topk_idx, t0 * krow),
                        at(topk_w, t0 * krow), workspace, workspace_bytes, (hipStream_t)stream, kStageAll);
    }
    return rc;
}

// The stage entry points keep their routing state in the workspace between calls,
// so each call covers one chunk: at most chunk_limit() tokens.
static int stage_batch_ok(const physllm_moe_config* cfg, int batch) {
    int rc = validate(cfg, batch);
    if (rc) return rc;
    if (batch > chunk_limit(*cfg))
        return set_error(PHYSLLM_MOE_EINVAL, "stage: batch above the chunk limit (use physllm_moe_layer_forward)");
    return PHYSLLM_MOE_OK;
}

extern "C" int physllm_moe_stage_route(const physllm_moe_config* cfg, const physllm_moe_weights* w, const void* x,
                                       int batch, void* topk_idx, void* topk_w, void* workspace,
                                       size_t workspace_bytes, void* stream) {
    if (int rc = stage_batch_ok(cfg, batch)) return rc;
    return run_stages(cfg, w, x, batch, nullptr, topk_idx, topk_w, workspace, workspace_bytes, (hipStream_t)stream,
                      kStageRoute);
}

extern "C" int physllm_moe_stage_gate_up(const physllm_moe_config* cfg, const physllm_moe_weights* w, const void* x,
                                         int batch, void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = stage_batch_ok(cfg, batch)) return rc;
    return run_stages(cfg, w, x, batch, nullptr, nullptr, nullptr, workspace, workspace_bytes, (hipStream_t)stream,
                      kStageGateUp);
}

extern "C" int physllm_moe_stage_down(const physllm_moe_config* cfg, const physllm_moe_weights* w, int batch,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = stage_batch_ok(cfg, batch)) return rc;
    return run_stages(cfg, w, nullptr, batch, nullptr, nullptr, nullptr, workspace, workspace_bytes,
                      (hipStream_t)stream, kStageDown);
}

extern "C" int physllm_moe_stage_combine(const physllm_moe_config* cfg, int batch, void* out, const void* topk_w,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = stage_batch_ok(cfg, batch)) return rc;
    return run_stages(cfg, nullptr, nullptr, batch, out, nullptr, (void*)topk_w, workspace, workspace_bytes,
                      (hipStream_t)stream, kStageCombine);
}

// One launch of the batch-1 layer (the layer at one or two tokens, when its
// launches fit the shape), on the state the earlier launches left in the workspace.
extern "C" int physllm_moe_stage_batch1(const physllm_moe_config* cfg, const physllm_moe_weights* w, const void* x,
                                        int batch, int launch, void* out, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    if (int rc = stage_batch_ok(cfg, batch)) return rc;
    if (batch == 0) return ok();
    const physllm_moe_config& c = *cfg;
    if (!w || !w->router_w || !w->gate_up_blocks || !w->gate_up_scales || !w->down_blocks || !w->down_scales)
        return set_error(PHYSLLM_MOE_EINVAL, "stage_batch1: null weight pointer");
    if (!x || !out) return set_error(PHYSLLM_MOE_EINVAL, "stage_batch1: null x or out");
    if (!b1_layer_path(c, batch, kStageAll, x, w, nullptr, nullptr))
        return set_error(PHYSLLM_MOE_EINVAL, "stage_batch1: the batch-1 launches do not serve this shape or batch");
    if (!workspace || workspace_bytes < carve(c, batch, nullptr).bytes)
        return set_error(PHYSLLM_MOE_EWORKSPACE, "stage_batch1: workspace too small");
    const Workspace ws = carve(c, batch, (char*)workspace);
    const B1Layer a = b1_layer(c, w, x, batch, out, ws.idx, ws.wts, ws, nullptr, nullptr, 0.f, nullptr);
    if (int rc = b1_layer_launch(a, (hipStream_t)stream, launch)) return rc;
    return ok();
}

// The MoE sub-layer of a transformer block (crates/llm-core/src/moe.rs:238-313):
// h = rms_norm(x) into the tail of the workspace, the layer on h, and the residual
// add of x fused into the combine; chunked like the layer (norm, layer, residual
// add per chunk). out may equal x (the reference updates its residual buffer in
// place): x is read by the norm and, per element, by the combine thread that then
// writes that element.
static size_t block_ws_bytes(const physllm_moe_config& c, int batch) {
    const Chunks ch = chunks(c, batch);
    return layer_ws_bytes(c, batch) + align256((size_t)ch.size(0) * c.hidden * 2);
}

extern "C" size_t physllm_moe_block_workspace_bytes(const physllm_moe_config* cfg, int batch) {
    if (validate(cfg, batch) != PHYSLLM_MOE_OK) return 0;
    ok();
    return block_ws_bytes(*cfg, batch);
}

static int block_chunk(const physllm_moe_config* cfg, const physllm_moe_weights* w, const void* x,
                       const void* norm_w, float eps, int batch, void* out, void* topk_idx, void* topk_w,
                       void* workspace, size_t lay, hipStream_t s) {
    void* h = (char*)workspace + lay;
    // a single token's norm runs inside its route launch
    if (route1_path(*cfg, batch) && cfg->hidden <= kRoute1NormMaxH)
        return run_stages(cfg, w, h, batch, out, topk_idx, topk_w, workspace, lay, s, kStageAll, x, norm_w, eps, x);
    if (int rc = rms_norm_launch(x, norm_w, h, batch, cfg->hidden, eps, s)) return rc;
    return run_stages(cfg, w, h, batch, out, topk_idx, topk_w, workspace, lay, s, kStageAll, x);
}

extern "C" int physllm_moe_block_forward(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                                         const void* x, const void* norm_w, float eps, int batch, void* out,
                                         void* topk_idx, void* topk_w, void* workspace, size_t workspace_bytes,
                                         void* stream) {
    int rc = validate(cfg, batch);
    if (rc) return rc;
    if (batch == 0) return ok();
    if (!x || !norm_w || !out) return set_error(PHYSLLM_MOE_EINVAL, "block: null x, norm_w or out");
    if (!workspace || workspace_bytes < block_ws_bytes(*cfg, batch))
        return set_error(PHYSLLM_MOE_EWORKSPACE, "block: workspace too small");
    if (!w || !w->router_w || !w->gate_up_blocks || !w->gate_up_scales || !w->down_blocks || !w->down_scales)
        return set_error(PHYSLLM_MOE_EINVAL, "layer: null weight pointer");
    const size_t lay = layer_ws_bytes(*cfg, batch);
    const Chunks ch = chunks(*cfg, batch);
    const int64_t row = (int64_t)cfg->hidden * 2, krow = (int64_t)cfg->top_k * 4;
    for (int i = 0; i < ch.n && !rc; ++i) {
        const int64_t t0 = ch.first(i);
        rc = block_chunk(cfg, w, at(x, t0 * row), norm_w, eps, ch.size(i), at(out, t0 * row),
                         at(topk_idx, t0 * krow), at(topk_w, t0 * krow), workspace, lay, (hipStream_t)stream);
    }
    return rc;
}

// ---------------------------------------------------------------------------
// No-allocation entry point: physllm_moe_layer_forward with a file-scope device
// array in place of the caller's workspace, for callers that cannot allocate
// (code under HIP graph capture, tight serving loops). Every device the library
// runs on holds its own copy of the array until the process ends. Each call
// writes every workspace region it reads before reading it, so the contents a
// previous call left behind never matter and nothing needs clearing; calls that
// overlap on one device share the array and race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The array's device address on each device, looked up once per device with that
// device current (the array's name in host code is only a host-side handle).
static std::once_flag g_scratch_once[kMaxDevices];
static void* g_scratch_ptr[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

static int scratch_for_current_device(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PHYSLLM_MOE_ELAUNCH, "noalloc: no current HIP device");
    if (dev < 0 || dev >= kMaxDevices) return set_error(PHYSLLM_MOE_EINVAL, "noalloc: device index above 63");
    std::call_once(g_scratch_once[dev], [dev] {
        void* p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = p;
    });
    if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev]) {
        char buf[200];
        snprintf(buf, sizeof(buf), "noalloc: hipGetSymbolAddress(scratch) failed: %s",
                 hipGetErrorString(g_scratch_err[dev]));
        return set_error(PHYSLLM_MOE_ELAUNCH, buf);
    }
    *out = g_scratch_ptr[dev];
    return PHYSLLM_MOE_OK;
}

extern "C" int physllm_moe_layer_forward_noalloc(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                                                 const void* x, int batch, void* out, void* topk_idx,
                                                 void* topk_w, void* stream) {
    int rc = validate(cfg, batch);
    if (rc) return rc;
    if (batch == 0) return ok();
    const size_t need = layer_ws_bytes(*cfg, batch);
    if (need > kScratchBytes) {
        char buf[256];
        snprintf(buf, sizeof(buf),
                 "noalloc: %d tokens need %zu bytes of scratch, above its %zu (lower max_chunk_tokens or use "
                 "physllm_moe_layer_forward)",
                 batch, need, kScratchBytes);
        return set_error(PHYSLLM_MOE_EINVAL, buf);
    }
    void* ws = nullptr;
    if ((rc = scratch_for_current_device(&ws))) return rc;
    return physllm_moe_layer_forward(cfg, w, x, batch, out, topk_idx, topk_w, ws, kScratchBytes, stream);
}
