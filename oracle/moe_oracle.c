/*
 * CPU oracle for the MXFP4 MoE expert path — TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference algorithm (PhysLLM @ /root/reference) with the
 * benchmark's bf16 / E8M0 / bias / clamped-SwiGLU semantics.  Every function
 * names the reference lines it follows.  Rounding points:
 *   dequant : bf16_rne(e2m1(code) * 2^(s-127)), s = 255 -> NaN (exact otherwise)
 *   router  : fp64 serial sum of exact fp32 bf16*bf16 products, + bias;
 *             top-k on fp64 (strict >, lowest index wins ties); softmax in fp64 -> fp32
 *   gate_up : fp32 serial sum, + bias (fp32), clamped SwiGLU in fp32, -> bf16
 *   down    : fp32 serial sum, + bias (fp32), kept fp32
 *   combine : fp32 fmaf over k in k order, -> bf16 once
 *   rms_norm: fp32 256-way strided partial sums of squares (fmaf) + the kernel's tree,
 *             sqrtf(sum/H + eps), (v / rms) * weight -> bf16
 *   residual: bf16(float(a) + float(b))
 * Built with -ffp-contract=off so that "serial fp32 sum" means one rounding
 * per multiply and one per add.
 *
 * Parity status per function (how each is pinned, tests/test_oracle.py):
 *   or_mxfp4_value_bf16 / or_mxfp4_dequant : exhaustive 16x256 KAT derived from
 *       the OCP e2m1 bit definition with exact rationals; hand-built nibble-order
 *       and flat-block-index vectors.
 *   or_router / or_topk_softmax : fp64 numpy brute force (argsort-based top-k),
 *       hand-built ties, NaN, -inf; agreement with the reference's fp32 serial
 *       logits wherever the k/k+1 gap exceeds the fp32 error bound.
 *   or_bucket : permutation invariants + numpy stable argsort.
 *   or_swiglu : closed-form points (clamp corners, NaN propagation).
 *   or_moe_layer / or_moe_experts : float64 numpy brute force on tiny shapes
 *       using weights decoded by an independent decoder; the committed fixture
 *       tests/golden/tiny_layer.npz freezes that brute force for one seeded layer.
 *   or_legacy_* : float64 numpy brute force.
 *   or_rms_norm : closed forms (constant rows, a single nonzero element, power-of-two
 *       scaling of a row with eps = 0 leaves it unchanged), the float64 brute force
 *       within the fp32 error of the 256-way sum, and the summation order itself
 *       (a row built so that another order rounds differently).
 *   or_residual_add : exact float64 sums rounded to bf16 by an independent
 *       (numpy) rounding.
 *   or_moe_block : composition of the pinned functions above.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                         */
/* ------------------------------------------------------------------------- */

float or_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* e2m1 table: kernels/mxfp4_dequant.hip:12-17 (bit 3 = sign, code 8 = -0.0). */
static const float k_e2m1[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

float or_e2m1_value(int code) { return k_e2m1[code & 15]; }

/* value = LUT[code] * scale (kernels/mxfp4_dequant.hip:43-47), with the scale an
 * E8M0 byte 2^(s-127) instead of the reference's 16-bit float scale. */
uint16_t or_mxfp4_value_bf16(int code, int scale) {
    if ((scale & 255) == 255) return 0x7fc0u;
    float s = ldexpf(1.0f, (scale & 255) - 127); /* exact, 2^-127 is an fp32 subnormal */
    return or_f32_to_bf16(k_e2m1[code & 15] * s);
}

/* 256 scales x 16 codes table of bf16 results, built once. */
static uint16_t g_dq_tab[256][16];
static float g_dq_tab_f32[256][16];
static int g_dq_ready = 0;

static void dq_init(void) {
    if (g_dq_ready) return;
#ifdef _OPENMP
#pragma omp critical(or_dq_init)
#endif
    {
        if (!g_dq_ready) {
            for (int s = 0; s < 256; ++s)
                for (int c = 0; c < 16; ++c) {
                    g_dq_tab[s][c] = or_mxfp4_value_bf16(c, s);
                    g_dq_tab_f32[s][c] = or_bf16_to_f32(g_dq_tab[s][c]);
                }
            g_dq_ready = 1;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* standalone dequant: kernels/mxfp4_dequant.hip:19-51                         */
/* byte i low nibble -> element 2i, high nibble -> element 2i+1 (:35-36,47-49) */
/* scale index = element / block_size over the flat tensor (:43)              */
/* ------------------------------------------------------------------------- */
void or_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, uint16_t* out,
                      int64_t numel, int block_size, int nthreads) {
    dq_init();
    int64_t npairs = (numel + 1) / 2;
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
#endif
    for (int64_t i = 0; i < npairs; ++i) {
        int64_t v = 2 * i;
        uint8_t b = packed[i];
        int s = scales[v / block_size];
        out[v] = g_dq_tab[s][b & 15];
        if (v + 1 < numel) {
            /* the reference uses the scale of element 2i for both nibbles (:43,47-49) */
            out[v + 1] = g_dq_tab[s][b >> 4];
        }
    }
}

/* ------------------------------------------------------------------------- */
/* router: kernels/moe_router.hip:24-78                                        */
/* ------------------------------------------------------------------------- */

/* a ranks above b: strict '>' (moe_router.hip:50) with NaN ranked lowest. */
static int rank_gt(double a, double b) {
    if (isnan(a)) return 0;
    if (isnan(b)) return 1;
    return a > b;
}

/* Selection (moe_router.hip:45-59): k rounds, each taking the unused expert with the
 * largest logit; scanning e upward with a strict '>' keeps the lowest index on ties.
 * The reference starts each round from (-1e38, index 0) and can therefore return a
 * used index when no logit beats -1e38; here the first unused expert seeds the round,
 * so the k indices are always distinct.  Softmax over the selected k (:61-78):
 * subtract the max, exponentiate, divide by the k-order sum — computed in fp64 and
 * rounded to fp32 once. */
void or_topk_softmax(const double* lg, int E, int K, int32_t* idx, float* wts) {
    unsigned char used_small[1024];
    unsigned char* used = E <= 1024 ? used_small : (unsigned char*)calloc((size_t)E, 1);
    if (E <= 1024) memset(used, 0, (size_t)E);
    double sel[64];
    for (int j = 0; j < K; ++j) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (used[e]) continue;
            if (best < 0 || rank_gt(lg[e], lg[best])) best = e;
        }
        idx[j] = best;
        used[best] = 1;
        sel[j] = lg[best];
    }
    if (E > 1024) free(used);
    double m = sel[0];
    for (int j = 1; j < K; ++j) m = fmax(m, sel[j]);
    double ex[64], sum = 0.0;
    for (int j = 0; j < K; ++j) {
        ex[j] = exp(sel[j] - m);
        sum += ex[j];
    }
    for (int j = 0; j < K; ++j) wts[j] = (float)(ex[j] / sum);
}

void or_router(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int B, int H, int E,
               int K, int32_t* idx, float* wts, double* logits, int nthreads) {
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
#endif
    for (int b = 0; b < B; ++b) {
        double* lg = (double*)malloc(sizeof(double) * (size_t)E);
        const uint16_t* xr = x + (size_t)b * H;
        for (int e = 0; e < E; ++e) {
            const uint16_t* wr = w + (size_t)e * H;
            double acc = 0.0;
            for (int d = 0; d < H; ++d) {
                /* bf16*bf16 is exact in fp32 (8-bit x 8-bit significands). */
                float p = or_bf16_to_f32(xr[d]) * or_bf16_to_f32(wr[d]);
                acc += (double)p;
            }
            if (bias) acc += (double)or_bf16_to_f32(bias[e]);
            lg[e] = acc;
        }
        if (logits) memcpy(logits + (size_t)b * E, lg, sizeof(double) * (size_t)E);
        or_topk_softmax(lg, E, K, idx + (size_t)b * K, wts + (size_t)b * K);
        free(lg);
    }
}

/* moe_router.hip:25-35 as written: fp32 accumulator, serial d, no bias. */
void or_router_logits_fp32_serial(const uint16_t* x, const uint16_t* w, int B, int H, int E,
                                  float* logits) {
    for (int b = 0; b < B; ++b)
        for (int e = 0; e < E; ++e) {
            float acc = 0.0f;
            for (int d = 0; d < H; ++d)
                acc += or_bf16_to_f32(x[(size_t)b * H + d]) * or_bf16_to_f32(w[(size_t)e * H + d]);
            logits[(size_t)b * E + e] = acc;
        }
}

/* ------------------------------------------------------------------------- */
/* bucketing (no reference counterpart: the reference loops over k on the     */
/* host for one token, crates/llm-core/src/moe.rs:274-299)                     */
/* ------------------------------------------------------------------------- */
void or_bucket(const int32_t* idx, int B, int K, int E, int32_t* counts, int32_t* offsets,
               int32_t* perm, int32_t* pos) {
    int N = B * K;
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (int p = 0; p < N; ++p) counts[idx[p]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* fill = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    for (int p = 0; p < N; ++p) {
        int e = idx[p];
        int q = offsets[e] + fill[e]++;
        perm[q] = p;
        if (pos) pos[p] = q;
    }
    free(fill);
}

/* ------------------------------------------------------------------------- */
/* expert math                                                                 */
/* ------------------------------------------------------------------------- */

/* Clamped SwiGLU: g = min(g, limit); u = clamp(u, -limit, limit);
 * out = g * sigmoid(alpha*g) * (u + 1).  Comparisons are written so that NaN
 * propagates (a min/max instruction would drop it).  The reference's activation
 * is plain SiLU(g)*u (kernels/moe_expert_forward.hip:31-32); this clamped form is
 * the benchmark contract's replacement. */
float or_swiglu(float g, float u, float alpha, float limit) {
    g = (g > limit) ? limit : g;
    u = (u > limit) ? limit : ((u < -limit) ? -limit : u);
    float sig = 1.0f / (1.0f + expf(-alpha * g));
    return (g * sig) * (u + 1.0f);
}

/* Dequantize one MXFP4 row of `cols` elements to fp32 (row-local block index;
 * equal to the flat index because cols % 32 == 0). */
static void dequant_row_f32(const uint8_t* prow, const uint8_t* srow, int cols, float* out) {
    for (int blk = 0; blk < cols / 32; ++blk) {
        const float* t = g_dq_tab_f32[srow[blk]];
        const uint8_t* p = prow + blk * 16;
        float* o = out + blk * 32;
        for (int j = 0; j < 16; ++j) {
            o[2 * j] = t[p[j] & 15];
            o[2 * j + 1] = t[p[j] >> 4];
        }
    }
}

#define OR_TB 8 /* tokens per vector block: 8 independent serial fp32 chains */

/* acc[j] = sum_d act[j][d] * wrow[d] for OR_TB tokens, each a serial fp32 chain
 * (the per-row dot of kernels/moe_expert_forward.hip:24-28 / :48-50). */
static void dot_block(const float* restrict actT /* [cols][OR_TB] */,
                      const float* restrict wrow, int cols, float* restrict acc) {
    float a[OR_TB];
    for (int j = 0; j < OR_TB; ++j) a[j] = 0.0f;
    for (int d = 0; d < cols; ++d) {
        float wv = wrow[d];
        const float* xr = actT + (size_t)d * OR_TB;
        for (int j = 0; j < OR_TB; ++j) a[j] = a[j] + xr[j] * wv;
    }
    for (int j = 0; j < OR_TB; ++j) acc[j] = a[j];
}

/* Expert stage for a given routing, grouped by expert (each weight row is
 * dequantized once and applied to every token routed to the expert; each output
 * keeps the reference's serial order, so grouping does not change any bit). */
int or_moe_experts(const or_moe_cfg* cfg, const or_moe_weights* w, const uint16_t* x, int B,
                   const int32_t* idx, const float* wts, uint16_t* out, uint16_t* h_pairs,
                   float* y_pairs, int nthreads) {
    const int H = cfg->hidden, I = cfg->intermediate, E = cfg->num_experts, K = cfg->top_k;
    const int R = 2 * I, N = B * K;
    if (H % 32 || I % 32 || B < 0 || K < 1 || K > E) return -1;
    if (B == 0) return 0;
    if (nthreads < 1) nthreads = 1;
    dq_init();

    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
    or_bucket(idx, B, K, E, counts, offsets, perm, NULL);

    uint16_t* h = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)N * I); /* by sorted position */
    float* y = (float*)malloc(sizeof(float) * (size_t)N * H);          /* by sorted position */

    for (int e = 0; e < E; ++e) {
        int ne = counts[e];
        if (!ne) continue;
        int p0 = offsets[e];
        int nblk = (ne + OR_TB - 1) / OR_TB;
        /* transposed activations: [nblk][H][OR_TB] */
        float* xt = (float*)calloc((size_t)nblk * H * OR_TB, sizeof(float));
        for (int r = 0; r < ne; ++r) {
            int t = perm[p0 + r] / K;
            float* dst = xt + (size_t)(r / OR_TB) * H * OR_TB + (r % OR_TB);
            for (int d = 0; d < H; ++d) dst[(size_t)d * OR_TB] = or_bf16_to_f32(x[(size_t)t * H + d]);
        }
        float* G = (float*)malloc(sizeof(float) * (size_t)ne * R); /* pre-activation [ne][2I] */
        const uint8_t* gp = w->gate_up_blocks + (size_t)e * R * (H / 2);
        const uint8_t* gs = w->gate_up_scales + (size_t)e * R * (H / 32);
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
        {
            float* wrow = (float*)malloc(sizeof(float) * (size_t)H);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int r = 0; r < R; ++r) {
                dequant_row_f32(gp + (size_t)r * (H / 2), gs + (size_t)r * (H / 32), H, wrow);
                float bias = w->gate_up_bias ? or_bf16_to_f32(w->gate_up_bias[(size_t)e * R + r]) : 0.0f;
                for (int b = 0; b < nblk; ++b) {
                    float acc[OR_TB];
                    dot_block(xt + (size_t)b * H * OR_TB, wrow, H, acc);
                    for (int j = 0; j < OR_TB && b * OR_TB + j < ne; ++j)
                        G[(size_t)(b * OR_TB + j) * R + r] = acc[j] + bias;
                }
            }
            free(wrow);
        }
        for (int r = 0; r < ne; ++r)
            for (int i = 0; i < I; ++i)
                h[(size_t)(p0 + r) * I + i] = or_f32_to_bf16(
                    or_swiglu(G[(size_t)r * R + 2 * i], G[(size_t)r * R + 2 * i + 1], cfg->alpha, cfg->limit));
        free(G);
        free(xt);

        /* down projection: y[p][r] = sum_i h[p][i] * Wd[r][i] + bias */
        float* ht = (float*)calloc((size_t)nblk * I * OR_TB, sizeof(float));
        for (int r = 0; r < ne; ++r) {
            float* dst = ht + (size_t)(r / OR_TB) * I * OR_TB + (r % OR_TB);
            for (int i = 0; i < I; ++i) dst[(size_t)i * OR_TB] = or_bf16_to_f32(h[(size_t)(p0 + r) * I + i]);
        }
        const uint8_t* dp = w->down_blocks + (size_t)e * H * (I / 2);
        const uint8_t* ds = w->down_scales + (size_t)e * H * (I / 32);
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
        {
            float* wrow = (float*)malloc(sizeof(float) * (size_t)I);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int r = 0; r < H; ++r) {
                dequant_row_f32(dp + (size_t)r * (I / 2), ds + (size_t)r * (I / 32), I, wrow);
                float bias = w->down_bias ? or_bf16_to_f32(w->down_bias[(size_t)e * H + r]) : 0.0f;
                for (int b = 0; b < nblk; ++b) {
                    float acc[OR_TB];
                    dot_block(ht + (size_t)b * I * OR_TB, wrow, I, acc);
                    for (int j = 0; j < OR_TB && b * OR_TB + j < ne; ++j)
                        y[(size_t)(p0 + b * OR_TB + j) * H + r] = acc[j] + bias;
                }
            }
            free(wrow);
        }
        free(ht);
    }

    /* pair-id views */
    int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
    for (int q = 0; q < N; ++q) pos[perm[q]] = q;
    if (h_pairs)
        for (int p = 0; p < N; ++p) memcpy(h_pairs + (size_t)p * I, h + (size_t)pos[p] * I, sizeof(uint16_t) * (size_t)I);
    if (y_pairs)
        for (int p = 0; p < N; ++p) memcpy(y_pairs + (size_t)p * H, y + (size_t)pos[p] * H, sizeof(float) * (size_t)H);

    /* combine: kernels/moe_combine.hip:16-20 — fp32 sum in k order, one rounding. */
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
    for (int t = 0; t < B; ++t) {
        for (int d = 0; d < H; ++d) {
            float acc = 0.0f;
            for (int j = 0; j < K; ++j) acc = fmaf(wts[(size_t)t * K + j], y[(size_t)pos[t * K + j] * H + d], acc);
            out[(size_t)t * H + d] = or_f32_to_bf16(acc);
        }
    }
    free(pos);
    free(h);
    free(y);
    free(counts);
    free(offsets);
    free(perm);
    return 0;
}

/* Layer order of crates/llm-core/src/moe.rs:246-307: router -> experts -> combine
 * (the rms_norm before and the residual add after are outside this path). */
int or_moe_layer(const or_moe_cfg* cfg, const or_moe_weights* w, const uint16_t* x, int B,
                 uint16_t* out, int32_t* idx, float* wts, uint16_t* h_pairs, float* y_pairs,
                 int nthreads) {
    const int E = cfg->num_experts, K = cfg->top_k, H = cfg->hidden;
    if (B < 0 || K < 1 || K > E || K > 64) return -1;
    if (B == 0) return 0;
    int32_t* ix = idx ? idx : (int32_t*)malloc(sizeof(int32_t) * (size_t)B * K);
    float* ws = wts ? wts : (float*)malloc(sizeof(float) * (size_t)B * K);
    or_router(x, w->router_w, w->router_b, B, H, E, K, ix, ws, NULL, nthreads);
    int rc = or_moe_experts(cfg, w, x, B, ix, ws, out, h_pairs, y_pairs, nthreads);
    if (!idx) free(ix);
    if (!wts) free(ws);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* the steps either side of the layer: rms_norm before, residual add after      */
/* ------------------------------------------------------------------------- */

/* kernels/rms_norm_gpu.hip:4-31 with bf16 data: per row, thread j of the
 * 256-thread block sums v*v over i = j, j + 256, ... in order (:11-15); the block
 * adds the 256 partials by its shared-memory tree, s = 128, 64, ..., 1:
 * p[j] += p[j + s] for j < s (:18-21); rms = sqrtf(p[0] / H + eps) (:24);
 * out[i] = round((v / rms) * weight[i]) (:30). fp32 throughout. `tsum += v * v` (:14)
 * is one fmaf: hipcc contracts it so under HIP's default -ffp-contract=fast-honor-pragmas.
 * For bf16 v the product is exact in fp32 unless |v| < 2^-63, so only rows that small
 * can tell the fused from the unfused form. */
void or_rms_norm(const uint16_t* x, const uint16_t* wt, uint16_t* out, int B, int H, float eps) {
    for (int b = 0; b < B; ++b) {
        const uint16_t* row = x + (size_t)b * H;
        float p[256];
        for (int j = 0; j < 256; ++j) {
            float t = 0.0f;
            for (int i = j; i < H; i += 256) {
                const float v = or_bf16_to_f32(row[i]);
                t = fmaf(v, v, t);
            }
            p[j] = t;
        }
        for (int s2 = 128; s2 > 0; s2 >>= 1)
            for (int j = 0; j < s2; ++j) p[j] = p[j] + p[j + s2];
        const float rms = sqrtf(p[0] / (float)H + eps);
        for (int i = 0; i < H; ++i) {
            const float v = or_bf16_to_f32(row[i]);
            const float q = v / rms;
            out[(size_t)b * H + i] = or_f32_to_bf16(q * or_bf16_to_f32(wt[i]));
        }
    }
}

/* kernels/residual_add.hip:4-10 with bf16 data: out[i] = round(out[i] + res[i]) in fp32. */
void or_residual_add(uint16_t* out, const uint16_t* res, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(or_bf16_to_f32(out[i]) + or_bf16_to_f32(res[i]));
}

/* The MoE sub-layer of crates/llm-core/src/moe.rs:238-313: h = rms_norm(x) (:240-244),
 * the layer (or_moe_layer, :246-307), then the residual add into the hidden state
 * (:310): out = round(moe(h) + x). */
int or_moe_block(const or_moe_cfg* cfg, const or_moe_weights* w, const uint16_t* x, const uint16_t* norm_w,
                 float eps, int B, uint16_t* out, int32_t* idx, float* wts, int nthreads) {
    const int H = cfg->hidden;
    if (B < 0) return -1;
    if (B == 0) return 0;
    uint16_t* h = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * H);
    or_rms_norm(x, norm_w, h, B, H, eps);
    const int rc = or_moe_layer(cfg, w, h, B, out, idx, wts, NULL, NULL, nthreads);
    free(h);
    if (rc) return rc;
    or_residual_add(out, x, (size_t)B * H);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* legacy single-token kernels                                                 */
/* ------------------------------------------------------------------------- */

/* kernels/moe_expert_forward.hip:19-32: g = x.Wg[i], u = x.Wu[i] (fp32 serial),
 * inter[i] = 16-bit(SiLU(g) * u). */
void or_legacy_expert_silu(const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
                           uint16_t* out, int H, int I) {
    for (int i = 0; i < I; ++i) {
        float g = 0.0f, u = 0.0f;
        for (int d = 0; d < H; ++d) {
            float xv = or_bf16_to_f32(x[d]);
            g = g + xv * or_bf16_to_f32(wg[(size_t)i * H + d]);
            u = u + xv * or_bf16_to_f32(wu[(size_t)i * H + d]);
        }
        float silu = g / (1.0f + expf(-g));
        out[i] = or_f32_to_bf16(silu * u);
    }
}

/* kernels/moe_expert_forward.hip:44-51: y[h] = inter . Wd[h] (fp32 serial) -> 16-bit. */
void or_legacy_expert_down(const uint16_t* inter, const uint16_t* wd, uint16_t* out, int H, int I) {
    for (int r = 0; r < H; ++r) {
        float s = 0.0f;
        for (int i = 0; i < I; ++i) s = s + or_bf16_to_f32(inter[i]) * or_bf16_to_f32(wd[(size_t)r * I + i]);
        out[r] = or_f32_to_bf16(s);
    }
}

/* kernels/moe_combine.hip:16-20: out[d] = sum_k w[k] * y[k][d] in k order -> 16-bit. */
void or_legacy_combine(const uint16_t* y, const float* w, uint16_t* out, int H, int K) {
    for (int d = 0; d < H; ++d) {
        float s = 0.0f;
        for (int k = 0; k < K; ++k) s = fmaf(w[k], or_bf16_to_f32(y[(size_t)k * H + d]), s);
        out[d] = or_f32_to_bf16(s);
    }
}
