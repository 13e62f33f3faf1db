/*
 * CPU oracle for the MXFP4 MoE expert path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference algorithm (PhysLLM,
 * kernels/moe_router.hip, kernels/mxfp4_dequant.hip, kernels/moe_expert_forward.hip,
 * kernels/moe_combine.hip, crates/llm-core/src/moe.rs) with the bf16 / E8M0 /
 * bias / clamped-SwiGLU semantics that the benchmark contract specifies.
 * Only the test suite, the smoke check and the CPU-baseline leg of the bench
 * may load it; the product library never links or calls it.
 *
 * All 16-bit activations and weights are bf16 bit patterns (uint16_t).
 * All functions are thread-safe and deterministic; the OpenMP-parallel ones
 * keep every output element's serial arithmetic order, so results do not
 * depend on the thread count.
 */
#ifndef PHYSLLM_MOE_ORACLE_H
#define PHYSLLM_MOE_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions --------------------------------------------------- */
float    or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_bf16(float f);                  /* round-to-nearest-even, NaN -> quiet NaN */
float    or_e2m1_value(int code);                  /* 4-bit e2m1 code -> value (code 8 = -0.0) */
uint16_t or_mxfp4_value_bf16(int code, int scale); /* bf16(e2m1(code) * 2^(scale-127)); scale 255 -> NaN */

/* ---- standalone dequant (flat block index = element / block_size) -------- */
void or_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, uint16_t* out,
                      int64_t numel, int block_size, int nthreads);

/* ---- router ----------------------------------------------------------------*/
/* logits[b,e] = sum_d x[b,d]*w[e,d] (fp64, serial d) + bias[e]; top-k; softmax over k. */
void or_router(const uint16_t* x, const uint16_t* w, const uint16_t* bias /* nullable */,
               int B, int H, int E, int K, int32_t* idx, float* wts,
               double* logits /* nullable [B,E] */, int nthreads);
/* The reference's own logit arithmetic: fp32, serial d, no bias. */
void or_router_logits_fp32_serial(const uint16_t* x, const uint16_t* w, int B, int H, int E,
                                  float* logits);
/* Selection + softmax given logits (exposed for tie/NaN tests). */
void or_topk_softmax(const double* logits, int E, int K, int32_t* idx, float* wts);

/* ---- bucketing ----------------------------------------------------------- */
/* counts[E], offsets[E+1], perm[N] (sorted position -> pair id t*K+j),
 * pos[N] (pair id -> sorted position); sorted by expert, then by pair id. */
void or_bucket(const int32_t* idx, int B, int K, int E, int32_t* counts, int32_t* offsets,
               int32_t* perm, int32_t* pos);

/* ---- expert math ---------------------------------------------------------- */
float or_swiglu(float g, float u, float alpha, float limit);

typedef struct or_moe_cfg {
    int hidden;        /* H */
    int intermediate;  /* I */
    int num_experts;   /* E */
    int top_k;         /* K */
    float alpha;       /* 1.702 */
    float limit;       /* 7.0 */
} or_moe_cfg;

typedef struct or_moe_weights {
    const uint16_t* router_w;      /* [E,H] bf16 */
    const uint16_t* router_b;      /* [E] bf16, nullable */
    const uint8_t*  gate_up_blocks;/* [E,2I,H/2]; row 2i = gate_i, row 2i+1 = up_i */
    const uint8_t*  gate_up_scales;/* [E,2I,H/32] E8M0 */
    const uint16_t* gate_up_bias;  /* [E,2I] bf16, nullable */
    const uint8_t*  down_blocks;   /* [E,H,I/2] */
    const uint8_t*  down_scales;   /* [E,H,I/32] */
    const uint16_t* down_bias;     /* [E,H] bf16, nullable */
} or_moe_weights;

/* Full layer: router -> bucket -> gate_up+SwiGLU -> down -> combine.
 * out [B,H] bf16. Optional outputs (nullable): idx/wts [B,K]; h_pairs [B*K, I] bf16 and
 * y_pairs [B*K, H] fp32, both indexed by pair id t*K+j. Returns 0 on success. */
int or_moe_layer(const or_moe_cfg* cfg, const or_moe_weights* w, const uint16_t* x, int B,
                 uint16_t* out, int32_t* idx, float* wts, uint16_t* h_pairs, float* y_pairs,
                 int nthreads);

/* Expert stage given a routing (used to time/compare the expert math alone). */
int or_moe_experts(const or_moe_cfg* cfg, const or_moe_weights* w, const uint16_t* x, int B,
                   const int32_t* idx, const float* wts, uint16_t* out, uint16_t* h_pairs,
                   float* y_pairs, int nthreads);

/* ---- legacy single-token kernels (dense bf16 weights, reference arithmetic) --- */
void or_legacy_expert_silu(const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
                           uint16_t* out, int H, int I);
void or_legacy_expert_down(const uint16_t* inter, const uint16_t* wd, uint16_t* out,
                           int H, int I);
void or_legacy_combine(const uint16_t* y, const float* w, uint16_t* out, int H, int K);

/* the steps either side of the layer (kernels/rms_norm_gpu.hip, kernels/residual_add.hip)
 * and the sub-layer they bracket (crates/llm-core/src/moe.rs:238-313) */
void or_rms_norm(const uint16_t* x, const uint16_t* wt, uint16_t* out, int B, int H, float eps);
void or_residual_add(uint16_t* out, const uint16_t* res, size_t n);
int or_moe_block(const or_moe_cfg* cfg, const or_moe_weights* w, const uint16_t* x, const uint16_t* norm_w,
                 float eps, int B, uint16_t* out, int32_t* idx, float* wts, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
