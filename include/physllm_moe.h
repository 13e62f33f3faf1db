/*
 * physllm_moe.h — C ABI of the MI355X (gfx950) MXFP4 Mixture-of-Experts expert path.
 *
 * Drop-in for PhysLLM's MoE kernels. The five MoE legacy launchers keep the exact
 * prototypes that crates/rocm-backend/src/ops.rs:554-594 binds, and the RMSNorm and
 * residual-add launchers those of ops.rs:315-332, so the Rust wrappers
 * (ops.rs:366-384, :421-435, :597-696) link against this library unchanged. The extension
 * entry points carry what the legacy ABI cannot express: biases, MXFP4 expert
 * weights with E8M0 scales, batched and grouped tokens, and a caller-owned
 * workspace.
 *
 * Conventions (all entry points):
 *  - Every pointer is caller-owned device memory (hipMalloc); nothing here
 *    allocates device memory. `stream` is a hipStream_t (NULL = default stream).
 *  - Launches are asynchronous. Sizes are int32 unless stated.
 *  - 16-bit activations and weights are bf16 bit patterns (the Rust side carries
 *    them in DeviceTensor<f16> storage). Routing weights are fp32, indices int32.
 *  - MXFP4: one byte holds two e2m1 codes, the element with the lower index in the
 *    low nibble; one E8M0 scale byte (value 2^(s-127), 255 = NaN) per 32
 *    consecutive elements along the row (the input dimension).
 *  - Legacy launchers return void (as the reference's do); argument errors are
 *    reported through physllm_moe_last_error(). Extension entry points return
 *    0 on success or a negative PHYSLLM_MOE_E* code and also set the last error.
 *  - Calls on one stream are ordered; two calls that share a workspace must be
 *    on the same stream or be ordered by the caller.
 */
#ifndef PHYSLLM_MOE_H
#define PHYSLLM_MOE_H

#include <stddef.h>
#include <stdint.h>

#if defined(PHYSLLM_MOE_BUILD)
#define PHYSLLM_MOE_API __attribute__((visibility("default")))
#else
#define PHYSLLM_MOE_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------- */
/* Error channel                                                              */
/* ------------------------------------------------------------------------- */
#define PHYSLLM_MOE_OK 0
#define PHYSLLM_MOE_EINVAL (-1)     /* bad argument (size, null pointer, limit) */
#define PHYSLLM_MOE_EWORKSPACE (-2) /* workspace missing or too small */
#define PHYSLLM_MOE_ELAUNCH (-3)    /* HIP launch error */

/* Code of the last error on the calling thread (0 if the last call succeeded). */
PHYSLLM_MOE_API int physllm_moe_last_error(void);
/* Message of the last error on the calling thread ("" if none). */
PHYSLLM_MOE_API const char* physllm_moe_last_error_message(void);

/* ------------------------------------------------------------------------- */
/* Legacy launchers — prototypes of crates/rocm-backend/src/ops.rs:554-594     */
/* ------------------------------------------------------------------------- */

/* Replaces kernels/moe_router.hip:82-104 (bound at ops.rs:556-563).
 * hidden [batch,hidden_dim] bf16, router_weight [num_experts,hidden_dim] bf16,
 * expert_indices [batch,top_k] int32, expert_weights [batch,top_k] fp32.
 * logits = hidden . W^T accumulated in fp64 (no bias); top_k in descending logit
 * order, ties to the lowest index; softmax over the selected k.
 * Limits: 1 <= top_k <= min(num_experts, 32), num_experts <= 1024. */
PHYSLLM_MOE_API void launch_moe_router(const void* hidden, const void* router_weight, void* expert_indices,
                       void* expert_weights, int batch_size, int hidden_dim, int num_experts,
                       int top_k, void* stream);

/* Replaces kernels/moe_expert_forward.hip:54-68 (bound at ops.rs:564-570).
 * One token: input [hidden_dim] bf16, w_gate/w_up dense [intermediate_dim,hidden_dim]
 * bf16 row-major, output [intermediate_dim] bf16 = SiLU(x.Wg) * (x.Wu), fp32 sums. */
PHYSLLM_MOE_API void launch_moe_expert_silu(const void* input, const void* w_gate, const void* w_up,
                            void* output, int hidden_dim, int intermediate_dim, void* stream);

/* Replaces kernels/moe_expert_forward.hip:70-82 (bound at ops.rs:571-576).
 * input [intermediate_dim] bf16, w_down [hidden_dim,intermediate_dim] bf16,
 * output [hidden_dim] bf16. */
PHYSLLM_MOE_API void launch_moe_expert_down(const void* input, const void* w_down, void* output,
                            int hidden_dim, int intermediate_dim, void* stream);

/* Replaces kernels/moe_combine.hip:23-37 (bound at ops.rs:577-582).
 * expert_outputs [top_k,hidden_dim] bf16, expert_weights [top_k] fp32,
 * output [hidden_dim] bf16 = sum over k in k order (fp32), rounded once. */
PHYSLLM_MOE_API void launch_moe_combine(const void* expert_outputs, const void* expert_weights, void* output,
                        int hidden_dim, int top_k, void* stream);

/* Replaces kernels/mxfp4_dequant.hip:53-68 (bound at ops.rs:583-589).
 * packed_data [ceil(numel/2)] u8, scales [ceil(numel/block_size)] E8M0 u8,
 * output [numel] bf16 = e2m1(code) * 2^(s-127), bit-exact (s = 255 gives NaN 0x7FC0).
 * The scale of element 2i also serves element 2i+1 (the reference's indexing). */
PHYSLLM_MOE_API void launch_mxfp4_dequant(const void* packed_data, const void* scales, void* output, int numel,
                          int block_size, void* stream);

/* Replaces kernels/rms_norm_gpu.hip:36-45 (bound at crates/rocm-backend/src/ops.rs:315-319,
 * wrapped at ops.rs:366-384 and called before the router at moe.rs:239-244).
 * input [batch_size,hidden_dim] bf16, weight [hidden_dim] bf16, output like input
 * (may equal input). Per row: sum of v*v in the reference kernel's order (256
 * strided fp32 partials, one fma per element, then its shared-memory tree),
 * rms = sqrtf(sum / hidden_dim + eps), output = bf16((v / rms) * weight).
 * Bit-identical to that order for bf16 data. */
PHYSLLM_MOE_API void launch_rms_norm(const void* input, const void* weight, void* output, int batch_size,
                     int hidden_dim, float eps, void* stream);

/* Replaces kernels/residual_add.hip:12-19 (bound at ops.rs:329-332, wrapped at
 * ops.rs:421-435, called after the combine at moe.rs:310-311).
 * output[i] = bf16(output[i] + residual[i]) in fp32, for i < size (bf16 data). */
PHYSLLM_MOE_API void launch_residual_add(void* output, const void* residual, int size, void* stream);

/* ------------------------------------------------------------------------- */
/* Extension entry points (no reference counterpart; they carry the benchmark */
/* semantics: biases, MXFP4 experts, batching). Callers: the bench/test       */
/* drivers and Rust wrappers written in the ops.rs:597-696 style.             */
/* ------------------------------------------------------------------------- */

typedef struct physllm_moe_config {
    int hidden;         /* H, multiple of 32 (GPT-OSS: 2880) */
    int intermediate;   /* I, multiple of 32 (GPT-OSS: 2880) */
    int num_experts;    /* E, <= 1024 */
    int top_k;          /* k, 1 <= k <= min(E, 32) */
    float swiglu_alpha; /* 1.702 */
    float swiglu_limit; /* 7.0 */
    /* Tokens per internal chunk (0 = automatic). The layer and block entry points run
     * a batch as consecutive chunks over one workspace, because every buffer range a
     * kernel reads must stay below 2^31 bytes: x [b,H] and h [b*k,I] bf16 give
     * b <= (2^31 - 2^20) / max(2H, 2kI), 93,161 tokens at the GPT-OSS shape (k = 4).
     * A positive value lowers the chunk size (and the workspace) further. Results do
     * not depend on the chunking as long as every chunk takes the same kernels. */
    int max_chunk_tokens;
} physllm_moe_config;

/* Expert weights, all device pointers. Layout:
 *  router_w       [E,H] bf16          router_b     [E] bf16 (nullable)
 *  gate_up_blocks [E,2I,H/2] u8       row 2i = gate_i, row 2i+1 = up_i (interleaved)
 *  gate_up_scales [E,2I,H/32] u8      gate_up_bias [E,2I] bf16 (nullable)
 *  down_blocks    [E,H,I/2] u8        down_scales  [E,H,I/32] u8
 *  down_bias      [E,H] bf16 (nullable) */
typedef struct physllm_moe_weights {
    const void* router_w;
    const void* router_b;
    const void* gate_up_blocks;
    const void* gate_up_scales;
    const void* gate_up_bias;
    const void* down_blocks;
    const void* down_scales;
    const void* down_bias;
} physllm_moe_weights;

/* Workspace bytes physllm_moe_layer_forward needs for `batch` tokens (sized for one
 * chunk; see max_chunk_tokens). Limits (EINVAL, and 0 from the size queries): one
 * expert's codes, I * H bytes, and the router rows, E * H * 2 bytes, below 2^31. */
PHYSLLM_MOE_API size_t physllm_moe_workspace_bytes(const physllm_moe_config* cfg, int batch);

/* Whole MoE layer (the MoE half of crates/llm-core/src/moe.rs:246-307, without the
 * rms_norm before and the residual add after):
 *   router (fp64 logits + bias, top-k, softmax) -> bucketing by expert ->
 *   gate_up MXFP4 GEMV/GEMM + bias + clamped SwiGLU -> down MXFP4 + bias ->
 *   weighted combine in k order.
 * x [batch,H] bf16, out [batch,H] bf16. topk_idx [batch,k] int32 and topk_w
 * [batch,k] fp32 are optional outputs (nullable). No host synchronisation. */
PHYSLLM_MOE_API int physllm_moe_layer_forward(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                              const void* x, int batch, void* out, void* topk_idx,
                              void* topk_w, void* workspace, size_t workspace_bytes,
                              void* stream);

/* physllm_moe_layer_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops); it has
 * no counterpart in the reference. It calls no allocating routine: the workspace is a
 * 64 MiB array in the library's device code object, one per device, held until the
 * process ends (looked up once per device on the first call there: make one call on a
 * device before capturing this entry point into a HIP graph). A batch whose
 * workspace (physllm_moe_workspace_bytes) exceeds 64 MiB is EINVAL: up to about 950
 * tokens at the GPT-OSS-20B shape, more with a smaller max_chunk_tokens. Calls that
 * overlap on one device share that array and race: order them on one stream. */
PHYSLLM_MOE_API int physllm_moe_layer_forward_noalloc(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                                      const void* x, int batch, void* out, void* topk_idx,
                                      void* topk_w, void* stream);

/* The same layer as four stages over one workspace, in this order on one stream
 * (used to time each stage and to run them from separate call sites):
 *   route   : router + bucketing; routing kept in the workspace (or topk_idx/topk_w);
 *   gate_up : MXFP4 gate_up + bias + clamped SwiGLU -> h [batch*k, I] in the workspace;
 *   down    : MXFP4 down + bias -> y [batch*k, H] fp32 in the workspace;
 *   combine : out [batch,H] bf16 = sum over k (k order) of w * y.
 * topk_w passed to combine must be the topk_w given to route (NULL if none was).
 * Each stage call covers one chunk: batch above the chunk limit is EINVAL. */
PHYSLLM_MOE_API int physllm_moe_stage_route(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                            const void* x, int batch, void* topk_idx, void* topk_w,
                            void* workspace, size_t workspace_bytes, void* stream);
PHYSLLM_MOE_API int physllm_moe_stage_gate_up(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                              const void* x, int batch, void* workspace, size_t workspace_bytes,
                              void* stream);
PHYSLLM_MOE_API int physllm_moe_stage_down(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                           int batch, void* workspace, size_t workspace_bytes, void* stream);
PHYSLLM_MOE_API int physllm_moe_stage_combine(const physllm_moe_config* cfg, int batch, void* out,
                              const void* topk_w, void* workspace, size_t workspace_bytes,
                              void* stream);

/* The layer at one or two tokens runs as three launches when its shape allows
 * (E <= 256, k <= 4, H and I <= 2944, 16-byte aligned x and router rows): 0 the
 * router logits, 1 gate_up with the top-k selection made inside every workgroup,
 * 2 down with the weighted combine. This runs launch `launch` alone on the state the
 * earlier launches left in the workspace (0, 1, 2 in order reproduce
 * physllm_moe_layer_forward's output bit for bit; routing stays in the workspace).
 * It has no counterpart in the reference: it exists to time and inspect the
 * batch-1 launches. EINVAL when the batch-1 launches do not serve cfg and batch. */
PHYSLLM_MOE_API int physllm_moe_stage_batch1(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                             const void* x, int batch, int launch, void* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Workspace bytes physllm_moe_block_forward needs for `batch` tokens (the layer's
 * workspace plus the normalised activations). */
PHYSLLM_MOE_API size_t physllm_moe_block_workspace_bytes(const physllm_moe_config* cfg, int batch);

/* The MoE sub-layer of a transformer block, crates/llm-core/src/moe.rs:238-313:
 *   h = rms_norm(x, norm_w, eps)   (moe.rs:239-244, kernels/rms_norm_gpu.hip:4-31)
 *   m = physllm_moe_layer_forward(h)                    (moe.rs:246-307)
 *   out = bf16(m + x)              (moe.rs:310-311, kernels/residual_add.hip:4-10)
 * x, out [batch,H] bf16; norm_w [H] bf16. out may equal x (in place, as the
 * reference updates its residual buffer). topk_idx / topk_w as for the layer. */
PHYSLLM_MOE_API int physllm_moe_block_forward(const physllm_moe_config* cfg, const physllm_moe_weights* w,
                              const void* x, const void* norm_w, float eps, int batch, void* out,
                              void* topk_idx, void* topk_w, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Router with bias: x [batch,H] bf16, router_w [E,H] bf16, router_b [E] bf16
 * (nullable); writes idx [batch,k] int32 and w [batch,k] fp32. */
PHYSLLM_MOE_API int physllm_moe_route_topk(const void* x, const void* router_w, const void* router_b, int batch,
                           int hidden, int num_experts, int top_k, void* idx, void* w,
                           void* stream);

/* Bucketing of idx [batch,k] by expert (counting sort, stable in pair id t*k+j):
 * counts [E], offsets [E+1], perm [batch*k] (sorted position -> pair id),
 * pos [batch*k] (pair id -> sorted position). */
PHYSLLM_MOE_API int physllm_moe_bucket(const void* idx, int batch, int top_k, int num_experts, void* counts,
                       void* offsets, void* perm, void* pos, void* stream);

/* MXFP4 -> bf16 dequant with a 64-bit element count; block size 32. */
PHYSLLM_MOE_API int physllm_moe_mxfp4_dequant(const void* packed, const void* scales, void* out, int64_t numel,
                              void* stream);

/* Replaces the transposing dequant of kernels/mxfp4_dequant_v2.hip:41-70 (a kernel the
 * reference declares without a host launcher). blocks / scales hold [num_experts,
 * out_dim, in_dim] as the flat dequant reads them: element f = (e*out_dim + o)*in_dim + i
 * has its code in the low (f even) or high nibble of byte f/2 and its E8M0 scale at
 * scales[f / block_size] (per element, as at :60-63). output [num_experts, in_dim,
 * out_dim] bf16 receives element f at (e*in_dim + i)*out_dim + o, bit-exact as in the
 * flat dequant. Any shape and block_size >= 1; block_size 32 with in_dim % 32 == 0,
 * out_dim % 8 == 0, 16-byte-aligned blocks and 16-byte-aligned output takes the
 * LDS-tiled kernel. */
PHYSLLM_MOE_API int physllm_moe_mxfp4_dequant_transpose(const void* blocks, const void* scales, void* output,
                                        int num_experts, int out_dim, int in_dim, int block_size,
                                        void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PHYSLLM_MOE_H */
