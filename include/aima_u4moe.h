/*
 * aima_u4moe.h -- C ABI of the MI355X U4 MoE expert hot path.
 *
 * One shared library, libaima_u4moe.so, hand-written HIP for gfx950.  Every
 * entry point:
 *   - takes caller-owned DEVICE pointers and plain sizes (no framework types);
 *   - enqueues asynchronously on `stream` (a hipStream_t, NULL = default
 *     stream) and never synchronizes the host;
 *   - returns AIMA_OK or a negative AIMA_E_* code, with a thread-local message
 *     in aima_last_error(); nothing is thrown across the ABI;
 *   - is re-entrant across distinct streams when given distinct workspaces.
 * Entry points that need scratch memory take a caller-owned workspace whose
 * size the matching *_workspace_size function reports; they allocate nothing.
 *
 * U4 group-quantized matrix W[N][K] (the boundary layout, from the OpenVINO IR
 * constants traced by tools/intel_qwen36_openvino_fixed_fc.py:107-144,241-265
 * and consumed by engine/openvino/custom/iq36_fixed_fc_multi_output.cl:118-127):
 *   qweight  u8 [N][K/2]     low nibble = even k, high nibble = odd k
 *   scale    f16[N][K/g]     row-major per (row, group)
 *   zp       u4 over the flat [N*(K/g)] index, two per byte, low nibble = even
 *   w[n][k] = f32(q - z) * f32(s)
 * Expert stacks are E such matrices back to back.  A routed gate/up stack has
 * 2*I rows per expert: rows 0..I-1 gate, I..2I-1 up (the CPU reference's
 * convention, engine/src/gguf_loader.cpp:4654-4660).
 *
 * f16 values travel as uint16_t bit patterns.
 */
#ifndef AIMA_U4MOE_H_
#define AIMA_U4MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIMA_OK 0
#define AIMA_E_INVALID (-1)   /* bad size, shape, alignment or null pointer */
#define AIMA_E_RANGE (-2)     /* expert id out of range / duplicated (device flag) */
#define AIMA_E_HIP (-3)       /* a HIP runtime call failed */
#define AIMA_E_WORKSPACE (-4) /* workspace missing or too small */
#define AIMA_E_UNSUPPORTED (-5) /* shape outside what the kernels implement */

/* Bits of the device error word kept at the start of every workspace.  They
 * mirror the reference device-schedule error bits (1 = out of range,
 * 2 = duplicated within a token; grouped_s8_u4_f16_contribution_moe.cl:38-53). */
#define AIMA_DEVERR_EXPERT_RANGE 1u
#define AIMA_DEVERR_EXPERT_DUPLICATE 2u
#define AIMA_DEVERR_TIMEOUT 4u /* a persistent-kernel wait hit its spin limit */

#define AIMA_OUT_F16 0
#define AIMA_OUT_F32 1
/* Most outputs of one aima_u4_matvec_multi call. */
#define AIMA_MAX_MULTI_OUT 4

/* Device pointers of one U4 matrix or expert stack. */
typedef struct aima_u4_tensor {
  const uint8_t* qweight;
  const uint16_t* scale;
  const uint8_t* zp;
} aima_u4_tensor;

/* One MoE FFN layer, all device pointers.
 *   gate_up        E x [2*inter][hidden]  (rows 0..inter-1 gate, then up)
 *   down           E x [hidden][inter]
 *   shared_gate_up 1 x [2*shared_inter][hidden]
 *   shared_down    1 x [hidden][shared_inter]
 *   shared_gate_vec f16[hidden]; the shared expert is scaled by
 *                   sigmoid(dot(shared_gate_vec, h))
 *   norm_weight    f32[hidden] RMSNorm weight applied before the layer by the
 *                   stack entry points (may be NULL for single-layer calls).
 *   up, shared_up  optional separate up projections, the operand form of the
 *                   OpenVINO op MOE3GemmFusedCompressed(hidden, routing_logits,
 *                   gate_w, gate_scale, gate_zp, up_w, up_scale, up_zp, down_*)
 *                   (engine/openvino/iq36-fixed-fc-moe-router-compat.patch:49-56):
 *                   when up.qweight is non-NULL, gate_up holds ONLY the gate
 *                   rows, E x [inter][hidden], and up the up rows,
 *                   E x [inter][hidden] (likewise shared_up / shared_gate_up
 *                   with 1 x [shared_inter][hidden]).  All-NULL (zeroed) = the
 *                   concatenated form.  No entry point repacks either form. */
typedef struct aima_moe_layer {
  aima_u4_tensor gate_up;
  aima_u4_tensor down;
  aima_u4_tensor shared_gate_up;
  aima_u4_tensor shared_down;
  const uint16_t* shared_gate_vec;
  const float* norm_weight;
  int32_t hidden;
  int32_t inter;
  int32_t shared_inter;
  int32_t experts;
  int32_t group;
  aima_u4_tensor up;
  aima_u4_tensor shared_up;
} aima_moe_layer;

/* Thread-local description of the last failure on this thread. */
const char* aima_last_error(void);

/* Library ABI version (major*100 + minor); 101 added the split up tensors of
 * aima_moe_layer and aima_moe_grouped_prefill_ex. */
int aima_version(void);

/* Exact dequantization out[n][k] = f32(q - z) * f32(s) (bit-exact with the
 * OpenVINO decompression subgraph Convert -> Subtract(zp) -> Multiply(scale),
 * tools/intel_qwen36_openvino_fixed_fc.py:111-119).  K % group == 0,
 * group % 32 == 0. */
int aima_u4_dequant(const uint8_t* qweight, const uint16_t* scale,
                    const uint8_t* zp, int64_t n, int64_t k, int32_t group,
                    float* out, void* stream);

/* The same dequantization rounded once to f16: out[n][k] = f16(f32(q - z) *
 * f32(s)) (round to nearest even, f16 subnormals kept), computed by the very
 * routine that builds the grouped prefill GEMM's f16 MFMA weight operand --
 * the weight form of the reference's f16 decompression path
 * (engine/openvino/custom/iq36_fixed_fc_multi_output.cl:118-128 dequantizes
 * in f32; OpenVINO's f16 inference precision rounds the product to f16).
 * Same size rules as aima_u4_dequant; out 16-byte aligned. */
int aima_u4_dequant_f16(const uint8_t* qweight, const uint16_t* scale,
                        const uint8_t* zp, int64_t n, int64_t k, int32_t group,
                        uint16_t* out, void* stream);

/* Batch-1 U4 weight-only matvec y[n] = sum_k w[n][k] * x[k], f32 accumulate,
 * output f16 (round to nearest even) or f32.  Replaces the U4 fixed-FC op
 * iq36_fixed_fc1 (engine/openvino/custom/iq36_fixed_fc_multi_output.cl:32-40,
 * arguments input, weight, out, scale, zp) and the CPU matvec_tensor
 * (engine/include/intel_qwen36/gguf_loader.hpp:379-382).
 * K = 32 * 2^j with 128 <= K <= 8192, group in {32,64,128,256}, 16-byte
 * aligned qweight. */
int aima_u4_matvec(const uint16_t* x, const uint8_t* qweight,
                   const uint16_t* scale, const uint8_t* zp, int64_t n,
                   int64_t k, int32_t group, void* y, int32_t out_dtype,
                   void* stream);

/* Multi-output U4 matvec over one input: y_j = W_j x for j < count (1 to
 * AIMA_MAX_MULTI_OUT), W_j = weights[j] with n[j] rows of k, output f16 or f32
 * per out_dtype[j]; one launch, every block owning rows of one matrix.
 * Replaces the multi-output fixed FC iq36_fixed_fc3 / iq36_fixed_fc4
 * (engine/openvino/custom/iq36_fixed_fc_multi_output.cl:9-60: one input,
 * then weight, out, scale, zp per projection, each workgroup selecting its
 * projection), which serves the K = 2048 fanout N = [1, 512, 512, 256]
 * (shared-expert gate scalar, shared gate, shared up, router).  Each y_j is
 * bit-identical to aima_u4_matvec of W_j; K and group rules as there. */
int aima_u4_matvec_multi(const uint16_t* x, int32_t count,
                         const aima_u4_tensor* weights, const int64_t* n,
                         int64_t k, int32_t group, void* const* y,
                         const int32_t* out_dtype, void* stream);

/* RMSNorm per row, out = f16(x * (1/sqrt(mean(x^2) + eps)) * weight) with f32
 * arithmetic.  Replaces apply_rms_norm
 * (engine/include/intel_qwen36/gguf_loader.hpp:355-357). */
int aima_rmsnorm(const uint16_t* x, const float* weight, int64_t rows,
                 int64_t hidden, float eps, uint16_t* out, void* stream);

/* Router selection per token: softmax over `experts` logits (f64), top-k
 * (value descending, lower id on ties), weights renormalized over the k by
 * max(sum, min_weight_sum).  Replaces select_router_topk
 * (engine/include/intel_qwen36/gguf_loader.hpp:371-373) and the device
 * iq36_router_topk8_1024 (grouped_s8_u4_f16_contribution_moe.cl:222-291).
 * experts <= 1024, k <= 16. */
int aima_router_topk(const float* logits, int64_t tokens, int32_t experts,
                     int32_t k, float min_weight_sum, int32_t* ids,
                     float* weights, void* stream);

/* Router on device for one token: logits = f32 U4 FC of h (router weight
 * [experts][hidden]), then the selection of aima_router_topk.  Replaces the
 * reference's routing step router_logits = matvec_tensor(ffn_gate_inp.weight,
 * ffn_norm); select_router_topk(router_logits, 8, 6.103515625e-5)
 * (engine/src/gguf_loader.cpp:5708-5711).  logits (experts floats) is a
 * caller buffer and keeps the logits.  experts <= 1024, k <= 16. */
int aima_router_fc_topk(const uint16_t* h, const aima_u4_tensor* router,
                        int32_t experts, int64_t hidden, int32_t group,
                        int32_t k, float min_weight_sum, float* logits,
                        int32_t* ids, float* weights, void* stream);

/* Workspace bytes for aima_router_gemm_topk (0 for an f32 input). */
int aima_router_gemm_workspace_size(int64_t tokens, int64_t hidden,
                                    int32_t input_f32, size_t* bytes);

/* Router for a batch of tokens (the grouped prefill's native router,
 * grouped_s8_u4_prefill_runtime.cpp:1085-1101; its weights are f32,
 * kRouterWeightBytes = experts x hidden x 4 at :35): logits[T][E] =
 * hidden_states[T][H] . router_weight[E][H]^T in f32 (f32 matrix-core
 * GEMM on `stream`), then the selection of aima_router_topk per token:
 * ids[T][k], weights[T][k] (normalized).  hidden_states is f32
 * (input_f32 = 1) or f16 (0: widened to f32 in the workspace first).
 * hidden % 16 == 0, hidden_states and router_weight 16-byte aligned,
 * experts <= 1024, k <= 16. */
int aima_router_gemm_topk(const void* hidden_states, int32_t input_f32,
                          int64_t tokens, int64_t hidden,
                          const float* router_weight, int32_t experts, int32_t k,
                          float min_weight_sum, float* logits, int32_t* ids,
                          float* weights, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Scale / zero-point order conversions for an [n][groups] U4 matrix: the
 * boundary order is row-major (scale f16[n][groups], zero points over the
 * flat n*groups index, low nibble first), which is also the order of an
 * OpenVINO IR U4 FC (tools/intel_qwen36_openvino_fixed_fc.py:107-144); the
 * reference's fixed-FC package stores both group-major, [groups][n]
 * (tools/intel_qwen36_openvino_fixed_fc.py:218-265, same nibble packing).
 * n * groups must be even (as the reference requires).  qweight is the same
 * in both orders. */
int aima_u4_group_major_to_rows(const uint16_t* scale_gm, const uint8_t* zp_gm,
                                int64_t n, int64_t groups, uint16_t* scale,
                                uint8_t* zp, void* stream);
int aima_u4_rows_to_group_major(const uint16_t* scale, const uint8_t* zp,
                                int64_t n, int64_t groups, uint16_t* scale_gm,
                                uint8_t* zp_gm, void* stream);

/* GGUF Q4_K unpack of a [rows][cols] tensor (144-byte super-blocks of 256
 * values): codes in the boundary packing (qweight u8[rows][cols/2]), the
 * group-32 scale f16(d * sc) (f16[rows][cols/32]) and min dmin * m
 * (f32[rows][cols/32]); the value is scale * q - min.  The package the
 * reference's prepack builds from Q4_K
 * (tools/intel-qwen36-openvino-moe-micro-prepack.py:76-124), row-major.
 * cols % 256 == 0.  aima_q4s_matvec consumes this form directly. */
int aima_q4k_unpack(const uint8_t* blocks, int64_t rows, int64_t cols,
                    uint8_t* qweight, uint16_t* scale, float* mins,
                    void* stream);

/* Matvec over the scale-and-min form that aima_q4k_unpack produces (the
 * reference's prepacked Q4_K, tools/intel-qwen36-openvino-moe-micro-prepack.py
 * :91-176): y[n] = sum_k (f32(scale[n][k/32]) * q[n][k] - mins[n][k/32]) * x[k],
 * computed per 32-wide group as scale * sum(q x) - min * sum(x) -- the
 * reference's micro runtime applies the mins to the per-group input sums
 * after its GEMM (engine/tools/openvino_moe_micro_runtime.cpp:735-745).
 * codes u8 [n][k/2] (aima_u4_matvec's packing), scale f16 and mins f32
 * [n][k/32] row-major; f16 or f32 output.  K = 32 * 2^j with
 * 128 <= K <= 8192; codes and x 16-byte aligned. */
int aima_q4s_matvec(const uint16_t* x, const uint8_t* codes,
                    const uint16_t* scale, const float* mins, int64_t n,
                    int64_t k, void* y, int32_t out_dtype, void* stream);

/* Workspace bytes for aima_topk_f32 / aima_u4_lm_head_topk over n values. */
int aima_topk_workspace_size(int64_t n, int32_t k, size_t* bytes);

/* Top-k of n f32 values (an LM head's logits): ids[r], values[r] for ranks
 * r < k, value descending, the lower index first among equal values (the
 * order of the reference's LM-head partial top-8, q4x8_matvec.cl:973-1021).
 * NaNs are never chosen; ranks past the last number hold (-inf, 0x7fffffff).
 * n <= 1,048,576, k <= 16; the workspace may be null when n <= 4096.  One
 * launch: each block stores its picks in the workspace, both 64-bit words of
 * each tagged with a 32-bit launch number kept in the workspace header
 * (bytes 132..135: any start value, every call advances it), and block 0
 * merges them once every word carries this launch's tag, so whatever the
 * pick region held before (zeros, earlier picks, other entry points' data)
 * is never taken for a pick.  Calls sharing a workspace must not overlap. */
int aima_topk_f32(const float* values, int64_t n, int32_t k, int32_t* ids,
                  float* out_values, void* workspace, size_t workspace_bytes,
                  void* stream);

/* U4 LM head with top-k: logits = f32 U4 matvec of x (as aima_u4_matvec,
 * kept in the caller's logits buffer of n floats), then aima_topk_f32 over
 * them (same results and workspace rules).  Replaces the reference's
 * q4s_group128_lm_head_topk8_f32 (engine/gpu/opencl/q4x8_matvec.cl:973-1021:
 * logits out plus per-block partial top-8 ids and values) with its merge.
 * At K = 2048 with a workspace (and ceil(n / 2048) * topk <= 1024) it is one
 * launch: the matvec's blocks also store each logit in the workspace as a
 * 64-bit word {bits, tag of (bits, launch number)}, and the selection's
 * blocks, dispatched after them, read their chunk once every word carries
 * this launch's tag.  AIMA_LM_HEAD_FUSED=0 selects the two launches. */
int aima_u4_lm_head_topk(const uint16_t* x, const uint8_t* qweight,
                         const uint16_t* scale, const uint8_t* zp, int64_t n,
                         int64_t k, int32_t group, int32_t topk, float* logits,
                         int32_t* ids, float* values, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Workspace bytes for aima_moe_ffn_decode / aima_moe_stack_decode. */
int aima_moe_decode_workspace_size(const aima_moe_layer* layer, int32_t k,
                                   size_t* bytes);

/* One MoE FFN block for one token (batch-1 decode):
 *   out = f16(residual + sum_r w[r] * down_{ids[r]}(swiglu(gate_up_{ids[r]} h))
 *             + sigmoid(shared_gate_vec . h) * shared_down(swiglu(shared_gate_up h)))
 * h = x (f16[hidden]); residual may be NULL (then it is 0); ids/weights are
 * device arrays of k entries (the router's top-k output).  Replaces
 * run_qwen36_moe_ffn_layer's expert part (gguf_loader.hpp:519-524,
 * gguf_loader.cpp:5711-5780) and the decode runner
 * RunResidentPackedQ4X8Expert8PlusSharedThenSwiGlu
 * (engine/src/gpu_q4x8_matvec.cpp:3464-3664).  Invalid expert ids set
 * AIMA_DEVERR_EXPERT_RANGE in the workspace error word and contribute 0. */
int aima_moe_ffn_decode(const aima_moe_layer* layer, const uint16_t* x,
                        const uint16_t* residual, const int32_t* ids,
                        const float* weights, int32_t k, uint16_t* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Every intermediate of one decode FFN layer, as device buffers the caller
 * owns: the counterpart of Qwen36MoeFfnLayerResult and RouterTopKSelection
 * (engine/include/intel_qwen36/gguf_loader.hpp:138-161), filled by
 * aima_moe_ffn_layer_trace.  Sizes: H = hidden, I = inter, E = experts. */
typedef struct aima_ffn_trace {
  uint16_t* ffn_norm;             /* f16[H]  rmsnorm(residual): the layer's input */
  float* router_logits;           /* f32[E] */
  int32_t* expert_ids;            /* [k]     RouterTopKSelection.expert_ids */
  float* router_weights;          /* [k]     .weights (softmax probabilities) */
  float* normalized_weights;      /* [k]     .normalized_weights */
  float* selected_gate_up;        /* [k][2I] gate rows, then up rows, per pick */
  uint16_t* selected_swiglu;      /* f16[k][I] (the down projections' input) */
  float* selected_down;           /* [k][H]  unweighted */
  float* weighted_selected_down;  /* [k][H] */
  float* moe_out;                 /* [H]     rank-order sum of the weighted rows */
  float* shared_gate;             /* [1]     shared_gate_vec . ffn_norm */
  float* shared_gate_sigmoid;     /* [1] */
  float* shared_gate_up;          /* [2I] */
  uint16_t* shared_swiglu;        /* f16[I] */
  float* shared_down;             /* [H] */
  float* shared_gated;            /* [H] */
  float* ffn_out;                 /* [H]     moe_out + shared_gated */
  uint16_t* residual;             /* f16[H]  the layer's output, as aima_moe_ffn_decode */
} aima_ffn_trace;

/* Workspace bytes for aima_moe_ffn_layer_trace. */
int aima_moe_ffn_layer_trace_workspace_size(const aima_moe_layer* layer, int32_t k,
                                            size_t* bytes);

/* One decode FFN layer with every intermediate kept (a debugging path, not
 * the fast one): ffn_norm = rmsnorm(residual, layer->norm_weight, eps); the
 * router (U4 [experts][hidden], the layer's group) and its selection as
 * aima_router_fc_topk; then aima_moe_ffn_decode's two kernels with their
 * gate/up rows, activations, per-pick down rows and shared gate captured,
 * and the weighted sums formed in rank order.  Mirrors
 * run_qwen36_moe_ffn_layer (engine/src/gguf_loader.cpp:5654-5782).  `residual`
 * is the kernels' own output (their summation order differs from the rank
 * order of moe_out/ffn_out by f32 rounding only).  Every buffer of *trace is
 * required; experts <= 1024, k <= 16. */
int aima_moe_ffn_layer_trace(const aima_moe_layer* layer, const aima_u4_tensor* router,
                             const uint16_t* residual, float eps, int32_t k,
                             float min_weight_sum, const aima_ffn_trace* trace,
                             void* workspace, size_t workspace_bytes, void* stream);

/* The two launches of aima_moe_ffn_decode, separately.
 * Gate/up: act[r][j] = f16(silu(g) * u) for the k routed experts (slot r =
 * ids[r]) and the shared expert (slot k), act f16 [k+1][inter], plus the
 * shared gate *shared_sigma = sigmoid(shared_gate_vec . x).  Replaces the
 * decode runner's expert8-plus-shared gate/up matvec with the SwiGLU
 * (engine/src/gpu_q4x8_matvec.cpp:3464-3664, kernels
 * q4k_x8_matvec_rowlane_expert8_plus_shared_localq8 and ffn_moe_swiglu_f32,
 * engine/gpu/opencl/q4x8_matvec.cl:1908-2008,2679-2694).  Invalid ids set
 * AIMA_DEVERR_EXPERT_RANGE in *error_word. */
int aima_moe_decode_gate_up(const aima_moe_layer* layer, const uint16_t* x,
                            const int32_t* ids, int32_t k, uint16_t* act,
                            float* shared_sigma, uint32_t* error_word,
                            void* stream);

/* Down + aggregate: out = f16(residual + sum_r weights[r] * down_{ids[r]} act[r]
 * + shared_sigma * shared_down act[k]), rank order fixed, no atomics.
 * Replaces the selected-down + FFN tail (q4s_group128_all_expert_down_topk8_plus_shared,
 * ffn_moe_weighted_aggregate_f32, shared_expert_gate_apply_f32,
 * ffn_output_add_f32, post_ffn_residual_add_f32;
 * engine/gpu/opencl/q4x8_matvec.cl:1023-1052,4358-4418). */
int aima_moe_decode_down(const aima_moe_layer* layer, const uint16_t* act,
                         const float* shared_sigma, const int32_t* ids,
                         const float* weights, int32_t k,
                         const uint16_t* residual, uint16_t* out, void* stream);

/* Workspace bytes for aima_moe_grouped_prefill / aima_moe_stack_prefill. */
int aima_moe_prefill_workspace_size(const aima_moe_layer* layer,
                                    int64_t tokens, int32_t k, size_t* bytes);

/* Grouped MoE FFN over T tokens (prefill): tokens are sorted by expert on the
 * device (stable by token), each expert runs a grouped gate/up GEMM with the
 * SwiGLU epilogue and a grouped down GEMM scaled by the router weight on
 * MFMA, and every token's output is the rank-ordered sum of its k
 * contributions plus the sigmoid-gated shared expert (plus residual, if not
 * NULL).  x, residual, out: f16 [T][hidden]; ids, weights: [T][k].
 * Replaces GroupedS8U4PrefillRuntime::RunLayer
 * (engine/include/intel_qwen36/grouped_s8_u4_prefill_runtime.hpp:148-150,
 * top-k int32[T][8] + float[T*8] in, per-token routed sum out) and the
 * OpenVINO MOE3GemmFusedCompressed op
 * (engine/openvino/iq36-fixed-fc-moe-router-compat.patch:49-56; gate and up
 * may be separate tensors, see aima_moe_layer).  RunLayer's exact output (f32
 * routed-only sum, strided top-k, f32 input) is aima_moe_grouped_prefill_ex.
 * Requires group 128, shared_inter == inter, hidden % 256 == 0,
 * inter % 128 == 0. */
int aima_moe_grouped_prefill(const aima_moe_layer* layer, const uint16_t* x,
                             const uint16_t* residual, int64_t tokens,
                             const int32_t* ids, const float* weights,
                             int32_t k, uint16_t* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Output forms of aima_moe_grouped_prefill_ex. */
#define AIMA_PREFILL_FULL_F16 0   /* f16 routed + sigmoid-gated shared (+ residual) */
#define AIMA_PREFILL_ROUTED_F32 1 /* f32 routed sum only: RunLayer's output */

/* Options of aima_moe_grouped_prefill_ex (zero-initialized = the defaults). */
typedef struct aima_prefill_options {
  int32_t output_mode;    /* AIMA_PREFILL_FULL_F16 (0) or AIMA_PREFILL_ROUTED_F32 */
  int32_t input_f32;      /* 1: x is f32 [T][hidden], RunLayer's hidden_states type
                             (rounded to f16 on the device); 0: x is f16 */
  int64_t topk_stride;    /* bytes between consecutive tokens' int32 top-k rows
                             (a multiple of 4, >= 4 * k); 0 = 4 * k (dense) */
  void* stage_events[5];  /* optional hipEvent_t, recorded on `stream` before the
                             schedule and after the schedule, the gate/up GEMM,
                             the down GEMM and the combine (NULL entries skipped) */
  float* swiglu_f32;      /* optional f32 [rows][inter], 16-byte aligned: the SwiGLU
                             rows before their f16 rounding (RunLayer's
                             grouped_swiglu_f32); rows in schedule order, T*k routed
                             rows (+ T shared rows in the full mode) */
  float* contributions_f32; /* optional f32 [rows][hidden], 16-byte aligned: w_row *
                             down(row) before its f16 rounding (RunLayer's
                             grouped_contributions_f32; shared rows unweighted) */
} aima_prefill_options;

/* Grouped MoE FFN over T tokens with GroupedS8U4PrefillRuntime::RunLayer's
 * contract (engine/include/intel_qwen36/grouped_s8_u4_prefill_runtime.hpp:62-84,
 * 100-121; validation grouped_s8_u4_prefill_runtime.cpp:1040-1061):
 *   topk     int32 ids, token t's k ids at byte offset t * topk_stride
 *   weights  f32 [T*k] normalized router weights (RunLayer's router_weights)
 *   x        f16 or (input_f32) f32 hidden states [T][hidden]
 *   out      AIMA_PREFILL_ROUTED_F32: f32 [T][hidden],
 *              out[t] = sum_r f32(f16(w_r * down_r(swiglu(gate_up_r x_t))))
 *              summed in rank order from 0 (the reference's grouped output,
 *              grouped_s8_u4_f16_contribution_moe.cl:831-845); no shared
 *              expert (its tensors may be NULL) and no residual;
 *            AIMA_PREFILL_FULL_F16: f16 [T][hidden] as aima_moe_grouped_prefill.
 * The arithmetic follows the reference's grouped kernels
 * (grouped_s8_u4_f16_contribution_moe.cl:627-683): each row's SwiGLU is
 * rounded to f16 unweighted, the down projection consumes it, and the router
 * weight multiplies the down output before its f16 rounding.
 * Out-of-range or duplicated ids set the workspace error word (RunLayer
 * throws).  Workspace as aima_moe_prefill_workspace_size; the schedule, the
 * f16 SwiGLU rows and the contributions of the call stay in it (see
 * aima_moe_prefill_workspace_views); f32 copies go to the option buffers. */
int aima_moe_grouped_prefill_ex(const aima_moe_layer* layer, const void* x,
                                const uint16_t* residual, int64_t tokens,
                                const int32_t* topk, const float* weights, int32_t k,
                                void* out, const aima_prefill_options* options,
                                void* workspace, size_t workspace_bytes, void* stream);

/* The grouped prefill fed router logits, as OpenVINO's fused MoE op
 * MOE3GemmFusedCompressed(hidden, routing_logits, gate_*, up_*, down_*)
 * (engine/openvino/iq36-fixed-fc-moe-router-compat.patch:31-56,183-193):
 * routing_logits f32 [T][experts] -> per token the selection of
 * aima_router_topk (select_router_topk: f64 softmax, k largest, lower id on
 * ties, renormalized by max(sum, min_weight_sum)) written to ids_out [T][k]
 * and weights_out [T][k], then aima_moe_grouped_prefill_ex on those dense
 * routes (options as there; topk_stride must be 0; stage event 0 is
 * recorded before the selection).  Workspace as
 * aima_moe_prefill_workspace_size.  One launch more than the layer (the
 * selection); the routes pass through ids_out / weights_out. */
int aima_moe_grouped_prefill_logits(const aima_moe_layer* layer, const void* x,
                                    const uint16_t* residual, int64_t tokens,
                                    const float* routing_logits, int32_t k,
                                    float min_weight_sum, int32_t* ids_out,
                                    float* weights_out, void* out,
                                    const aima_prefill_options* options,
                                    void* workspace, size_t workspace_bytes,
                                    void* stream);

/* Device pointers into a prefill workspace: the intermediates the last
 * aima_moe_grouped_prefill(_ex) call on it left there (RunLayer's
 * capture_intermediates outputs, grouped_s8_u4_prefill_runtime.hpp:100-121).
 * Rows are in schedule order (expert-major, tokens ascending within an
 * expert); routed rows 0 .. T*k-1, then (full mode) the shared expert's rows
 * T*k + t. */
typedef struct aima_prefill_views {
  int32_t* offsets;          /* [experts] exclusive end row of each expert */
  int32_t* token_map;        /* [T*k] source token of each routed row */
  int32_t* inverse_map;      /* [T*k] row of (token, rank) */
  float* compact_weights;    /* [T*k] router weight of each routed row */
  uint16_t* swiglu;          /* f16 [T*k + T][inter]: silu(gate) * up, unweighted
                                (RunLayer's grouped_swiglu_f16) */
  uint16_t* contributions;   /* f16 [T*k + T][hidden]: w_row * down of the row
                                above (shared rows unweighted; RunLayer's
                                grouped_contributions_f16) */
  int32_t* tiles;            /* [tile_count][4] expert, first row, rows, 0 */
  int32_t* tile_count;       /* one int */
} aima_prefill_views;
int aima_moe_prefill_workspace_views(const aima_moe_layer* layer, int64_t tokens,
                                     int32_t k, void* workspace,
                                     aima_prefill_views* views);

/* Workspace bytes for aima_grouped_schedule. */
int aima_grouped_schedule_workspace_size(int64_t tokens, int32_t k,
                                         int32_t experts, size_t* bytes);

/* The grouped schedule alone (the step the prefill runs first): a stable
 * device counting sort of the T*k assignments by expert.  Outputs, all
 * device arrays: offsets[E] = exclusive end row of each expert, token_map[A]
 * = source token of each sorted row, inverse_map[A] = sorted row of each
 * (token, rank), compact_weights[A] = router weight of each sorted row.
 * Same results as the host BuildGroupedSchedule
 * (engine/src/grouped_s8_u4_prefill_runtime.cpp:231-346: rows of one expert
 * in (token, rank) order); out-of-range or duplicated ids set the workspace
 * error word (the reference throws). */
int aima_grouped_schedule(const int32_t* ids, const float* weights,
                          int64_t tokens, int32_t k, int32_t experts,
                          int32_t* offsets, int32_t* token_map,
                          int32_t* inverse_map, float* compact_weights,
                          void* workspace, size_t workspace_bytes, void* stream);

/* n_layers MoE FFN layers for one token: r_0 = residual_in and for each
 * layer L, h = f16(rmsnorm(r_L, layers[L].norm_weight, eps)),
 * r_{L+1} = f16(r_L + ffn_L(h)).  ids/weights: [n_layers][k].  `layers` is a
 * HOST array of layer descriptors.  out = r_{n_layers}. */
int aima_moe_stack_decode(const aima_moe_layer* layers, int32_t n_layers,
                          float eps, const uint16_t* residual_in,
                          const int32_t* ids, const float* weights, int32_t k,
                          uint16_t* out, void* workspace,
                          size_t workspace_bytes, void* stream);

/* True decode: aima_moe_stack_decode with each layer's routing computed on
 * the device from its own normalized input -- logits = U4 FC (routers[l],
 * [experts][hidden], the layer's group) of h_l, then the selection of
 * aima_router_topk -- as run_qwen36_moe_ffn_layer does per layer
 * (engine/src/gguf_loader.cpp:5704-5711).  The chosen ids / weights of every
 * layer are written to ids / weights ([n_layers][k]).  experts <= 1024,
 * k <= 16; workspace as aima_moe_stack_decode. */
int aima_moe_stack_decode_routed(const aima_moe_layer* layers,
                                 const aima_u4_tensor* routers, int32_t n_layers,
                                 float eps, const uint16_t* residual_in, int32_t k,
                                 float min_weight_sum, int32_t* ids, float* weights,
                                 uint16_t* out, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* aima_moe_stack_decode_routed without a workspace and without any
 * allocation: the scratch (normalized input, residual ping-pong, router
 * logits, activations) is a fixed 128 KiB device array inside this library,
 * one per GPU, held until the process ends.  No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Device-detected errors
 * are OR-ed into the caller's device word *error_word (never cleared here).
 * The scratch takes (k + 1) * inter * 2 + 3 * hidden * 2 + 4.6 KiB: at most
 * 97 KiB for every shape the decode kernels accept (hidden <= 4096,
 * inter <= 2048, k <= 16); a shape past 128 KiB would return
 * AIMA_E_UNSUPPORTED.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialized by the caller.  The first call on each device
 * resolves the array's device address (hipGetSymbolAddress, once per device):
 * make that call outside graph capture; later calls may be captured. */
int aima_moe_stack_decode_routed_noalloc(const aima_moe_layer* layers,
                                         const aima_u4_tensor* routers, int32_t n_layers,
                                         float eps, const uint16_t* residual_in, int32_t k,
                                         float min_weight_sum, int32_t* ids, float* weights,
                                         uint16_t* out, uint32_t* error_word, void* stream);

/* Resident decode plan: the whole n_layers-layer decode step in ONE
 * persistent launch (hidden 2048, inter 512, k <= 8; see
 * moe_decode_persistent.hip).  create() validates the shapes, checks that
 * the device has 256 CUs (8 XCDs x 32) and keeps one 512-thread block
 * resident on each, allocates the plan's
 * device buffers, uploads the layer table and copies each layer's
 * shared-expert down weights into an XCD-slice-major layout (512 KB per
 * layer; the plan reads that copy, so changed shared-down weights need a
 * new plan) (synchronous, setup time only;
 * AIMA_E_UNSUPPORTED when the shape or device does not fit, in which case
 * aima_moe_stack_decode is the general path).  run() is asynchronous,
 * allocates nothing and can be captured in a HIP graph: routing comes from
 * router_logits [n_layers][experts] (the select_router_topk rule) or, when
 * that is NULL, from ids/weights [n_layers][k]; out = r_{n_layers} as in
 * aima_moe_stack_decode.  Calls on one plan must not overlap, and no other
 * plan's run may execute concurrently on the same device (another stream):
 * all 256 blocks must be resident at once, and two persistent launches
 * sharing the CUs can each wait for blocks the other holds, which the
 * kernel's spin limits report as AIMA_DEVERR_TIMEOUT.  Mirrors the
 * reference's resident native loop (engine/include/intel_qwen36/
 * native_carrier_loop.hpp:38-100) for the MoE FFN stack. */
typedef struct aima_moe_decode_plan aima_moe_decode_plan;
int aima_moe_decode_plan_create(const aima_moe_layer* layers, int32_t n_layers,
                                int32_t k, aima_moe_decode_plan** plan);
int aima_moe_decode_plan_run(aima_moe_decode_plan* plan, float eps,
                             const uint16_t* residual_in,
                             const float* router_logits, const int32_t* ids,
                             const float* weights, float min_weight_sum,
                             uint16_t* out, void* stream);
/* True decode in the resident plan.  set_routers registers one U4 router
 * per layer (routers[n_layers], each [experts][hidden] at the layer's
 * group; experts <= 256; qweight 16-byte, scale and zp 4-byte aligned;
 * setup time: waits for the device, then uploads).  run_routed then routes
 * every layer from its own normalized input inside the same launch, as
 * run_qwen36_moe_ffn_layer does per layer (engine/src/gguf_loader.cpp:
 * 5704-5711): h = f16(rmsnorm(r_L)), logits = U4 FC(router_L, h) in f32,
 * then the select_router_topk rule (gguf_loader.hpp:371-373), then the
 * layer's experts.  Optional outputs (NULL to skip): ids / weights
 * [n_layers][k] (rank order, normalized weights) and logits
 * [n_layers][experts].  Asynchronous, allocates nothing, graph-capturable,
 * with the same concurrency rules as aima_moe_decode_plan_run.  Non-finite
 * logits select no expert: AIMA_DEVERR_EXPERT_RANGE is set and the slot
 * contributes nothing.  AIMA_E_INVALID before set_routers. */
int aima_moe_decode_plan_set_routers(aima_moe_decode_plan* plan,
                                     const aima_u4_tensor* routers);
int aima_moe_decode_plan_run_routed(aima_moe_decode_plan* plan, float eps,
                                    const uint16_t* residual_in, float min_weight_sum,
                                    int32_t* ids, float* weights, float* logits,
                                    uint16_t* out, void* stream);
/* Device error bits of the plan (AIMA_DEVERR_*; synchronizes, then clears). */
int aima_moe_decode_plan_error(aima_moe_decode_plan* plan, uint32_t* error_bits,
                               void* stream);
int aima_moe_decode_plan_destroy(aima_moe_decode_plan* plan);

/* Workspace bytes for aima_moe_stack_prefill (one layer's prefill workspace
 * plus the normalized activations). */
int aima_moe_stack_prefill_workspace_size(const aima_moe_layer* layer,
                                          int64_t tokens, int32_t k,
                                          size_t* bytes);

/* The same stack for T tokens: x_in, out f16 [T][hidden]; ids/weights
 * [n_layers][T][k]. */
int aima_moe_stack_prefill(const aima_moe_layer* layers, int32_t n_layers,
                           float eps, const uint16_t* x_in, int64_t tokens,
                           const int32_t* ids, const float* weights, int32_t k,
                           uint16_t* out, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Copy the device error word of a workspace to the host (synchronizes
 * `stream`).  0 = no error; otherwise AIMA_DEVERR_* bits.  Clears it. */
int aima_workspace_error(void* workspace, uint32_t* error_bits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AIMA_U4MOE_H_ */
