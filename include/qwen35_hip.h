/*
 * qwen35_hip.h -- C ABI of the MI355X (gfx950) fused per-layer kernels.
 *
 * Plain pointers and sizes only. Every pointer argument that names a tensor is a
 * device pointer owned by the caller; `stream` is a hipStream_t (NULL = the
 * default stream). Every function validates its arguments on the host before
 * anything is enqueued, enqueues asynchronously, never allocates, frees or
 * synchronises, and returns a qwen_status. It never throws. On failure,
 * qwen_last_error() returns a message for the calling thread.
 *
 * Citations "ref: file:line" name the reference interface (sahan974/qwen-3.5-cuda)
 * that each entry point replaces. The C++ drop-in headers (ops.hpp, rope.hpp,
 * gdn.hpp, matmul_q4.hpp, layer_kernels.hpp) wrap these in namespace qwen with
 * the reference signatures and its exception behaviour.
 *
 * Layouts: "rows" are tokens. A [rows x n] tensor is row-major and contiguous.
 * bf16 tensors are uint16_t holding the top half of an IEEE binary32.
 * The vectorised paths use 16-byte loads when every pointer is 16-byte aligned
 * and the row length is a multiple of 4 (fp32) or 8 (bf16); other shapes take a
 * scalar path with the same results.
 */
#ifndef QWEN35_HIP_H
#define QWEN35_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qwen_status {
    QWEN_STATUS_OK = 0,
    QWEN_STATUS_INVALID_ARGUMENT = 1, /* bad pointer, size or parameter       */
    QWEN_STATUS_UNSUPPORTED_TYPE = 2, /* GGML type without a dequant path     */
    QWEN_STATUS_OUT_OF_RANGE = 3,     /* row/element range outside the tensor */
    QWEN_STATUS_LAUNCH_FAILED = 4,    /* the HIP runtime rejected the launch  */
    QWEN_STATUS_IO_ERROR = 5,         /* GGUF: file unreadable or not GGUF    */
    QWEN_STATUS_MALFORMED = 6,        /* GGUF: content rejected by the parser */
    QWEN_STATUS_OUT_OF_MEMORY = 7     /* GGUF: device or pinned allocation    */
};

/* ABI version of this header (bumped on any signature change). */
int qwen_abi_version(void);
/* Message describing the calling thread's most recent failure ("" if none). */
const char* qwen_last_error(void);
/* Constant name of a status code. */
const char* qwen_status_name(int status);

/* ===================================================================== norms
 * out = (x * r) * w, r = rsqrtf(sum(x^2)/n + eps), per row.
 * ref: include/ops.hpp:11-18 (rmsnorm_forward), src/cuda/ops.cu:25-65,143-154 */
int qwen_rmsnorm_forward(const float* x, const float* weight, float* out, int n, float eps,
                         void* stream);
/* Row-batched form of the above: x, out [rows x n]. */
int qwen_rmsnorm_rows(const float* x, const float* weight, float* out, int rows, int n, float eps,
                      void* stream);

/* out = ((x * r) * w) * silu(gate), full-row r.
 * ref: include/ops.hpp:21-29 (rmsnorm_gated_forward), src/cuda/ops.cu:68-109 */
int qwen_rmsnorm_gated_forward(const float* x, const float* gate, const float* weight, float* out,
                               int n, float eps, void* stream);
int qwen_rmsnorm_gated_rows(const float* x, const float* gate, const float* weight, float* out,
                            int rows, int n, float eps, void* stream);

/* out = x1 + x2.  ref: include/ops.hpp:32-38, src/cuda/ops.cu:115-125,170-181 */
int qwen_residual_add(const float* x1, const float* x2, float* out, int size, void* stream);

/* Fused residual add + RMSNorm: resid = x + branch; normed = rmsnorm(resid) * w.
 * Replaces the pair residual_add (src/model.cpp:205) + rmsnorm_forward
 * (src/model.cpp:208); both outputs are written. */
int qwen_residual_rmsnorm_rows_f32(const float* x, const float* branch, const float* weight,
                                   float* resid, float* normed, int rows, int n, float eps,
                                   void* stream);
/* bf16 storage, fp32 math: resid = bf16(x + branch); the norm reads the rounded
 * resid back, so the result equals the unfused pair run on bf16 buffers. */
int qwen_residual_rmsnorm_rows_bf16(const uint16_t* x, const uint16_t* branch, const float* weight,
                                    uint16_t* resid, uint16_t* normed, int rows, int n, float eps,
                                    void* stream);

/* out = table[token_id * d_model : +d_model] (fp32 rows). token_id is not range
 * checked (the reference has no vocabulary bound here either).
 * ref: include/ops.hpp:41-47 (encoder_forward), src/cuda/ops.cu:128-138 */
int qwen_encoder_forward(int token_id, const float* table, float* out, int d_model, void* stream);

/* ================================================================ attention
 * Per-head RMSNorm in place: x = x * (r * w), w shared by all heads [dim].
 * ref: src/layer_attn.cpp:11 (attn_head_norm decl), src/cuda/attn_kernels.cu:34-68 */
int qwen_attn_head_norm(float* x, const float* weight, int heads, int dim, float eps, void* stream);

/* Split-half partial RoPE in place on the first rope_dim dims of every head:
 * theta_i = pos / powf(theta, 2i/rope_dim); (a, b) -> (a c - b s, b c + a s).
 * Rejects (INVALID_ARGUMENT) exactly what the reference throws on.
 * ref: include/rope.hpp:13-21 (rope_forward), src/cuda/rope.cu:9-47 */
int qwen_rope_forward(float* x, int pos, int heads, int head_dim, int rope_dim, float theta,
                      void* stream);

/* Fused Q/K per-head RMSNorm + partial RoPE over `rows` tokens, in place:
 * q [rows x q_heads x head_dim] with q_weight [head_dim], k [rows x k_heads x
 * head_dim] with k_weight [head_dim]. Row t uses position pos[t] (device int32
 * array) or, when pos is NULL, pos0 + t. rope_dim 0 skips the rotation.
 * Replaces src/layer_attn.cpp:91-96 (two attn_head_norm + two rope_forward). */
int qwen_attn_qk_norm_rope_rows(float* q, float* k, const float* q_weight, const float* k_weight,
                                const int32_t* pos, int pos0, int rows, int q_heads, int k_heads,
                                int head_dim, int rope_dim, float theta, float eps, void* stream);

/* ========================================================= Gated DeltaNet
 * One decode step of the causal depthwise conv + SiLU; history [channels x
 * (kernel-1)] is shifted in place.
 * ref: include/gdn.hpp:9-17 (gdn_conv_step), src/cuda/gdn.cu:9-32 */
int qwen_gdn_conv_step(const float* input, const float* weight, float* history, float* output,
                       int channels, int kernel, void* stream);

/* Per-head L2 norm in place; q is also scaled by rsqrtf(dim); eps on the sum.
 * ref: include/gdn.hpp:20-27 (gdn_qk_normalize), src/cuda/gdn.cu:36-86 */
int qwen_gdn_qk_normalize(float* q, float* k, int heads, int dim, float eps, void* stream);

/* Fused GDN front end over `rows` tokens: y = silu(causal depthwise conv(x))
 * with weights [channels x kernel] and history hist_in [channels x (kernel-1)];
 * then the L2 norm of gdn_qk_normalize on q = channels [0, k_heads*key_dim) and
 * k = [k_heads*key_dim, 2*k_heads*key_dim) of every row. hist_out receives the
 * history after the last row (hist_out may equal hist_in). k_heads 0 skips the
 * norm. Equals `rows` sequential gdn_conv_step calls followed by
 * gdn_qk_normalize on each row (src/layer_gdn.cpp:89-97). */
int qwen_gdn_frontend_rows(const float* x, const float* weight, const float* hist_in,
                           float* hist_out, float* y, int rows, int channels, int kernel,
                           int k_heads, int key_dim, float eps, void* stream);

/* Gated per-head RMSNorm: out = ((x * r) * w) * silu(z), r per head of `dim`.
 * ref: include/gdn.hpp:58-67 (gdn_norm_gate), src/cuda/gdn.cu:176-215 */
int qwen_gdn_norm_gate(const float* x, const float* z, const float* weight, float* out, int heads,
                       int dim, float eps, void* stream);
/* Row-batched form: x, z, out [rows x heads x dim]. */
int qwen_gdn_norm_gate_rows(const float* x, const float* z, const float* weight, float* out,
                            int rows, int heads, int dim, float eps, void* stream);

/* The gated norm and the output projection of a GDN decode step in one launch:
 * normed = qwen_gdn_norm_gate(x, z, norm_weight) over heads of dim, then
 * y = qwen_matmul_dispatch(weight, type, num_elements, normed, M, K = heads * dim,
 * element_offset). Results are the bits of those two calls (normed included). One
 * launch for Q4_K weights on the per-row GEMV path, dim 64 / 128 / 256, K a multiple
 * of 2048 and 16-byte aligned pointers: every workgroup normalises the x it reads;
 * otherwise the two calls. Statuses as those calls.
 * ref: src/layer_gdn.cpp:109-112 (gdn_norm_gate, matmul_dispatch) */
int qwen_gdn_norm_gate_matmul(const float* x, const float* z, const float* norm_weight, float* normed,
                              int heads, int dim, float eps, const void* weight, int type,
                              uint64_t num_elements, float* y, int M, uint64_t element_offset,
                              void* stream);

/* Gates of the delta rule: beta = 1/(1+expf(-beta_raw)),
 * decay = expf(a * softplus(alpha_raw + dt_bias)), softplus(x) = x > 20 ? x : log1p(exp(x)).
 * beta_raw, alpha_raw, beta, decay [heads]; a, dt_bias [heads].
 * ref: include/gdn.hpp:29-38 (gdn_gate_values), src/cuda/gdn.cu:90-104 */
int qwen_gdn_gate_values(const float* beta_raw, const float* alpha_raw, const float* a,
                         const float* dt_bias, float* beta, float* decay, int heads, void* stream);
/* Row-batched form: beta_raw, alpha_raw, beta, decay [rows x heads]; a, dt_bias [heads]. */
int qwen_gdn_gate_values_rows(const float* beta_raw, const float* alpha_raw, const float* a,
                              const float* dt_bias, float* beta, float* decay, int rows, int heads,
                              void* stream);

/* One delta-rule step per value head h (key head h % key_heads), state
 * [value_heads x key_dim x value_dim] updated in place:
 *   S *= decay[h]; delta = (v - k^T S) * beta[h]; S += k delta^T; out = q^T S.
 * q, k [key_heads x key_dim]; v, out [value_heads x value_dim]; beta, decay [value_heads].
 * value_dim > 256 -> QWEN_STATUS_INVALID_ARGUMENT ("GDN value dimension exceeds kernel limit").
 * ref: include/gdn.hpp:41-54 (gdn_recurrent_step), src/cuda/gdn.cu:108-172 */
int qwen_gdn_recurrent_step(float* state, const float* q, const float* k, const float* v,
                            const float* beta, const float* decay, float* out, int key_heads,
                            int value_heads, int key_dim, int value_dim, void* stream);
/* `rows` consecutive steps in one launch (the reference's per-token loop,
 * src/layer_gdn.cpp:100-106): token t reads q, k, v at t * qkv_stride elements
 * (e.g. the q | k | v slices of the GDN front end's output rows), beta and decay
 * at t * value_heads, and writes out at t * out_stride. */
int qwen_gdn_recurrent_rows(float* state, const float* q, const float* k, const float* v,
                            const float* beta, const float* decay, float* out, int rows,
                            int key_heads, int value_heads, int key_dim, int value_dim,
                            int64_t qkv_stride, int64_t out_stride, void* stream);

/* qwen_gdn_gate_values_rows fused into qwen_gdn_recurrent_rows: the gates of
 * token t and value head h are evaluated where the recurrence uses them, from
 * beta_raw and alpha_raw [rows x value_heads] (at t * value_heads) and a,
 * dt_bias [value_heads], with the same expressions, so the results are the
 * bits of the two calls in sequence; one launch instead of two per decode step,
 * and no beta / decay buffers. Other arguments and statuses as
 * qwen_gdn_recurrent_rows.
 * ref: src/layer_gdn.cpp:100-106 (gdn_gate_values, then gdn_recurrent_step) */
int qwen_gdn_gated_recurrent_rows(float* state, const float* q, const float* k, const float* v,
                                  const float* beta_raw, const float* alpha_raw, const float* a,
                                  const float* dt_bias, float* out, int rows, int key_heads,
                                  int value_heads, int key_dim, int value_dim, int64_t qkv_stride,
                                  int64_t out_stride, void* stream);

/* One decode token of a GDN layer after its input projections, in one launch:
 * qwen_gdn_frontend_rows on the row x [C] (C = 2 key_heads key_dim + value_heads
 * value_dim; conv weights [C x kernel], history hist_in -> hist_out) writing y [C],
 * then qwen_gdn_gated_recurrent_rows on y's q | k | v with beta_raw, alpha_raw
 * [value_heads] into state and out [value_heads x value_dim]. Results are the
 * bits of those two calls. One launch for kernel 4, key_dim 128, value_dim a
 * multiple of 4, value_heads a multiple of key_heads, 16-byte aligned pointers and
 * hist_out not overlapping hist_in; otherwise the two calls (which also allow
 * hist_out == hist_in). Statuses as those calls.
 * ref: src/layer_gdn.cpp:89-106 (gdn_conv_step, gdn_qk_normalize, gdn_gate_values,
 * gdn_recurrent_step) */
int qwen_gdn_decode_step(const float* x, const float* conv_weight, const float* hist_in, float* hist_out,
                         float* y, float* state, const float* beta_raw, const float* alpha_raw,
                         const float* a, const float* dt_bias, float* out, int key_heads, int value_heads,
                         int key_dim, int value_dim, int kernel, float eps, void* stream);

/* Chunked form of qwen_gdn_recurrent_rows for many tokens (prefill): the same
 * recurrence re-associated over chunks of 64 tokens (decay ratios as running
 * products, a 64 x 64 triangular solve per chunk and head, the state updated
 * once per chunk; the products over 128 keys or 64 tokens on fp16 MFMA with each
 * fp32 operand held as a scaled pair of fp16 values);
 * equal to the token loop within fp32 rounding.
 * Arguments as qwen_gdn_recurrent_rows plus a caller-owned device workspace of
 * at least qwen_gdn_recurrent_chunked_workspace_bytes(rows, value_heads)
 * (16-byte aligned; contents scratch). Shapes the chunked kernels do not cover
 * (key_dim != 128, value_dim not a multiple of 16, unaligned q / k) run the
 * token loop and leave the workspace untouched.
 * No reference counterpart: the reference runs the per-token step for every
 * token (src/layer_gdn.cpp:100-106). */
size_t qwen_gdn_recurrent_chunked_workspace_bytes(int rows, int value_heads);
int qwen_gdn_recurrent_chunked(float* state, const float* q, const float* k, const float* v,
                               const float* beta, const float* decay, float* out, int rows,
                               int key_heads, int value_heads, int key_dim, int value_dim,
                               int64_t qkv_stride, int64_t out_stride, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ====================================================================== attention core (decode)
 * One query position against the KV cache, rows [t][kv_heads][dim]; query head h
 * reads kv head h / (heads / kv_heads) (heads a multiple of kv_heads). */

/* q[h] = qg[h][0:dim], gate[h] = qg[h][dim:2*dim].
 * ref: src/layer_attn.cpp:10 (attn_split_qg decl), src/cuda/attn_kernels.cu:16-31 */
int qwen_attn_split_qg(const float* qg, float* q, float* gate, int heads, int dim, void* stream);

/* scores[h][t] = (q_h . k_t) * (1/sqrt(dim)), t <= pos, scores [heads x (pos+1)].
 * ref: src/layer_attn.cpp:12 (attn_scores decl), src/cuda/attn_kernels.cu:72-96 */
int qwen_attn_scores(const float* q, const float* k_cache, float* scores, int heads, int kv_heads,
                     int dim, int pos, void* stream);

/* Row softmax in place: s = exp(s - max) / sum over valid_len entries per head.
 * ref: src/layer_attn.cpp:13 (attn_softmax decl), src/cuda/attn_kernels.cu:99-158 */
int qwen_attn_softmax(float* scores, int heads, int valid_len, void* stream);

/* out[h][j] = sum_{t<=pos} scores[h][t] * v_cache[t][kv(h)][j].
 * ref: src/layer_attn.cpp:14 (attn_values decl), src/cuda/attn_kernels.cu:162-181 */
int qwen_attn_values(const float* scores, const float* v_cache, float* out, int heads, int kv_heads,
                     int dim, int pos, void* stream);

/* out = x / (1 + exp(-gate)) over n elements (out may equal x).
 * ref: src/layer_attn.cpp:15 (attn_sigmoid_gate decl), src/cuda/attn_kernels.cu:185-195 */
int qwen_attn_sigmoid_gate(const float* x, const float* gate, float* out, int n, void* stream);

/* k, v [kv_dim] stored to row pos of the caches; pos outside [0, max_seq_len) ->
 * QWEN_STATUS_OUT_OF_RANGE ("attention position exceeds configured context").
 * ref: src/layer_attn.cpp:76-78 (check), :99-100 (cudaMemcpyAsync of k and v) */
int qwen_attn_kv_store(const float* k, const float* v, float* k_cache, float* v_cache, int pos,
                       int kv_dim, int max_seq_len, void* stream);

/* Workspace bytes qwen_attn_decode needs for this shape (0 for an invalid shape). */
size_t qwen_attn_decode_workspace_bytes(int heads, int kv_heads, int dim, int pos);

/* scores -> softmax -> values -> sigmoid gate (gate may be NULL) in one call:
 * out[h] = sum_t softmax_t(q_h . k_t / sqrt(dim)) v_t (* sigmoid(gate[h])).
 * workspace: device memory of at least qwen_attn_decode_workspace_bytes, owned by
 * the caller (the per-split partial results; the reference's scores buffer plays
 * this role, src/layer_attn.cpp:57).
 * ref: src/layer_attn.cpp:103-108 */
int qwen_attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* gate,
                     float* out, int heads, int kv_heads, int dim, int pos, void* workspace,
                     size_t workspace_bytes, void* stream);

/* The attention front end folded into the decode: q_normed = q with
 * qwen_attn_qk_norm_rope_rows applied (q_weight, rope at position pos), the cache
 * row of pos (k_cache + pos * kv_heads * dim) normalised and rotated in place with
 * k_weight, then qwen_attn_decode of q_normed. q is read only; q_normed [heads x
 * dim] receives the normalised queries (q_normed == q normalises in place; any
 * other overlap is rejected). Outputs are the bits of those calls. One split pass
 * for head dim 256, rope_dim 64, 8 or 16 query heads per kv head, 16-byte aligned
 * pointers and q_normed apart from q: every workgroup normalises the query heads it
 * reads, the one holding key pos that row; otherwise a copy of q and the calls.
 * Workspace and statuses as qwen_attn_decode, plus the front end's.
 * ref: src/layer_attn.cpp:91-96 (attn_head_norm, rope_forward) and :103-108 */
int qwen_attn_decode_norm_rope(const float* q, float* q_normed, float* k_cache, const float* v_cache,
                               const float* gate, float* out, int heads, int kv_heads, int dim, int pos,
                               const float* q_weight, const float* k_weight, int rope_dim, float theta,
                               float eps, void* workspace, size_t workspace_bytes, void* stream);

/* qwen_attn_decode without a workspace argument and without any allocation: the
 * split-K partials live in a fixed device array of
 * qwen_attn_decode_noalloc_max_scratch_bytes() bytes (8 MiB) inside the library,
 * one copy per GPU, held until the process ends. No counterpart in the reference:
 * this entry point is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Shapes whose qwen_attn_decode_workspace_bytes exceed the array are rejected with
 * INVALID_ARGUMENT (16 query / 2 kv heads of 256: up to 16,256 keys; 8 query heads
 * per kv head: 516 bytes per key for 16 query heads). Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (several streams or host threads)
 * race and must be serialised by the caller. Nothing in the array has to start at
 * zero. Output equals qwen_attn_decode's bit for bit. */
size_t qwen_attn_decode_noalloc_max_scratch_bytes(void);
int qwen_attn_decode_noalloc(const float* q, const float* k_cache, const float* v_cache,
                             const float* gate, float* out, int heads, int kv_heads, int dim,
                             int pos, void* stream);

/* ====================================================================== MoE routing
 * The reference picks experts on the device, copies them to the host and syncs
 * (src/layer_moe.cpp:98-106); these entry points keep the routing on the device. */

/* Top-k of n router logits, then softmax over the k picks: idx int32 [k] (strictly
 * greater wins, ties to the lower index), weights [k]; a non-finite logit gives
 * idx[0] = -1, weights[0] = NaN. 0 < k <= min(n, 64), n <= 1024.
 * ref: src/layer_moe.cpp:9 (moe_topk decl), src/cuda/moe.cu:7-57 */
int qwen_moe_topk(const float* logits, int32_t* idx, float* weights, int n, int k, void* stream);
/* Row-batched form: logits [rows x n] -> idx, weights [rows x k]. */
int qwen_moe_topk_rows(const float* logits, int32_t* idx, float* weights, int rows, int n, int k,
                       void* stream);

/* out += a * x over n elements (a from the host).
 * ref: src/layer_moe.cpp:11 (moe_add decl), src/cuda/moe.cu:76-86 */
int qwen_moe_add(float* out, const float* x, float a, int n, void* stream);

/* out[t] += sum_j weights[t][j] * expert_out[t][j] for j < k (weights on the device):
 * the layer's k moe_add calls per token, src/layer_moe.cpp:127-142.
 * out [rows x dim], expert_out [rows x k x dim], weights [rows x k]. */
int qwen_moe_weighted_sum_rows(float* out, const float* expert_out, const float* weights, int rows,
                               int k, int dim, void* stream);

/* n_sel expert GEMVs in one launch with the expert ids on the device:
 * y[j] = W_e x_j, e = idx[j], W_e = the M x K rows at element offset e * expert_stride
 * of a GGML tensor of n_experts experts; x_j = x + j * x_stride; y [n_sel x M]. An id
 * outside [0, n_experts) gives a NaN row. Statuses as qwen_matmul_dispatch.
 * ref: src/layer_moe.cpp:131-138 (matmul_dispatch at element offset e * stride) */
int qwen_moe_expert_matmul(const void* weight, int type, uint64_t num_elements, uint64_t expert_stride,
                           int n_experts, const int32_t* idx, int n_sel, const float* x,
                           int64_t x_stride, float* y, int M, int K, void* stream);

/* The routed experts' gate and up projections of one token in one launch (the
 * reference's 2 x n_sel matmul_dispatch calls, src/layer_moe.cpp:131-132):
 * gate_out[j] = Wg_e x, up_out[j] = Wu_e x, e = idx[j] (on the device), j < n_sel;
 * gate_out, up_out [n_sel x M]. Both tensors of one type and element count, expert e
 * at element offset e * expert_stride. Bit-equal to two qwen_moe_expert_matmul calls
 * (x_stride 0); an id outside [0, n_experts) gives NaN rows. */
int qwen_moe_expert_gate_up(const void* w_gate, const void* w_up, int type, uint64_t num_elements,
                            uint64_t expert_stride, int n_experts, const int32_t* idx, int n_sel,
                            const float* x, float* gate_out, float* up_out, int M, int K, void* stream);

/* The SwiGLU hidden rows of a MoE layer's decode step in one launch
 * (src/layer_moe.cpp:131-133 per routed expert, :146-148 for the shared expert):
 *   hidden[j]     = SiLU(Wg_e x) * (Wu_e x)       e = idx[j] (on the device), j < n_sel
 *   shared_hidden = SiLU(Wsg x) * (Wsu x)          (when w_shared_gate / w_shared_up are given)
 * hidden [n_sel x inter], shared_hidden [shared_dim], x [K]. Routed expert e at element
 * offset e * expert_stride of w_gate / w_up (one type and element count); the shared
 * tensors may have another type. Bit-equal to the separate calls (two GEMVs each, then
 * qwen_moe_silu_mul); an invalid id gives NaN rows. Q4_K / Q6_K with K a multiple of
 * 2048 run in one launch; other shapes take the separate kernels through `workspace`
 * (qwen_moe_expert_swiglu_workspace_bytes() bytes, required in every case). No
 * counterpart entry point in the reference (it fuses the calls cited above). */
size_t qwen_moe_expert_swiglu_workspace_bytes(int n_sel, int inter, int shared_dim);
int qwen_moe_expert_swiglu(const void* w_gate, const void* w_up, int type, uint64_t num_elements,
                           uint64_t expert_stride, int n_experts, const int32_t* idx, int n_sel, int inter,
                           const void* w_shared_gate, const void* w_shared_up, int shared_type,
                           uint64_t shared_elements, int shared_dim, const float* x, int K, float* hidden,
                           float* shared_hidden, void* workspace, size_t workspace_bytes, void* stream);

/* The routing of a MoE decode step fused into qwen_moe_expert_swiglu: the ids and
 * weights of the k experts come from the n_experts router logits (top-k then softmax
 * over the picks, src/layer_moe.cpp:99, src/cuda/moe.cu:7-51, computed by the code of
 * qwen_moe_topk_rows) and are written to idx, weights [k] for the later calls; the
 * hidden rows are those of qwen_moe_expert_swiglu with these ids. Equals
 * qwen_moe_topk_rows (one row) followed by qwen_moe_expert_swiglu, bit for bit, for
 * finite logits; a non-finite logit gives idx[0] = -1, weights[0] = NaN (the rest
 * untouched, as the top-k call) and a NaN hidden row 0 (on the one-launch path every
 * routed row is NaN). n_experts <= 256, k <= 64.
 * Other arguments and statuses as qwen_moe_expert_swiglu. No counterpart entry point in
 * the reference (it fuses the calls cited above). */
int qwen_moe_route_swiglu(const float* logits, int32_t* idx, float* weights, int k, const void* w_gate,
                          const void* w_up, int type, uint64_t num_elements, uint64_t expert_stride,
                          int n_experts, int inter, const void* w_shared_gate, const void* w_shared_up,
                          int shared_type, uint64_t shared_elements, int shared_dim, const float* x, int K,
                          float* hidden, float* shared_hidden, void* workspace, size_t workspace_bytes,
                          void* stream);

/* The rest of a MoE layer's decode step after the SwiGLU hidden rows,
 * src/layer_moe.cpp:135-147 (the down projection per routed expert, moe_add from a
 * zeroed accumulator in routing order, the shared expert's down projection, the
 * sigmoid-gated shared add):
 *   out = sum_j weights[j] * Wd_e hidden[j]  (e = idx[j], j < n_sel)
 *       + sigmoid(shared_logit[0]) * Wsd shared_hidden
 * hidden [n_sel x inter], shared_hidden [shared_dim], out [d_model] (written, not
 * accumulated). Down expert e at element offset e * expert_stride. One launch for
 * inter = 512, shared_dim a multiple of 2048 up to 4096, n_sel <= 8 and Q4_K / Q6_K
 * weights; other shapes run the same steps as separate launches through `workspace`,
 * which must hold qwen_moe_down_combine_workspace_bytes() bytes in every case.
 * Bit-equal to the separate calls (qwen_moe_expert_matmul, qwen_matmul_dispatch,
 * qwen_moe_weighted_sum_rows into a zeroed out, qwen_moe_shared_add_rows); an invalid
 * expert id makes out NaN. No counterpart entry point in the reference (it fuses the
 * calls cited above). */
size_t qwen_moe_down_combine_workspace_bytes(int n_sel, int d_model);
int qwen_moe_down_combine(const void* w_down, int down_type, uint64_t down_elements, uint64_t expert_stride,
                          int n_experts, const int32_t* idx, const float* weights, int n_sel,
                          const float* hidden, int inter, const void* w_shared_down, int shared_type,
                          uint64_t shared_elements, const float* shared_hidden, int shared_dim,
                          const float* shared_logit, float* out, int d_model, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ====================================================================== MoE
 * h = silu(g) * u (fp32).  ref: src/layer_moe.cpp:10 (moe_silu_mul decl),
 * src/cuda/moe.cu:61-72 */
int qwen_moe_silu_mul(const float* gate, const float* up, float* hidden, int n, void* stream);

/* accum += x * sigmoid(gate[0]); gate is a device scalar.
 * ref: src/layer_moe.cpp:12 (moe_shared_add decl), src/cuda/moe.cu:90-101 */
int qwen_moe_shared_add(float* accum, const float* shared_out, const float* gate, int n,
                        void* stream);
/* Row-batched: accum, shared_out [rows x n], gate [rows] (one logit per token). */
int qwen_moe_shared_add_rows(float* accum, const float* shared_out, const float* gate, int rows,
                             int n, void* stream);

/* SwiGLU on bf16 storage with fp32 math: h = bf16(silu(g) * u), n elements
 * (e.g. [tokens x experts x moe_dim] flattened). Batched moe_silu_mul
 * (src/layer_moe.cpp:135). */
int qwen_swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n,
                     void* stream);
/* Shared expert SwiGLU with its sigmoid gate folded in:
 * h[t] = bf16((silu(g[t]) * u[t]) * sigmoid(logits[t])), rows x dim.
 * Equals moe_silu_mul (layer_moe.cpp:149) followed by moe_shared_add's scale
 * (layer_moe.cpp:153) moved before the (linear) down projection. */
int qwen_shared_swiglu_sigmoid_rows_bf16(const uint16_t* gate, const uint16_t* up,
                                         const float* logits, uint16_t* hidden, int rows, int dim,
                                         void* stream);
/* Both SwiGLUs of a MoE layer in one launch: the routed experts'
 * hidden = bf16(silu(gate) * up) over n elements (as qwen_swiglu_bf16) and the
 * shared expert's shared_hidden[t] = bf16((silu(shared_gate[t]) * shared_up[t]) *
 * sigmoid(logits[t])) over rows x dim (as qwen_shared_swiglu_sigmoid_rows_bf16);
 * each output equals its separate entry point bit for bit. Replaces the calls at
 * src/layer_moe.cpp:135 (per expert), :149 and :153 (src/cuda/moe.cu:61-101).
 * Either part may be empty (n == 0 or rows * dim == 0); pointers of an empty part
 * may be NULL. Shapes or pointers outside the 16-byte vector kernel (n or dim not
 * a multiple of 8, pointers not 16-byte aligned) run as the two separate launches. */
int qwen_swiglu_routed_shared_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden,
                                   int64_t n, const uint16_t* shared_gate,
                                   const uint16_t* shared_up, const float* logits,
                                   uint16_t* shared_hidden, int rows, int dim, void* stream);

/* ================================================================== dequant
 * GGML type ids as in include/quantized.hpp:12-35 (F32 0, F16 1, Q4_0 2,
 * Q5_0 6, Q8_0 8, Q4_K 12, Q5_K 13, Q6_K 14, BF16 30).
 * Returns 1 if `type` has a dequant path.
 * ref: include/matmul_q4.hpp:10 (matmul_type_supported), src/cuda/matmul_q4.cu:179-183 */
int qwen_type_supported(int type);

/* out[i] = element (row*cols + i) of the tensor, i < cols.
 * Errors: data NULL or type unsupported -> UNSUPPORTED_TYPE (reference message
 * "cannot dequantize tensor"); row < 0, cols <= 0 or the span past
 * num_elements -> OUT_OF_RANGE ("row is outside tensor").
 * ref: include/matmul_q4.hpp:24-30 (dequantize_row), src/cuda/matmul_q4.cu:209-227 */
int qwen_dequantize_row(const void* data, int type, uint64_t num_elements, float* out, int row,
                        int cols, void* stream);

/* Embedding gather: out[t] = dequantize_row(table, ids[t], cols) for t < n_ids,
 * ids a device int32 array. A table of num_elements holds num_elements/cols
 * rows; an id outside [0, rows) yields a row of quiet NaNs instead of a read
 * outside the table. Batched form of src/model.cpp:190. */
int qwen_dequant_gather_rows(const void* table, int type, uint64_t num_elements,
                             const int32_t* ids, int n_ids, int cols, float* out, void* stream);

/* ================================================================== quantized GEMV
 * ref: include/matmul_q4.hpp:10-21, src/cuda/matmul_q4.cu:140-167 (gemv_kernel), :179-207 */

/* Returns 1 if `type` has a GEMV path (the dequant types).
 * ref: include/matmul_q4.hpp:10 (matmul_type_supported), src/cuda/matmul_q4.cu:179-183 */
int qwen_matmul_type_supported(int type);

/* y[m] = sum_{k<K} W[element_offset + m*K + k] * x[k] for m < M: weight is the
 * device pointer of a GGML tensor of `type` holding num_elements elements
 * (row-major, K elements per row), x fp32 [K], y fp32 [M], fp32 accumulation.
 * Statuses, in the reference's order of checks: weight NULL ->
 * QWEN_STATUS_INVALID_ARGUMENT ("tensor is not loaded"); type without a path ->
 * QWEN_STATUS_UNSUPPORTED_TYPE; M <= 0, K <= 0 or element_offset + M*K past
 * num_elements -> QWEN_STATUS_OUT_OF_RANGE ("GEMV shape exceeds tensor").
 * ref: include/matmul_q4.hpp:13-21 (matmul_dispatch), src/cuda/matmul_q4.cu:185-207 */
int qwen_matmul_dispatch(const void* weight, int type, uint64_t num_elements, const float* x,
                         float* y, int M, int K, uint64_t element_offset, void* stream);

/* rows GEMVs of one matrix: y[t][m] = sum_{k<K} W[element_offset + m*K + k] * x[t][k]
 * for t < rows, m < M (x fp32 [rows x K], y fp32 [rows x M], row-major) -- the
 * reference's per-token matmul_dispatch over a prompt as one call. Q4_K and
 * Q6_K with K % 256 == 0, element_offset % 256 == 0, x 16-byte aligned and
 * rows >= 16 run on the matrix cores: each token row is scaled by a power of
 * two and split exactly into two fp16 parts (prep kernel, into the workspace),
 * the quants enter as exact fp16 integers, products are exact and sums fp32 --
 * an fp32 dot product's accuracy, not the reference's bits. Those cases need a
 * 16-byte aligned workspace of qwen_matmul_rows_workspace_bytes(rows, K)
 * bytes (QWEN_STATUS_INVALID_ARGUMENT otherwise); the other cases run
 * qwen_matmul_dispatch once per token and ignore it. A row of x holding an
 * infinity gives non-finite outputs (the NaN / infinity pattern may differ
 * from the reference's). rows == 0 is a no-op. Statuses and messages as
 * qwen_matmul_dispatch; rows < 0 or a NULL x / y -> QWEN_STATUS_INVALID_ARGUMENT.
 * ref: src/cuda/matmul_q4.cu:140-167,185-207 (the GEMV it batches), called per
 * token by the layers (src/layer_gdn.cpp:83-86, src/layer_attn.cpp:85-87) */
int qwen_matmul_rows(const void* weight, int type, uint64_t num_elements, const float* x, float* y,
                     int rows, int M, int K, uint64_t element_offset, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Workspace bytes qwen_matmul_rows needs for rows tokens of K elements (0 when
 * the call takes the per-token path: rows < 16 or K % 256 != 0). */
size_t qwen_matmul_rows_workspace_bytes(int rows, int K);

/* One projection of qwen_matmul_dispatch_multi: the arguments of one
 * qwen_matmul_dispatch call except x, K and the stream. */
typedef struct qwen_gemv_desc {
    const void* weight;       /* device GGML tensor */
    int type;                 /* GGML type id */
    int M;                    /* rows */
    uint64_t num_elements;    /* elements of the tensor */
    uint64_t element_offset;  /* first element of row 0 */
    float* y;                 /* output, fp32 [M] */
    int split;                /* 0: y[m] = row m. s > 0: the rows are M / (2 s) pairs of s-row
                                 halves (attention's fused query | gate projection, one pair per
                                 head) written as y[0 .. M/2) = the first halves, y[M/2 .. M) =
                                 the second: the projection followed by attn_split_qg
                                 (src/layer_attn.cpp:85,90), bit for bit. M % (2 s) == 0. */
} qwen_gemv_desc;

/* n GEMVs of the same x (K elements): y_j = W_j x for each descriptor, with the
 * results of n qwen_matmul_dispatch calls. The Q4_K / Q6_K projections of one
 * type run in one launch (up to 8 per launch); other types and shapes take
 * qwen_matmul_dispatch's kernels one by one. Every descriptor is validated
 * first, in order, with qwen_matmul_dispatch's statuses and messages (naming
 * the descriptor); nothing is launched if one fails. 0 <= n <= 64.
 * The reference issues these as consecutive matmul_dispatch calls on one
 * input: src/layer_gdn.cpp:83-86 (qkv, z, beta, alpha), src/layer_attn.cpp:85-87
 * (q|gate, k, v), src/layer_moe.cpp:98 (router), :145-147 (shared expert gate logit, gate, up). */
int qwen_matmul_dispatch_multi(const qwen_gemv_desc* descs, int n, const float* x, int K, void* stream);

/* qwen_matmul_rows for n matrices of the same x [rows x K]: y_j [rows x M_j] =
 * x W_j^T for each descriptor (split must be 0), with the results of n
 * qwen_matmul_rows calls bit for bit. x is prepared once (one prep launch) and
 * the Q4_K / Q6_K matrices of one type run in one GEMM launch (up to 8 per
 * launch), so small matrices (a layer's 32-row gate projections) share the
 * launch of the large ones; other types and offsets take the per-token path.
 * Validation as qwen_matmul_dispatch_multi; workspace as qwen_matmul_rows
 * (qwen_matmul_rows_workspace_bytes(rows, K)). 0 <= n <= 64.
 * ref: the per-token calls of src/layer_gdn.cpp:83-86, src/layer_attn.cpp:85-87 over a prompt */
int qwen_matmul_rows_multi(const qwen_gemv_desc* descs, int n, const float* x, int rows, int K,
                           void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN35_HIP_H */
