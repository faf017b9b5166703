// Kernels the reference's layer code forward-declares instead of including a
// header (src/layer_attn.cpp:10-15, src/layer_moe.cpp:9-12). The names and
// parameter lists match those declarations, with hipStream_t in place of
// cudaStream_t, so the layer code links against this library unchanged apart
// from the stream type.
#ifndef QWEN35_LAYER_KERNELS_HPP
#define QWEN35_LAYER_KERNELS_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace qwen {

// Per-head RMSNorm in place, x = x * (r * w).  ref: src/layer_attn.cpp:11
void attn_head_norm(float* x, const float* weight, int heads, int dim, float eps, hipStream_t stream);

// q[h] = qg[h][0:dim], gate[h] = qg[h][dim:2*dim].  ref: src/layer_attn.cpp:10
void attn_split_qg(const float* qg, float* q, float* gate, int heads, int dim, hipStream_t stream);

// scores[h][t] = (q_h . k_cache[t][h / (heads / kv_heads)]) / sqrt(dim), t <= pos.
// ref: src/layer_attn.cpp:12
void attn_scores(const float* q, const float* k_cache, float* scores, int q_heads, int kv_heads, int dim, int pos,
                 hipStream_t stream);

// Row softmax of scores [heads x valid_len] in place.  ref: src/layer_attn.cpp:13
void attn_softmax(float* scores, int heads, int valid_len, hipStream_t stream);

// out[h][j] = sum_t scores[h][t] * v_cache[t][h / (heads / kv_heads)][j].  ref: src/layer_attn.cpp:14
void attn_values(const float* scores, const float* v_cache, float* out, int q_heads, int kv_heads, int dim, int pos,
                 hipStream_t stream);

// out = attn / (1 + exp(-gate)).  ref: src/layer_attn.cpp:15
void attn_sigmoid_gate(const float* attn, const float* gate, float* out, int dim, hipStream_t stream);

// hidden = silu(gate) * up.  ref: src/layer_moe.cpp:10
void moe_silu_mul(const float* gate, const float* up, float* hidden, int dim, hipStream_t stream);

// Top-k experts of the router logits and softmax weights over the picks
// (idx[0] = -1, weight[0] = NaN for a non-finite logit).  ref: src/layer_moe.cpp:9
void moe_topk(const float* router, int* top_idx, float* top_weight, int experts, int k, hipStream_t stream);

// accum += weight * expert_out.  ref: src/layer_moe.cpp:11
void moe_add(float* accum, const float* expert_out, float weight, int dim, hipStream_t stream);

// accum += shared_out * sigmoid(sgate[0]) (sgate on the device).  ref: src/layer_moe.cpp:12
void moe_shared_add(float* accum, const float* shared_out, const float* sgate, int dim, hipStream_t stream);

// ---- row-batched and fused forms

// Cache store of src/layer_attn.cpp:99-100: k, v [kv_dim] to row pos; throws
// "attention position exceeds configured context" unless 0 <= pos < max_seq_len.
void attn_kv_store(const float* k, const float* v, float* k_cache, float* v_cache, int pos, int kv_dim,
                   int max_seq_len, hipStream_t stream);

// Bytes of workspace attn_decode needs for this shape.
size_t attn_decode_workspace_bytes(int heads, int kv_heads, int dim, int pos);

// scores -> softmax -> values -> (gate) of src/layer_attn.cpp:103-108 in one
// split-K pass and a combine; gate may be null.
void attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* gate, float* out, int heads,
                 int kv_heads, int dim, int pos, void* workspace, size_t workspace_bytes, hipStream_t stream);

// The Q/K norm + RoPE of src/layer_attn.cpp:91-96 folded into attn_decode: q_normed
// receives the normalised queries (q read only; q_normed == q normalises in place),
// the cache row of pos is normalised in place, then the decode of q_normed. The
// same bits as those calls; one split pass at the production head shape.
void attn_decode_norm_rope(const float* q, float* q_normed, float* k_cache, const float* v_cache, const float* gate,
                           float* out, int heads, int kv_heads, int dim, int pos, const float* q_weight,
                           const float* k_weight, int rope_dim, float theta, float eps, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

// moe_shared_add per row: accum, shared_out [rows x dim], sgate [rows].
void moe_shared_add_rows(float* accum, const float* shared_out, const float* sgate, int rows, int dim,
                         hipStream_t stream);

// moe_topk per row: router [rows x experts] -> top_idx, top_weight [rows x k].
void moe_topk_rows(const float* router, int* top_idx, float* top_weight, int rows, int experts, int k,
                   hipStream_t stream);

// accum[t] += sum_j weight[t][j] * expert_out[t][j] with the weights on the device.
void moe_weighted_sum_rows(float* accum, const float* expert_out, const float* weight, int rows, int k, int dim,
                           hipStream_t stream);

// bf16 SwiGLU over n elements: hidden = bf16(silu(gate) * up).
void swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n, hipStream_t stream);

// Shared-expert SwiGLU with the sigmoid gate folded in, rows x dim, one logit per row.
void shared_swiglu_sigmoid_rows_bf16(const uint16_t* gate, const uint16_t* up, const float* logits,
                                     uint16_t* hidden, int rows, int dim, hipStream_t stream);

// Routed SwiGLU over n elements and the shared expert's gated SwiGLU (rows x dim)
// in one launch; each output equals the separate call.
void swiglu_routed_shared_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n,
                               const uint16_t* shared_gate, const uint16_t* shared_up, const float* logits,
                               uint16_t* shared_hidden, int rows, int dim, hipStream_t stream);

}  // namespace qwen

#endif  // QWEN35_LAYER_KERNELS_HPP
