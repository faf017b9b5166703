// C++ drop-in layer (namespace qwen) over the C ABI: the reference's function
// names and signatures (with hipStream_t), throwing std::runtime_error where the
// reference throws. Each function forwards to its qwen_* C entry point.
#include <stdexcept>
#include <vector>
#include <string>

#include "gdn.hpp"
#include "layer_kernels.hpp"
#include "matmul_q4.hpp"
#include "ops.hpp"
#include "qwen35_hip.h"
#include "rope.hpp"

namespace qwen {
namespace {

void* st(hipStream_t s) { return reinterpret_cast<void*>(s); }

// Throws the C ABI's message for a failed call.
void check(int status) {
    if (status != QWEN_STATUS_OK) throw std::runtime_error(qwen_last_error());
}

}  // namespace

// ---- ops.hpp
void rmsnorm_forward(const float* x, const float* weight, float* out, int N, float eps, hipStream_t stream) {
    check(qwen_rmsnorm_forward(x, weight, out, N, eps, st(stream)));
}

void rmsnorm_gated_forward(const float* x, const float* gate, const float* weight, float* out, int N, float eps,
                           hipStream_t stream) {
    check(qwen_rmsnorm_gated_forward(x, gate, weight, out, N, eps, st(stream)));
}

void residual_add(const float* x1, const float* x2, float* out, int size, hipStream_t stream) {
    check(qwen_residual_add(x1, x2, out, size, st(stream)));
}

void encoder_forward(int token_id, const float* embed_table, float* out, int d_model, hipStream_t stream) {
    check(qwen_encoder_forward(token_id, embed_table, out, d_model, st(stream)));
}

void rmsnorm_rows(const float* x, const float* weight, float* out, int rows, int N, float eps, hipStream_t stream) {
    check(qwen_rmsnorm_rows(x, weight, out, rows, N, eps, st(stream)));
}

void residual_rmsnorm_rows(const float* x, const float* branch, const float* weight, float* resid, float* normed,
                           int rows, int N, float eps, hipStream_t stream) {
    check(qwen_residual_rmsnorm_rows_f32(x, branch, weight, resid, normed, rows, N, eps, st(stream)));
}

void residual_rmsnorm_rows_bf16(const uint16_t* x, const uint16_t* branch, const float* weight, uint16_t* resid,
                                uint16_t* normed, int rows, int N, float eps, hipStream_t stream) {
    check(qwen_residual_rmsnorm_rows_bf16(x, branch, weight, resid, normed, rows, N, eps, st(stream)));
}

// ---- rope.hpp
void rope_forward(float* q_or_k, int pos, int num_heads, int head_dim, int partial_rope_dim, float rope_theta,
                  hipStream_t stream) {
    // The C ABI reports the reference's own message, "invalid RoPE arguments".
    check(qwen_rope_forward(q_or_k, pos, num_heads, head_dim, partial_rope_dim, rope_theta, st(stream)));
}

void attn_qk_norm_rope_rows(float* q, float* k, const float* q_weight, const float* k_weight, const int32_t* pos,
                            int pos0, int rows, int q_heads, int k_heads, int head_dim, int partial_rope_dim,
                            float rope_theta, float eps, hipStream_t stream) {
    check(qwen_attn_qk_norm_rope_rows(q, k, q_weight, k_weight, pos, pos0, rows, q_heads, k_heads, head_dim,
                                      partial_rope_dim, rope_theta, eps, st(stream)));
}

// ---- gdn.hpp
void gdn_conv_step(const float* input, const float* weight, float* history, float* output, int channels, int kernel,
                   hipStream_t stream) {
    check(qwen_gdn_conv_step(input, weight, history, output, channels, kernel, st(stream)));
}

void gdn_qk_normalize(float* q, float* k, int heads, int dim, float eps, hipStream_t stream) {
    check(qwen_gdn_qk_normalize(q, k, heads, dim, eps, st(stream)));
}

void gdn_norm_gate(const float* x, const float* z, const float* weight, float* out, int heads, int dim, float eps,
                   hipStream_t stream) {
    check(qwen_gdn_norm_gate(x, z, weight, out, heads, dim, eps, st(stream)));
}

void gdn_gate_values(const float* beta_raw, const float* alpha_raw, const float* a, const float* dt_bias, float* beta,
                     float* decay, int heads, hipStream_t stream) {
    check(qwen_gdn_gate_values(beta_raw, alpha_raw, a, dt_bias, beta, decay, heads, st(stream)));
}

void gdn_gate_values_rows(const float* beta_raw, const float* alpha_raw, const float* a, const float* dt_bias,
                          float* beta, float* decay, int rows, int heads, hipStream_t stream) {
    check(qwen_gdn_gate_values_rows(beta_raw, alpha_raw, a, dt_bias, beta, decay, rows, heads, st(stream)));
}

void gdn_recurrent_step(float* state, const float* q, const float* k, const float* v, const float* beta,
                        const float* decay, float* out, int key_heads, int value_heads, int key_dim, int value_dim,
                        hipStream_t stream) {
    check(qwen_gdn_recurrent_step(state, q, k, v, beta, decay, out, key_heads, value_heads, key_dim, value_dim,
                                  st(stream)));
}

void gdn_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta,
                        const float* decay, float* out, int rows, int key_heads, int value_heads, int key_dim,
                        int value_dim, int64_t qkv_stride, int64_t out_stride, hipStream_t stream) {
    check(qwen_gdn_recurrent_rows(state, q, k, v, beta, decay, out, rows, key_heads, value_heads, key_dim, value_dim,
                                  qkv_stride, out_stride, st(stream)));
}

void gdn_gated_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta_raw,
                              const float* alpha_raw, const float* a, const float* dt_bias, float* out, int rows,
                              int key_heads, int value_heads, int key_dim, int value_dim, int64_t qkv_stride,
                              int64_t out_stride, hipStream_t stream) {
    check(qwen_gdn_gated_recurrent_rows(state, q, k, v, beta_raw, alpha_raw, a, dt_bias, out, rows, key_heads,
                                        value_heads, key_dim, value_dim, qkv_stride, out_stride, st(stream)));
}

void gdn_decode_step(const float* x, const float* conv_weight, const float* hist_in, float* hist_out, float* y,
                     float* state, const float* beta_raw, const float* alpha_raw, const float* a,
                     const float* dt_bias, float* out, int key_heads, int value_heads, int key_dim, int value_dim,
                     int kernel, float eps, hipStream_t stream) {
    check(qwen_gdn_decode_step(x, conv_weight, hist_in, hist_out, y, state, beta_raw, alpha_raw, a, dt_bias, out,
                               key_heads, value_heads, key_dim, value_dim, kernel, eps, st(stream)));
}

void gdn_frontend_rows(const float* x, const float* weight, const float* hist_in, float* hist_out, float* y, int rows,
                       int channels, int kernel, int k_heads, int key_dim, float eps, hipStream_t stream) {
    check(qwen_gdn_frontend_rows(x, weight, hist_in, hist_out, y, rows, channels, kernel, k_heads, key_dim, eps,
                                 st(stream)));
}

void gdn_norm_gate_rows(const float* x, const float* z, const float* weight, float* out, int rows, int heads, int dim,
                        float eps, hipStream_t stream) {
    check(qwen_gdn_norm_gate_rows(x, z, weight, out, rows, heads, dim, eps, st(stream)));
}

// ---- layer_kernels.hpp
void attn_head_norm(float* x, const float* weight, int heads, int dim, float eps, hipStream_t stream) {
    check(qwen_attn_head_norm(x, weight, heads, dim, eps, st(stream)));
}

void attn_split_qg(const float* qg, float* q, float* gate, int heads, int dim, hipStream_t stream) {
    check(qwen_attn_split_qg(qg, q, gate, heads, dim, st(stream)));
}

void attn_scores(const float* q, const float* k_cache, float* scores, int q_heads, int kv_heads, int dim, int pos,
                 hipStream_t stream) {
    check(qwen_attn_scores(q, k_cache, scores, q_heads, kv_heads, dim, pos, st(stream)));
}

void attn_softmax(float* scores, int heads, int valid_len, hipStream_t stream) {
    check(qwen_attn_softmax(scores, heads, valid_len, st(stream)));
}

void attn_values(const float* scores, const float* v_cache, float* out, int q_heads, int kv_heads, int dim, int pos,
                 hipStream_t stream) {
    check(qwen_attn_values(scores, v_cache, out, q_heads, kv_heads, dim, pos, st(stream)));
}

void attn_sigmoid_gate(const float* attn, const float* gate, float* out, int dim, hipStream_t stream) {
    check(qwen_attn_sigmoid_gate(attn, gate, out, dim, st(stream)));
}

void attn_kv_store(const float* k, const float* v, float* k_cache, float* v_cache, int pos, int kv_dim,
                   int max_seq_len, hipStream_t stream) {
    check(qwen_attn_kv_store(k, v, k_cache, v_cache, pos, kv_dim, max_seq_len, st(stream)));
}

size_t attn_decode_workspace_bytes(int heads, int kv_heads, int dim, int pos) {
    return qwen_attn_decode_workspace_bytes(heads, kv_heads, dim, pos);
}

void attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* gate, float* out, int heads,
                 int kv_heads, int dim, int pos, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    check(qwen_attn_decode(q, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, workspace, workspace_bytes,
                           st(stream)));
}

void attn_decode_norm_rope(const float* q, float* q_normed, float* k_cache, const float* v_cache, const float* gate,
                           float* out, int heads, int kv_heads, int dim, int pos, const float* q_weight,
                           const float* k_weight, int rope_dim, float theta, float eps, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
    check(qwen_attn_decode_norm_rope(q, q_normed, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, q_weight,
                                     k_weight, rope_dim, theta, eps, workspace, workspace_bytes, st(stream)));
}

void moe_topk(const float* router, int* top_idx, float* top_weight, int experts, int k, hipStream_t stream) {
    check(qwen_moe_topk(router, top_idx, top_weight, experts, k, st(stream)));
}

void moe_topk_rows(const float* router, int* top_idx, float* top_weight, int rows, int experts, int k,
                   hipStream_t stream) {
    check(qwen_moe_topk_rows(router, top_idx, top_weight, rows, experts, k, st(stream)));
}

void moe_add(float* accum, const float* expert_out, float weight, int dim, hipStream_t stream) {
    check(qwen_moe_add(accum, expert_out, weight, dim, st(stream)));
}

void moe_weighted_sum_rows(float* accum, const float* expert_out, const float* weight, int rows, int k, int dim,
                           hipStream_t stream) {
    check(qwen_moe_weighted_sum_rows(accum, expert_out, weight, rows, k, dim, st(stream)));
}

void moe_silu_mul(const float* gate, const float* up, float* hidden, int dim, hipStream_t stream) {
    check(qwen_moe_silu_mul(gate, up, hidden, dim, st(stream)));
}

void moe_shared_add(float* accum, const float* shared_out, const float* sgate, int dim, hipStream_t stream) {
    check(qwen_moe_shared_add(accum, shared_out, sgate, dim, st(stream)));
}

void moe_shared_add_rows(float* accum, const float* shared_out, const float* sgate, int rows, int dim,
                         hipStream_t stream) {
    check(qwen_moe_shared_add_rows(accum, shared_out, sgate, rows, dim, st(stream)));
}

void swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n, hipStream_t stream) {
    check(qwen_swiglu_bf16(gate, up, hidden, n, st(stream)));
}

void shared_swiglu_sigmoid_rows_bf16(const uint16_t* gate, const uint16_t* up, const float* logits, uint16_t* hidden,
                                     int rows, int dim, hipStream_t stream) {
    check(qwen_shared_swiglu_sigmoid_rows_bf16(gate, up, logits, hidden, rows, dim, st(stream)));
}

void swiglu_routed_shared_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n,
                               const uint16_t* shared_gate, const uint16_t* shared_up, const float* logits,
                               uint16_t* shared_hidden, int rows, int dim, hipStream_t stream) {
    check(qwen_swiglu_routed_shared_bf16(gate, up, hidden, n, shared_gate, shared_up, logits, shared_hidden, rows,
                                         dim, st(stream)));
}

// ---- matmul_q4.hpp
namespace {
// matmul_dispatch's messages for tensor w (src/cuda/matmul_q4.cu:187-195).
void throw_tensor_status(int status, const QuantTensor& w) {
    if (status == QWEN_STATUS_INVALID_ARGUMENT && !w.device_ptr)
        throw std::runtime_error("tensor '" + w.name + "' is not loaded");
    if (status == QWEN_STATUS_UNSUPPORTED_TYPE)
        throw std::runtime_error("unsupported GGML type for tensor '" + w.name + "'");
    if (status == QWEN_STATUS_OUT_OF_RANGE) throw std::runtime_error("GEMV shape exceeds tensor '" + w.name + "'");
}
}  // namespace

bool matmul_type_supported(GgmlType type) { return qwen_matmul_type_supported(static_cast<int>(type)) != 0; }

void matmul_dispatch(const QuantTensor& w, const float* x, float* y, int M, int K, hipStream_t stream,
                     uint64_t element_offset) {
    const int status = qwen_matmul_dispatch(w.device_ptr, static_cast<int>(w.type), w.num_elements, x, y, M, K,
                                            element_offset, st(stream));
    throw_tensor_status(status, w);
    check(status);
}

void gdn_norm_gate_matmul(const float* x, const float* z, const float* norm_weight, float* normed, int heads, int dim,
                          float eps, const QuantTensor& w, float* y, int M, hipStream_t stream,
                          uint64_t element_offset) {
    const int status = qwen_gdn_norm_gate_matmul(x, z, norm_weight, normed, heads, dim, eps, w.device_ptr,
                                                 static_cast<int>(w.type), w.num_elements, y, M, element_offset,
                                                 st(stream));
    throw_tensor_status(status, w);
    check(status);
}

size_t matmul_rows_workspace_bytes(int rows, int K) { return qwen_matmul_rows_workspace_bytes(rows, K); }

void matmul_rows(const QuantTensor& w, const float* x, float* y, int rows, int M, int K, void* workspace,
                 size_t workspace_bytes, hipStream_t stream, uint64_t element_offset) {
    const int status = qwen_matmul_rows(w.device_ptr, static_cast<int>(w.type), w.num_elements, x, y, rows, M, K,
                                        element_offset, workspace, workspace_bytes, st(stream));
    throw_tensor_status(status, w);
    check(status);
}

void moe_expert_matmul(const QuantTensor& w, uint64_t expert_stride, int n_experts, const int32_t* idx, int n_sel,
                       const float* x, int64_t x_stride, float* y, int M, int K, hipStream_t stream) {
    const int status = qwen_moe_expert_matmul(w.device_ptr, static_cast<int>(w.type), w.num_elements, expert_stride,
                                              n_experts, idx, n_sel, x, x_stride, y, M, K, st(stream));
    throw_tensor_status(status, w);
    check(status);
}

void moe_expert_gate_up(const QuantTensor& w_gate, const QuantTensor& w_up, uint64_t expert_stride, int n_experts,
                        const int32_t* idx, int n_sel, const float* x, float* gate_out, float* up_out, int M, int K,
                        hipStream_t stream) {
    if (w_gate.type != w_up.type || w_gate.num_elements != w_up.num_elements) {
        moe_expert_matmul(w_gate, expert_stride, n_experts, idx, n_sel, x, 0, gate_out, M, K, stream);
        moe_expert_matmul(w_up, expert_stride, n_experts, idx, n_sel, x, 0, up_out, M, K, stream);
        return;
    }
    const int status = qwen_moe_expert_gate_up(w_gate.device_ptr, w_up.device_ptr, static_cast<int>(w_gate.type),
                                               w_gate.num_elements, expert_stride, n_experts, idx, n_sel, x, gate_out,
                                               up_out, M, K, st(stream));
    throw_tensor_status(status, w_gate.device_ptr && !w_up.device_ptr ? w_up : w_gate);
    check(status);
}

size_t moe_expert_swiglu_workspace_bytes(int n_sel, int inter, int shared_dim) {
    return qwen_moe_expert_swiglu_workspace_bytes(n_sel, inter, shared_dim);
}

namespace {
void swiglu_checks(const QuantTensor& w_gate, const QuantTensor& w_up, const QuantTensor* shared_gate,
                   const QuantTensor* shared_up) {
    if (!shared_gate != !shared_up) throw std::invalid_argument("moe_expert_swiglu: shared gate without shared up");
    // matmul_dispatch's checks in the order the reference's calls meet the tensors
    std::vector<const QuantTensor*> ts{&w_gate, &w_up};
    if (shared_gate) ts.insert(ts.end(), {shared_gate, shared_up});
    for (const QuantTensor* w : ts) {
        if (!w->device_ptr) throw std::runtime_error("tensor '" + w->name + "' is not loaded");
        if (!matmul_type_supported(w->type))
            throw std::runtime_error("unsupported GGML type for tensor '" + w->name + "'");
    }
    if (w_gate.type != w_up.type || w_gate.num_elements != w_up.num_elements ||
        (shared_gate && (shared_gate->type != shared_up->type || shared_gate->num_elements != shared_up->num_elements)))
        throw std::invalid_argument("moe_expert_swiglu: gate and up tensors differ in type or size");
}

void swiglu_status(int status, const QuantTensor& w_gate, const QuantTensor* shared_gate, uint64_t expert_stride,
                   int n_experts, int inter, int K) {
    if (status == QWEN_STATUS_OUT_OF_RANGE) {
        const bool routed = static_cast<uint64_t>(inter) * static_cast<uint64_t>(K) > expert_stride || n_experts <= 0 ||
                            expert_stride > w_gate.num_elements / static_cast<uint64_t>(n_experts);
        throw std::runtime_error("GEMV shape exceeds tensor '" + (routed ? w_gate : *shared_gate).name + "'");
    }
    check(status);
}
}  // namespace

void moe_expert_swiglu(const QuantTensor& w_gate, const QuantTensor& w_up, uint64_t expert_stride, int n_experts,
                       const int32_t* idx, int n_sel, int inter, const QuantTensor* shared_gate,
                       const QuantTensor* shared_up, int shared_dim, const float* x, int K, float* hidden,
                       float* shared_hidden, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    swiglu_checks(w_gate, w_up, shared_gate, shared_up);
    const int status = qwen_moe_expert_swiglu(
        w_gate.device_ptr, w_up.device_ptr, static_cast<int>(w_gate.type), w_gate.num_elements, expert_stride,
        n_experts, idx, n_sel, inter, shared_gate ? shared_gate->device_ptr : nullptr,
        shared_up ? shared_up->device_ptr : nullptr, shared_gate ? static_cast<int>(shared_gate->type) : 0,
        shared_gate ? shared_gate->num_elements : 0, shared_dim, x, K, hidden, shared_hidden, workspace,
        workspace_bytes, st(stream));
    swiglu_status(status, w_gate, shared_gate, expert_stride, n_experts, inter, K);
}

void moe_route_swiglu(const float* logits, int32_t* idx, float* weights, int k, const QuantTensor& w_gate,
                      const QuantTensor& w_up, uint64_t expert_stride, int n_experts, int inter,
                      const QuantTensor* shared_gate, const QuantTensor* shared_up, int shared_dim, const float* x,
                      int K, float* hidden, float* shared_hidden, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
    swiglu_checks(w_gate, w_up, shared_gate, shared_up);
    const int status = qwen_moe_route_swiglu(
        logits, idx, weights, k, w_gate.device_ptr, w_up.device_ptr, static_cast<int>(w_gate.type),
        w_gate.num_elements, expert_stride, n_experts, inter, shared_gate ? shared_gate->device_ptr : nullptr,
        shared_up ? shared_up->device_ptr : nullptr, shared_gate ? static_cast<int>(shared_gate->type) : 0,
        shared_gate ? shared_gate->num_elements : 0, shared_dim, x, K, hidden, shared_hidden, workspace,
        workspace_bytes, st(stream));
    swiglu_status(status, w_gate, shared_gate, expert_stride, n_experts, inter, K);
}

size_t moe_down_combine_workspace_bytes(int n_sel, int d_model) {
    return qwen_moe_down_combine_workspace_bytes(n_sel, d_model);
}

void moe_down_combine(const QuantTensor& w_down, uint64_t expert_stride, int n_experts, const int32_t* idx,
                      const float* weights, int n_sel, const float* hidden, int inter,
                      const QuantTensor& w_shared_down, const float* shared_hidden, int shared_dim,
                      const float* shared_logit, float* out, int d_model, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
    // Tensor checks in the order the reference's calls meet them: the routed
    // down projection first, then the shared expert's.
    for (const QuantTensor* w : {&w_down, &w_shared_down}) {
        if (!w->device_ptr) throw std::runtime_error("tensor '" + w->name + "' is not loaded");
        if (!matmul_type_supported(w->type))
            throw std::runtime_error("unsupported GGML type for tensor '" + w->name + "'");
    }
    const int status = qwen_moe_down_combine(
        w_down.device_ptr, static_cast<int>(w_down.type), w_down.num_elements, expert_stride, n_experts, idx, weights,
        n_sel, hidden, inter, w_shared_down.device_ptr, static_cast<int>(w_shared_down.type),
        w_shared_down.num_elements, shared_hidden, shared_dim, shared_logit, out, d_model, workspace, workspace_bytes,
        st(stream));
    if (status == QWEN_STATUS_OUT_OF_RANGE) {
        const bool routed = static_cast<uint64_t>(d_model) * static_cast<uint64_t>(inter) > expert_stride ||
                            n_experts <= 0 || expert_stride > w_down.num_elements / static_cast<uint64_t>(n_experts);
        throw std::runtime_error("GEMV shape exceeds tensor '" + (routed ? w_down : w_shared_down).name + "'");
    }
    check(status);
}

namespace {
// matmul_dispatch's checks and messages per job, then the C descriptor table.
std::vector<qwen_gemv_desc> gemv_descs(const GemvJob* jobs, int n, int K) {
    std::vector<qwen_gemv_desc> d(static_cast<size_t>(n));
    for (int j = 0; j < n; ++j) {
        const QuantTensor& w = *jobs[j].weight;
        // matmul_dispatch's checks and messages per job (src/cuda/matmul_q4.cu:187-195)
        if (!w.device_ptr) throw std::runtime_error("tensor '" + w.name + "' is not loaded");
        if (!matmul_type_supported(w.type)) throw std::runtime_error("unsupported GGML type for tensor '" + w.name + "'");
        const uint64_t need = static_cast<uint64_t>(jobs[j].M) * static_cast<uint64_t>(K);
        if (jobs[j].M <= 0 || K <= 0 || jobs[j].element_offset > w.num_elements ||
            need > w.num_elements - jobs[j].element_offset)
            throw std::runtime_error("GEMV shape exceeds tensor '" + w.name + "'");
        d[j] = qwen_gemv_desc{w.device_ptr, static_cast<int>(w.type), jobs[j].M, w.num_elements,
                              jobs[j].element_offset, jobs[j].y, jobs[j].split};
    }
    return d;
}
}  // namespace

void matmul_dispatch_multi(const GemvJob* jobs, int n, const float* x, int K, hipStream_t stream) {
    if (n <= 0) return;
    const std::vector<qwen_gemv_desc> d = gemv_descs(jobs, n, K);
    check(qwen_matmul_dispatch_multi(d.data(), n, x, K, st(stream)));
}

void matmul_rows_multi(const GemvJob* jobs, int n, const float* x, int rows, int K, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
    if (n <= 0) return;
    const std::vector<qwen_gemv_desc> d = gemv_descs(jobs, n, K);
    check(qwen_matmul_rows_multi(d.data(), n, x, rows, K, workspace, workspace_bytes, st(stream)));
}

void dequantize_row(const QuantTensor& tensor, float* out, int row, int cols, hipStream_t stream) {
    const int status = qwen_dequantize_row(tensor.device_ptr, static_cast<int>(tensor.type), tensor.num_elements, out,
                                           row, cols, st(stream));
    // Reference messages, src/cuda/matmul_q4.cu:210-217.
    if (status == QWEN_STATUS_UNSUPPORTED_TYPE)
        throw std::runtime_error("cannot dequantize tensor '" + tensor.name + "'");
    if (status == QWEN_STATUS_OUT_OF_RANGE) throw std::runtime_error("row is outside tensor '" + tensor.name + "'");
    check(status);
}

void dequant_gather_rows(const QuantTensor& tensor, const int32_t* ids, int n_ids, int cols, float* out,
                         hipStream_t stream) {
    const int status = qwen_dequant_gather_rows(tensor.device_ptr, static_cast<int>(tensor.type), tensor.num_elements,
                                                ids, n_ids, cols, out, st(stream));
    if (status == QWEN_STATUS_UNSUPPORTED_TYPE)
        throw std::runtime_error("cannot dequantize tensor '" + tensor.name + "'");
    check(status);
}

}  // namespace qwen
