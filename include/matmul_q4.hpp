// Drop-in for include/matmul_q4.hpp of the reference (sahan974/qwen-3.5-cuda,
// :10-30), hipStream_t in place of cudaStream_t. matmul_dispatch and
// dequantize_row throw std::runtime_error with the reference's messages
// ("tensor '<name>' is not loaded", "unsupported GGML type for tensor '<name>'",
// "GEMV shape exceeds tensor '<name>'"; "cannot dequantize tensor '<name>'",
// "row is outside tensor '<name>'").
#ifndef QWEN35_MATMUL_Q4_HPP
#define QWEN35_MATMUL_Q4_HPP

#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "quantized.hpp"

namespace qwen {

// True for F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K.  ref: include/matmul_q4.hpp:10
bool matmul_type_supported(GgmlType type);

// y[m] = sum_k W[element_offset + m*K + k] * x[k], m < M (x, y device fp32).
// ref: include/matmul_q4.hpp:13-21
void matmul_dispatch(const QuantTensor& weight, const float* x, float* y, int M, int K, hipStream_t stream = nullptr,
                     uint64_t element_offset = 0);

// matmul_dispatch for each of `rows` tokens in one call: y[t*M + m] = sum_k
// W[element_offset + m*K + k] * x[t*K + k] (matrix cores for Q4_K / Q6_K at
// rows >= 16, fp32 accuracy), with a device workspace of
// matmul_rows_workspace_bytes(rows, K) bytes. Throws as matmul_dispatch.
// gdn_norm_gate of x, z [heads x dim] into normed, then matmul_dispatch of weight on
// normed (K = heads * dim): the same bits, one launch for Q4_K weights on the per-row
// path. Throws as the two calls.  ref: src/layer_gdn.cpp:109-112
void gdn_norm_gate_matmul(const float* x, const float* z, const float* norm_weight, float* normed, int heads, int dim,
                          float eps, const QuantTensor& weight, float* y, int M, hipStream_t stream = nullptr,
                          uint64_t element_offset = 0);

size_t matmul_rows_workspace_bytes(int rows, int K);
void matmul_rows(const QuantTensor& weight, const float* x, float* y, int rows, int M, int K, void* workspace,
                 size_t workspace_bytes, hipStream_t stream = nullptr, uint64_t element_offset = 0);

// n_sel expert GEMVs with the expert ids on the device: y[j] = W_{idx[j]} x_j,
// expert e at element offset e * expert_stride, x_j = x + j * x_stride, y
// [n_sel x M]; an invalid id gives a NaN row. Throws as matmul_dispatch.
void moe_expert_matmul(const QuantTensor& weight, uint64_t expert_stride, int n_experts, const int32_t* idx,
                       int n_sel, const float* x, int64_t x_stride, float* y, int M, int K,
                       hipStream_t stream = nullptr);

// The routed experts' gate and up GEMVs of one token in one launch (both
// tensors of one type and size): gate_out[j] = Wg_{idx[j]} x, up_out[j] =
// Wu_{idx[j]} x, [n_sel x M] each (src/layer_moe.cpp:131-132). Throws as
// matmul_dispatch, naming the gate tensor (or the up tensor if only it fails).
void moe_expert_gate_up(const QuantTensor& w_gate, const QuantTensor& w_up, uint64_t expert_stride, int n_experts,
                        const int32_t* idx, int n_sel, const float* x, float* gate_out, float* up_out, int M, int K,
                        hipStream_t stream = nullptr);

// The SwiGLU hidden rows of a MoE layer's decode step in one launch
// (src/layer_moe.cpp:131-133, :146-148): hidden[j] = SiLU(Wg_{idx[j]} x) *
// (Wu_{idx[j]} x) [n_sel x inter], and, when shared_gate is non-null,
// shared_hidden = SiLU(Wsg x) * (Wsu x) [shared_dim]. workspace:
// moe_expert_swiglu_workspace_bytes(n_sel, inter, shared_dim) bytes of device
// memory. Throws as matmul_dispatch, naming the tensor.
size_t moe_expert_swiglu_workspace_bytes(int n_sel, int inter, int shared_dim);
void moe_expert_swiglu(const QuantTensor& w_gate, const QuantTensor& w_up, uint64_t expert_stride, int n_experts,
                       const int32_t* idx, int n_sel, int inter, const QuantTensor* shared_gate,
                       const QuantTensor* shared_up, int shared_dim, const float* x, int K, float* hidden,
                       float* shared_hidden, void* workspace, size_t workspace_bytes, hipStream_t stream = nullptr);

// moe_topk (src/layer_moe.cpp:99) fused into moe_expert_swiglu: the k ids and
// weights come from the router logits [n_experts] and are written to idx,
// weights for the later calls. Throws as moe_expert_swiglu.
void moe_route_swiglu(const float* logits, int32_t* idx, float* weights, int k, const QuantTensor& w_gate,
                      const QuantTensor& w_up, uint64_t expert_stride, int n_experts, int inter,
                      const QuantTensor* shared_gate, const QuantTensor* shared_up, int shared_dim, const float* x,
                      int K, float* hidden, float* shared_hidden, void* workspace, size_t workspace_bytes,
                      hipStream_t stream = nullptr);

// The rest of a MoE layer's decode step after the SwiGLU hidden rows
// (src/layer_moe.cpp:135-147): out = sum_j weights[j] Wd_{idx[j]} hidden[j] +
// sigmoid(shared_logit[0]) Wsd shared_hidden. workspace:
// moe_down_combine_workspace_bytes(n_sel, d_model) bytes of device memory.
// Throws as matmul_dispatch, naming the tensor.
size_t moe_down_combine_workspace_bytes(int n_sel, int d_model);
void moe_down_combine(const QuantTensor& w_down, uint64_t expert_stride, int n_experts, const int32_t* idx,
                      const float* weights, int n_sel, const float* hidden, int inter,
                      const QuantTensor& w_shared_down, const float* shared_hidden, int shared_dim,
                      const float* shared_logit, float* out, int d_model, void* workspace, size_t workspace_bytes,
                      hipStream_t stream = nullptr);

// Several GEMVs of one x (K elements) in as few launches as possible: y_j =
// W_j x for each job, the results of n matmul_dispatch calls (the reference
// makes these calls one after another on one input, src/layer_gdn.cpp:83-86,
// src/layer_attn.cpp:85-87, src/layer_moe.cpp:145-147). Throws as
// matmul_dispatch, naming the first job that fails; nothing runs then.
struct GemvJob {
    const QuantTensor* weight;
    float* y;
    int M;
    uint64_t element_offset = 0;
    // s > 0: write the rows in attn_split_qg's layout (pairs of s-row halves,
    // first halves to y[0, M/2), second halves to y[M/2, M)), M % (2 s) == 0.
    int split = 0;
};
void matmul_dispatch_multi(const GemvJob* jobs, int n, const float* x, int K, hipStream_t stream = nullptr);

// matmul_rows for the n jobs of one x [rows x K] (one prep, one GEMM launch per
// K-quant type): job j writes y_j [rows x M_j]; split must be 0. Bit-equal to n
// matmul_rows calls. Throws as matmul_dispatch_multi.
void matmul_rows_multi(const GemvJob* jobs, int n, const float* x, int rows, int K, void* workspace,
                       size_t workspace_bytes, hipStream_t stream = nullptr);

// out[i] = element (row * cols + i) of `tensor`.  ref: include/matmul_q4.hpp:24-30
void dequantize_row(const QuantTensor& tensor, float* out, int row, int cols, hipStream_t stream = nullptr);

// Batched embedding gather: out[t] = dequantize_row(tensor, ids[t], cols) for
// t < n_ids; ids is a device int32 array. Ids outside the table give NaN rows.
void dequant_gather_rows(const QuantTensor& tensor, const int32_t* ids, int n_ids, int cols, float* out,
                         hipStream_t stream = nullptr);

}  // namespace qwen

#endif  // QWEN35_MATMUL_Q4_HPP
