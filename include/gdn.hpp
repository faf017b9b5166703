// Drop-in for the Gated DeltaNet kernels of include/gdn.hpp of the reference
// (sahan974/qwen-3.5-cuda, :9-67), hipStream_t in place of cudaStream_t.
#ifndef QWEN35_GDN_HPP
#define QWEN35_GDN_HPP

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace qwen {

// One decode step of the causal depthwise conv + SiLU; history [channels x
// (kernel-1)] shifted in place.  ref: include/gdn.hpp:9-17
void gdn_conv_step(const float* input, const float* weight, float* history, float* output, int channels,
                   int kernel, hipStream_t stream);

// Per-head L2 norm of q and k in place, q also scaled by 1/sqrt(dim).
// ref: include/gdn.hpp:20-27
void gdn_qk_normalize(float* q, float* k, int heads, int dim, float eps, hipStream_t stream);

// beta = sigmoid(beta_raw); decay = exp(a * softplus(alpha_raw + dt_bias)) per
// value head.  ref: include/gdn.hpp:29-38
void gdn_gate_values(const float* beta_raw, const float* alpha_raw, const float* a, const float* dt_bias,
                     float* beta, float* decay, int heads, hipStream_t stream);

// One delta-rule step of the [value_heads x key_dim x value_dim] state, in
// place; throws "GDN value dimension exceeds kernel limit" for value_dim > 256.
// ref: include/gdn.hpp:41-54
void gdn_recurrent_step(float* state, const float* q, const float* k, const float* v, const float* beta,
                        const float* decay, float* out, int key_heads, int value_heads, int key_dim, int value_dim,
                        hipStream_t stream);

// out = norm(x) * weight * silu(z) per head.  ref: include/gdn.hpp:58-67
void gdn_norm_gate(const float* x, const float* z, const float* weight, float* out, int heads, int dim,
                   float eps, hipStream_t stream);

// ---- row-batched and fused forms

// `rows` conv steps + the q/k L2 norm of every row in one pass
// (src/layer_gdn.cpp:89-97); hist_out may equal hist_in.
void gdn_frontend_rows(const float* x, const float* weight, const float* hist_in, float* hist_out, float* y,
                       int rows, int channels, int kernel, int k_heads, int key_dim, float eps,
                       hipStream_t stream);

// gdn_gate_values over rows x heads (a, dt_bias per head).
void gdn_gate_values_rows(const float* beta_raw, const float* alpha_raw, const float* a, const float* dt_bias,
                          float* beta, float* decay, int rows, int heads, hipStream_t stream);

// `rows` consecutive recurrent steps in one launch; token t reads q, k, v at
// t * qkv_stride and beta, decay at t * value_heads, writes out at t * out_stride.
void gdn_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta,
                        const float* decay, float* out, int rows, int key_heads, int value_heads, int key_dim,
                        int value_dim, int64_t qkv_stride, int64_t out_stride, hipStream_t stream);

// gdn_gate_values fused into gdn_recurrent_rows (one launch per decode step,
// the same bits): beta_raw, alpha_raw [rows x value_heads], a, dt_bias
// [value_heads]. ref: src/layer_gdn.cpp:100-106
void gdn_gated_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta_raw,
                              const float* alpha_raw, const float* a, const float* dt_bias, float* out, int rows,
                              int key_heads, int value_heads, int key_dim, int value_dim, int64_t qkv_stride = 0,
                              int64_t out_stride = 0, hipStream_t stream = nullptr);

// One decode token after the input projections (src/layer_gdn.cpp:89-106):
// gdn_frontend_rows on x [C] (history hist_in -> hist_out, output y [C]) then
// gdn_gated_recurrent_rows on y, the same bits, one launch when hist_out does
// not overlap hist_in (key dim 128, conv kernel 4).
void gdn_decode_step(const float* x, const float* conv_weight, const float* hist_in, float* hist_out, float* y,
                     float* state, const float* beta_raw, const float* alpha_raw, const float* a,
                     const float* dt_bias, float* out, int key_heads, int value_heads, int key_dim, int value_dim,
                     int kernel, float eps = 1e-6f, hipStream_t stream = nullptr);

// gdn_norm_gate over rows x heads x dim.
void gdn_norm_gate_rows(const float* x, const float* z, const float* weight, float* out, int rows, int heads,
                        int dim, float eps, hipStream_t stream);

}  // namespace qwen

#endif  // QWEN35_GDN_HPP
