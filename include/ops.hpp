// Drop-in for include/ops.hpp of the reference (sahan974/qwen-3.5-cuda,
// :11-47): same names, argument order, defaults and exception behaviour, with
// hipStream_t in place of cudaStream_t. Implemented over the C ABI in
// qwen35_hip.h; a failing call throws std::runtime_error with the C ABI's
// message. Every call is asynchronous on `stream`.
#ifndef QWEN35_OPS_HPP
#define QWEN35_OPS_HPP

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace qwen {

// out = norm(x) * weight (GGUF RMSNorm weights are already 1-centred).
// ref: include/ops.hpp:11-18
void rmsnorm_forward(const float* x, const float* weight, float* out, int N, float eps = 1e-6f,
                     hipStream_t stream = nullptr);

// out = norm(x) * weight * silu(gate).  ref: include/ops.hpp:21-29
void rmsnorm_gated_forward(const float* x, const float* gate, const float* weight, float* out, int N,
                           float eps = 1e-6f, hipStream_t stream = nullptr);

// out = x1 + x2.  ref: include/ops.hpp:32-38
void residual_add(const float* x1, const float* x2, float* out, int size, hipStream_t stream = nullptr);

// out = embed_table[token_id].  ref: include/ops.hpp:41-47
void encoder_forward(int token_id, const float* embed_table, float* out, int d_model,
                     hipStream_t stream = nullptr);

// ---- row-batched and fused forms (no reference counterpart; same per-row semantics)

// rmsnorm_forward over rows x N.
void rmsnorm_rows(const float* x, const float* weight, float* out, int rows, int N, float eps = 1e-6f,
                  hipStream_t stream = nullptr);

// residual_add then rmsnorm_forward on the sum (src/model.cpp:205,208), both outputs written.
void residual_rmsnorm_rows(const float* x, const float* branch, const float* weight, float* resid,
                           float* normed, int rows, int N, float eps = 1e-6f, hipStream_t stream = nullptr);

// bf16 storage (uint16_t), fp32 math.
void residual_rmsnorm_rows_bf16(const uint16_t* x, const uint16_t* branch, const float* weight,
                                uint16_t* resid, uint16_t* normed, int rows, int N, float eps = 1e-6f,
                                hipStream_t stream = nullptr);

}  // namespace qwen

#endif  // QWEN35_OPS_HPP
