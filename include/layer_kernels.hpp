// Kernels the reference's layer code forward-declares instead of including a
// header (src/layer_attn.cpp:10-15, src/layer_moe.cpp:9-12). The names and
// parameter lists match those declarations, with hipStream_t in place of
// cudaStream_t, so the layer code links against this library unchanged apart
// from the stream type.
#ifndef QWEN35_LAYER_KERNELS_HPP
#define QWEN35_LAYER_KERNELS_HPP

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace qwen {

// Per-head RMSNorm in place, x = x * (r * w).  ref: src/layer_attn.cpp:11
void attn_head_norm(float* x, const float* weight, int heads, int dim, float eps, hipStream_t stream);

// hidden = silu(gate) * up.  ref: src/layer_moe.cpp:10
void moe_silu_mul(const float* gate, const float* up, float* hidden, int dim, hipStream_t stream);

// accum += shared_out * sigmoid(sgate[0]) (sgate on the device).  ref: src/layer_moe.cpp:12
void moe_shared_add(float* accum, const float* shared_out, const float* sgate, int dim, hipStream_t stream);

// ---- row-batched forms

// moe_shared_add per row: accum, shared_out [rows x dim], sgate [rows].
void moe_shared_add_rows(float* accum, const float* shared_out, const float* sgate, int rows, int dim,
                         hipStream_t stream);

// bf16 SwiGLU over n elements: hidden = bf16(silu(gate) * up).
void swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n, hipStream_t stream);

// Shared-expert SwiGLU with the sigmoid gate folded in, rows x dim, one logit per row.
void shared_swiglu_sigmoid_rows_bf16(const uint16_t* gate, const uint16_t* up, const float* logits,
                                     uint16_t* hidden, int rows, int dim, hipStream_t stream);

}  // namespace qwen

#endif  // QWEN35_LAYER_KERNELS_HPP
