// Drop-in for include/rope.hpp of the reference (sahan974/qwen-3.5-cuda,
// :13-21), hipStream_t in place of cudaStream_t. Throws
// std::runtime_error("invalid RoPE arguments") on the reference's conditions.
#ifndef QWEN35_ROPE_HPP
#define QWEN35_ROPE_HPP

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace qwen {

// Partial split-half RoPE in place on q_or_k [num_heads x head_dim].
// ref: include/rope.hpp:13-21
void rope_forward(float* q_or_k, int pos, int num_heads, int head_dim, int partial_rope_dim = 64,
                  float rope_theta = 1000000.0f, hipStream_t stream = nullptr);

// Fused replacement of src/layer_attn.cpp:91-96 (attn_head_norm on q and k, then
// rope_forward on q and k) over `rows` tokens; row t is at position pos[t]
// (device int32 array) or pos0 + t when pos is null.
void attn_qk_norm_rope_rows(float* q, float* k, const float* q_weight, const float* k_weight,
                            const int32_t* pos, int pos0, int rows, int q_heads, int k_heads, int head_dim,
                            int partial_rope_dim, float rope_theta, float eps, hipStream_t stream = nullptr);

}  // namespace qwen

#endif  // QWEN35_ROPE_HPP
