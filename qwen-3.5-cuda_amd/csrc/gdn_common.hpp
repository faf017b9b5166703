// Gated DeltaNet pieces shared by the front-end kernels (gdn.hip) and the
// fused decode step (gdn_state.hip), so both evaluate the same expressions, and
// the limit the recurrent entry points share (gdn_state.hip, gdn_chunk.hip).
#ifndef QWEN35_GDN_COMMON_HPP
#define QWEN35_GDN_COMMON_HPP

#include <hip/hip_runtime.h>

#include <cmath>

namespace qk {

// Largest value-head dimension the recurrence accepts; every recurrent entry
// point rejects more with the reference's message (src/cuda/gdn.cu:167-169).
constexpr int kMaxValueDim = 256;

// Exactly-rounded 1/sqrt(n) for the q scale, so the device multiplies by the
// same constant as the host oracle (src/cuda/gdn.cu:76).
inline float host_rsqrt(int n) { return static_cast<float>(1.0 / std::sqrt(static_cast<double>(n))); }

__device__ __forceinline__ float conv4(float h0, float h1, float h2, float xv, float4 w) {
    // sum = 0; sum += h0*w0; sum += h1*w1; sum += h2*w2; sum += x*w3, each a
    // fused multiply-add as nvcc contracts it (src/cuda/gdn.cu:13-17).
    float s = __builtin_fmaf(h0, w.x, 0.0f);
    s = __builtin_fmaf(h1, w.y, s);
    s = __builtin_fmaf(h2, w.z, s);
    return __builtin_fmaf(xv, w.w, s);
}

// History of 4 consecutive channels, [c][3] floats each (12 floats from
// hist), as the three previous inputs h0 = x[t-3], h1 = x[t-2], h2 = x[t-1].
__device__ __forceinline__ void history4(const float4 a, const float4 b, const float4 d, float4& h0, float4& h1,
                                         float4& h2) {
    // [ch0: j0 j1 j2 | ch1: j0 j1 j2 | ch2 ... | ch3 ...]
    h0 = make_float4(a.x, a.w, b.z, d.y);
    h1 = make_float4(a.y, b.x, b.w, d.z);
    h2 = make_float4(a.z, b.y, d.x, d.w);
}

}  // namespace qk

#endif  // QWEN35_GDN_COMMON_HPP
