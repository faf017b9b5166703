// RoPE pieces shared by the attention front end (attn.hip) and the decode
// attention that folds the front end in (attn_core.hip): the host-side table of
// inverse-frequency denominators and, for the production head shape (head_dim
// 256 held as one float4 per lane of a wave, rope_dim 64), the per-lane angles
// and the in-register norm + rotation of one head. One copy of the arithmetic,
// so both kernels give the same bits.
#ifndef QWEN35_ATTN_COMMON_HPP
#define QWEN35_ATTN_COMMON_HPP

#include <cmath>

#include "device_common.hpp"

namespace qk {
namespace {

constexpr int kMaxDen = 128;  // pairs per kernel-argument table

struct RopeDen {
    float den[kMaxDen];
};

// den[i - lo] = powf(theta, (2i)/rope_dim) for i in [lo, lo + count): the
// exponent is formed in float as the reference does (src/cuda/rope.cu:19).
inline RopeDen make_den(int lo, int count, int rope_dim, float theta) {
    RopeDen d{};
    for (int j = 0; j < count; ++j) {
        const float e = (2.0f * static_cast<float>(lo + j)) / static_cast<float>(rope_dim);
        d.den[j] = static_cast<float>(std::pow(static_cast<double>(theta), static_cast<double>(e)));
    }
    return d;
}

__device__ __forceinline__ float pl16_hi(float v) {  // lane m (even row) <- lane m + 16
    return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
}
__device__ __forceinline__ float pl32_hi(float v) {  // lane m (< 32) <- lane m + 32
    return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
}

// head_dim 256, rope_dim 64: the denominator lane L evaluates (pair
// 4 (L % 8) + L / 16 of lane 16 r + m), read before the angle math.
__device__ __forceinline__ float rope256_den(const RopeDen& den, int lane) {
    return den.den[4 * (lane & 7) + (lane >> 4)];
}

// cos / sin of the four pairs rotary lane m (m < 16) needs: lane 16 r + m
// evaluates the angle of pair 4 (m % 8) + r, and rotary lane m gathers its four
// from lanes m, m+16, m+32, m+48 (v_permlane16_swap / v_permlane32_swap).
struct Rope256 {
    float cs[4], sn[4];
};
__device__ __forceinline__ Rope256 rope256_angles(float fp, float dn0) {
    float s0, c0;
    sincosf(fp / dn0, &s0, &c0);
    const float c01 = pl16_hi(c0), s01 = pl16_hi(s0);
    return Rope256{{c0, c01, pl32_hi(c0), pl32_hi(c01)}, {s0, s01, pl32_hi(s0), pl32_hi(s01)}};
}

// One head (float4 `lane` of it in x): RMSNorm x * (r * w) (src/cuda/attn_kernels.cu:
// 34-63) when NORM, then the split-half rotation of dims 0..63 (src/cuda/rope.cu:9-29):
// lanes 0..7 hold dims 0..31, their partners (dims 32..63) sit 8 lanes away in
// the same 16-lane row (DPP row_ror:8).
template <bool NORM>
__device__ __forceinline__ float4 norm_rope256(float4 x, float4 wv, const Rope256& rp, float eps, int lane) {
    if constexpr (NORM) {
        const float ss = group_sum<kWave>(sumsq4(x));
        const float r = rsqrtf(ss / 256.0f + eps);
        x.x = x.x * (r * wv.x);
        x.y = x.y * (r * wv.y);
        x.z = x.z * (r * wv.z);
        x.w = x.w * (r * wv.w);
    }
    const float pv[4] = {dpp_move<0x128>(x.x), dpp_move<0x128>(x.y), dpp_move<0x128>(x.z), dpp_move<0x128>(x.w)};
    const float a[4] = {x.x, x.y, x.z, x.w};
    const bool first = lane < 8, second = lane >= 8 && lane < 16;
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (first)
            o[i] = a[i] * rp.cs[i] - pv[i] * rp.sn[i];  // x[i]      = a c - b s
        else if (second)
            o[i] = a[i] * rp.cs[i] + pv[i] * rp.sn[i];  // x[i+half] = b c + a s
        else
            o[i] = a[i];
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

}  // namespace
}  // namespace qk

#endif  // QWEN35_ATTN_COMMON_HPP
