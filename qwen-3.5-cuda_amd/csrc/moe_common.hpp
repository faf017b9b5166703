// MoE top-k of one logit row by one wave, shared by the routing kernel
// (moe_route.hip) and the fused routing + SwiGLU GEMV (gemv.hip), so both
// produce the same ids and weights.
//
// Reference semantics (src/cuda/moe.cu:7-51): any non-finite logit makes the
// row invalid; else k rounds of "largest unused logit, strictly greater wins"
// (ties to the lower index), then w = softmax over the k picks. Lane L holds
// the VPL consecutive logits VPL*L .. VPL*L+VPL-1 and sorts them once, larger
// value first and lower index first among equal values. Each round is one wave
// max over the lanes' heads; among lanes whose head equals it the lowest lane
// wins (a ballot), which is the lowest index because lanes own increasing
// index ranges; the winner lane shifts its list. The softmax over the picks
// runs in the first k lanes.
#ifndef QWEN35_MOE_COMMON_HPP
#define QWEN35_MOE_COMMON_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "device_common.hpp"

namespace qk {

// Wave max with DPP inside 16-lane rows, permlane swaps across rows.
__device__ __forceinline__ float wave_maxf(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// (v, i) before (w, j): larger value, then lower index (a total order on a
// row's finite logits, so the sorted order is unique).
__device__ __forceinline__ bool topk_ahead(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

// Top-k of the n logits at xr (n <= 64 VPL, k <= min(n, 64)), called by all 64
// lanes of a wave. Returns false if any logit is non-finite (nothing picked);
// else lane j < k gets pick j's index and softmax weight.
template <int VPL>
__device__ __forceinline__ bool topk_row(const float* __restrict__ xr, int n, int k, int& pick_i, float& weight) {
    const int lane = threadIdx.x & 63;
    const int i0 = VPL * lane;
    float v[VPL];
    int vi[VPL];
    if (VPL % 4 == 0 && n == VPL * kWave && (reinterpret_cast<uintptr_t>(xr) & 15) == 0) {
#pragma unroll
        for (int s = 0; s < VPL; s += 4) {
            const float4 q = ld4(xr + i0 + s);
            v[s] = q.x;
            v[s + 1] = q.y;
            v[s + 2] = q.z;
            v[s + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < VPL; ++s) v[s] = i0 + s < n ? xr[i0 + s] : -INFINITY;
    }
    bool finite = true;
#pragma unroll
    for (int s = 0; s < VPL; ++s) {
        vi[s] = i0 + s;
        if (i0 + s < n && !isfinite(v[s])) finite = false;
    }
    if (__any(!finite)) return false;
    // Odd-even transposition sort of the lane's list. Padding (-inf, index >= n)
    // sorts last and is never picked: k <= n and every logit is finite.
#pragma unroll
    for (int r = 0; r < VPL; ++r) {
#pragma unroll
        for (int s = r & 1; s + 1 < VPL; s += 2) {
            if (topk_ahead(v[s + 1], vi[s + 1], v[s], vi[s])) {
                const float tv = v[s];
                const int ti = vi[s];
                v[s] = v[s + 1];
                vi[s] = vi[s + 1];
                v[s + 1] = tv;
                vi[s + 1] = ti;
            }
        }
    }
    float pick_v = 0.f;     // lane j < k: value of pick j
    pick_i = -1;
    for (int j = 0; j < k; ++j) {
        const float m = wave_maxf(v[0]);
        const uint64_t tied = __ballot(v[0] == m);
        const int wl = __builtin_ctzll(tied);            // lowest lane holding the max
        const int wi = __builtin_amdgcn_readlane(vi[0], wl);
        if (lane == wl) {
#pragma unroll
            for (int s = 0; s + 1 < VPL; ++s) {
                v[s] = v[s + 1];
                vi[s] = vi[s + 1];
            }
            v[VPL - 1] = -INFINITY;
            vi[VPL - 1] = 0x7fffffff;
        }
        if (lane == j) {
            pick_v = m;
            pick_i = wi;
        }
    }
    // softmax over the picks (lanes < k); the first pick is the largest
    const float mx = __shfl(pick_v, 0);
    const float e = lane < k ? expf(pick_v - mx) : 0.0f;
    const float sum = group_sum<64>(e);
    weight = e / sum;
    return true;
}

}  // namespace qk

#endif  // QWEN35_MOE_COMMON_HPP
