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
// runs in the first k lanes. The comparisons run on integer keys that order
// like the (finite) logits, so the wave max is v_max_i32 with its DPP operand
// folded in, not fmaxf with NaN canonicalisation around every step.
#ifndef QWEN35_MOE_COMMON_HPP
#define QWEN35_MOE_COMMON_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "device_common.hpp"

namespace qk {

// Integer key of a finite logit with the same order as the reference's
// float comparison: x + 0 turns -0 into +0 (the two compare equal), then the
// sign-magnitude bits become two's-complement order. topk_value inverts it.
__device__ __forceinline__ int topk_key(float x) {
    const int b = __float_as_int(x + 0.0f);
    return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float topk_value(int key) { return __int_as_float(key ^ ((key >> 31) & 0x7fffffff)); }

// A candidate as one signed 64-bit entry: key in the high half, the bitwise
// complement of its index in the low half, so entry a > entry b exactly when a
// comes first (larger value, then lower index): one v_cmp_gt_i64 per
// comparison. The padding entry (-inf, index 2^31 - 1) sorts after every logit.
typedef long long topk_entry;
__device__ __forceinline__ topk_entry topk_make(int key, int index) {
    return static_cast<topk_entry>((static_cast<uint64_t>(static_cast<uint32_t>(key)) << 32) |
                                   static_cast<uint32_t>(~index));
}
__device__ __forceinline__ int topk_entry_key(topk_entry e) { return static_cast<int>(e >> 32); }
__device__ __forceinline__ int topk_entry_low(topk_entry e) { return static_cast<int>(static_cast<uint32_t>(e)); }
__device__ __forceinline__ int topk_low_index(int low) { return static_cast<int>(~static_cast<uint32_t>(low)); }

template <int CTRL>
__device__ __forceinline__ int dpp_move_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Max of integer keys over aligned groups of G lanes (16, 32 or 64): DPP
// within 16-lane rows (v_max_i32 takes the DPP operand directly), permlane
// swaps across rows.
template <int G>
__device__ __forceinline__ int group_max_key(int v) {
    static_assert(G == 16 || G == 32 || G == 64, "group");
    v = max(v, dpp_move_i<0xB1>(v));
    v = max(v, dpp_move_i<0x4E>(v));
    v = max(v, dpp_move_i<0x141>(v));
    v = max(v, dpp_move_i<0x140>(v));
    if constexpr (G >= 32) {
        const auto p = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false,
                                                        false);
        v = max(static_cast<int>(p[0]), static_cast<int>(p[1]));
    }
    if constexpr (G == 64) {
        const auto p = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false,
                                                        false);
        v = max(static_cast<int>(p[0]), static_cast<int>(p[1]));
    }
    return v;
}

// Sort a lane's VPL entries (VPL a power of two), first entry first:
// Batcher's odd-even merge network (1, 5, 19 and 63 compare-exchanges for 2,
// 4, 8 and 16 entries), unrolled at compile time.
__device__ __forceinline__ void topk_ce(topk_entry& a, topk_entry& b) {
    const bool swap = b > a;
    const topk_entry t = a;
    a = swap ? b : a;
    b = swap ? t : b;
}

template <int VPL>
__device__ __forceinline__ void topk_sort(topk_entry (&e)[VPL]) {
    static_assert((VPL & (VPL - 1)) == 0, "power of two");
#pragma unroll
    for (int p = 1; p < VPL; p <<= 1) {
#pragma unroll
        for (int k = p; k >= 1; k >>= 1) {
#pragma unroll
            for (int j = k % p; j + k < VPL; j += 2 * k) {
#pragma unroll
                for (int i = 0; i < k && i + j + k < VPL; ++i) {
                    if ((i + j) / (2 * p) == (i + j + k) / (2 * p)) topk_ce(e[i + j], e[i + j + k]);
                }
            }
        }
    }
}

// Loads the VPL logits of lane slot `hl` (VPL hl .. VPL hl + VPL - 1, -inf
// past n) as sorted entries; false if any of them is non-finite. VEC: every
// slot lies inside the row (n = lanes x VPL) and the row is 16-byte aligned,
// so the loads are unconditional 16-byte loads.
template <int VPL, bool VEC = false>
__device__ __forceinline__ bool topk_load(const float* __restrict__ xr, int n, int hl, topk_entry (&e)[VPL]) {
    const int i0 = VPL * hl;
    float v[VPL];
    if constexpr (VEC) {
        static_assert(VPL % 4 == 0, "16-byte loads");
#pragma unroll
        for (int s = 0; s < VPL; s += 4) {
            const float4 q = ld4(xr + i0 + s);
            v[s] = q.x;
            v[s + 1] = q.y;
            v[s + 2] = q.z;
            v[s + 3] = q.w;
        }
        // finite: no exponent field all ones
        uint32_t ex = 0;
#pragma unroll
        for (int s = 0; s < VPL; ++s) ex = max(ex, __float_as_uint(v[s]) & 0x7fffffffu);
#pragma unroll
        for (int s = 0; s < VPL; ++s) e[s] = topk_make(topk_key(v[s]), i0 + s);
        topk_sort<VPL>(e);
        return ex < 0x7f800000u;
    } else {
#pragma unroll
        for (int s = 0; s < VPL; ++s) v[s] = i0 + s < n ? xr[i0 + s] : -INFINITY;
        bool finite = true;
#pragma unroll
        for (int s = 0; s < VPL; ++s) {
            if (i0 + s < n && !isfinite(v[s])) finite = false;
            e[s] = i0 + s < n ? topk_make(topk_key(v[s]), i0 + s) : topk_make(topk_key(-INFINITY), 0x7fffffff);
        }
        topk_sort<VPL>(e);
        return finite;
    }
}

// One round over groups of G lanes (a row per group; G = 64: one row per
// wave): the group's largest head key; among the lanes holding it the lowest
// wins (a ballot: lanes own increasing index ranges, so this is the lowest
// index), shifts its list, and the pick goes to lane j of the group. The
// winners' lanes and indices are found once per group on the scalar unit.
template <int G, int VPL>
__device__ __forceinline__ int topk_round(topk_entry (&e)[VPL], int j, int& pick_k, int& pick_i) {
    constexpr int R = kWave / G;
    const int lane = threadIdx.x & 63;
    const int m = group_max_key<G>(topk_entry_key(e[0]));
    const uint64_t tied = __ballot(topk_entry_key(e[0]) == m);
    int wl = 0, wi = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint64_t grp = G == 64 ? tied : (tied >> (r * G)) & ((uint64_t{1} << (G & 63)) - 1);
        const int wlr = r * G + __builtin_ctzll(grp | (uint64_t{1} << (G - 1)));   // lowest tied lane
        const int wir = topk_low_index(__builtin_amdgcn_readlane(topk_entry_low(e[0]), wlr));
        if (r == 0 || lane / G == r) {
            wl = wlr;
            wi = wir;
        }
    }
    if (lane == wl) {
#pragma unroll
        for (int s = 0; s + 1 < VPL; ++s) e[s] = e[s + 1];
        e[VPL - 1] = topk_make(topk_key(-INFINITY), 0x7fffffff);
    }
    if ((lane & (G - 1)) == j) {
        pick_k = m;
        pick_i = wi;
    }
    return m;
}

// k rounds: unrolled when the count is known at compile time (KC > 0, the
// lists then need no register moves between rounds), else a loop. Returns the
// first round's key (the group's largest logit, its first pick).
template <int G, int VPL, int KC>
__device__ __forceinline__ int topk_rounds(topk_entry (&e)[VPL], int k, int& pick_k, int& pick_i) {
    const int m0 = topk_round<G, VPL>(e, 0, pick_k, pick_i);
    if constexpr (KC > 0) {
#pragma unroll
        for (int j = 1; j < KC; ++j) topk_round<G, VPL>(e, j, pick_k, pick_i);
    } else {
        for (int j = 1; j < k; ++j) topk_round<G, VPL>(e, j, pick_k, pick_i);
    }
    return m0;
}

// Softmax over a group's picks (lanes j < k of each group of G); m0: the key
// of the group's first (largest) pick.
template <int G>
__device__ __forceinline__ float topk_softmax(int pick_k, int m0, int k) {
    const int lane = threadIdx.x & 63;
    const float e = (lane & (G - 1)) < k ? expf(topk_value(pick_k) - topk_value(m0)) : 0.0f;
    return e / group_sum<G>(e);
}

// Top-k of the n logits at xr (n <= 64 VPL, k <= min(n, 64)), called by all 64
// lanes of a wave. Returns false if any logit is non-finite (nothing picked);
// else lane j < k gets pick j's index and softmax weight. KC: k when known at
// compile time (must then equal k), else 0.
template <int VPL, int KC = 0>
__device__ __forceinline__ bool topk_row(const float* __restrict__ xr, int n, int k, int& pick_i, float& weight) {
    topk_entry e[VPL];
    const bool finite = topk_load<VPL>(xr, n, threadIdx.x & 63, e);
    if (__any(!finite)) return false;
    int pick_k = 0;
    pick_i = -1;
    const int m0 = topk_rounds<64, VPL, KC>(e, k, pick_k, pick_i);
    weight = topk_softmax<64>(pick_k, m0, k);
    return true;
}

// Top-k of R = 64 / G logit rows per wave, one per group of G lanes (xr: the
// calling lane's row; n <= G VPL, k <= min(n, G)), the same selection
// as topk_row; each round's max runs over all groups at once, so a round serves
// R rows. Lane G r + j < k gets pick j of row r. Bit r of the result: row r has
// only finite logits (else nothing of it is picked).
template <int G, int VPL, int KC = 0, bool VEC = false>
__device__ __forceinline__ uint32_t topk_rows_group(const float* __restrict__ xr, int n, int k, int& pick_i,
                                                    float& weight) {
    constexpr int R = kWave / G;
    const int lane = threadIdx.x & 63;
    topk_entry e[VPL];
    const bool finite = topk_load<VPL, VEC>(xr, n, lane & (G - 1), e);
    const uint64_t bad = __ballot(!finite);
    uint32_t ok = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint64_t grp = G == 64 ? bad : (bad >> (r * G)) & ((uint64_t{1} << (G & 63)) - 1);
        if (grp == 0) ok |= 1u << r;
    }
    int pick_k = 0;
    pick_i = -1;
    const int m0 = topk_rounds<G, VPL, KC>(e, k, pick_k, pick_i);
    weight = topk_softmax<G>(pick_k, m0, k);
    return ok;
}

}  // namespace qk

#endif  // QWEN35_MOE_COMMON_HPP
