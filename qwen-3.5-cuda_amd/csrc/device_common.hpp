// Device-side building blocks shared by every kernel: wave64 reductions over
// DPP, bf16 packing, and the SiLU / sigmoid forms the reference uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qk {

constexpr int kWave = 64;

// Index of the calling wave inside its workgroup, as a wave-uniform (scalar)
// value: the compiler cannot prove threadIdx.x / 64 uniform by itself, and
// without this the row / head arithmetic and the per-wave loads that depend on
// it are done per lane (vector ALU, vector loads) instead of once per wave.
__device__ __forceinline__ int wave_in_block() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------- reductions
// DPP row-local move (gfx9 encodings): quad_perm, row_half_mirror, row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G a power of two, 1..64). Every lane of a
// group ends with the same bits: each step adds a lane and its partner, and both
// partners evaluate the same sum with the same operand order (or a commutative
// pair). Everything stays in the VALU: DPP within 16-lane rows, then gfx950's
// v_permlane16_swap / v_permlane32_swap, which with both operands = v return
// (even row, odd row) and (lower half, upper half) values in every lane.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group");
    if constexpr (G >= 2) v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (G >= 4) v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (G >= 8) v += dpp_move<0x141>(v);  // row_half_mirror: 8-lane halves
    if constexpr (G >= 16) v += dpp_move<0x140>(v); // row_mirror: 16-lane rows
    if constexpr (G >= 32) {                        // rows (0,1) and (2,3)
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if constexpr (G >= 64) {                        // halves (0..31) and (32..63)
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}

// Value of `v` held by lane `src` (any lane of the wave).
__device__ __forceinline__ float lane_fetch(float v, int src) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

// ---------------------------------------------------------------- activations
// SiLU, x / (1 + expf(-x)) in the reference (src/cuda/ops.cu:9-11).
//
// Fast form: x * rcp(1 + 2^(-x log2 e)) on the transcendental unit
// (v_exp_f32, v_rcp_f32; 2 quarter-rate + 3 full-rate ops instead of ~40 for
// the accurate expf and the IEEE divide). Relative error against the exact
// SiLU: rounding -x*log2(e) perturbs the exponent by |x| * 2^-24 (relative
// error |x| * 2^-24 in e^-x), plus ~1 ulp each for v_exp_f32, the add,
// v_rcp_f32 and the final multiply: at most ~2.8e-6 for x >= -40.
// Below -40, 1 + e^-x approaches the range where v_rcp_f32's result would be
// a flushed denormal, so those inputs take the reference formula.
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kSiluFastMin = -40.0f;

__device__ __forceinline__ float silu_exact(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float silu_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * kLog2e);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// SiLU of N register values: the fast form, then the exact form for any value
// below kSiluFastMin (a branch that activations of normal magnitude never take).
// NaN stays NaN (fminf ignores it; the fast form propagates it).
template <int N>
__device__ __forceinline__ void silu_n(float (&v)[N]) {
    float lo = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) lo = fminf(lo, v[i]);
    float r[N];
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = silu_fast(v[i]);
    if (lo < kSiluFastMin) {
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (v[i] < kSiluFastMin) r[i] = silu_exact(v[i]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = r[i];
}

__device__ __forceinline__ float silu(float x) {
    float v[1] = {x};
    silu_n<1>(v);
    return v[0];
}

__device__ __forceinline__ float4 silu4(float4 x) {
    float v[4] = {x.x, x.y, x.z, x.w};
    silu_n<4>(v);
    return make_float4(v[0], v[1], v[2], v[3]);
}

// Sigmoid, 1 / (1 + expf(-x)) in the reference (src/cuda/moe.cu:94): the same
// fast form and guard as silu (rcp(1 + 2^(-x log2 e)); the reference formula
// below kSiluFastMin, where the reciprocal would approach the denormal range).
__device__ __forceinline__ float sigmoid(float x) {
    float r = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
    if (x < kSiluFastMin) r = 1.0f / (1.0f + expf(-x));
    return r;
}

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (lo in bits 0..15), round to nearest even
// (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    float2_t f = {lo, hi};
    bf16x2_t b = __builtin_convertvector(f, bf16x2_t);
    return __builtin_bit_cast(uint32_t, b);
}

// ---------------------------------------------------------------- memory
// Tile of workgroup b in a grid of exactly `tiles` workgroups. Workgroups are
// dealt to the 8 XCDs round robin (b % 8), so tiles 2 l and 2 l + 1 (two
// halves of a 128-byte line segment) go to workgroups b and b + 8 of a group
// of 16, on one XCD, whose L2 then fetches the line once; the last tiles % 16
// keep their own index. A bijection on [0, tiles).
__device__ __forceinline__ int tile_of_block(int b, int tiles) {
    if (b >= (tiles & ~15)) return b;
    const int idx = b >> 3;
    return (((idx >> 1) << 3) + (b & 7)) * 2 + (idx & 1);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

// Streaming (nontemporal) 16-byte accesses for data touched exactly once per
// call: the loads and stores carry the nontemporal hint, so the lines are not
// kept in L2 / MALL at the expense of reused data (weights). On gfx950 this
// lifts a plain copy from ~5.5 to ~6.1 TB/s at 256 MB and up.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4_nt(const float* p) {
    const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st4_nt(float* p, float4 v) {
    const f32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4_t*>(p));
}
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
    const u32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t*>(p));
}

__device__ __forceinline__ float sumsq4(float4 v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }

}  // namespace qk
