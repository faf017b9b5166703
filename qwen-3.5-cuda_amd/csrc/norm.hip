// RMSNorm family on gfx950: plain / gated RMSNorm rows, fused residual add +
// RMSNorm (fp32 and bf16 storage), residual add and the fp32 embedding copy.
//
// Reference semantics: src/cuda/ops.cu:25-138 (rmsnorm_kernel,
// rmsnorm_gated_kernel, residual_add_kernel, encoder_kernel). The reference
// launches one 256-thread block per call and re-reads x for the second pass;
// here one wave64 owns a row (two waves when there are few rows), holds the row
// in VGPRs between the reduction and the scale (x is read from HBM once),
// reduces with DPP row ops and permlane swaps, and moves data in 16-byte
// vectors.
#include <algorithm>
#include <type_traits>

#include "capi_common.hpp"
#include "device_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;

// Launch shape. Few rows: one wave (one row) per workgroup, so rows land on
// different CUs, each wave loading its own weights. Many rows: kStageWaves rows
// per workgroup sharing one copy of the weight row in LDS, loaded once per
// workgroup instead of once per wave (the per-wave reload is as many L2 bytes
// as half a bf16 row's HBM traffic).
constexpr int kStageWaves = 8;
inline bool stage_weights(int rows) { return rows >= 1024; }

// Cooperative copy of n4 float4 weights into LDS, then a barrier. Every wave of
// the workgroup must call it (no early return before).
__device__ __forceinline__ void stage_rows_weights(float4* wl, const float* __restrict__ w, int n4) {
    for (int i = threadIdx.x; i < n4; i += blockDim.x) wl[i] = ld4(w + 4 * i);
    __syncthreads();
}

// ss / n, the mean of the squares (src/cuda/ops.cu:56 divides). For n a power of
// two the quotient equals ss * 2^-log2(n) bit for bit (division and
// multiplication both round the same real number), one multiply instead of the
// IEEE division sequence on the row's critical path.
__device__ __forceinline__ float div_n(float ss, int n) {
    if ((n & (n - 1)) == 0) return ss * __int_as_float((127 - __builtin_ctz(static_cast<unsigned>(n))) << 23);
    return ss / static_cast<float>(n);
}

// Sum-of-squares order shared by every vector row form, so that a row gives the
// same bits whether it is normalised alone or among many rows (the launch shape
// depends on the row count): with the row in 16-byte chunks c = 0, 1, ... and
// chunk c on lane c % 64, lane l adds its chunks in two sets, c / 64 even and
// c / 64 odd, each in order; each set is summed over the 64 lanes by
// group_sum<64>, and the odd set's total is added to the even set's. The
// two-wave form (rmsnorm_rows_split) holds one set per wave.
__device__ __forceinline__ float row_sumsq(float even, float odd) {
    return group_sum<kWave>(even) + group_sum<kWave>(odd);
}

// ------------------------------------------------------------- fp32 rows
// One wave per row; lane l holds float4 chunks l, l+64, ... (up to MAXC).
// Lanes past the row end load a clamped in-row address and use zeros, so every
// load is issued unconditionally; the weights are loaded with the row (or, when
// staged, read from LDS after it), ahead of the reduction, so the second pass
// waits on nothing. Waves past the last row clamp to it and leave after the
// staging barrier.
template <int MAXC, bool GATED, bool STAGE>
__global__ __launch_bounds__(STAGE ? kStageWaves * kWave : kWave) void rmsnorm_rows_v4(
    const float* __restrict__ x, const float* __restrict__ gate, const float* __restrict__ w, float* __restrict__ out,
    int rows, int n, float eps) {
    extern __shared__ float4 wl[];
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + wave_in_block();
    const bool live = row < rows;  // wave-uniform
    const int n4 = n >> 2;
    const size_t base = static_cast<size_t>(live ? row : rows - 1) * n;
    float4 v[MAXC], wv[MAXC];
    float4 g[GATED ? MAXC : 1];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int ic = min(c * kWave + lane, n4 - 1);
        v[c] = ld4_nt(x + base + 4 * ic);
        if constexpr (!STAGE) wv[c] = ld4(w + 4 * ic);
        if constexpr (GATED) g[c] = ld4_nt(gate + base + 4 * ic);
    }
    if constexpr (STAGE) {
        stage_rows_weights(wl, w, n4);
#pragma unroll
        for (int c = 0; c < MAXC; ++c) wv[c] = wl[min(c * kWave + lane, n4 - 1)];
    }
    if (!live) return;
    // Chunks past the row end (clamped loads) are left out of the sum by a
    // select once every load is issued: overwriting a load's destination
    // registers in the load loop would make each load wait for the previous one.
    float se = 0.f, so = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const float q = c * kWave + lane < n4 ? sumsq4(v[c]) : 0.f;
        if (c % 2 == 0)
            se += q;
        else
            so += q;
    }
    const float r = rsqrtf(div_n(row_sumsq(se, so), n) + eps);
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = c * kWave + lane;
        float4 o;
        o.x = v[c].x * r * wv[c].x;
        o.y = v[c].y * r * wv[c].y;
        o.z = v[c].z * r * wv[c].z;
        o.w = v[c].w * r * wv[c].w;
        if constexpr (GATED) {
            const float4 sg = silu4(g[c]);
            o.x *= sg.x;
            o.y *= sg.y;
            o.z *= sg.z;
            o.w *= sg.w;
        }
        if (i < n4) st4_nt(out + base + 4 * i, o);
    }
}

// Few rows (fewer than kSplitRows, e.g. the 36 rows of one prompt's final
// norm): kSplitWaves waves share a row, wave v holding the 64-float4 chunks
// v, v + kSplitWaves, ...; the two wave sums meet in LDS and are added in wave
// order. Twice the waves in flight for the same bytes: at 36 x 2048 it measured
// 2.16 us against 2.50 us with one wave per row (a plain copy of the same bytes
// takes 1.87 us).
constexpr int kSplitWaves = 2;   // the two chunk sets of row_sumsq
constexpr int kSplitRows = 256;

// FULL: n4 == MAXC * kSplitWaves * 64 (every chunk inside the row: no clamps or
// masks, so the loads take immediate offsets and the sum needs no selects).
template <int MAXC, bool GATED, bool FULL>
__global__ __launch_bounds__(kSplitWaves * kWave) void rmsnorm_rows_split(
    const float* __restrict__ x, const float* __restrict__ gate, const float* __restrict__ w, float* __restrict__ out,
    int n, float eps) {
    __shared__ float part[kSplitWaves];
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int n4 = n >> 2;
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    auto chunk = [&](int c) { return (c * kSplitWaves + wv) * kWave + lane; };
    auto at = [&](int c) { return FULL ? chunk(c) : min(chunk(c), n4 - 1); };  // clamped: loads never branch
    float4 v[MAXC], wt[MAXC];
    float4 g[GATED ? MAXC : 1];
    // the row (from HBM) first, then the gate and the weights (shared by every
    // row, so mostly cache hits): the row's round trip starts earliest
#pragma unroll
    for (int c = 0; c < MAXC; ++c) v[c] = ld4_nt(x + base + 4 * at(c));
    if constexpr (GATED) {
#pragma unroll
        for (int c = 0; c < MAXC; ++c) g[c] = ld4_nt(gate + base + 4 * at(c));
    }
#pragma unroll
    for (int c = 0; c < MAXC; ++c) wt[c] = ld4(w + 4 * at(c));
    float ss = 0.f;  // chunks past the row end left out by a select (see rmsnorm_rows_v4)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) ss += (FULL || chunk(c) < n4) ? sumsq4(v[c]) : 0.f;
    ss = group_sum<kWave>(ss);
    if (lane == 0) part[wv] = ss;
    __syncthreads();
    ss = part[0] + part[1];   // the set order of row_sumsq: wave 0 holds the even chunk set
    const float r = rsqrtf(div_n(ss, n) + eps);
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        float4 o;
        o.x = v[c].x * r * wt[c].x;
        o.y = v[c].y * r * wt[c].y;
        o.z = v[c].z * r * wt[c].z;
        o.w = v[c].w * r * wt[c].w;
        if constexpr (GATED) {
            const float4 sg = silu4(g[c]);
            o.x *= sg.x;
            o.y *= sg.y;
            o.z *= sg.z;
            o.w *= sg.w;
        }
        if (FULL || chunk(c) < n4) st4_nt(out + base + 4 * chunk(c), o);
    }
}

// Cross-wave sum for a block of kBlock threads: wave sums meet in LDS.
__device__ __forceinline__ float block_sum(float v, float* lds) {
    v = group_sum<kWave>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kBlock / kWave; ++i) t += lds[i];
    return t;
}

// Any n, any alignment: one block per row, two passes (the second pass re-reads
// x, which the first pass left in cache).
template <bool GATED>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_any(const float* __restrict__ x, const float* __restrict__ gate,
                                                           const float* __restrict__ w, float* __restrict__ out, int n,
                                                           float eps) {
    __shared__ float lds[kBlock / kWave];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) ss += x[base + i] * x[base + i];
    ss = block_sum(ss, lds);
    const float r = rsqrtf(div_n(ss, n) + eps);
    for (int i = threadIdx.x; i < n; i += kBlock) {
        float o = x[base + i] * r * w[i];
        if constexpr (GATED) o *= silu(gate[base + i]);
        out[base + i] = o;
    }
}

// ------------------------------------------------- fused residual + RMSNorm, fp32
template <int MAXC, bool STAGE>
__global__ __launch_bounds__(STAGE ? kStageWaves * kWave : kWave) void residual_rmsnorm_f32_v4(
    const float* __restrict__ x, const float* __restrict__ b, const float* __restrict__ w, float* __restrict__ resid,
    float* __restrict__ normed, int rows, int n, float eps) {
    extern __shared__ float4 wl[];
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + wave_in_block();
    const bool live = row < rows;  // wave-uniform
    const int n4 = n >> 2;
    const size_t base = static_cast<size_t>(live ? row : rows - 1) * n;
    float4 v[MAXC], wv[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int ic = min(c * kWave + lane, n4 - 1);
        const float4 a = ld4_nt(x + base + 4 * ic);
        const float4 d = ld4_nt(b + base + 4 * ic);
        if constexpr (!STAGE) wv[c] = ld4(w + 4 * ic);
        v[c] = make_float4(a.x + d.x, a.y + d.y, a.z + d.z, a.w + d.w);
    }
    if constexpr (STAGE) {
        stage_rows_weights(wl, w, n4);
#pragma unroll
        for (int c = 0; c < MAXC; ++c) wv[c] = wl[min(c * kWave + lane, n4 - 1)];
    }
    if (!live) return;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = c * kWave + lane;
        if (i < n4) {
            st4_nt(resid + base + 4 * i, v[c]);
            ss += sumsq4(v[c]);
        }
    }
    ss = group_sum<kWave>(ss);
    const float r = rsqrtf(div_n(ss, n) + eps);
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = c * kWave + lane;
        if (i < n4)
            st4_nt(normed + base + 4 * i, make_float4(v[c].x * r * wv[c].x, v[c].y * r * wv[c].y,
                                                      v[c].z * r * wv[c].z, v[c].w * r * wv[c].w));
    }
}

__global__ __launch_bounds__(kBlock) void residual_rmsnorm_f32_any(const float* __restrict__ x,
                                                                   const float* __restrict__ b,
                                                                   const float* __restrict__ w,
                                                                   float* __restrict__ resid,
                                                                   float* __restrict__ normed, int n, float eps) {
    __shared__ float lds[kBlock / kWave];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) {
        const float s = x[base + i] + b[base + i];
        resid[base + i] = s;
        ss += s * s;
    }
    ss = block_sum(ss, lds);
    const float r = rsqrtf(div_n(ss, n) + eps);
    // Each thread re-reads only the elements it wrote itself.
    for (int i = threadIdx.x; i < n; i += kBlock) normed[base + i] = resid[base + i] * r * w[i];
}

// ------------------------------------------------- fused residual + RMSNorm, bf16
// 8 bf16 per 16-byte chunk; lane l holds chunks l, l+64, ... The rounded sum is
// what the norm reads, so the result equals the unfused pair on bf16 buffers.
template <int MAXC, bool STAGE>
__global__ __launch_bounds__(STAGE ? kStageWaves * kWave : kWave) void residual_rmsnorm_bf16_v8(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ b, const float* __restrict__ w,
    uint16_t* __restrict__ resid, uint16_t* __restrict__ normed, int rows, int n, float eps) {
    extern __shared__ float4 wl[];
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + wave_in_block();
    const bool live = row < rows;  // wave-uniform
    const int n8 = n >> 3;
    const size_t base = static_cast<size_t>(live ? row : rows - 1) * n;
    uint4 xa[MAXC], ba[MAXC];
    float4 w0[MAXC], w1[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int ic = min(c * kWave + lane, n8 - 1);
        xa[c] = ld16_nt(x + base + 8 * ic);
        ba[c] = ld16_nt(b + base + 8 * ic);
        if constexpr (!STAGE) {
            w0[c] = ld4(w + 8 * ic);
            w1[c] = ld4(w + 8 * ic + 4);
        }
    }
    if constexpr (STAGE) {
        stage_rows_weights(wl, w, 2 * n8);
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            const int ic = min(c * kWave + lane, n8 - 1);
            w0[c] = wl[2 * ic];
            w1[c] = wl[2 * ic + 1];
        }
    }
    if (!live) return;
    uint4 s[MAXC];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const uint32_t xs[4] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w};
        const uint32_t bs[4] = {ba[c].x, ba[c].y, ba[c].z, ba[c].w};
        uint32_t ps[4];
        float part = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ps[k] = pack_bf16(bf16_lo(xs[k]) + bf16_lo(bs[k]), bf16_hi(xs[k]) + bf16_hi(bs[k]));
            const float lo = bf16_lo(ps[k]);
            const float hi = bf16_hi(ps[k]);
            part += lo * lo + hi * hi;
        }
        s[c] = make_uint4(ps[0], ps[1], ps[2], ps[3]);
        const int i = c * kWave + lane;
        if (i < n8) {
            st16_nt(resid + base + 8 * i, s[c]);
            ss += part;
        }
    }
    ss = group_sum<kWave>(ss);
    const float r = rsqrtf(div_n(ss, n) + eps);
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = c * kWave + lane;
        if (i < n8) {
            const uint4 o = make_uint4(pack_bf16(bf16_lo(s[c].x) * r * w0[c].x, bf16_hi(s[c].x) * r * w0[c].y),
                                       pack_bf16(bf16_lo(s[c].y) * r * w0[c].z, bf16_hi(s[c].y) * r * w0[c].w),
                                       pack_bf16(bf16_lo(s[c].z) * r * w1[c].x, bf16_hi(s[c].z) * r * w1[c].y),
                                       pack_bf16(bf16_lo(s[c].w) * r * w1[c].z, bf16_hi(s[c].w) * r * w1[c].w));
            st16_nt(normed + base + 8 * i, o);
        }
    }
}

__device__ __forceinline__ uint16_t to_bf16(float f) { return static_cast<uint16_t>(pack_bf16(f, 0.f) & 0xffffu); }
__device__ __forceinline__ float from_bf16(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

__global__ __launch_bounds__(kBlock) void residual_rmsnorm_bf16_any(const uint16_t* __restrict__ x,
                                                                    const uint16_t* __restrict__ b,
                                                                    const float* __restrict__ w,
                                                                    uint16_t* __restrict__ resid,
                                                                    uint16_t* __restrict__ normed, int n, float eps) {
    __shared__ float lds[kBlock / kWave];
    const size_t base = static_cast<size_t>(blockIdx.x) * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) {
        const uint16_t s = to_bf16(from_bf16(x[base + i]) + from_bf16(b[base + i]));
        resid[base + i] = s;
        const float f = from_bf16(s);
        ss += f * f;
    }
    ss = block_sum(ss, lds);
    const float r = rsqrtf(div_n(ss, n) + eps);
    for (int i = threadIdx.x; i < n; i += kBlock) normed[base + i] = to_bf16(from_bf16(resid[base + i]) * r * w[i]);
}

// ------------------------------------------------------------- elementwise
__global__ __launch_bounds__(kBlock) void add_v4(const float* __restrict__ a, const float* __restrict__ b,
                                                 float* __restrict__ out, int64_t n4) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n4;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        const float4 p = ld4(a + 4 * i);
        const float4 q = ld4(b + 4 * i);
        st4(out + 4 * i, make_float4(p.x + q.x, p.y + q.y, p.z + q.z, p.w + q.w));
    }
}

__global__ __launch_bounds__(kBlock) void add_any(const float* __restrict__ a, const float* __restrict__ b,
                                                  float* __restrict__ out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(kBlock) void copy_row(const float* __restrict__ src, float* __restrict__ dst, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        dst[i] = src[i];
}

// ------------------------------------------------------------- launchers
// Calls launch(stage, grid, block, lds_bytes) with the row-kernel launch shape
// for `rows`; stage is std::true_type / std::false_type (the kernel's STAGE).
template <typename L>
void launch_row_shape(int rows, size_t weight_bytes, L&& launch) {
    if (stage_weights(rows))
        launch(std::true_type{}, dim3(blocks_for(rows, kStageWaves)), dim3(kStageWaves * kWave), weight_bytes);
    else
        launch(std::false_type{}, dim3(rows), dim3(kWave), size_t{0});
}

template <bool GATED>
int launch_rmsnorm(const float* x, const float* gate, const float* w, float* out, int rows, int n, float eps,
                   hipStream_t s) {
    const int n4 = n / 4;
    const bool vec = (n % 4 == 0) && aligned16(x) && aligned16(w) && aligned16(out) && (!GATED || aligned16(gate));
    constexpr int kSplit = kSplitWaves * kWave;
    if (vec && rows < kSplitRows && n4 <= 8 * kSplit) {
        const dim3 grid(rows), block(kSplit);
        const auto go = [&](auto maxc) {
            constexpr int M = decltype(maxc)::value;
            if (n4 == M * kSplit)
                rmsnorm_rows_split<M, GATED, true><<<grid, block, 0, s>>>(x, gate, w, out, n, eps);
            else
                rmsnorm_rows_split<M, GATED, false><<<grid, block, 0, s>>>(x, gate, w, out, n, eps);
        };
        if (n4 <= kSplit)
            go(std::integral_constant<int, 1>{});
        else if (n4 <= 2 * kSplit)
            go(std::integral_constant<int, 2>{});
        else if (n4 <= 4 * kSplit)
            go(std::integral_constant<int, 4>{});
        else
            go(std::integral_constant<int, 8>{});
    } else if (vec && n4 <= 16 * kWave) {
        launch_row_shape(rows, size_t(n4) * 16, [&](auto stage, dim3 grid, dim3 block, size_t lds) {
            constexpr bool S = decltype(stage)::value;
            if (n4 <= kWave)
                rmsnorm_rows_v4<1, GATED, S><<<grid, block, lds, s>>>(x, gate, w, out, rows, n, eps);
            else if (n4 <= 2 * kWave)
                rmsnorm_rows_v4<2, GATED, S><<<grid, block, lds, s>>>(x, gate, w, out, rows, n, eps);
            else if (n4 <= 4 * kWave)
                rmsnorm_rows_v4<4, GATED, S><<<grid, block, lds, s>>>(x, gate, w, out, rows, n, eps);
            else if (n4 <= 8 * kWave)
                rmsnorm_rows_v4<8, GATED, S><<<grid, block, lds, s>>>(x, gate, w, out, rows, n, eps);
            else
                rmsnorm_rows_v4<16, GATED, S><<<grid, block, lds, s>>>(x, gate, w, out, rows, n, eps);
        });
    } else {
        rmsnorm_rows_any<GATED><<<rows, kBlock, 0, s>>>(x, gate, w, out, n, eps);
    }
    return check_launch(GATED ? "rmsnorm_gated" : "rmsnorm");
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_rmsnorm_rows(const float* x, const float* weight, float* out, int rows, int n, float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && n >= 0, "rmsnorm: negative size (rows=%d, n=%d)", rows, n);
    if (rows == 0 || n == 0) return ok();
    QK_REQUIRE(x && weight && out, "rmsnorm: null pointer");
    return launch_rmsnorm<false>(x, nullptr, weight, out, rows, n, eps, as_stream(stream));
}

int qwen_rmsnorm_forward(const float* x, const float* weight, float* out, int n, float eps, void* stream) {
    return qwen_rmsnorm_rows(x, weight, out, 1, n, eps, stream);
}

int qwen_rmsnorm_gated_rows(const float* x, const float* gate, const float* weight, float* out, int rows, int n,
                            float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && n >= 0, "rmsnorm_gated: negative size (rows=%d, n=%d)", rows, n);
    if (rows == 0 || n == 0) return ok();
    QK_REQUIRE(x && gate && weight && out, "rmsnorm_gated: null pointer");
    return launch_rmsnorm<true>(x, gate, weight, out, rows, n, eps, as_stream(stream));
}

int qwen_rmsnorm_gated_forward(const float* x, const float* gate, const float* weight, float* out, int n, float eps,
                               void* stream) {
    return qwen_rmsnorm_gated_rows(x, gate, weight, out, 1, n, eps, stream);
}

int qwen_residual_add(const float* x1, const float* x2, float* out, int size, void* stream) {
    QK_REQUIRE(size >= 0, "residual_add: negative size %d", size);
    if (size == 0) return ok();
    QK_REQUIRE(x1 && x2 && out, "residual_add: null pointer");
    hipStream_t s = as_stream(stream);
    if (size % 4 == 0 && aligned16(x1) && aligned16(x2) && aligned16(out)) {
        const int n4 = size / 4;
        add_v4<<<std::min<unsigned>(blocks_for(n4, kBlock), 4096u), kBlock, 0, s>>>(x1, x2, out, n4);
    } else {
        add_any<<<std::min<unsigned>(blocks_for(size, kBlock), 4096u), kBlock, 0, s>>>(x1, x2, out, size);
    }
    return check_launch("residual_add");
}

int qwen_residual_rmsnorm_rows_f32(const float* x, const float* branch, const float* weight, float* resid,
                                   float* normed, int rows, int n, float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && n >= 0, "residual_rmsnorm_f32: negative size (rows=%d, n=%d)", rows, n);
    if (rows == 0 || n == 0) return ok();
    QK_REQUIRE(x && branch && weight && resid && normed, "residual_rmsnorm_f32: null pointer");
    hipStream_t s = as_stream(stream);
    const int n4 = n / 4;
    const bool vec = n % 4 == 0 && aligned16(x) && aligned16(branch) && aligned16(weight) && aligned16(resid) &&
                     aligned16(normed);
    if (vec && n4 <= 16 * kWave) {
        launch_row_shape(rows, size_t(n4) * 16, [&](auto stage, dim3 grid, dim3 block, size_t lds) {
            constexpr bool S = decltype(stage)::value;
            if (n4 <= kWave)
                residual_rmsnorm_f32_v4<1, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else if (n4 <= 2 * kWave)
                residual_rmsnorm_f32_v4<2, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else if (n4 <= 4 * kWave)
                residual_rmsnorm_f32_v4<4, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else if (n4 <= 8 * kWave)
                residual_rmsnorm_f32_v4<8, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else
                residual_rmsnorm_f32_v4<16, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
        });
    } else {
        residual_rmsnorm_f32_any<<<rows, kBlock, 0, s>>>(x, branch, weight, resid, normed, n, eps);
    }
    return check_launch("residual_rmsnorm_f32");
}

int qwen_residual_rmsnorm_rows_bf16(const uint16_t* x, const uint16_t* branch, const float* weight, uint16_t* resid,
                                    uint16_t* normed, int rows, int n, float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && n >= 0, "residual_rmsnorm_bf16: negative size (rows=%d, n=%d)", rows, n);
    if (rows == 0 || n == 0) return ok();
    QK_REQUIRE(x && branch && weight && resid && normed, "residual_rmsnorm_bf16: null pointer");
    hipStream_t s = as_stream(stream);
    const int n8 = n / 8;
    const bool vec = n % 8 == 0 && aligned16(x) && aligned16(branch) && aligned16(weight) && aligned16(resid) &&
                     aligned16(normed);
    if (vec && n8 <= 8 * kWave) {
        launch_row_shape(rows, size_t(n8) * 32, [&](auto stage, dim3 grid, dim3 block, size_t lds) {
            constexpr bool S = decltype(stage)::value;
            if (n8 <= kWave)
                residual_rmsnorm_bf16_v8<1, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else if (n8 <= 2 * kWave)
                residual_rmsnorm_bf16_v8<2, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else if (n8 <= 4 * kWave)
                residual_rmsnorm_bf16_v8<4, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
            else
                residual_rmsnorm_bf16_v8<8, S><<<grid, block, lds, s>>>(x, branch, weight, resid, normed, rows, n, eps);
        });
    } else {
        residual_rmsnorm_bf16_any<<<rows, kBlock, 0, s>>>(x, branch, weight, resid, normed, n, eps);
    }
    return check_launch("residual_rmsnorm_bf16");
}

int qwen_encoder_forward(int token_id, const float* table, float* out, int d_model, void* stream) {
    QK_REQUIRE(d_model >= 0 && token_id >= 0, "encoder_forward: bad token %d or d_model %d", token_id, d_model);
    if (d_model == 0) return ok();
    QK_REQUIRE(table && out, "encoder_forward: null pointer");
    hipStream_t s = as_stream(stream);
    copy_row<<<blocks_for(d_model, kBlock), kBlock, 0, s>>>(table + static_cast<size_t>(token_id) * d_model, out,
                                                            d_model);
    return check_launch("encoder_forward");
}

}  // extern "C"
