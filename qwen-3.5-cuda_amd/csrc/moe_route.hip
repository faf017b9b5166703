// MoE routing and weighted accumulate on gfx950.
//
// Reference semantics (src/cuda/moe.cu):
//   topk_kernel :7-51   one thread: any non-finite logit -> idx[0] = -1,
//                       w[0] = NaN (rest untouched); else k rounds of "largest
//                       unused logit, strictly greater wins" (ties to the lower
//                       index), then w = softmax over the k picks
//   add_kernel :76-86   out += a * x
// The layer (src/layer_moe.cpp:98-142) copies idx / w to the host, waits on
// the stream, and launches k expert GEMV chains with host-side offsets and k
// moe_add calls with host-side weights.
//
// Here top-k runs on 32 lanes per token row, two rows per wave
// (topk_rows_group, moe_common.hpp; one wave per row for rows past 256 logits
// or k past 32). Routing
// stays on the device: qwen_moe_expert_matmul (gemv.hip) reads the expert ids,
// and qwen_moe_weighted_sum_rows reads the weights, so no host round trip is
// needed.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "moe_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxExperts = 16 * kWave;  // logits per row held in VGPRs (16 per lane)

template <int VPL, int KC>
__global__ __launch_bounds__(kBlock) void topk_rows_kernel(const float* __restrict__ x, int32_t* __restrict__ idx,
                                                           float* __restrict__ w, int rows, int n, int k) {
    const int row = blockIdx.x * kWaves + wave_in_block();
    if (row >= rows) return;  // wave-uniform
    const int lane = threadIdx.x & 63;
    int pick_i;
    float weight;
    const bool ok = topk_row<VPL, KC>(x + static_cast<size_t>(row) * n, n, k, pick_i, weight);
    int32_t* ir = idx + static_cast<size_t>(row) * k;
    float* wr = w + static_cast<size_t>(row) * k;
    if (!ok) {   // a non-finite logit: idx[0] = -1, w[0] = NaN, the rest untouched
        if (lane == 0) {
            ir[0] = -1;
            wr[0] = __builtin_nanf("");
        }
        return;
    }
    if (lane < k) {
        ir[lane] = pick_i;
        wr[lane] = weight;
    }
}

// R = 64 / G rows per wave (topk_rows_group): row R w + r in lane group r.
// VEC: rows of exactly G x VPL logits, 16-byte aligned.
template <int G, int VPL, int KC, bool VEC>
__global__ __launch_bounds__(kBlock) void topk_group_kernel(const float* __restrict__ x, int32_t* __restrict__ idx,
                                                            float* __restrict__ w, int rows, int n, int k) {
    constexpr int R = kWave / G;
    const int row0 = R * (blockIdx.x * kWaves + wave_in_block());
    if (row0 >= rows) return;  // wave-uniform
    const int lane = threadIdx.x & 63, grp = lane / G, gl = lane & (G - 1);
    const int row = row0 + grp;   // a row past the end repeats the last row and writes nothing
    int pick_i;
    float weight;
    const uint32_t ok = topk_rows_group<G, VPL, KC, VEC>(x + static_cast<size_t>(min(row, rows - 1)) * n, n, k,
                                                         pick_i, weight);
    if (row >= rows) return;
    int32_t* ir = idx + static_cast<size_t>(row) * k;
    float* wr = w + static_cast<size_t>(row) * k;
    if (!((ok >> grp) & 1)) {   // a non-finite logit: idx[0] = -1, w[0] = NaN, the rest untouched
        if (gl == 0) {
            ir[0] = -1;
            wr[0] = __builtin_nanf("");
        }
        return;
    }
    if (gl < k) {
        ir[gl] = pick_i;
        wr[gl] = weight;
    }
}

__global__ __launch_bounds__(kBlock) void moe_add_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                         float a, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        out[i] = __builtin_fmaf(a, x[i], out[i]);
}

// out[t][d] += sum_j w[t][j] * y[t][j][d], j in order (the reference's k
// moe_add calls, each a fused multiply-add). Vector form: 4 columns per
// thread, the k expert rows streamed with 16-byte nontemporal loads.
__global__ __launch_bounds__(kBlock) void weighted_sum_v4(float* __restrict__ out, const float* __restrict__ y,
                                                          const float* __restrict__ w, int rows, int k, int dim4) {
    const int64_t n = static_cast<int64_t>(rows) * dim4;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        const int64_t t = i / dim4, d4 = i - t * dim4;
        float4 o = ld4_nt(out + 4 * i);
        const float* yt = y + (t * k) * dim4 * 4 + 4 * d4;
        for (int j = 0; j < k; ++j) {
            const float4 yy = ld4_nt(yt + static_cast<int64_t>(j) * dim4 * 4);
            const float a = w[t * k + j];
            o.x = __builtin_fmaf(a, yy.x, o.x);
            o.y = __builtin_fmaf(a, yy.y, o.y);
            o.z = __builtin_fmaf(a, yy.z, o.z);
            o.w = __builtin_fmaf(a, yy.w, o.w);
        }
        st4_nt(out + 4 * i, o);
    }
}

__global__ __launch_bounds__(kBlock) void weighted_sum_kernel(float* __restrict__ out, const float* __restrict__ y,
                                                              const float* __restrict__ w, int rows, int k, int dim) {
    const int64_t n = static_cast<int64_t>(rows) * dim;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        const int64_t t = i / dim, d = i - t * dim;
        float o = out[i];
        for (int j = 0; j < k; ++j) o = __builtin_fmaf(w[t * k + j], y[(t * k + j) * dim + d], o);
        out[i] = o;
    }
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_moe_topk_rows(const float* logits, int32_t* idx, float* weights, int rows, int n, int k, void* stream) {
    QK_REQUIRE(rows >= 0, "moe_topk: negative rows %d", rows);
    QK_REQUIRE(n > 0 && n <= kMaxExperts && k > 0 && k <= n && k <= kWave,
               "moe_topk: need 0 < k <= min(n, 64) and n <= %d (n=%d, k=%d)", kMaxExperts, n, k);
    if (rows == 0) return ok();
    QK_REQUIRE(logits && idx && weights, "moe_topk: null pointer");
    hipStream_t s = as_stream(stream);
    // Rows of up to 256 logits and k <= 32: 32 lanes per row (two rows per wave),
    // 16-byte loads when a row fills the 32 lanes exactly, the rounds unrolled
    // for k = 8 (Qwen3.5's experts per token).
    if (n <= 256 && k <= 32) {
        const unsigned grid2 = blocks_for((rows + 1) / 2, kWaves);
        const bool vec = aligned16(logits);
        const auto group = [&](auto vpl_c) {
            constexpr int V = decltype(vpl_c)::value;
            if (vec && n == 32 * V && V % 4 == 0) {
                if (k == 8)
                    topk_group_kernel<32, V, 8, (V % 4 == 0)><<<grid2, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
                else
                    topk_group_kernel<32, V, 0, (V % 4 == 0)><<<grid2, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
            } else {
                if (k == 8)
                    topk_group_kernel<32, V, 8, false><<<grid2, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
                else
                    topk_group_kernel<32, V, 0, false><<<grid2, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
            }
        };
        if (n <= 32)
            group(std::integral_constant<int, 1>{});
        else if (n <= 64)
            group(std::integral_constant<int, 2>{});
        else if (n <= 128)
            group(std::integral_constant<int, 4>{});
        else
            group(std::integral_constant<int, 8>{});
        return check_launch("moe_topk");
    }
    const unsigned grid = blocks_for(rows, kWaves);
    const int vpl = (n + kWave - 1) / kWave;
    if (vpl <= 1)
        topk_rows_kernel<1, 0><<<grid, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
    else if (vpl <= 2)
        topk_rows_kernel<2, 0><<<grid, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
    else if (vpl <= 4)
        topk_rows_kernel<4, 0><<<grid, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
    else if (vpl <= 8)
        topk_rows_kernel<8, 0><<<grid, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
    else
        topk_rows_kernel<16, 0><<<grid, kBlock, 0, s>>>(logits, idx, weights, rows, n, k);
    return check_launch("moe_topk");
}

int qwen_moe_topk(const float* logits, int32_t* idx, float* weights, int n, int k, void* stream) {
    return qwen_moe_topk_rows(logits, idx, weights, 1, n, k, stream);
}

int qwen_moe_add(float* out, const float* x, float a, int n, void* stream) {
    QK_REQUIRE(n >= 0, "moe_add: negative size %d", n);
    if (n == 0) return ok();
    QK_REQUIRE(out && x, "moe_add: null pointer");
    moe_add_kernel<<<std::min<unsigned>(blocks_for(n, kBlock), 4096u), kBlock, 0, as_stream(stream)>>>(out, x, a, n);
    return check_launch("moe_add");
}

int qwen_moe_weighted_sum_rows(float* out, const float* expert_out, const float* weights, int rows, int k, int dim,
                               void* stream) {
    QK_REQUIRE(rows >= 0 && k >= 0 && dim >= 0, "moe_weighted_sum: negative size");
    if (rows == 0 || k == 0 || dim == 0) return ok();
    QK_REQUIRE(out && expert_out && weights, "moe_weighted_sum: null pointer");
    const int64_t n = static_cast<int64_t>(rows) * dim;
    if (dim % 4 == 0 && aligned16(out) && aligned16(expert_out)) {
        const int64_t n4 = n / 4;
        weighted_sum_v4<<<std::min<unsigned>(blocks_for(n4, kBlock), 16384u), kBlock, 0, as_stream(stream)>>>(
            out, expert_out, weights, rows, k, dim / 4);
    } else {
        weighted_sum_kernel<<<std::min<unsigned>(blocks_for(n, kBlock), 8192u), kBlock, 0, as_stream(stream)>>>(
            out, expert_out, weights, rows, k, dim);
    }
    return check_launch("moe_weighted_sum");
}

}  // extern "C"
