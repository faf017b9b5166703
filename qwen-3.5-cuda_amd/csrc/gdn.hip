// Gated DeltaNet front and back end on gfx950.
//
// Front end (reference: conv_step_kernel src/cuda/gdn.cu:9-27 then
// qk_norm_kernel src/cuda/gdn.cu:36-81, called at src/layer_gdn.cpp:89,97):
// per channel c, y[t] = silu(sum_j x[t-K+1+j] * w[c][j]) with x[<0] taken from
// the history, then q = y[0:H*dk] and k = y[H*dk:2*H*dk] are L2-normalised per
// head (eps on the sum, q also scaled by 1/sqrt(dk)). The reference runs one
// launch per token and a second pass over y; here one wave owns 256 channels
// (float4 per lane) over a tile of TT tokens, keeps the K-1 previous inputs in
// registers as a sliding window, so x is read once (plus a 3-token halo per
// tile) and y is written once, already normalised. The channel/time tiling puts
// the previous time tile of the same channels 8 workgroups earlier, i.e. on the
// same XCD, so the halo rows come from that XCD's L2.
//
// Back end (reference: norm_gate_kernel src/cuda/gdn.cu:176-210):
// out = ((x * r) * w) * silu(z) per head; one lane group of dim/4 lanes per
// head, U head groups per wave with all loads issued before any math.
#include <algorithm>
#include <cmath>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "gdn_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;
constexpr int kConvTile = 64;    // tokens per thread tile (generic front end)
// Vector front end: rows per wave and waves per workgroup. Swept at C4a (4096 x
// 8192): 3 x 8 = 44.5 us, 4 x 8 = 44.9, 4 x 4 = 45.9, 6 x 8 = 46.4, 8 x 8 = 50.2;
// one or two rows per wave (halo rows then come from two or three waves back,
// through LDS) 45.3-57 us. Three is the fewest rows a wave can hand on whole.
constexpr int kConvRows = 3;
constexpr int kConvWaves = 8;
constexpr int kGateUnroll = 4;   // head groups in flight per wave (norm_gate)

// ---------------------------------------------------- front end, kernel size 4
// Workgroup = 256 channels (float4 per lane) x W waves x R rows: wave v owns
// rows T0 + v*R .. +R-1 and issues all R row loads at once. The three rows
// before a wave's first row are the previous wave's last three, handed over
// through LDS, so only wave 0 reads rows outside its tile (the rows before T0,
// or the history when T0 == 0). Lanes past the last channel address a clamped
// channel and skip their stores, so loads never branch.
template <int LPH, int R, int W>
__global__ __launch_bounds__(W * kWave) void gdn_frontend_k4(const float* __restrict__ x, const float* __restrict__ w,
                                                          const float* hist_in, float* hist_out, float* __restrict__ y,
                                                          int rows, int C, int q_ch, int qk_ch, float eps, float qscale,
                                                          int n_ctiles) {
    static_assert(R >= 3, "a wave hands its last three rows to the next wave");
    __shared__ float4 halo[W][3][kWave];
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int cbase = (blockIdx.x % n_ctiles) * (4 * kWave);
    const int T0 = (blockIdx.x / n_ctiles) * (W * R);       // first row of the workgroup
    const int t0 = T0 + wv * R;                             // first row of this wave
    const int c = cbase + 4 * lane;
    const bool on = c < C;
    const int cc = on ? c : C - 4;         // clamped channel for addressing
    const bool norm_wave = cbase < qk_ch;  // wave-uniform
    const bool is_q = c < q_ch;
    const bool is_qk = c < qk_ch;

    // Loads return in order: the small reused operands first, then the rows.
    const float4 w0 = ld4(w + 4 * static_cast<size_t>(cc));  // taps of channels c..c+3
    const float4 w1 = ld4(w + 4 * static_cast<size_t>(cc) + 4);
    const float4 w2 = ld4(w + 4 * static_cast<size_t>(cc) + 8);
    const float4 w3 = ld4(w + 4 * static_cast<size_t>(cc) + 12);
    float4 h0 = make_float4(0.f, 0.f, 0.f, 0.f), h1 = h0, h2 = h0;  // x[t-3], x[t-2], x[t-1]
    if (wv == 0) {
        if (T0 == 0) {
            history4(ld4(hist_in + 3 * static_cast<size_t>(cc)), ld4(hist_in + 3 * static_cast<size_t>(cc) + 4),
                     ld4(hist_in + 3 * static_cast<size_t>(cc) + 8), h0, h1, h2);
        } else {
            h0 = ld4(x + static_cast<size_t>(T0 - 3) * C + cc);
            h1 = ld4(x + static_cast<size_t>(T0 - 2) * C + cc);
            h2 = ld4(x + static_cast<size_t>(T0 - 1) * C + cc);
        }
    }
    float4 xv[R];
#pragma unroll
    for (int u = 0; u < R; ++u) xv[u] = ld4_nt(x + static_cast<size_t>(min(t0 + u, rows - 1)) * C + cc);

    // Hand the last three rows to the next wave. A wave whose rows run past the
    // end publishes clamped rows, read only by waves with no rows at all.
    halo[wv][0][lane] = xv[R - 3];
    halo[wv][1][lane] = xv[R - 2];
    halo[wv][2][lane] = xv[R - 1];
    __syncthreads();
    if (wv > 0) {
        h0 = halo[wv - 1][0][lane];
        h1 = halo[wv - 1][1][lane];
        h2 = halo[wv - 1][2][lane];
    }

#pragma unroll
    for (int u = 0; u < R; ++u) {
        if (t0 + u >= rows) break;  // wave-uniform
        float4 v = silu4(make_float4(conv4(h0.x, h1.x, h2.x, xv[u].x, w0), conv4(h0.y, h1.y, h2.y, xv[u].y, w1),
                                     conv4(h0.z, h1.z, h2.z, xv[u].z, w2), conv4(h0.w, h1.w, h2.w, xv[u].w, w3)));
        if (norm_wave) {
            const float ss = group_sum<LPH>(sumsq4(v));
            const float r = rsqrtf(ss + eps);
            const float sc = is_q ? r * qscale : r;  // q *= rq * scale; k *= rk
            if (is_qk) {
                v.x *= sc;
                v.y *= sc;
                v.z *= sc;
                v.w *= sc;
            }
        }
        if (on) st4_nt(y + static_cast<size_t>(t0 + u) * C + c, v);
        h0 = h1;
        h1 = h2;
        h2 = xv[u];
    }

    // Wave 0 of the first workgroup in time owns the history: it read hist_in
    // first and writes hist_out last, so hist_out may alias hist_in.
    if (T0 == 0 && wv == 0 && on) {
        if (rows > R) {  // the last three inputs (when rows <= R the window already holds them)
            h0 = ld4(x + static_cast<size_t>(rows - 3) * C + c);
            h1 = ld4(x + static_cast<size_t>(rows - 2) * C + c);
            h2 = ld4(x + static_cast<size_t>(rows - 1) * C + c);
        }
        st4(hist_out + 3 * static_cast<size_t>(c), make_float4(h0.x, h1.x, h2.x, h0.y));
        st4(hist_out + 3 * static_cast<size_t>(c) + 4, make_float4(h1.y, h2.y, h0.z, h1.z));
        st4(hist_out + 3 * static_cast<size_t>(c) + 8, make_float4(h2.z, h0.w, h1.w, h2.w));
    }
}

// ---------------------------------------------------- front end, generic
// Any kernel size and alignment: one thread per (channel, tile of kConvTile
// tokens); inputs before the tile are re-read from x (or the history).
__global__ __launch_bounds__(kBlock) void gdn_conv_any(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* hist_in, float* hist_out, float* __restrict__ y,
                                                       int rows, int C, int K, int n_ttiles) {
    const int64_t id = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (id >= static_cast<int64_t>(C) * n_ttiles) return;
    const int c = static_cast<int>(id % C);
    const int t0 = static_cast<int>(id / C) * kConvTile;
    const int t1 = min(t0 + kConvTile, rows);
    const int hk = K - 1;
    const float* wc = w + static_cast<size_t>(c) * K;
    auto input = [&](int tau) -> float {  // x[tau] of channel c, history for tau < 0
        return tau >= 0 ? x[static_cast<size_t>(tau) * C + c] : hist_in[static_cast<size_t>(c) * hk + hk + tau];
    };
    for (int t = t0; t < t1; ++t) {
        float s = 0.0f;
        for (int j = 0; j < hk; ++j) s = __builtin_fmaf(input(t - hk + j), wc[j], s);
        s = __builtin_fmaf(x[static_cast<size_t>(t) * C + c], wc[hk], s);
        y[static_cast<size_t>(t) * C + c] = silu(s);
    }
    if (t0 == 0) {
        // hist_out[j] = input(rows - hk + j); for in-place use every read index
        // (j + rows when negative) is ahead of the index being written.
        for (int j = 0; j < hk; ++j) hist_out[static_cast<size_t>(c) * hk + j] = input(rows - hk + j);
    }
}

// ---------------------------------------------------- Q/K L2 norm
// Lane groups of LPH lanes (dim = 4*LPH); slot s -> (row, q-or-k, head).
template <int LPH>
__global__ __launch_bounds__(kBlock) void qk_l2_v4(float* q, float* k, int64_t stride, int rows, int heads, float eps,
                                                   float qscale) {
    constexpr int HPW = kWave / LPH;
    const int lane = threadIdx.x & 63;
    const int lg = lane % LPH;
    const int64_t total = static_cast<int64_t>(rows) * heads * 2;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave_in_block();
    if (wave * HPW >= total) return;
    const int64_t slot = wave * HPW + lane / LPH;
    const bool active = slot < total;
    const int64_t t = slot / (2 * heads);
    const int rem = static_cast<int>(slot % (2 * heads));
    const bool is_q = rem < heads;
    float* p = (is_q ? q : k) + t * stride + static_cast<int64_t>(is_q ? rem : rem - heads) * (4 * LPH) + 4 * lg;
    float4 v = active ? ld4(p) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float ss = group_sum<LPH>(sumsq4(v));
    const float r = rsqrtf(ss + eps);
    const float sc = is_q ? r * qscale : r;
    if (active) st4(p, make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc));
}

// One block per head (any dim / alignment): blockIdx = (row * 2 + {q,k}) * heads + head.
__global__ __launch_bounds__(kBlock) void qk_l2_any(float* q, float* k, int64_t stride, int heads, int dim, float eps,
                                                    float qscale) {
    __shared__ float lds[kBlock / kWave];
    const int64_t t = blockIdx.x / (2 * heads);
    const int rem = static_cast<int>(blockIdx.x % (2 * heads));
    const bool is_q = rem < heads;
    float* p = (is_q ? q : k) + t * stride + static_cast<int64_t>(is_q ? rem : rem - heads) * dim;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kBlock) ss += p[i] * p[i];
    ss = group_sum<kWave>(ss);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    const float r = rsqrtf(ss + eps);
    const float sc = is_q ? r * qscale : r;
    for (int i = threadIdx.x; i < dim; i += kBlock) p[i] *= sc;
}

// ---------------------------------------------------- gated per-head RMSNorm
// Lane groups of LPH lanes per head (dim = 4*LPH); a wave handles kGateUnroll
// consecutive head groups with every x and z load issued before any math.
template <int LPH>
__global__ __launch_bounds__(kBlock) void norm_gate_v4(const float* __restrict__ x, const float* __restrict__ z,
                                                       const float* __restrict__ w, float* __restrict__ out,
                                                       int64_t heads_total, float eps) {
    constexpr int HPW = kWave / LPH;
    constexpr int D = 4 * LPH;
    const int lane = threadIdx.x & 63;
    const int lg = lane % LPH;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave_in_block();
    const int64_t h_first = wave * (HPW * kGateUnroll);
    if (h_first >= heads_total) return;
    const float4 wv = ld4(w + 4 * lg);
    float4 xv[kGateUnroll], zv[kGateUnroll];
#pragma unroll
    for (int u = 0; u < kGateUnroll; ++u) {
        const int64_t h = min(h_first + u * HPW + lane / LPH, heads_total - 1);
        xv[u] = ld4_nt(x + h * D + 4 * lg);
        zv[u] = ld4_nt(z + h * D + 4 * lg);
    }
#pragma unroll
    for (int u = 0; u < kGateUnroll; ++u) {
        const int64_t h = h_first + u * HPW + lane / LPH;
        const float ss = group_sum<LPH>(sumsq4(xv[u]));
        const float r = rsqrtf(ss / static_cast<float>(D) + eps);
        const float4 sz = silu4(zv[u]);
        float4 o;
        o.x = xv[u].x * r * wv.x * sz.x;
        o.y = xv[u].y * r * wv.y * sz.y;
        o.z = xv[u].z * r * wv.z * sz.z;
        o.w = xv[u].w * r * wv.w * sz.w;
        if (h < heads_total) st4_nt(out + h * D + 4 * lg, o);
    }
}

__global__ __launch_bounds__(kBlock) void norm_gate_any(const float* __restrict__ x, const float* __restrict__ z,
                                                        const float* __restrict__ w, float* __restrict__ out, int dim,
                                                        float eps) {
    __shared__ float lds[kBlock / kWave];
    const size_t base = static_cast<size_t>(blockIdx.x) * dim;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kBlock) ss += x[base + i] * x[base + i];
    ss = group_sum<kWave>(ss);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    const float r = rsqrtf(ss / static_cast<float>(dim) + eps);
    for (int i = threadIdx.x; i < dim; i += kBlock) out[base + i] = x[base + i] * r * w[i] * silu(z[base + i]);
}

// ---------------------------------------------------- launchers
int lph_of(int dim) {
    if (dim % 4 != 0) return 0;
    const int l = dim / 4;
    return (l == 16 || l == 32 || l == 64) ? l : 0;
}

void launch_qk_l2(float* q, float* k, int64_t stride, int rows, int heads, int dim, float eps, hipStream_t s) {
    const float qscale = host_rsqrt(dim);
    const int lph = lph_of(dim);
    const bool vec = lph && aligned16(q) && aligned16(k) && stride % 4 == 0;
    if (vec) {
        const int64_t slots = static_cast<int64_t>(rows) * heads * 2;
        const int64_t waves = (slots + (kWave / lph) - 1) / (kWave / lph);
        const unsigned grid = blocks_for(waves, kBlock / kWave);
        if (lph == 64)
            qk_l2_v4<64><<<grid, kBlock, 0, s>>>(q, k, stride, rows, heads, eps, qscale);
        else if (lph == 32)
            qk_l2_v4<32><<<grid, kBlock, 0, s>>>(q, k, stride, rows, heads, eps, qscale);
        else
            qk_l2_v4<16><<<grid, kBlock, 0, s>>>(q, k, stride, rows, heads, eps, qscale);
    } else {
        qk_l2_any<<<static_cast<unsigned>(rows) * heads * 2, kBlock, 0, s>>>(q, k, stride, heads, dim, eps, qscale);
    }
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_gdn_frontend_rows(const float* x, const float* weight, const float* hist_in, float* hist_out, float* y,
                           int rows, int channels, int kernel, int k_heads, int key_dim, float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && channels >= 0, "gdn_frontend: negative size (rows=%d, channels=%d)", rows, channels);
    // kernel - 1 <= kConvTile keeps every history read inside the first time
    // tile, whose thread alone writes hist_out (in-place safety).
    QK_REQUIRE(kernel >= 2 && kernel <= kConvTile + 1, "gdn_frontend: kernel size %d outside [2, %d]", kernel,
               kConvTile + 1);
    QK_REQUIRE(k_heads >= 0 && (k_heads == 0 || key_dim > 0), "gdn_frontend: bad k_heads %d / key_dim %d", k_heads,
               key_dim);
    QK_REQUIRE(static_cast<int64_t>(2) * k_heads * key_dim <= channels,
               "gdn_frontend: q and k (%d heads x %d) exceed %d channels", k_heads, key_dim, channels);
    if (rows == 0 || channels == 0) return ok();
    QK_REQUIRE(x && weight && hist_in && hist_out && y, "gdn_frontend: null pointer");
    hipStream_t s = as_stream(stream);
    const int q_ch = k_heads * key_dim;
    const int qk_ch = 2 * q_ch;
    const int lph = k_heads > 0 ? lph_of(key_dim) : 64;
    const bool vec = kernel == 4 && channels % 4 == 0 && lph && aligned16(x) && aligned16(weight) &&
                     aligned16(hist_in) && aligned16(hist_out) && aligned16(y);
    const int n_ttiles = (rows + kConvTile - 1) / kConvTile;
    if (vec) {
        constexpr int R = kConvRows, W = kConvWaves;
        const int n_ctiles = (channels + 4 * kWave - 1) / (4 * kWave);
        const int n_wtiles = (rows + W * R - 1) / (W * R);
        const unsigned grid = static_cast<unsigned>(n_ctiles) * n_wtiles;
        const float qscale = k_heads > 0 ? host_rsqrt(key_dim) : 1.0f;
        if (lph == 64)
            gdn_frontend_k4<64, R, W><<<grid, W * kWave, 0, s>>>(x, weight, hist_in, hist_out, y, rows, channels, q_ch,
                                                                qk_ch, eps, qscale, n_ctiles);
        else if (lph == 32)
            gdn_frontend_k4<32, R, W><<<grid, W * kWave, 0, s>>>(x, weight, hist_in, hist_out, y, rows, channels, q_ch,
                                                                qk_ch, eps, qscale, n_ctiles);
        else
            gdn_frontend_k4<16, R, W><<<grid, W * kWave, 0, s>>>(x, weight, hist_in, hist_out, y, rows, channels, q_ch,
                                                                qk_ch, eps, qscale, n_ctiles);
    } else {
        const int64_t threads = static_cast<int64_t>(channels) * n_ttiles;
        gdn_conv_any<<<blocks_for(threads, kBlock), kBlock, 0, s>>>(x, weight, hist_in, hist_out, y, rows, channels,
                                                                    kernel, n_ttiles);
        if (k_heads > 0) launch_qk_l2(y, y + q_ch, channels, rows, k_heads, key_dim, eps, s);
    }
    return check_launch("gdn_frontend");
}

int qwen_gdn_conv_step(const float* input, const float* weight, float* history, float* output, int channels,
                       int kernel, void* stream) {
    return qwen_gdn_frontend_rows(input, weight, history, history, output, 1, channels, kernel, 0, 0, 0.0f, stream);
}

int qwen_gdn_qk_normalize(float* q, float* k, int heads, int dim, float eps, void* stream) {
    QK_REQUIRE(heads >= 0 && dim >= 0, "gdn_qk_normalize: negative size (heads=%d, dim=%d)", heads, dim);
    if (heads == 0 || dim == 0) return ok();
    QK_REQUIRE(q && k, "gdn_qk_normalize: null pointer");
    launch_qk_l2(q, k, 0, 1, heads, dim, eps, as_stream(stream));
    return check_launch("gdn_qk_normalize");
}

int qwen_gdn_norm_gate_rows(const float* x, const float* z, const float* weight, float* out, int rows, int heads,
                            int dim, float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && heads >= 0 && dim >= 0, "gdn_norm_gate: negative size");
    if (rows == 0 || heads == 0 || dim == 0) return ok();
    QK_REQUIRE(x && z && weight && out, "gdn_norm_gate: null pointer");
    hipStream_t s = as_stream(stream);
    const int64_t total = static_cast<int64_t>(rows) * heads;
    const int lph = lph_of(dim);
    const bool vec = lph && aligned16(x) && aligned16(z) && aligned16(weight) && aligned16(out);
    if (vec) {
        const int64_t per_wave = (kWave / lph) * kGateUnroll;
        const unsigned grid = blocks_for((total + per_wave - 1) / per_wave, kBlock / kWave);
        if (lph == 64)
            norm_gate_v4<64><<<grid, kBlock, 0, s>>>(x, z, weight, out, total, eps);
        else if (lph == 32)
            norm_gate_v4<32><<<grid, kBlock, 0, s>>>(x, z, weight, out, total, eps);
        else
            norm_gate_v4<16><<<grid, kBlock, 0, s>>>(x, z, weight, out, total, eps);
    } else {
        norm_gate_any<<<static_cast<unsigned>(total), kBlock, 0, s>>>(x, z, weight, out, dim, eps);
    }
    return check_launch("gdn_norm_gate");
}

int qwen_gdn_norm_gate(const float* x, const float* z, const float* weight, float* out, int heads, int dim, float eps,
                       void* stream) {
    return qwen_gdn_norm_gate_rows(x, z, weight, out, 1, heads, dim, eps, stream);
}

}  // extern "C"
