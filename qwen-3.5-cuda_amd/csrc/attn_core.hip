// Decode attention core on gfx950: one query position against the KV cache.
//
// Reference semantics (src/cuda/attn_kernels.cu, called from
// src/layer_attn.cpp:82-109 once per token per full-attention layer):
//   split_qg_kernel :16-31     q[h][j] = qg[h][j], g[h][j] = qg[h][d + j]
//   score_kernel :72-96        s[h][t] = (q_h . k_t) * rsqrtf(D), t <= pos,
//                              kv head h / (H / Hkv); cache rows [t][kv][D]
//   softmax_kernel :99-158     s = expf(s - max) / sum, per head row
//   value_kernel :162-181      out[h][j] = sum_t s[h][t] * v[t][kv][j]
//   sigmoid_mul_kernel :185-195 out = x / (1 + expf(-g))
// plus the cache store of layer_attn.cpp:99-100 (k, v copied to row pos).
// The reference runs these as separate launches (scores with 32-thread
// blocks per (head, key), values with one block per head).
//
// The separate entry points are kept as drop-ins. The fused decode path is a
// split-K pass plus a combine: workgroup (split, kv head) takes the G = H/Hkv
// (8 or 16) query heads that share kv head and 32 or 16 keys (thread = (head,
// key) for the scores, thread = value column for P.V), so every key and value
// row of the cache is read from HBM once per call; it writes per-split softmax
// statistics (max, sum of exp) and unnormalised P.V rows to a caller-provided
// workspace, and the combine rescales the splits to the global max, divides by
// the total and applies the sigmoid gate.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "attn_common.hpp"
#include "capi_common.hpp"
#include "device_common.hpp"

// Scratch of qwen_attn_decode_noalloc (its split-K partials): a device array,
// one copy on every GPU the library runs on, held until the process ends. In
// host code this name is a host-side stand-in, not a device address: the host
// uses the address hipGetSymbolAddress returns for the current device.
constexpr size_t kDecodeScratchBytes = size_t{8} << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

namespace qk {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxDim = 256;  // fused path: one thread per value column

float host_rsqrt(int n) { return static_cast<float>(1.0 / std::sqrt(static_cast<double>(n))); }

// ---------------------------------------------------------------- elementwise
__global__ __launch_bounds__(kBlock) void split_qg_kernel(const float* __restrict__ in, float* __restrict__ q,
                                                          float* __restrict__ g, int heads, int dim) {
    const int64_t n = static_cast<int64_t>(heads) * dim;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        const int64_t h = i / dim, j = i - h * dim;
        q[i] = in[h * 2 * dim + j];
        g[i] = in[h * 2 * dim + dim + j];
    }
}

__global__ __launch_bounds__(kBlock) void sigmoid_gate_kernel(const float* x, const float* __restrict__ g,
                                                              float* out, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        out[i] = x[i] / (1.0f + expf(-g[i]));
}

__global__ __launch_bounds__(kBlock) void kv_store_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                          float* __restrict__ kc, float* __restrict__ vc, int n) {
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) {
        kc[i] = k[i];
        vc[i] = v[i];
    }
}

// ---------------------------------------------------------------- drop-in stages (other shapes)
// attn_scores outside the tiled form's shapes (scores_split): one wave per
// (head, key), dot over dim, lanes strided.
__global__ __launch_bounds__(kBlock) void scores_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                        float* __restrict__ s, int heads, int kv_heads, int dim,
                                                        int n_keys, float scale) {
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave_in_block();
    if (wave >= static_cast<int64_t>(heads) * n_keys) return;
    const int lane = threadIdx.x & 63;
    const int h = static_cast<int>(wave / n_keys);
    const int t = static_cast<int>(wave - static_cast<int64_t>(h) * n_keys);
    const int kv = h / (heads / kv_heads);
    const float* qh = q + static_cast<size_t>(h) * dim;
    const float* kt = kc + (static_cast<size_t>(t) * kv_heads + kv) * dim;
    float sum = 0.f;
    for (int i = lane; i < dim; i += kWave) sum = __builtin_fmaf(qh[i], kt[i], sum);
    sum = group_sum<64>(sum);
    if (lane == 0) s[static_cast<size_t>(h) * n_keys + t] = sum * scale;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}

// Softmax of one head row per workgroup for rows longer than the register
// form takes (softmax_regs): three passes over the row in global memory.
__global__ __launch_bounds__(kBlock) void softmax_loop(float* __restrict__ s, int n) {
    __shared__ float red[kBlock / kWave];
    float* r = s + static_cast<size_t>(blockIdx.x) * n;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kBlock) m = fmaxf(m, r[i]);
    m = wave_max(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) {
        const float e = expf(r[i] - m);
        r[i] = e;
        sum += e;
    }
    sum = group_sum<64>(sum);
    if (lane == 0) red[w] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);
    for (int i = threadIdx.x; i < n; i += kBlock) r[i] /= sum;
}

// ---------------------------------------------------------------- fused decode
// Workgroup (split, kv head): G query heads x L keys, G * L = 256 threads,
// thread (head, key) for the softmax (32 keys per split for 8 heads per kv
// head, 16 for 16: larger splits halve the partial rows the combine reads).
// The scores are 16 x 16 fp32 MFMA tiles over the queries and keys staged in
// LDS (see below). All of the split's loads go out before the first wait (a
// wait on one load waits for all loads issued before it). Keys go through LDS
// (rows padded to kKeyStride floats so the 16 rows of a tile hit different
// banks); values stay in VGPRs, thread (group, column) holding its column of
// one group of keys; groups of P.V (when the workgroup has more threads than
// columns) meet in LDS. Workspace: acc [H][D / 16][splits][16] (query head
// h = kv G + head of the group), then m and l [H][splits].
constexpr int kKeyStride = kMaxDim + 4;
constexpr int kPairLanes = 1;

// Scores of G query heads x L keys on the matrix cores
// (v_mfma_f32_16x16x4_f32), from the queries and keys staged in LDS: 16 keys
// x 16 heads tiles (for 8 query heads, columns 8..15 repeat them and are not
// read), the head dim split in P parts over the NT / 64 waves; wave w takes
// tile w % T, part w / T. In a 16x16x4 product lane l gives A[key l % 16][k =
// l / 16] and B[k][head l % 16]; lane group g = l / 16 runs over dims part DP
// + g DP/4 + j (j < DP/4), four at a time from one 16-byte LDS read of the key
// row and of the query row. Partial tile `part` goes to sc[part]; the caller
// waits at a barrier and adds the P parts in part order for (head, key).
template <int G, int L, int NT>
struct ScoreTiles {
    static constexpr int T = L / 16, P = (NT / kWave) / T, DP = kMaxDim / P;
    static_assert(T * 16 == L && P * T == NT / kWave && G <= 16 && DP % 16 == 0, "score tiles");
    typedef float Part[T][16][17];

    static __device__ __forceinline__ void run(const float4 (*q_lds)[kMaxDim / 4], const float (*k_lds)[kKeyStride],
                                               Part* sc, int tid) {
        typedef float v4f_t __attribute__((ext_vector_type(4)));
        const int w = wave_in_block(), l = tid & (kWave - 1);
        const int tile = w % T, part = w / T;
        const int m = l & 15, g = l >> 4;
        const float* krow = &k_lds[tile * 16 + m][part * DP + g * (DP / 4)];
        const float4* qrow = &q_lds[m % G][(part * DP + g * (DP / 4)) / 4];
        v4f_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int s = 0; s < DP / 16; ++s) {
            const float4 ka = *reinterpret_cast<const float4*>(krow + 4 * s);
            const float4 qb = qrow[s];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.x, qb.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.y, qb.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.z, qb.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.w, qb.w, acc, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[part][tile][4 * g + i][m] = acc[i];   // key 4g + i, head m
    }

    // q . k of (head hh, key tt) from the P partial tiles, in part order.
    static __device__ __forceinline__ float dot(const Part* sc, int hh, int tt) {
        float d = 0.f;
#pragma unroll
        for (int p = 0; p < P; ++p) d += sc[p][tt >> 4][tt & 15][hh];
        return d;
    }
};

// ---------------------------------------------------------------- drop-in stages
// The reference's three launches keep their signatures and meaning (scores
// [H][n] in HBM between them) with bodies shaped for the whole GPU.
//
// attn_scores: workgroup (split of L keys, kv head), thread (head, key): the G
// query heads of the kv head and the split's key rows staged in LDS, the dot
// products on the matrix cores (ScoreTiles, the tiles of the fused decode), so
// every key row is read from HBM once per call (256 workgroups at 4096 keys).
template <int G, int L>
__global__ __launch_bounds__(G * L) void scores_split(const float* __restrict__ q, const float* __restrict__ kc,
                                                      float* __restrict__ s, int kv_heads, int n_keys, float scale) {
    constexpr int D = kMaxDim, D4 = D / 4, NT = G * L;
    constexpr int QCH = G * D4 / NT, KCH = L * D4 / NT;
    static_assert((G * D4) % NT == 0 && (L * D4) % NT == 0, "scores_split shape");
    using Tiles = ScoreTiles<G, L, NT>;
    __shared__ float4 q_lds[G][D4];
    __shared__ __align__(16) float k_lds[L][kKeyStride];
    __shared__ typename Tiles::Part sc_lds[Tiles::P];
    const int split = blockIdx.x, kv = blockIdx.y, tid = threadIdx.x;
    const int t0 = split * L;
    const size_t row_stride = static_cast<size_t>(kv_heads) * D;
    const float* kbase = kc + static_cast<size_t>(kv) * D;
    float4 qr[QCH], kr[KCH];
#pragma unroll
    for (int i = 0; i < QCH; ++i) qr[i] = ld4(q + static_cast<size_t>(kv) * G * D + 4 * (tid + i * NT));
#pragma unroll
    for (int i = 0; i < KCH; ++i) {  // rows past the end clamped (their scores are not stored)
        const int c = tid + i * NT;
        kr[i] = ld4(kbase + static_cast<size_t>(min(t0 + c / D4, n_keys - 1)) * row_stride + 4 * (c % D4));
    }
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
        const int c = tid + i * NT;
        q_lds[c / D4][c % D4] = qr[i];
    }
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
        const int c = tid + i * NT;
        *reinterpret_cast<float4*>(&k_lds[c / D4][4 * (c % D4)]) = kr[i];
    }
    __syncthreads();
    Tiles::run(q_lds, k_lds, sc_lds, tid);
    __syncthreads();
    const int hh = tid / L, tt = tid % L;
    if (t0 + tt < n_keys)
        s[(static_cast<size_t>(kv) * G + hh) * n_keys + t0 + tt] = Tiles::dot(sc_lds, hh, tt) * scale;
}

// attn_softmax: one workgroup of 1024 threads per head row, the row held in
// registers (element tid + 1024 k in value k), so it is read once and written
// once: row max (DPP within waves, then the 16 wave maxima in LDS), expf(s -
// max), the sum (each thread over its values in order, then lanes, then waves
// in wave order), then exp / sum as the reference divides.
constexpr int kSoftmaxThreads = 1024;

template <int VPT>
__global__ __launch_bounds__(kSoftmaxThreads) void softmax_regs(float* __restrict__ s, int n) {
    constexpr int NW = kSoftmaxThreads / kWave;
    __shared__ float wmax[NW], wsum[NW];
    float* r = s + static_cast<size_t>(blockIdx.x) * n;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = wave_in_block();
    float v[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int i = tid + k * kSoftmaxThreads;
        v[k] = i < n ? r[i] : -INFINITY;
    }
    float m = v[0];
#pragma unroll
    for (int k = 1; k < VPT; ++k) m = fmaxf(m, v[k]);
    m = wave_max(m);
    if (lane == 0) wmax[w] = m;
    __syncthreads();
    m = wmax[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) m = fmaxf(m, wmax[i]);
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        v[k] = tid + k * kSoftmaxThreads < n ? expf(v[k] - m) : 0.f;
        sum += v[k];
    }
    sum = group_sum<64>(sum);
    if (lane == 0) wsum[w] = sum;
    __syncthreads();
    sum = wsum[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) sum += wsum[i];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int i = tid + k * kSoftmaxThreads;
        if (i < n) r[i] = v[k] / sum;
    }
}

// attn_values: workgroup (query head, 16-column block), the keys split over
// its threads and the partial sums added in a fixed order (lane swaps within a
// wave, then the waves in wave order through LDS), so the result does not
// depend on scheduling. VEC (head dim a multiple of 4, 16-byte aligned
// cache): thread (key lane kq = tid / 4, column quad tid % 4) adds p[t] v[t]
// for t = kq, kq + 64, ... (one 16-byte load of 64-byte key segments); else
// thread (key lane tid / 16, column tid % 16) with scalar loads. Workgroups
// are mapped so that the G query heads of a kv head and neighbouring column
// blocks run on one XCD (workgroup b on XCD b % 8), whose L2 then serves the
// value rows G times from one HBM read.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void values_cols(const float* __restrict__ s, const float* __restrict__ vc,
                                                      float* __restrict__ out, int heads, int kv_heads, int dim,
                                                      int n_keys, int ncb) {
    constexpr int NW = kBlock / kWave;
    constexpr int KL = VEC ? kBlock / 4 : kBlock / 16;   // key lanes per workgroup
    constexpr int CW = VEC ? 4 : 1;                       // columns per thread
    __shared__ float part[NW][16];
    const int nblk = gridDim.x, b = blockIdx.x;
    const int idx = (nblk & 7) ? b : (b & 7) * (nblk >> 3) + (b >> 3);
    const int G = heads / kv_heads;
    const int g = idx % G, unit = idx / G;
    const int cb = unit % ncb, kv = unit / ncb;
    const int h = kv * G + g;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = wave_in_block();
    const int kq = VEC ? tid >> 2 : tid >> 4;
    const int cidx = VEC ? tid & 3 : tid & 15;
    const int col = cb * 16 + CW * cidx;
    const bool live = col < dim;
    const float* sh = s + static_cast<size_t>(h) * n_keys;
    const size_t stride = static_cast<size_t>(kv_heads) * dim;
    const float* vp = vc + static_cast<size_t>(kv) * dim + (live ? col : 0);
    float acc[CW];
#pragma unroll
    for (int c = 0; c < CW; ++c) acc[c] = 0.f;
    auto load = [&](int t, float (&vv)[CW]) {
        if constexpr (VEC) {
            const float4 x = ld4(vp + static_cast<size_t>(t) * stride);
            vv[0] = x.x, vv[1] = x.y, vv[2] = x.z, vv[3] = x.w;
        } else {
            vv[0] = vp[static_cast<size_t>(t) * stride];
        }
    };
    if (live) {
        constexpr int U = 4;   // keys in flight per thread
        int t = kq;
        for (; t + (U - 1) * KL < n_keys; t += U * KL) {
            float p[U], vv[U][CW];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                p[u] = sh[t + u * KL];
                load(t + u * KL, vv[u]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int c = 0; c < CW; ++c) acc[c] = __builtin_fmaf(p[u], vv[u][c], acc[c]);
        }
        for (; t < n_keys; t += KL) {
            float vv[CW];
            const float p = sh[t];
            load(t, vv);
#pragma unroll
            for (int c = 0; c < CW; ++c) acc[c] = __builtin_fmaf(p, vv[c], acc[c]);
        }
    }
    // key lanes of one column (lanes cidx + (kWave / KL_w) j) within the wave
#pragma unroll
    for (int o = VEC ? 4 : 16; o < kWave; o <<= 1)
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[c] += __shfl_xor(acc[c], o);
    if (lane < 16 / CW) {
#pragma unroll
        for (int c = 0; c < CW; ++c) part[w][CW * lane + c] = acc[c];
    }
    __syncthreads();
    if (w == 0 && lane < 16 / CW && live) {
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            float z = part[0][CW * lane + c];
#pragma unroll
            for (int i = 1; i < NW; ++i) z += part[i][CW * lane + c];
            out[static_cast<size_t>(h) * dim + col + c] = z;
        }
    }
}

// NR: the attention front end folded in (qwen_attn_decode_norm_rope): q and
// the cache row of key pos = n_keys - 1 arrive unnormalised; each workgroup
// applies the per-head RMSNorm and RoPE (head_dim 256, rope_dim 64;
// norm_rope256, the arithmetic of qk_norm_rope_grouped) to its G query heads in
// registers, the workgroup whose keys hold pos does the same to that row and
// writes it back to the cache, and split 0 of each kv head writes its G
// normalised query heads to q_out (when set).
struct NormRopeArgs {
    const float* qw;
    const float* kw;
    float* q_out;
    float eps;
};

// The key cache argument: read-only (and __restrict__) for the plain decode; a
// plain float* for NR, whose kernel also writes the cache row of pos.
template <bool NR>
struct KeyCache {
    typedef const float* __restrict__ type;
};
template <>
struct KeyCache<true> {
    typedef float* type;
};

template <int G, int L, bool NR = false>
__global__ __launch_bounds__(G * L * kPairLanes) void decode_split(
    const float* __restrict__ q, typename KeyCache<NR>::type kc, const float* __restrict__ vc,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l, int kv_heads, int n_keys,
    int splits, float scale, NormRopeArgs nr = NormRopeArgs{}, RopeDen den = RopeDen{}) {
    constexpr int D = kMaxDim;                 // this path: head dim 256
    constexpr int D4 = D / 4;
    constexpr int NT = G * L * kPairLanes;
    constexpr int HALVES = NT / D;             // P.V: key groups, one thread per (group, column)
    constexpr int LH = L / HALVES;             // keys per group
    constexpr int QCH = G * D4 / NT;           // float4 chunks of q per thread
    constexpr int KCH = L * D4 / NT;           // float4 chunks of the key tile per thread
    static_assert(NT % D == 0 && L % HALVES == 0 && (G * D4) % NT == 0 && (L * D4) % NT == 0 &&
                  L * kPairLanes <= kWave && kWave % (L * kPairLanes) == 0, "decode_split shape");
    __shared__ float4 q_lds[G][D4];
    __shared__ __align__(16) float k_lds[L][kKeyStride];
    __shared__ __align__(16) float p_lds[G][L];
    __shared__ typename ScoreTiles<G, L, NT>::Part sc_lds[ScoreTiles<G, L, NT>::P];   // partial score tiles
    __shared__ float acc_lds[HALVES > 1 ? HALVES - 1 : 1][HALVES > 1 ? G : 1][HALVES > 1 ? D : 1];
    const int split = blockIdx.x, kv = blockIdx.y;
    const int tid = threadIdx.x;
    const int t0 = split * L;
    const size_t row_stride = static_cast<size_t>(kv_heads) * D;  // floats between consecutive keys
    const float* kbase = kc + static_cast<size_t>(kv) * D;
    const float* vbase = vc + static_cast<size_t>(kv) * D;
    const int col = tid % D, half = tid / D;

    float4 qr[QCH], kr[KCH];
    float vcol[LH];
#pragma unroll
    for (int i = 0; i < QCH; ++i) qr[i] = ld4(q + static_cast<size_t>(kv) * G * D + 4 * (tid + i * NT));
    // NR: the front end's operands right behind q, so that the queries'
    // norm + rotation runs while the keys and values are still arriving.
    const int lane = tid & (kWave - 1);
    float dn0 = 0.f;
    float4 wq = make_float4(0.f, 0.f, 0.f, 0.f), wk = wq;
    if constexpr (NR) {
        dn0 = rope256_den(den, lane);
        wq = ld4(nr.qw + 4 * lane);
        wk = ld4(nr.kw + 4 * lane);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
        const int c = tid + i * NT;
        kr[i] = ld4(kbase + static_cast<size_t>(min(t0 + c / D4, n_keys - 1)) * row_stride + 4 * (c % D4));
    }
#pragma unroll
    for (int k2 = 0; k2 < LH; ++k2)  // rows past the end clamped (weight 0)
        vcol[k2] = vbase[static_cast<size_t>(min(t0 + half * LH + k2, n_keys - 1)) * row_stride + col];
    if constexpr (NR) {
        // Thread (wave w, lane) holds float4 `lane` of query head w + 4 i in qr[i]
        // and of key t0 + w + 4 i in kr[i] (NT = 256, D4 = 64): whole heads per
        // wave, the layout norm_rope256 takes.
        static_assert(NT == 4 * kWave && D4 == kWave, "front end layout");
        const int w = wave_in_block();
        const Rope256 rp = rope256_angles(static_cast<float>(n_keys - 1), dn0);
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
            qr[i] = norm_rope256<true>(qr[i], wq, rp, nr.eps, lane);
            if (split == 0 && nr.q_out) st4(nr.q_out + static_cast<size_t>(kv) * G * D + 4 * (tid + i * NT), qr[i]);
        }
        const int kk = n_keys - 1 - t0;   // key pos in this split's tile (wave-uniform)
        if (kk < L && (kk & 3) == w) {
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                if (i == kk >> 2) {
                    kr[i] = norm_rope256<true>(kr[i], wk, rp, nr.eps, lane);
                    st4(kc + static_cast<size_t>(kv) * D + static_cast<size_t>(n_keys - 1) * row_stride + 4 * lane,
                        kr[i]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
        const int c = tid + i * NT;
        q_lds[c / D4][c % D4] = qr[i];
    }
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
        const int c = tid + i * NT;
        *reinterpret_cast<float4*>(&k_lds[c / D4][4 * (c % D4)]) = kr[i];
    }
    __syncthreads();

    // scores on the matrix cores (ScoreTiles). (Per-thread dot products over
    // LDS read 2 KB per thread, 512 KB per workgroup: 11.0 against 10.25 us
    // per decode at 4096 keys.)
    const int pair = tid / kPairLanes, r = tid % kPairLanes;
    const int hh = pair / L, tt = pair % L;
    const bool valid = t0 + tt < n_keys;
    using Tiles = ScoreTiles<G, L, NT>;
    Tiles::run(q_lds, k_lds, sc_lds, tid);
    __syncthreads();
    const float dot = Tiles::dot(sc_lds, hh, tt);
    const float sc = valid ? dot * scale : -INFINITY;
    // max and sum over the L keys of head hh: 4*L consecutive lanes
    constexpr int HL = L * kPairLanes;
    float m = sc;  // equal across the kPairLanes lanes of a pair already
    if constexpr (kPairLanes < 2 && HL >= 2) m = fmaxf(m, dpp_move<0xB1>(m));
    if constexpr (kPairLanes < 4 && HL >= 4) m = fmaxf(m, dpp_move<0x4E>(m));
    if constexpr (HL >= 8) m = fmaxf(m, dpp_move<0x141>(m));
    if constexpr (HL >= 16) m = fmaxf(m, dpp_move<0x140>(m));
    if constexpr (HL >= 32) m = fmaxf(m, __shfl_xor(m, 16));
    if constexpr (HL >= 64) m = fmaxf(m, __shfl_xor(m, 32));
    const float p = valid ? expf(sc - m) : 0.0f;  // every split holds at least one valid key
    const float l = group_sum<HL>(r == 0 ? p : 0.0f);
    if (r == 0) p_lds[hh][tt] = p;
    const size_t stat = (static_cast<size_t>(kv) * G + hh) * splits + split;
    if (tt == 0 && r == 0) {
        ws_m[stat] = m;
        ws_l[stat] = l;
    }
    __syncthreads();

    // P.V: thread = (key group `half`, column), all G heads
    float acc[G];
#pragma unroll
    for (int h2 = 0; h2 < G; ++h2) acc[h2] = 0.f;
#pragma unroll
    for (int k4 = 0; k4 < LH; k4 += 4) {
#pragma unroll
        for (int h2 = 0; h2 < G; ++h2) {
            const float4 pp = *reinterpret_cast<const float4*>(&p_lds[h2][half * LH + k4]);
            acc[h2] = __builtin_fmaf(pp.x, vcol[k4], acc[h2]);
            acc[h2] = __builtin_fmaf(pp.y, vcol[k4 + 1], acc[h2]);
            acc[h2] = __builtin_fmaf(pp.z, vcol[k4 + 2], acc[h2]);
            acc[h2] = __builtin_fmaf(pp.w, vcol[k4 + 3], acc[h2]);
        }
    }
    if constexpr (HALVES > 1) {
        if (half > 0) {
#pragma unroll
            for (int h2 = 0; h2 < G; ++h2) acc_lds[half - 1][h2][col] = acc[h2];
        }
        __syncthreads();
        if (half > 0) return;
#pragma unroll
        for (int v = 0; v < HALVES - 1; ++v) {
#pragma unroll
            for (int h2 = 0; h2 < G; ++h2) acc[h2] += acc_lds[v][h2][col];
        }
    }
#pragma unroll
    // partials as [head][16-column block][split][16]: the combine's workgroup
    // (head, column block) then reads one contiguous run
    for (int h2 = 0; h2 < G; ++h2)
        ws_acc[((static_cast<size_t>(kv) * G + h2) * (D / 16) + col / 16) * splits * 16 + split * 16 + (col & 15)] =
            acc[h2];
}

// Workgroup (query head, 16 columns), 256 workgroups for 16 heads of 256
// columns. Every wave first reduces the head's largest split max M over all
// splits (lane-strided loads, a DPP max); thread (wave w, lane L) then adds
// exp(m_s - M) times the partial row of splits s = 16 w + L/4, + 64, + 128, ...
// for columns 4 (L % 4) .. + 3 of the block (one 16-byte load per split), and
// exp(m_s - M) l_s; the 16 lanes of a column quad add up by lane swaps and the
// 4 waves through LDS in wave order, then the sum is divided by the total
// weight and gated. One max and no rescaling chain: the merge of running
// (max, weight, sum) states split by split costs ~2 us of dependent exp/FMA
// latency at 128 splits, more than the kernel's loads.
// The split pass stores the partials as [head][16-column block][split][16],
// so a workgroup reads one contiguous run of splits x 64 bytes.
constexpr int kCombineCols = 16;
constexpr int kCombineBatch = 2;   // splits per thread and memory round trip

__global__ __launch_bounds__(kBlock) void decode_combine(const float* __restrict__ ws_acc,
                                                         const float* __restrict__ ws_m,
                                                         const float* __restrict__ ws_l,
                                                         const float* __restrict__ gate, float* __restrict__ out,
                                                         int splits) {
    constexpr int D = kMaxDim, NCB = D / kCombineCols, NW = kBlock / kWave;
    constexpr int SPW = kWave / 4;   // splits per wave and round (4 lanes per split)
    constexpr int STEP = SPW * NW * kCombineBatch;
    __shared__ float4 zpart[NW][4];
    __shared__ float tpart[NW][4];
    const int h = blockIdx.x / NCB, cb = blockIdx.x - h * NCB;
    const int lane = threadIdx.x & 63, w = wave_in_block();
    const int cq = lane & 3;
    const size_t s0 = static_cast<size_t>(h) * splits;   // stat of split s: s0 + s
    const float* accp = ws_acc + (s0 * NCB + static_cast<size_t>(cb) * splits) * kCombineCols + 4 * cq;  // + 16 s
    const int first = SPW * w + (lane >> 2);
    // the gate of the columns this lane stores (lanes 0-3 of wave 0), requested
    // first: loaded at the end it would add a memory round trip to the tail
    const size_t j0 = static_cast<size_t>(h) * D + cb * kCombineCols + 4 * cq;
    float gv[4] = {0.f, 0.f, 0.f, 0.f};
    if (gate) {
#pragma unroll
        for (int i = 0; i < 4; ++i) gv[i] = gate[j0 + i];
    }
    // the first batch's partials and statistics, requested with the max's loads
    float4 a[kCombineBatch];
    float mi[kCombineBatch], li[kCombineBatch];
    auto load_batch = [&](int base) {
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) {
            const size_t sc = static_cast<size_t>(min(base + i * SPW * NW, splits - 1));
            a[i] = ld4(accp + sc * kCombineCols);
            mi[i] = ws_m[s0 + sc];
            li[i] = ws_l[s0 + sc];
        }
    };
    load_batch(first);
    float M = -INFINITY;
    for (int s = lane; s < splits; s += kWave) M = fmaxf(M, ws_m[s0 + s]);
    M = wave_max(M);
    float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    float t = 0.f;
    for (int base = first;;) {
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) {
            const float e = base + i * SPW * NW < splits ? expf(mi[i] - M) : 0.f;
            t = __builtin_fmaf(e, li[i], t);
            z = make_float4(__builtin_fmaf(e, a[i].x, z.x), __builtin_fmaf(e, a[i].y, z.y),
                            __builtin_fmaf(e, a[i].z, z.z), __builtin_fmaf(e, a[i].w, z.w));
        }
        base += STEP;
        if (base >= splits) break;
        load_batch(base);
    }
#pragma unroll
    for (int o = 4; o < kWave; o <<= 1) {
        t += __shfl_xor(t, o);
        z.x += __shfl_xor(z.x, o);
        z.y += __shfl_xor(z.y, o);
        z.z += __shfl_xor(z.z, o);
        z.w += __shfl_xor(z.w, o);
    }
    if (lane < 4) {
        zpart[w][lane] = z;
        tpart[w][lane] = t;
    }
    __syncthreads();
    if (w == 0 && lane < 4) {
        float4 zz = zpart[0][lane];
        float tt = tpart[0][lane];
#pragma unroll
        for (int v = 1; v < NW; ++v) {
            zz = make_float4(zz.x + zpart[v][lane].x, zz.y + zpart[v][lane].y, zz.z + zpart[v][lane].z,
                             zz.w + zpart[v][lane].w);
            tt += tpart[v][lane];
        }
        const float o[4] = {zz.x / tt, zz.y / tt, zz.z / tt, zz.w / tt};
#pragma unroll
        for (int i = 0; i < 4; ++i) out[j0 + i] = gate ? o[i] / (1.0f + expf(-gv[i])) : o[i];
    }
}

// Keys per split of the fused path: 32 for 8 query heads per kv head, 16 for
// 16 (256-thread workgroups either way).
int split_keys(int group) { return group == 8 ? 32 : 16; }

int fused_splits(int heads, int kv_heads, int n_keys) {
    const int L = split_keys(heads / kv_heads);
    return (n_keys + L - 1) / L;
}

// Shapes of the fused path: head dim 256, 8 or 16 query heads per kv head.
bool fused_ok(int heads, int kv_heads, int dim, int n_keys) {
    const int g = heads / kv_heads;
    (void)n_keys;
    return dim == kMaxDim && (g == 8 || g == 16);
}

size_t fused_workspace_bytes(int heads, int kv_heads, int dim, int n_keys) {
    return static_cast<size_t>(fused_splits(heads, kv_heads, n_keys)) * heads * (dim + 2) * sizeof(float);
}

// The device address of `scratch` on the current device, looked up once per
// device (hipGetSymbolAddress with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int decode_scratch(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return fail(QWEN_STATUS_LAUNCH_FAILED, "attn_decode_noalloc: no current device");
    }
    QK_REQUIRE(dev >= 0 && dev < kMaxDevices, "attn_decode_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(QWEN_STATUS_LAUNCH_FAILED, "attn_decode_noalloc: hipGetSymbolAddress failed on device %d: %s",
                        dev, hipGetErrorString(e));
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return ok();
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_attn_split_qg(const float* qg, float* q, float* gate, int heads, int dim, void* stream) {
    QK_REQUIRE(heads >= 0 && dim >= 0, "attn_split_qg: negative size");
    if (heads == 0 || dim == 0) return ok();
    QK_REQUIRE(qg && q && gate, "attn_split_qg: null pointer");
    const int64_t n = static_cast<int64_t>(heads) * dim;
    split_qg_kernel<<<std::min<unsigned>(blocks_for(n, kBlock), 4096u), kBlock, 0, as_stream(stream)>>>(qg, q, gate,
                                                                                                       heads, dim);
    return check_launch("attn_split_qg");
}

int qwen_attn_sigmoid_gate(const float* x, const float* gate, float* out, int n, void* stream) {
    QK_REQUIRE(n >= 0, "attn_sigmoid_gate: negative size");
    if (n == 0) return ok();
    QK_REQUIRE(x && gate && out, "attn_sigmoid_gate: null pointer");
    sigmoid_gate_kernel<<<std::min<unsigned>(blocks_for(n, kBlock), 4096u), kBlock, 0, as_stream(stream)>>>(x, gate,
                                                                                                           out, n);
    return check_launch("attn_sigmoid_gate");
}

int qwen_attn_kv_store(const float* k, const float* v, float* k_cache, float* v_cache, int pos, int kv_dim,
                       int max_seq_len, void* stream) {
    QK_REQUIRE(kv_dim >= 0, "attn_kv_store: negative size");
    if (pos < 0 || pos >= max_seq_len)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "attention position exceeds configured context");
    if (kv_dim == 0) return ok();
    QK_REQUIRE(k && v && k_cache && v_cache, "attn_kv_store: null pointer");
    const size_t off = static_cast<size_t>(pos) * kv_dim;
    kv_store_kernel<<<std::min<unsigned>(blocks_for(kv_dim, kBlock), 1024u), kBlock, 0, as_stream(stream)>>>(
        k, v, k_cache + off, v_cache + off, kv_dim);
    return check_launch("attn_kv_store");
}

#define QK_ATTN_SHAPE(what)                                                                                     \
    QK_REQUIRE(heads > 0 && kv_heads > 0 && dim > 0 && pos >= 0, what ": bad shape (heads=%d kv_heads=%d "      \
               "dim=%d pos=%d)", heads, kv_heads, dim, pos);                                                    \
    QK_REQUIRE(heads % kv_heads == 0, what ": heads %d not a multiple of kv_heads %d", heads, kv_heads)

int qwen_attn_scores(const float* q, const float* k_cache, float* scores, int heads, int kv_heads, int dim, int pos,
                     void* stream) {
    QK_ATTN_SHAPE("attn_scores");
    QK_REQUIRE(q && k_cache && scores, "attn_scores: null pointer");
    const int n_keys = pos + 1;
    hipStream_t s = as_stream(stream);
    if (fused_ok(heads, kv_heads, dim, n_keys) && aligned16(q) && aligned16(k_cache)) {
        const int L = split_keys(heads / kv_heads);
        const dim3 grid((n_keys + L - 1) / L, kv_heads);
        if (heads / kv_heads == 8)
            scores_split<8, 32><<<grid, 8 * 32, 0, s>>>(q, k_cache, scores, kv_heads, n_keys, host_rsqrt(dim));
        else
            scores_split<16, 16><<<grid, 16 * 16, 0, s>>>(q, k_cache, scores, kv_heads, n_keys, host_rsqrt(dim));
        return check_launch("attn_scores");
    }
    const int64_t waves = static_cast<int64_t>(heads) * n_keys;
    scores_kernel<<<blocks_for(waves, kBlock / kWave), kBlock, 0, s>>>(q, k_cache, scores, heads, kv_heads, dim,
                                                                      n_keys, host_rsqrt(dim));
    return check_launch("attn_scores");
}

int qwen_attn_softmax(float* scores, int heads, int valid_len, void* stream) {
    QK_REQUIRE(heads >= 0 && valid_len >= 0, "attn_softmax: negative size");
    if (heads == 0 || valid_len == 0) return ok();
    QK_REQUIRE(scores, "attn_softmax: null pointer");
    hipStream_t s = as_stream(stream);
    const int vpt = (valid_len + kSoftmaxThreads - 1) / kSoftmaxThreads;
    if (vpt <= 1)
        softmax_regs<1><<<heads, kSoftmaxThreads, 0, s>>>(scores, valid_len);
    else if (vpt <= 2)
        softmax_regs<2><<<heads, kSoftmaxThreads, 0, s>>>(scores, valid_len);
    else if (vpt <= 4)
        softmax_regs<4><<<heads, kSoftmaxThreads, 0, s>>>(scores, valid_len);
    else if (vpt <= 8)
        softmax_regs<8><<<heads, kSoftmaxThreads, 0, s>>>(scores, valid_len);
    else if (vpt <= 16)
        softmax_regs<16><<<heads, kSoftmaxThreads, 0, s>>>(scores, valid_len);
    else
        softmax_loop<<<heads, kBlock, 0, s>>>(scores, valid_len);
    return check_launch("attn_softmax");
}

int qwen_attn_values(const float* scores, const float* v_cache, float* out, int heads, int kv_heads, int dim, int pos,
                     void* stream) {
    QK_ATTN_SHAPE("attn_values");
    QK_REQUIRE(scores && v_cache && out, "attn_values: null pointer");
    const int ncb = (dim + 15) / 16;
    const int64_t blocks = static_cast<int64_t>(heads) * ncb;
    QK_REQUIRE(blocks <= INT32_MAX, "attn_values: %d heads x %d columns is too large", heads, dim);
    hipStream_t s = as_stream(stream);
    if (dim % 4 == 0 && aligned16(v_cache))
        values_cols<true><<<static_cast<unsigned>(blocks), kBlock, 0, s>>>(scores, v_cache, out, heads, kv_heads, dim,
                                                                           pos + 1, ncb);
    else
        values_cols<false><<<static_cast<unsigned>(blocks), kBlock, 0, s>>>(scores, v_cache, out, heads, kv_heads,
                                                                            dim, pos + 1, ncb);
    return check_launch("attn_values");
}

size_t qwen_attn_decode_workspace_bytes(int heads, int kv_heads, int dim, int pos) {
    if (heads <= 0 || kv_heads <= 0 || dim <= 0 || pos < 0 || heads % kv_heads) return 0;
    const size_t staged = static_cast<size_t>(heads) * (pos + 1) * sizeof(float);  // scores of the staged path
    return fused_ok(heads, kv_heads, dim, pos + 1)
               ? std::max(staged, fused_workspace_bytes(heads, kv_heads, dim, pos + 1))
               : staged;
}

}  // extern "C"

namespace {

// The split pass and the combine (fused_ok shapes, 16-byte aligned q and
// cache); NR: the front end folded into the split pass.
template <bool NR>
int split_combine(const float* q, std::conditional_t<NR, float*, const float*> k_cache, const float* v_cache,
                  const float* gate, float* out,
                  int heads, int kv_heads, int dim, int pos, void* workspace, hipStream_t s,
                  const NormRopeArgs& nr = NormRopeArgs{}, const RopeDen& den = RopeDen{}) {
    const int n_keys = pos + 1;
    const int g = heads / kv_heads;
    const int splits = fused_splits(heads, kv_heads, n_keys);
    float* acc = static_cast<float*>(workspace);
    float* m = acc + static_cast<size_t>(splits) * heads * dim;
    float* l = m + static_cast<size_t>(splits) * heads;
    const dim3 grid(splits, kv_heads);
    const float scale = host_rsqrt(dim);
    if (g == 8)
        decode_split<8, 32, NR><<<grid, 8 * 32 * kPairLanes, 0, s>>>(q, k_cache, v_cache, acc, m, l, kv_heads, n_keys,
                                                                    splits, scale, nr, den);
    else
        decode_split<16, 16, NR><<<grid, 16 * 16 * kPairLanes, 0, s>>>(q, k_cache, v_cache, acc, m, l, kv_heads,
                                                                      n_keys, splits, scale, nr, den);
    int st = check_launch("attn_decode");
    if (st) return st;
    decode_combine<<<heads * (kMaxDim / kCombineCols), kBlock, 0, s>>>(acc, m, l, gate, out, splits);
    return check_launch("attn_decode");
}

// qwen_attn_decode on a workspace already checked against the shape.
int attn_decode_ws(const float* q, const float* k_cache, const float* v_cache, const float* gate, float* out,
                   int heads, int kv_heads, int dim, int pos, void* workspace, void* stream) {
    hipStream_t s = as_stream(stream);
    const int n_keys = pos + 1;
    if (fused_ok(heads, kv_heads, dim, n_keys) && aligned16(q) && aligned16(k_cache))
        return split_combine<false>(q, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, workspace, s);
    float* sc = static_cast<float*>(workspace);
    int st = qwen_attn_scores(q, k_cache, sc, heads, kv_heads, dim, pos, stream);
    if (!st) st = qwen_attn_softmax(sc, heads, n_keys, stream);
    if (!st) st = qwen_attn_values(sc, v_cache, out, heads, kv_heads, dim, pos, stream);
    if (!st && gate) st = qwen_attn_sigmoid_gate(out, gate, out, heads * dim, stream);
    return st;
}

}  // namespace

extern "C" {

int qwen_attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* gate, float* out,
                     int heads, int kv_heads, int dim, int pos, void* workspace, size_t workspace_bytes,
                     void* stream) {
    QK_ATTN_SHAPE("attn_decode");
    QK_REQUIRE(q && k_cache && v_cache && out && workspace, "attn_decode: null pointer");
    const size_t need = qwen_attn_decode_workspace_bytes(heads, kv_heads, dim, pos);
    QK_REQUIRE(workspace_bytes >= need, "attn_decode: workspace of %zu bytes, need %zu", workspace_bytes, need);
    return attn_decode_ws(q, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, workspace, stream);
}

int qwen_attn_decode_norm_rope(const float* q, float* q_normed, float* k_cache, const float* v_cache,
                               const float* gate, float* out, int heads, int kv_heads, int dim, int pos,
                               const float* q_weight, const float* k_weight, int rope_dim, float theta, float eps,
                               void* workspace, size_t workspace_bytes, void* stream) {
    QK_ATTN_SHAPE("attn_decode_norm_rope");
    QK_REQUIRE(q && q_normed && k_cache && v_cache && out && workspace && q_weight && k_weight,
               "attn_decode_norm_rope: null pointer");
    QK_REQUIRE(rope_dim >= 0 && rope_dim <= dim && (rope_dim & 1) == 0 && rope_dim / 2 <= 1024,
               "attn_decode_norm_rope: rope_dim %d invalid for head_dim %d", rope_dim, dim);
    QK_REQUIRE(rope_dim == 0 || theta > 0.0f, "attn_decode_norm_rope: theta must be positive");
    const size_t need = qwen_attn_decode_workspace_bytes(heads, kv_heads, dim, pos);
    QK_REQUIRE(workspace_bytes >= need, "attn_decode_norm_rope: workspace of %zu bytes, need %zu", workspace_bytes,
               need);
    const size_t qbytes = static_cast<size_t>(heads) * dim * sizeof(float);
    const auto qa = reinterpret_cast<uintptr_t>(q), na = reinterpret_cast<uintptr_t>(q_normed);
    const bool disjoint = na + qbytes <= qa || qa + qbytes <= na;
    QK_REQUIRE(disjoint || q_normed == q, "attn_decode_norm_rope: q_normed overlaps q without being q");
    hipStream_t s = as_stream(stream);
    float* krow = k_cache + static_cast<size_t>(pos) * kv_heads * dim;
    if (disjoint && rope_dim == 64 && fused_ok(heads, kv_heads, dim, pos + 1) && aligned16(q) && aligned16(q_normed) &&
        aligned16(k_cache) && aligned16(q_weight) && aligned16(k_weight)) {
        const NormRopeArgs nr{q_weight, k_weight, q_normed, eps};
        return split_combine<true>(q, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, workspace, s, nr,
                                   make_den(0, 32, 64, theta));
    }
    // Other shapes: the front end on a copy of q, then the decode.
    if (q_normed != q) {
        const hipError_t e = hipMemcpyAsync(q_normed, q, qbytes, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess)
            return fail(QWEN_STATUS_LAUNCH_FAILED, "attn_decode_norm_rope: copy of q failed: %s", hipGetErrorString(e));
    }
    int st = qwen_attn_qk_norm_rope_rows(q_normed, krow, q_weight, k_weight, nullptr, pos, 1, heads, kv_heads, dim,
                                         rope_dim, theta, eps, stream);
    if (!st) st = attn_decode_ws(q_normed, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, workspace, stream);
    return st;
}

size_t qwen_attn_decode_noalloc_max_scratch_bytes(void) { return kDecodeScratchBytes; }

int qwen_attn_decode_noalloc(const float* q, const float* k_cache, const float* v_cache, const float* gate,
                             float* out, int heads, int kv_heads, int dim, int pos, void* stream) {
    QK_ATTN_SHAPE("attn_decode_noalloc");
    QK_REQUIRE(q && k_cache && v_cache && out, "attn_decode_noalloc: null pointer");
    const size_t need = qwen_attn_decode_workspace_bytes(heads, kv_heads, dim, pos);
    QK_REQUIRE(need <= kDecodeScratchBytes,
               "attn_decode_noalloc: this shape needs %zu bytes of scratch, beyond the fixed %zu (heads=%d "
               "kv_heads=%d dim=%d pos=%d); use qwen_attn_decode with a workspace",
               need, kDecodeScratchBytes, heads, kv_heads, dim, pos);
    void* ws = nullptr;
    if (const int rc = decode_scratch(&ws)) return rc;
    return attn_decode_ws(q, k_cache, v_cache, gate, out, heads, kv_heads, dim, pos, ws, stream);
}

}  // extern "C"
