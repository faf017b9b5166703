// Gated DeltaNet gates and recurrent state update on gfx950.
//
// Reference semantics (src/cuda/gdn.cu):
//   gates_kernel :90-99      beta = 1 / (1 + expf(-b));
//                            decay = expf(a * softplus(alpha + dt)),
//                            softplus(x) = x > 20 ? x : log1pf(expf(x))
//   recurrent_kernel :108-151, per value head h (key head h % key_heads) and
//   value column j:
//       S[i][j] *= decay[h];  mem += k[i] * S[i][j]          (i < key_dim)
//       delta = (v[j] - mem) * beta[h]
//       S[i][j] += k[i] * delta
//       out[j] = sum_i q[i] * S[i][j]
// called once per token per GDN layer (src/layer_gdn.cpp:100-106). The
// reference walks the state three times per token (one thread per column, a
// block per head, 32 blocks).
//
// Here the state (value_heads x key_dim x value_dim fp32, 2 MB per layer at
// 32 x 128 x 128) is read once and written once per call: one wave owns a few
// value columns of one head, each column spread over a group of 16 or 32
// lanes that hold 4 or 8 of its rows in VGPRs, so a column sum over rows is a
// short per-lane partial plus a 4-5 step DPP reduction. The multi-token entry
// point keeps the state slice in VGPRs across all tokens of the call (the
// reference's per-token loop, one launch), reading each token's q, k, v
// straight from the GDN front end's output rows. A single token (the decode
// step) reads the state in row-major tiles instead: a workgroup of two waves
// per (value head, 16 columns), the two tiles of a 128-byte line segment on one
// XCD, column sums through DPP and LDS.
#include <algorithm>
#include <cmath>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "gdn_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;

// softplus with the reference's threshold; log1p(exp(x)) evaluated with the
// accurate device expf / log1pf.
__device__ __forceinline__ float softplus20(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// The gate pair of src/cuda/gdn.cu:93-97, shared by gates_kernel and the
// recurrence's fused-gate form so that both give the same bits.
__device__ __forceinline__ float gate_beta(float b) { return 1.0f / (1.0f + expf(-b)); }
__device__ __forceinline__ float gate_decay(float a, float alpha, float dt) { return expf(a * softplus20(alpha + dt)); }

// Fused-gate form of the recurrence: with `a` set, the kernels' beta / decay
// arguments hold beta_raw / alpha_raw and the gates are evaluated per token
// where they are used (a, dt_bias per value head).
struct RawGates {
    const float* a;
    const float* dt;
};

__global__ __launch_bounds__(kBlock) void gates_kernel(const float* __restrict__ b, const float* __restrict__ alpha,
                                                       const float* __restrict__ a, const float* __restrict__ dt,
                                                       float* __restrict__ beta, float* __restrict__ decay,
                                                       int64_t n, int heads) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        const int h = static_cast<int>(i % heads);
        beta[i] = gate_beta(b[i]);
        decay[i] = gate_decay(a[h], alpha[i], dt[h]);
    }
}

// One wave per (value head, NCOL value columns): column c = L / G of the wave
// (G = 64 / NCOL lanes per column), rows (L % G) * RPL .. + RPL - 1 of that
// column in VGPRs (RPL = DK / G). The per-token column sums over rows are a
// per-lane partial over RPL rows plus a G-lane DPP reduction (4 or 5 steps).
// Tokens t < rows run in order, the state slice staying in VGPRs; q/k/v of
// token t sit at t * qkv_stride, beta/decay at t * value_heads, out at
// t * out_stride. The inputs of token t + kPrefetch are loaded while token t
// is computed (a ring of kPrefetch register slots; loads past the last token
// re-read it and are never used).
constexpr int kPrefetch = 4;

template <int DK, int NCOL>
__global__ __launch_bounds__(kBlock) void gdn_recurrent_g(float* __restrict__ S, const float* __restrict__ q,
                                                          const float* __restrict__ k, const float* __restrict__ v,
                                                          const float* __restrict__ beta,
                                                          const float* __restrict__ decay, float* __restrict__ out,
                                                          int rows, int key_heads, int value_heads, int value_dim,
                                                          int64_t qkv_stride, int64_t out_stride, RawGates rg) {
    constexpr int G = kWave / NCOL;
    constexpr int RPL = DK / G;
    static_assert(RPL % 4 == 0 && RPL * G == DK, "rows per lane");
    constexpr int P = kPrefetch;
    const int cblocks = value_dim / NCOL;
    const int wave = blockIdx.x * kWaves + wave_in_block();
    if (wave >= value_heads * cblocks) return;  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int h = wave / cblocks;
    const int c = lane / G, r0 = (lane % G) * RPL;
    const int j = NCOL * (wave - h * cblocks) + c;   // this lane's value column
    const int src = h % key_heads;  // value heads tile as [subgroup][key head]
    const float ah = rg.a ? rg.a[h] : 0.0f, dth = rg.a ? rg.dt[h] : 0.0f;
    float* Sj = S + static_cast<size_t>(h) * DK * value_dim + static_cast<size_t>(r0) * value_dim + j;

    float kr[P][RPL], qr[P][RPL], vv[P], bt[P], dc[P];
    auto fetch = [&](int slot, int t) {
        t = min(t, rows - 1);
        const float* qt = q + t * qkv_stride + src * DK + r0;
        const float* kt = k + t * qkv_stride + src * DK + r0;
#pragma unroll
        for (int r = 0; r < RPL; r += 4) {
            const float4 kv = ld4(kt + r), qv = ld4(qt + r);
            kr[slot][r] = kv.x;
            kr[slot][r + 1] = kv.y;
            kr[slot][r + 2] = kv.z;
            kr[slot][r + 3] = kv.w;
            qr[slot][r] = qv.x;
            qr[slot][r + 1] = qv.y;
            qr[slot][r + 2] = qv.z;
            qr[slot][r + 3] = qv.w;
        }
        vv[slot] = v[t * qkv_stride + static_cast<size_t>(h) * value_dim + j];
        bt[slot] = beta[static_cast<int64_t>(t) * value_heads + h];
        dc[slot] = decay[static_cast<int64_t>(t) * value_heads + h];
    };
#pragma unroll
    for (int p = 0; p < P; ++p) fetch(p, p);

    // NCOL lanes of a row read NCOL consecutive floats (the same 16- or 8-byte
    // pieces per row as any column slicing of the row-major state).
    float s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) s[r] = __builtin_nontemporal_load(Sj + static_cast<size_t>(r) * value_dim);

    for (int t0 = 0; t0 < rows; t0 += P) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int t = t0 + p;
            if (t >= rows) break;  // wave-uniform
            // S *= decay; mem = sum_i k_i S_i (this column)
            const float d = rg.a ? gate_decay(ah, dc[p], dth) : dc[p];
            float m = 0.f;
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                s[r] *= d;
                m = __builtin_fmaf(kr[p][r], s[r], m);
            }
            m = group_sum<G>(m);
            const float dl = (vv[p] - m) * (rg.a ? gate_beta(bt[p]) : bt[p]);
            // S += k_i * delta; o = sum_i q_i S_i
            float o = 0.f;
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                s[r] = __builtin_fmaf(kr[p][r], dl, s[r]);
                o = __builtin_fmaf(qr[p][r], s[r], o);
            }
            o = group_sum<G>(o);
            if (lane % G == 0) out[t * out_stride + static_cast<size_t>(h) * value_dim + j] = o;
            fetch(p, t + P);
        }
    }

#pragma unroll
    for (int r = 0; r < RPL; ++r) __builtin_nontemporal_store(s[r], Sj + static_cast<size_t>(r) * value_dim);
}

// Single step with value_dim % 16 != 0 (gdn_step_tile takes the others): one
// wave per (value head, 4 value columns); RPL rows of the state per lane
// (key_dim = 64 * RPL). Tokens t < rows run in order, the state slice staying
// in VGPRs; q/k/v of token t sit at t * qkv_stride, beta/decay at
// t * value_heads, out at t * out_stride. The inputs of token t + kPrefetch
// are loaded while token t is computed (a ring of kPrefetch register slots;
// loads past the last token re-read it and are never used).

template <int RPL>
__global__ __launch_bounds__(kBlock) void gdn_recurrent_v4(float* __restrict__ S, const float* __restrict__ q,
                                                           const float* __restrict__ k, const float* __restrict__ v,
                                                           const float* __restrict__ beta,
                                                           const float* __restrict__ decay, float* __restrict__ out,
                                                           int rows, int key_heads, int value_heads, int value_dim,
                                                           int64_t qkv_stride, int64_t out_stride, RawGates rg) {
    constexpr int DK = 64 * RPL;
    constexpr int P = kPrefetch;
    const int cblocks = value_dim >> 2;
    const int wave = blockIdx.x * kWaves + wave_in_block();
    if (wave >= value_heads * cblocks) return;  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int h = wave / cblocks;
    const int j0 = 4 * (wave - h * cblocks);
    const int src = h % key_heads;  // value heads tile as [subgroup][key head]
    const float ah = rg.a ? rg.a[h] : 0.0f, dth = rg.a ? rg.dt[h] : 0.0f;
    float* Sh = S + static_cast<size_t>(h) * DK * value_dim + j0;

    float kr[P][RPL], qr[P][RPL], bt[P], dc[P];
    float4 vv[P];
    auto fetch = [&](int slot, int t) {
        t = min(t, rows - 1);
        const float* qt = q + t * qkv_stride + src * DK;
        const float* kt = k + t * qkv_stride + src * DK;
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            kr[slot][r] = kt[lane + 64 * r];
            qr[slot][r] = qt[lane + 64 * r];
        }
        vv[slot] = ld4(v + t * qkv_stride + static_cast<size_t>(h) * value_dim + j0);
        bt[slot] = beta[static_cast<int64_t>(t) * value_heads + h];
        dc[slot] = decay[static_cast<int64_t>(t) * value_heads + h];
    };
#pragma unroll
    for (int p = 0; p < P; ++p) fetch(p, p);

    float4 s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) s[r] = ld4_nt(Sh + static_cast<size_t>(lane + 64 * r) * value_dim);

    for (int t0 = 0; t0 < rows; t0 += P) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int t = t0 + p;
            if (t >= rows) break;  // wave-uniform
            // S *= decay; mem = sum_i k_i S_i  (per column)
            const float d = rg.a ? gate_decay(ah, dc[p], dth) : dc[p];
            float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                s[r].x *= d;
                s[r].y *= d;
                s[r].z *= d;
                s[r].w *= d;
                m.x = __builtin_fmaf(kr[p][r], s[r].x, m.x);
                m.y = __builtin_fmaf(kr[p][r], s[r].y, m.y);
                m.z = __builtin_fmaf(kr[p][r], s[r].z, m.z);
                m.w = __builtin_fmaf(kr[p][r], s[r].w, m.w);
            }
            m.x = group_sum<64>(m.x);
            m.y = group_sum<64>(m.y);
            m.z = group_sum<64>(m.z);
            m.w = group_sum<64>(m.w);
            const float b = rg.a ? gate_beta(bt[p]) : bt[p];
            const float4 dl = make_float4((vv[p].x - m.x) * b, (vv[p].y - m.y) * b, (vv[p].z - m.z) * b,
                                          (vv[p].w - m.w) * b);
            // S += k_i * delta; o = sum_i q_i S_i
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                s[r].x = __builtin_fmaf(kr[p][r], dl.x, s[r].x);
                s[r].y = __builtin_fmaf(kr[p][r], dl.y, s[r].y);
                s[r].z = __builtin_fmaf(kr[p][r], dl.z, s[r].z);
                s[r].w = __builtin_fmaf(kr[p][r], dl.w, s[r].w);
                o.x = __builtin_fmaf(qr[p][r], s[r].x, o.x);
                o.y = __builtin_fmaf(qr[p][r], s[r].y, o.y);
                o.z = __builtin_fmaf(qr[p][r], s[r].z, o.z);
                o.w = __builtin_fmaf(qr[p][r], s[r].w, o.w);
            }
            o.x = group_sum<64>(o.x);
            o.y = group_sum<64>(o.y);
            o.z = group_sum<64>(o.z);
            o.w = group_sum<64>(o.w);
            if (lane == 0) st4(out + t * out_stride + static_cast<size_t>(h) * value_dim + j0, o);
            fetch(p, t + P);
        }
    }

#pragma unroll
    for (int r = 0; r < RPL; ++r) st4_nt(Sh + static_cast<size_t>(lane + 64 * r) * value_dim, s[r]);
}

// Single token with value_dim % 16 == 0 (the decode path): one workgroup of
// kTileWaves = 2 waves per (value head h, kTileCols = 16 value columns). Lane L
// holds columns 4 * (L / 16) .. + 3 of the tile and wave w rows
// w * DK / 2 + L % 16 + 16 r (r < DK / 32): the 16 lanes of a column group read
// 16 rows and the 4 groups the 16 columns of each, so one float4 load
// instruction covers 16 64-byte halves of state lines. The two tiles that share
// a 128-byte line segment run on one XCD (tile_of_block), whose L2 then fetches
// the line once. A column's sums over rows: a per-lane partial, a 16-lane DPP
// sum, and the two waves' partials added through LDS in wave order. The state
// loads are issued before anything else the kernel loads.
//
// Measured at 32 x 128 x 128 against the earlier tiles of four waves x 32
// columns (8 lanes per column, whole 128-byte lines per workgroup, 128
// workgroups): 2.93 against 3.38 us per call, the same bytes on twice as many
// CUs; 16-column tiles in plain block order (line halves on two XCDs) take
// 3.66 us.
constexpr int kTileWaves = 2;
constexpr int kTileBlock = kTileWaves * kWave;
constexpr int kTileLanes = 16;                       // lanes per column group
constexpr int kTileGroups = kWave / kTileLanes;      // column groups per wave
constexpr int kTileCols = 4 * kTileGroups;           // value columns per workgroup

// One token on a lane's slice (RPL rows kr / qr of k / q, the state rows s at
// St + 8 r * value_dim, value columns vv, gates b / d): S *= d; m = k . S;
// delta = (v - m) b; S += k delta; o = q . S. Stores the state slice and
// returns o summed over the workgroup (wave 0; other waves get a partial).
// red: 2 * kTileWaves * kTileGroups float4 of LDS; every thread of the
// workgroup must call it (two barriers).
template <int RPL>
__device__ __forceinline__ float4 tile_step(float4 (&s)[RPL], const float (&kr)[RPL], const float (&qr)[RPL],
                                            float4 vv, float b, float d, float* St, int value_dim, float4* red,
                                            int w, int cg, int rl) {
    float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        s[r].x *= d;
        s[r].y *= d;
        s[r].z *= d;
        s[r].w *= d;
        m.x = __builtin_fmaf(kr[r], s[r].x, m.x);
        m.y = __builtin_fmaf(kr[r], s[r].y, m.y);
        m.z = __builtin_fmaf(kr[r], s[r].z, m.z);
        m.w = __builtin_fmaf(kr[r], s[r].w, m.w);
    }
    m.x = group_sum<kTileLanes>(m.x);
    m.y = group_sum<kTileLanes>(m.y);
    m.z = group_sum<kTileLanes>(m.z);
    m.w = group_sum<kTileLanes>(m.w);
    if (rl == 0) red[w * kTileGroups + cg] = m;
    __syncthreads();
    m = red[cg];
#pragma unroll
    for (int x = 1; x < kTileWaves; ++x) {
        const float4 u = red[x * kTileGroups + cg];
        m.x += u.x;
        m.y += u.y;
        m.z += u.z;
        m.w += u.w;
    }
    const float4 dl = make_float4((vv.x - m.x) * b, (vv.y - m.y) * b, (vv.z - m.z) * b, (vv.w - m.w) * b);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        s[r].x = __builtin_fmaf(kr[r], dl.x, s[r].x);
        s[r].y = __builtin_fmaf(kr[r], dl.y, s[r].y);
        s[r].z = __builtin_fmaf(kr[r], dl.z, s[r].z);
        s[r].w = __builtin_fmaf(kr[r], dl.w, s[r].w);
        o.x = __builtin_fmaf(qr[r], s[r].x, o.x);
        o.y = __builtin_fmaf(qr[r], s[r].y, o.y);
        o.z = __builtin_fmaf(qr[r], s[r].z, o.z);
        o.w = __builtin_fmaf(qr[r], s[r].w, o.w);
    }
#pragma unroll
    for (int r = 0; r < RPL; ++r) st4_nt(St + static_cast<size_t>(kTileLanes * r) * value_dim, s[r]);
    o.x = group_sum<kTileLanes>(o.x);
    o.y = group_sum<kTileLanes>(o.y);
    o.z = group_sum<kTileLanes>(o.z);
    o.w = group_sum<kTileLanes>(o.w);
    float4* ro = red + kTileWaves * kTileGroups;
    if (rl == 0) ro[w * kTileGroups + cg] = o;
    __syncthreads();
    if (w == 0) {
        o = ro[cg];
#pragma unroll
        for (int x = 1; x < kTileWaves; ++x) {
            const float4 u = ro[x * kTileGroups + cg];
            o.x += u.x;
            o.y += u.y;
            o.z += u.z;
            o.w += u.w;
        }
    }
    return o;
}

// The tile form of one token (key dim DK = 64 or 128). Grid: exactly
// value_heads * value_dim / kTileCols workgroups of kTileBlock threads.
template <int DK>
__global__ __launch_bounds__(kTileBlock) void gdn_step_tile(float* __restrict__ S, const float* __restrict__ q,
                                                            const float* __restrict__ k, const float* __restrict__ v,
                                                            const float* __restrict__ beta,
                                                            const float* __restrict__ decay, float* __restrict__ out,
                                                            int key_heads, int value_dim, RawGates rg) {
    constexpr int RPL = DK / (kTileWaves * kTileLanes);
    static_assert(RPL * kTileWaves * kTileLanes == DK, "key dim");
    __shared__ float4 red[2 * kTileWaves * kTileGroups];
    const int lane = threadIdx.x & 63;
    const int w = wave_in_block();
    const int cblocks = value_dim / kTileCols;
    const int tile = tile_of_block(blockIdx.x, gridDim.x);
    const int h = tile / cblocks;
    const int cg = lane / kTileLanes, rl = lane % kTileLanes;
    const int j0 = (tile - h * cblocks) * kTileCols + 4 * cg;
    const int r0 = w * (DK / kTileWaves) + rl;
    float* St = S + (static_cast<size_t>(h) * DK + r0) * value_dim + j0;
    float4 s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) s[r] = ld4_nt(St + static_cast<size_t>(kTileLanes * r) * value_dim);
    __builtin_amdgcn_sched_barrier(0);   // the state loads first
    const int src = h % key_heads;       // value heads tile as [subgroup][key head]
    const float* kt = k + src * DK + r0;
    const float* qt = q + src * DK + r0;
    float kr[RPL], qr[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        kr[r] = kt[kTileLanes * r];
        qr[r] = qt[kTileLanes * r];
    }
    const float4 vv = ld4(v + static_cast<size_t>(h) * value_dim + j0);
    const float br = beta[h], dr = decay[h];
    const float d = rg.a ? gate_decay(rg.a[h], dr, rg.dt[h]) : dr;
    const float b = rg.a ? gate_beta(br) : br;
    const float4 o = tile_step<RPL>(s, kr, qr, vv, b, d, St, value_dim, red, w, cg, rl);
    if (w == 0 && rl == 0) st4(out + static_cast<size_t>(h) * value_dim + j0, o);
}

// One decode token of a GDN layer after its input projections, in one launch:
// the front end (causal conv of kernel 4 + SiLU, Q/K L2 norm) and the
// fused-gate recurrence. Key dim 128, value_dim % kTileCols == 0. Each
// workgroup is a workgroup of gdn_step_tile<128> -- (value head h, columns
// cb * 16 ..), lane L of wave w holding columns j0 = cb * 16 + 4 (L / 16) .. + 3
// and rows w * 64 + L % 16 + 16 r -- whose waves first evaluate the front end for
// what they read: the 256 q | k channels of key head h % key_heads in
// gdn_frontend_k4<32>'s layout (lane L: channels 4L..4L+3 of q for L < 32, of k
// for L >= 32; a 32-lane sum of squares per head), moved to the recurrence's
// layout through a per-wave LDS copy, and each lane its 4 value channels. So every value
// equals what gdn_frontend_rows writes and the recurrence reads, bit for bit.
// Writes: the front end's output row y and the new history (q | k channels of
// key head g by wave 0 of the tile h = g, cb = 0; value channels by wave 0 of
// the workgroup that reads them), the state and the output. hist_out must not
// overlap hist_in: many waves read one key head's history while one of them
// writes it. Grid: exactly value_heads * value_dim / kTileCols workgroups.
__global__ __launch_bounds__(kTileBlock) void gdn_decode_fused(
        const float* __restrict__ x, const float* __restrict__ cw, const float* __restrict__ hin,
        float* __restrict__ hout, float* __restrict__ y, float* __restrict__ S, const float* __restrict__ beta_raw,
        const float* __restrict__ alpha_raw, const float* __restrict__ a, const float* __restrict__ dt,
        float* __restrict__ out, int key_heads, int value_dim, float eps, float qscale) {
    constexpr int DK = 128;
    constexpr int RPL = DK / (kTileWaves * kTileLanes);
    __shared__ float4 red[2 * kTileWaves * kTileGroups];
    const int lane = threadIdx.x & 63;
    const int w = wave_in_block();
    const int cblocks = value_dim / kTileCols;
    const int tile = tile_of_block(blockIdx.x, gridDim.x);
    const int h = tile / cblocks;
    const int cb = tile - h * cblocks;
    const int cg = lane / kTileLanes, rl = lane % kTileLanes;
    const int j0 = cb * kTileCols + 4 * cg;
    const int r0 = w * (DK / kTileWaves) + rl;
    float* St = S + (static_cast<size_t>(h) * DK + r0) * value_dim + j0;
    const int src = h % key_heads;
    const int kd = key_heads * DK;
    const bool is_q = lane < 32;
    const size_t c = static_cast<size_t>(is_q ? src * DK + 4 * lane : kd + src * DK + 4 * (lane - 32));
    const size_t cv = static_cast<size_t>(2 * kd + h * value_dim + j0);

    // Every load issued before the first use: taps, history and input of the
    // lane's q | k channels and of its value channels, the gates, then the
    // state slice. Loads return in order, so the front end's inputs come first
    // and its math runs while the state is still arriving (issued the other
    // way round, the front end waited for the state: 4.6 us against 4.3 per
    // step at 32 x 128 x 128).
    const float4 w0 = ld4(cw + 4 * c), w1 = ld4(cw + 4 * c + 4), w2 = ld4(cw + 4 * c + 8), w3 = ld4(cw + 4 * c + 12);
    const float4 ha = ld4(hin + 3 * c), hb = ld4(hin + 3 * c + 4), hd = ld4(hin + 3 * c + 8);
    const float4 xv = ld4(x + c);
    const float4 u0 = ld4(cw + 4 * cv), u1 = ld4(cw + 4 * cv + 4), u2 = ld4(cw + 4 * cv + 8), u3 = ld4(cw + 4 * cv + 12);
    const float4 va = ld4(hin + 3 * cv), vb = ld4(hin + 3 * cv + 4), vd = ld4(hin + 3 * cv + 8);
    const float4 vx = ld4(x + cv);
    const float br = beta_raw[h], ar = alpha_raw[h], ah = a[h], dth = dt[h];
    float4 s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) s[r] = ld4_nt(St + static_cast<size_t>(kTileLanes * r) * value_dim);
    __builtin_amdgcn_sched_barrier(0);

    // q | k front end (gdn_frontend_k4<32>, one row)
    float4 h0, h1, h2;
    history4(ha, hb, hd, h0, h1, h2);
    float4 f = silu4(make_float4(conv4(h0.x, h1.x, h2.x, xv.x, w0), conv4(h0.y, h1.y, h2.y, xv.y, w1),
                                 conv4(h0.z, h1.z, h2.z, xv.z, w2), conv4(h0.w, h1.w, h2.w, xv.w, w3)));
    const float ss = group_sum<32>(sumsq4(f));
    const float rr = rsqrtf(ss + eps);
    const float sc = is_q ? rr * qscale : rr;
    f.x *= sc;
    f.y *= sc;
    f.z *= sc;
    f.w *= sc;
    // value channels (no norm)
    float4 g0, g1, g2;
    history4(va, vb, vd, g0, g1, g2);
    const float4 vv = silu4(make_float4(conv4(g0.x, g1.x, g2.x, vx.x, u0), conv4(g0.y, g1.y, g2.y, vx.y, u1),
                                        conv4(g0.z, g1.z, g2.z, vx.z, u2), conv4(g0.w, g1.w, g2.w, vx.w, u3)));

    if (h == src && cb == 0 && w == 0) {   // one wave per key head writes its q | k channels
        st4(y + c, f);
        st4(hout + 3 * c, make_float4(h1.x, h2.x, xv.x, h1.y));
        st4(hout + 3 * c + 4, make_float4(h2.y, xv.y, h1.z, h2.z));
        st4(hout + 3 * c + 8, make_float4(xv.z, h1.w, h2.w, xv.w));
    }
    if (w == 0 && rl == 0) {   // each column group's value channels once
        st4(y + cv, vv);
        st4(hout + 3 * cv, make_float4(g1.x, g2.x, vx.x, g1.y));
        st4(hout + 3 * cv + 4, make_float4(g2.y, vx.y, g1.z, g2.z));
        st4(hout + 3 * cv + 8, make_float4(vx.z, g1.w, g2.w, vx.w));
    }

    // Recurrence layout: lane L needs q, k of rows i = r0 + 16 r. Lane L holds
    // channels 4L..4L+3 of q (L < 32) or of k (L >= 32) in f, so the wave's f
    // written to LDS as [lane][4] is the q | k head in channel order: q row i is
    // float i, k row i float 128 + i. Each wave uses its own copy (no barrier:
    // a wave's LDS accesses complete in order).
    __shared__ float qk_lds[kTileWaves][2 * DK];
    *reinterpret_cast<float4*>(&qk_lds[w][4 * lane]) = f;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float qr[RPL], kr[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        qr[r] = qk_lds[w][r0 + kTileLanes * r];
        kr[r] = qk_lds[w][DK + r0 + kTileLanes * r];
    }

    // gdn_step_tile<128>, gates from the raw projections
    const float d = gate_decay(ah, ar, dth);
    const float b = gate_beta(br);
    const float4 o = tile_step<RPL>(s, kr, qr, vv, b, d, St, value_dim, red, w, cg, rl);
    if (w == 0 && rl == 0) st4(out + static_cast<size_t>(h) * value_dim + j0, o);
}

// Any key / value dim (value_dim <= 256): one block per value head, thread j
// owns column j and walks the rows, as the reference does.
__global__ __launch_bounds__(kMaxValueDim) void gdn_recurrent_any(
    float* __restrict__ S, const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ beta, const float* __restrict__ decay, float* __restrict__ out, int rows, int key_heads,
    int value_heads, int key_dim, int value_dim, int64_t qkv_stride, int64_t out_stride, RawGates rg) {
    const int h = blockIdx.x;
    const int j = threadIdx.x;
    if (j >= value_dim) return;
    const int src = h % key_heads;
    float* Sh = S + static_cast<size_t>(h) * key_dim * value_dim + j;
    for (int t = 0; t < rows; ++t) {
        const float* qt = q + t * qkv_stride + static_cast<size_t>(src) * key_dim;
        const float* kt = k + t * qkv_stride + static_cast<size_t>(src) * key_dim;
        const float dr = decay[static_cast<int64_t>(t) * value_heads + h];
        const float dc = rg.a ? gate_decay(rg.a[h], dr, rg.dt[h]) : dr;
        float mem = 0.f;
        for (int i = 0; i < key_dim; ++i) {
            float c = Sh[static_cast<size_t>(i) * value_dim] * dc;
            Sh[static_cast<size_t>(i) * value_dim] = c;
            mem = __builtin_fmaf(kt[i], c, mem);
        }
        const float br = beta[static_cast<int64_t>(t) * value_heads + h];
        const float dl = (v[t * qkv_stride + static_cast<size_t>(h) * value_dim + j] - mem) *
                         (rg.a ? gate_beta(br) : br);
        float o = 0.f;
        for (int i = 0; i < key_dim; ++i) {
            const float c = __builtin_fmaf(kt[i], dl, Sh[static_cast<size_t>(i) * value_dim]);
            Sh[static_cast<size_t>(i) * value_dim] = c;
            o = __builtin_fmaf(qt[i], c, o);
        }
        out[t * out_stride + static_cast<size_t>(h) * value_dim + j] = o;
    }
}

int launch_recurrent(float* state, const float* q, const float* k, const float* v, const float* beta,
                     const float* decay, float* out, int rows, int key_heads, int value_heads, int key_dim,
                     int value_dim, int64_t qkv_stride, int64_t out_stride, hipStream_t s, const char* what,
                     RawGates rg = RawGates{nullptr, nullptr}) {
    const bool vec = value_dim % 4 == 0 && (key_dim == 64 || key_dim == 128) && aligned16(q) && aligned16(k) &&
                     qkv_stride % 4 == 0;
    if (vec && rows == 1 && value_dim % kTileCols == 0 && aligned16(state) && aligned16(v) && aligned16(out)) {
        // One token: the state traffic dominates, read as whole 128-byte lines.
        const unsigned grid = static_cast<unsigned>(value_heads * (value_dim / kTileCols));
        if (key_dim == 64)
            gdn_step_tile<64><<<grid, kTileBlock, 0, s>>>(state, q, k, v, beta, decay, out, key_heads, value_dim, rg);
        else
            gdn_step_tile<128><<<grid, kTileBlock, 0, s>>>(state, q, k, v, beta, decay, out, key_heads, value_dim, rg);
    } else if (vec && rows == 1 && aligned16(state) && aligned16(v) && aligned16(out)) {
        // One token, value_dim % 16 != 0: 4-column float4 slices.
        const unsigned grid = blocks_for(value_heads * (value_dim / 4), kWaves);
        if (key_dim == 64)
            gdn_recurrent_v4<1><<<grid, kBlock, 0, s>>>(state, q, k, v, beta, decay, out, rows, key_heads,
                                                        value_heads, value_dim, qkv_stride, out_stride, rg);
        else
            gdn_recurrent_v4<2><<<grid, kBlock, 0, s>>>(state, q, k, v, beta, decay, out, rows, key_heads,
                                                        value_heads, value_dim, qkv_stride, out_stride, rg);
    } else if (vec) {
        // Columns per wave: 2 for key dim 128 (two waves per SIMD at the Qwen3.5
        // shape, 32 value heads x 128 columns), 4 for key dim 64.
        constexpr int kNcol128 = 2;
        const int ncol = key_dim == 64 ? 4 : kNcol128;
        const unsigned grid = blocks_for(value_heads * (value_dim / ncol), kWaves);
        if (key_dim == 64)
            gdn_recurrent_g<64, 4><<<grid, kBlock, 0, s>>>(state, q, k, v, beta, decay, out, rows, key_heads,
                                                           value_heads, value_dim, qkv_stride, out_stride, rg);
        else
            gdn_recurrent_g<128, kNcol128><<<grid, kBlock, 0, s>>>(state, q, k, v, beta, decay, out, rows, key_heads,
                                                                   value_heads, value_dim, qkv_stride, out_stride, rg);
    } else {
        gdn_recurrent_any<<<value_heads, kMaxValueDim, 0, s>>>(state, q, k, v, beta, decay, out, rows, key_heads,
                                                               value_heads, key_dim, value_dim, qkv_stride,
                                                               out_stride, rg);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_gdn_gate_values_rows(const float* beta_raw, const float* alpha_raw, const float* a, const float* dt_bias,
                              float* beta, float* decay, int rows, int heads, void* stream) {
    QK_REQUIRE(rows >= 0 && heads >= 0, "gdn_gate_values: negative size (rows=%d, heads=%d)", rows, heads);
    if (rows == 0 || heads == 0) return ok();
    QK_REQUIRE(beta_raw && alpha_raw && a && dt_bias && beta && decay, "gdn_gate_values: null pointer");
    const int64_t n = static_cast<int64_t>(rows) * heads;
    gates_kernel<<<std::min<unsigned>(blocks_for(n, kBlock), 4096u), kBlock, 0, as_stream(stream)>>>(
        beta_raw, alpha_raw, a, dt_bias, beta, decay, n, heads);
    return check_launch("gdn_gate_values");
}

int qwen_gdn_gate_values(const float* beta_raw, const float* alpha_raw, const float* a, const float* dt_bias,
                         float* beta, float* decay, int heads, void* stream) {
    return qwen_gdn_gate_values_rows(beta_raw, alpha_raw, a, dt_bias, beta, decay, 1, heads, stream);
}

int qwen_gdn_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta,
                            const float* decay, float* out, int rows, int key_heads, int value_heads, int key_dim,
                            int value_dim, int64_t qkv_stride, int64_t out_stride, void* stream) {
    QK_REQUIRE(rows >= 0 && key_heads >= 0 && value_heads >= 0 && key_dim >= 0 && value_dim >= 0,
               "gdn_recurrent: negative size");
    QK_REQUIRE(value_dim <= kMaxValueDim, "GDN value dimension exceeds kernel limit");
    if (rows == 0 || value_heads == 0 || value_dim == 0) return ok();
    QK_REQUIRE(key_heads > 0 && key_dim > 0, "gdn_recurrent: key_heads and key_dim must be positive");
    QK_REQUIRE(state && q && k && v && beta && decay && out, "gdn_recurrent: null pointer");
    QK_REQUIRE(rows == 1 || (qkv_stride > 0 && out_stride > 0), "gdn_recurrent: non-positive row stride");
    return launch_recurrent(state, q, k, v, beta, decay, out, rows, key_heads, value_heads, key_dim, value_dim,
                            qkv_stride, out_stride, as_stream(stream), "gdn_recurrent");
}

int qwen_gdn_gated_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta_raw,
                                  const float* alpha_raw, const float* a, const float* dt_bias, float* out, int rows,
                                  int key_heads, int value_heads, int key_dim, int value_dim, int64_t qkv_stride,
                                  int64_t out_stride, void* stream) {
    QK_REQUIRE(rows >= 0 && key_heads >= 0 && value_heads >= 0 && key_dim >= 0 && value_dim >= 0,
               "gdn_gated_recurrent: negative size");
    QK_REQUIRE(value_dim <= kMaxValueDim, "GDN value dimension exceeds kernel limit");
    if (rows == 0 || value_heads == 0 || value_dim == 0) return ok();
    QK_REQUIRE(key_heads > 0 && key_dim > 0, "gdn_gated_recurrent: key_heads and key_dim must be positive");
    QK_REQUIRE(state && q && k && v && beta_raw && alpha_raw && a && dt_bias && out,
               "gdn_gated_recurrent: null pointer");
    QK_REQUIRE(rows == 1 || (qkv_stride > 0 && out_stride > 0), "gdn_gated_recurrent: non-positive row stride");
    return launch_recurrent(state, q, k, v, beta_raw, alpha_raw, out, rows, key_heads, value_heads, key_dim,
                            value_dim, qkv_stride, out_stride, as_stream(stream), "gdn_gated_recurrent",
                            RawGates{a, dt_bias});
}

int qwen_gdn_decode_step(const float* x, const float* conv_weight, const float* hist_in, float* hist_out, float* y,
                         float* state, const float* beta_raw, const float* alpha_raw, const float* a,
                         const float* dt_bias, float* out, int key_heads, int value_heads, int key_dim, int value_dim,
                         int kernel, float eps, void* stream) {
    QK_REQUIRE(key_heads > 0 && value_heads > 0 && key_dim > 0 && value_dim > 0 && kernel >= 2,
               "gdn_decode_step: bad shape (heads %d / %d, dims %d / %d, kernel %d)", key_heads, value_heads, key_dim,
               value_dim, kernel);
    QK_REQUIRE(value_dim <= kMaxValueDim, "GDN value dimension exceeds kernel limit");
    QK_REQUIRE(x && conv_weight && hist_in && hist_out && y && state && beta_raw && alpha_raw && a && dt_bias && out,
               "gdn_decode_step: null pointer");
    const int64_t C = 2 * static_cast<int64_t>(key_heads) * key_dim + static_cast<int64_t>(value_heads) * value_dim;
    QK_REQUIRE(C < (int64_t{1} << 31), "gdn_decode_step: %lld channels", static_cast<long long>(C));
    const auto lo = reinterpret_cast<uintptr_t>(hist_in), hi = lo + static_cast<uintptr_t>(C) * (kernel - 1) * 4;
    const auto olo = reinterpret_cast<uintptr_t>(hist_out), ohi = olo + static_cast<uintptr_t>(C) * (kernel - 1) * 4;
    const bool disjoint = ohi <= lo || hi <= olo;
    const bool fused = disjoint && kernel == 4 && key_dim == 128 && value_dim % kTileCols == 0 &&
                       value_heads % key_heads == 0 &&
                       aligned16(x) && aligned16(conv_weight) && aligned16(hist_in) && aligned16(hist_out) &&
                       aligned16(y) && aligned16(state) && aligned16(out);
    if (!fused) {   // the two calls it fuses (the front end may update the history in place)
        int rc = qwen_gdn_frontend_rows(x, conv_weight, hist_in, hist_out, y, 1, static_cast<int>(C), kernel,
                                        key_heads, key_dim, eps, stream);
        if (rc) return rc;
        const int64_t kd = static_cast<int64_t>(key_heads) * key_dim;
        return qwen_gdn_gated_recurrent_rows(state, y, y + kd, y + 2 * kd, beta_raw, alpha_raw, a, dt_bias, out, 1,
                                             key_heads, value_heads, key_dim, value_dim, 0, 0, stream);
    }
    const unsigned grid = static_cast<unsigned>(value_heads * (value_dim / kTileCols));
    gdn_decode_fused<<<grid, kTileBlock, 0, as_stream(stream)>>>(x, conv_weight, hist_in, hist_out, y, state, beta_raw,
                                                             alpha_raw, a, dt_bias, out, key_heads, value_dim, eps,
                                                             host_rsqrt(key_dim));
    return check_launch("gdn_decode_step");
}

int qwen_gdn_recurrent_step(float* state, const float* q, const float* k, const float* v, const float* beta,
                            const float* decay, float* out, int key_heads, int value_heads, int key_dim,
                            int value_dim, void* stream) {
    return qwen_gdn_recurrent_rows(state, q, k, v, beta, decay, out, 1, key_heads, value_heads, key_dim, value_dim,
                                   0, 0, stream);
}

}  // extern "C"
