// Chunked form of the Gated DeltaNet recurrence for many tokens (prefill).
//
// The reference updates the state one token at a time (src/cuda/gdn.cu:108-151,
// called per token by src/layer_gdn.cpp:100-106): per value head, with key
// vectors k_t, q_t (key head h % key_heads), value v_t, gates beta_t, d_t,
//     S <- d_t S;  delta_t = beta_t (v_t - S^T k_t);  S <- S + k_t delta_t^T;
//     o_t = S^T q_t.
// Over a chunk of C tokens starting from state S0, with
//     R[t][i] = d_{i+1} * ... * d_t  (i <= t; the decay between tokens i and t),
//     gamma_t = d_0 * ... * d_t,
// the state after token t is gamma_t S0 + sum_{i<=t} R[t][i] k_i delta_i^T, so
//     delta_t = beta_t (v_t - gamma_t S0^T k_t - sum_{i<t} R[t][i] (k_i.k_t) delta_i)
//     (I + A) Delta = diag(beta) (V - diag(gamma) K S0),  A[t][i] = beta_t R[t][i] (k_t.k_i), i < t
//     Delta = T' (V - diag(gamma) X),  T' = (I + A)^-1 diag(beta),  X = K S0
//     O = diag(gamma) Q S0 + Bm Delta,  Bm[t][i] = R[t][i] (q_t.k_i), i <= t
//     S_C = gamma_{C-1} S0 + sum_i R[C-1][i] k_i delta_i^T.
// This is the same sum re-associated (fp32 tolerance against the token loop).
// The decay ratios are running products, never quotients, so decays that
// underflow give exact zeros rather than 0/0.
//
// Kernel A (one workgroup per (chunk, key head), all chunks in parallel):
// K K^T and Q K^T on fp32 MFMA (v_mfma_f32_16x16x4f32) once, then for each value
// head that reads this key head the ratios and T as a blocked inverse (16 x 16 diagonal blocks by forward substitution, the others
// as MFMA products) -> T', Bm, gamma, R[C-1][.] to the caller's workspace.
// Kernel B (one workgroup per (value head, 16 state columns), chunks in order,
// the workgroups of one head on one XCD):
// X = K S0 and Y = Q S0 (each wave one 16-token M-tile, K = 128 over 32 MFMA
// steps), Delta = T' (V - gamma X), O = gamma Y + Bm Delta, then the 128 x 16
// state block updated from K~^T Delta; the block lives in LDS between chunks
// and is read from / written to the state once per call.
#include <algorithm>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "gdn_common.hpp"

namespace qk {
namespace {

constexpr int kC = 64;                        // tokens per chunk
constexpr int kDK = 128;                      // key dim of the chunked path
constexpr int kNB = 16;                       // state columns per workgroup (kernel B)
constexpr int kThreads = 256;
constexpr int kXcds = 8;                      // gfx950: 8 XCDs, workgroups dealt round-robin
constexpr int kLdA = kC + 4;                  // LDS row stride of the C x C matrices (16-byte rows)
constexpr size_t kWsFloats = 2 * kC * kC + 2 * kC;   // per (chunk, head): T', Bm, gamma, R[C-1][.]

typedef float v4f_t __attribute__((ext_vector_type(4)));

// D[m][n] += sum over the instruction's 4 k-slots of A[m][k] B[k][n]: lane L
// supplies A[L%16][L/16] and B[L/16][L%16]; D lane L, element r is
// D[4(L/16) + r][L%16].
__device__ __forceinline__ v4f_t mfma4(float a, float b, v4f_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The 32 dims of a 128-dim row that lane group g supplies as MFMA k-slots:
// r[4j + c] = row[16j + 4g + c]. The four groups of a 16-lane column read 64
// contiguous bytes per load (the same token's row), so a wave's load touches
// 16 half-lines instead of 64 scattered 16-byte pieces. Zeros for a padding
// token; `row` is always a real row (callers clamp the token), so the loads
// are unconditional and the zeros are selected afterwards.
__device__ __forceinline__ void load32(const float* __restrict__ row, int g, bool valid, float (&r)[32]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 v = ld4(row + 16 * j + 4 * g);
        r[4 * j] = valid ? v.x : 0.0f;
        r[4 * j + 1] = valid ? v.y : 0.0f;
        r[4 * j + 2] = valid ? v.z : 0.0f;
        r[4 * j + 3] = valid ? v.w : 0.0f;
    }
}

__global__ __launch_bounds__(kThreads) void gdn_chunk_prep(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ beta,
                                                           const float* __restrict__ decay, float* __restrict__ ws,
                                                           int rows, int key_heads, int value_heads,
                                                           int64_t qkv_stride) {
    // The chunk's K rows while the products run; after them the same storage
    // holds A (strictly lower) and T of the value head in hand.
    __shared__ __align__(16) float kat[2 * kC * kLdA];
    static_assert(kC * (kDK + 4) <= 2 * kC * kLdA, "K rows fit the A and T storage");
    __shared__ __align__(16) float G[kC][kLdA];    // K K^T
    __shared__ __align__(16) float Pm[kC][kLdA];   // Q K^T
    __shared__ __align__(16) float sb[kC], sd[kC];
    float(*Kl)[kDK + 4] = reinterpret_cast<float(*)[kDK + 4]>(kat);
    float(*Ab)[kLdA] = reinterpret_cast<float(*)[kLdA]>(kat);
    float(*T)[kLdA] = reinterpret_cast<float(*)[kLdA]>(kat + kC * kLdA);
    const int c = blockIdx.x, src = blockIdx.y;   // chunk, key head
    const int t0 = c * kC;
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int g = lane >> 4, n = lane & 15;

    // beta and decay of token t0 + threadIdx.x (threads < kC) for value head h,
    // held in registers: the next head's are requested while this head's work
    // runs. Padding tokens: beta 0 (no update), decay 1.
    float bn = 0.0f, dn = 1.0f;
    auto load_gates = [&](int h) {
        const int t = t0 + threadIdx.x;
        if (threadIdx.x < kC && t < rows) {
            bn = beta[static_cast<int64_t>(t) * value_heads + h];
            dn = decay[static_cast<int64_t>(t) * value_heads + h];
        }
    };
    load_gates(src);

    // Lower-triangle 16x16 tiles (mt >= nt) of K K^T and Q K^T. Wave w loads
    // the K and Q rows of tokens 16w .. 16w+15 once (lane: token 16w + L%16,
    // dims 32(L/16) .. +31, the MFMA k-slot map of both operands) and puts its
    // K rows in LDS; Q K^T tiles (w, nt <= w) stay with wave w (its Q rows in
    // VGPRs), the K K^T tiles are dealt so that every wave has five tiles.
    {
        const int tok = t0 + 16 * wv + n;
        const int64_t row = static_cast<int64_t>(min(tok, rows - 1)) * qkv_stride + src * kDK;
        float kr[32], qr[32];
        load32(k + row, g, tok < rows, kr);
        load32(q + row, g, tok < rows, qr);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            *reinterpret_cast<float4*>(&Kl[16 * wv + n][16 * j + 4 * g]) =
                make_float4(kr[4 * j], kr[4 * j + 1], kr[4 * j + 2], kr[4 * j + 3]);
        __syncthreads();
        auto tile = [&](const float (&a)[32], int mt, int nt, float (*D)[kLdA]) {
            v4f_t acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float4 b = *reinterpret_cast<const float4*>(&Kl[16 * nt + n][16 * j + 4 * g]);
                acc[0] = mfma4(a[4 * j], b.x, acc[0]);
                acc[1] = mfma4(a[4 * j + 1], b.y, acc[1]);
                acc[2] = mfma4(a[4 * j + 2], b.z, acc[2]);
                acc[3] = mfma4(a[4 * j + 3], b.w, acc[3]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                D[16 * mt + 4 * g + r][16 * nt + n] = (acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]);
        };
        for (int nt = 0; nt <= wv; ++nt) tile(qr, wv, nt, Pm);
        // K K^T tiles (mt, nt), mt >= nt: wave w takes 4 - w of them, A rows from LDS.
        static constexpr int kTiles[10][2] = {{3, 0}, {3, 1}, {3, 2}, {3, 3}, {2, 0}, {2, 1}, {2, 2}, {1, 0}, {1, 1}, {0, 0}};
        const int first = wv == 0 ? 0 : wv == 1 ? 4 : wv == 2 ? 7 : 9;
        for (int i = first; i < first + 4 - wv; ++i) {
            const int mt = kTiles[i][0], nt = kTiles[i][1];
            float a[32];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float4 v = *reinterpret_cast<const float4*>(&Kl[16 * mt + n][16 * j + 4 * g]);
                a[4 * j] = v.x;
                a[4 * j + 1] = v.y;
                a[4 * j + 2] = v.z;
                a[4 * j + 3] = v.w;
            }
            tile(a, mt, nt, G);
        }
    }

    // The products depend on the key head only: every value head h with
    // h % key_heads == src (the heads that read this key head) takes them from
    // here, so K and Q are read and multiplied once per key head.
    for (int h = src; h < value_heads; h += key_heads) {
        float* wsc = ws + (static_cast<size_t>(c) * value_heads + h) * kWsFloats;
        float* Tp = wsc;
        float* Bm = wsc + kC * kC;
        float* gam = wsc + 2 * kC * kC;
        float* rr = gam + kC;
        __syncthreads();   // the products are done; the previous head's readers of sb, sd, A, T too
        if (threadIdx.x < kC) {
            sb[threadIdx.x] = bn;
            sd[threadIdx.x] = dn;
        }
        if (h + key_heads < value_heads) load_gates(h + key_heads);
        __syncthreads();

        // Rows 16wv .. 16wv+15 per wave, lane i = column i: R[t][i] as a running
        // product (the factor up to the wave's first row rebuilt from the decays,
        // the same multiplication sequence as one pass over all rows), A and Bm.
        // The decays are read once into registers (broadcast LDS reads) and the
        // products run over all 64 positions with the factors outside a lane's
        // range replaced by 1.0 (exact), so the chains are plain multiplies
        // without an LDS round trip per step.
        {
            const int i = lane;
            const int ta = 16 * wv;
            float dall[kC];
#pragma unroll
            for (int t = 0; t < kC; t += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(&sd[t]);
                dall[t] = v4.x;
                dall[t + 1] = v4.y;
                dall[t + 2] = v4.z;
                dall[t + 3] = v4.w;
            }
            float r = 1.0f;
#pragma unroll
            for (int t = 1; t < kC - 16; ++t) r *= (t > i && t < ta) ? dall[t] : 1.0f;
            float dv16[16], bv16[16], gv[16], pv[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                dv16[u] = sd[ta + u];
                bv16[u] = sb[ta + u];
                gv[u] = G[ta + u][i];
                pv[u] = Pm[ta + u][i];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int t = ta + u;
                if (t > i) r *= dv16[u];
                Ab[t][i] = t > i ? (bv16[u] * gv[u]) * r : 0.0f;
                Bm[t * kC + i] = t >= i ? pv[u] * r : 0.0f;
            }
            if (wv == 3) rr[i] = r;  // R[C-1][i]
            if (wv == 0) {  // gamma_t = d_0 * ... * d_t in order, lane t
                float gm = 1.0f;
#pragma unroll
                for (int t = 0; t < kC; ++t) gm *= t <= lane ? dall[t] : 1.0f;
                gam[lane] = gm;
            }
        }
        __syncthreads();

        // T = (I + A)^-1 in 16 x 16 blocks (A strictly lower). Diagonal blocks by
        // forward substitution, lane L = block L/16, column L%16:
        //   T_II[t][j] = [t == j] - sum_{i<t} A_II[t][i] T_II[i][j];
        // then block rows I = 1..3, wave J computing
        //   T_IJ = -T_II (sum_{K=J}^{I-1} A_IK T_KJ)
        // on MFMA. The 4 k-slots of the MFMAs of one 16-deep product map to
        // k = 4g + q (q the MFMA's index): A operands are 4 consecutive floats of a
        // row, and a result in the D layout (lane: rows 4g + r) is directly the B
        // operand of the next product.
        if (wv == 0) {
            const int I = lane >> 4, j = lane & 15;
            float tc[16];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                float acc[4] = {t == j ? 1.0f : 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int i4 = 0; i4 < t; i4 += 4) {
                    const float4 a = *reinterpret_cast<const float4*>(&Ab[16 * I + t][16 * I + i4]);
                    acc[0] = __builtin_fmaf(-a.x, tc[i4], acc[0]);
                    if (i4 + 1 < t) acc[1] = __builtin_fmaf(-a.y, tc[i4 + 1], acc[1]);
                    if (i4 + 2 < t) acc[2] = __builtin_fmaf(-a.z, tc[i4 + 2], acc[2]);
                    if (i4 + 3 < t) acc[3] = __builtin_fmaf(-a.w, tc[i4 + 3], acc[3]);
                }
                tc[t] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
                T[16 * I + t][16 * I + j] = tc[t];
            }
        }
        __syncthreads();
        // 16 x 16 x 16 product: acc += X[16xa rows][16xa cols] * Y, X rows from LDS at
        // (xr, xc), Y given as its D-layout registers (rows 4g + q, column n).
        auto prod_regs = [&](v4f_t acc, const float(*X)[kLdA], int xr, int xc, const v4f_t& y) {
            const float4 a = *reinterpret_cast<const float4*>(&X[xr + n][xc + 4 * g]);
            acc = mfma4(a.x, y[0], acc);
            acc = mfma4(a.y, y[1], acc);
            acc = mfma4(a.z, y[2], acc);
            return mfma4(a.w, y[3], acc);
        };
        for (int I = 1; I < 4; ++I) {
            if (wv < I) {
                const int J = wv;
                v4f_t m = {0.f, 0.f, 0.f, 0.f};
                for (int K = J; K < I; ++K) {
                    v4f_t tkj;  // T_KJ rows 4g + q, column n
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) tkj[q4] = T[16 * K + 4 * g + q4][16 * J + n];
                    m = prod_regs(m, Ab, 16 * I, 16 * K, tkj);
                }
                v4f_t t = prod_regs(v4f_t{0.f, 0.f, 0.f, 0.f}, T, 16 * I, 16 * I, m);
#pragma unroll
                for (int r = 0; r < 4; ++r) T[16 * I + 4 * g + r][16 * J + n] = -t[r];
            }
            __syncthreads();
        }
        // T' = T diag(beta), zeros above the diagonal.
        for (int e = threadIdx.x; e < kC * kC; e += kThreads) {
            const int t = e / kC, jj = e % kC;
            Tp[e] = t >= jj ? T[t][jj] * sb[jj] : 0.0f;
        }
    }
}

// One workgroup per CU (51 KB of LDS): one wave per SIMD, so the scheduler may
// keep every operand load of a chunk in flight.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gdn_chunk_state(float* __restrict__ S, const float* __restrict__ q,
                                                            const float* __restrict__ k, const float* __restrict__ v,
                                                            const float* __restrict__ ws, float* __restrict__ out,
                                                            int rows, int key_heads, int value_heads, int value_dim,
                                                            int64_t qkv_stride, int64_t out_stride) {
    // The tiles a lane reads as MFMA operands along their K dimension are stored
    // transposed ([column][row]), so those operands are consecutive floats: one
    // 16-byte LDS read per 4 operands and one wait before the products.
    __shared__ __align__(16) float KsT[kDK][kC + 4];  // the chunk's R[C-1][t] k_t, [key][token]
    __shared__ __align__(16) float RvT[kNB][kC + 4];  // V - gamma X, [column][token]
    __shared__ __align__(16) float DlT[kNB][kC + 4];  // Delta, [column][token]
    __shared__ __align__(16) float SlT[kNB][kDK + 4]; // this block's 128 x 16 state, [column][key]
    // Workgroup i runs on XCD i % 8 (round-robin dispatch). With the value
    // heads a multiple of 8, head h's column blocks all get ids i with
    // i % 8 == h % 8, so the chunk data of a head (K, Q, T', Bm, V) is fetched
    // into one XCD's L2 instead of every XCD's.
    const int ncb = value_dim / kNB;
    int h, cb;
    if (value_heads % kXcds == 0) {
        const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
        h = x + kXcds * (j / ncb);
        cb = j % ncb;
    } else {
        h = blockIdx.x / ncb;
        cb = blockIdx.x % ncb;
    }
    const int j0 = cb * kNB;
    const int src = h % key_heads;
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int g = lane >> 4, n = lane & 15;
    float* Sg = S + static_cast<size_t>(h) * kDK * value_dim + j0;

    for (int e = threadIdx.x; e < kDK * kNB; e += kThreads)
        SlT[e % kNB][e / kNB] = Sg[static_cast<size_t>(e / kNB) * value_dim + e % kNB];
    __syncthreads();

    // Per-chunk inputs of this lane, each reloaded for the next chunk as soon as
    // it is dead in the current one (the state-free loads overlap the chain of
    // MFMAs that the state forces).
    const int nchunks = (rows + kC - 1) / kC;
    const int tok = 16 * wv + n;   // token row of this lane's A operands
    const int tres = 16 * wv + 4 * g;   // first of the 4 token rows of this lane's results
    float kA[32], qA[32], kB[32], qB[32], vv[4], gm[4], glast, gm_n[4], glast_n;
    float4 tpr[4], bmr[4];
    float rt, rt_n;   // R[C-1][tok]: the K rows go to LDS already scaled by it
    auto chunk_base = [&](int c) { return ws + (static_cast<size_t>(c) * value_heads + h) * kWsFloats; };
    // Padding tokens of the last chunk read the last real row and are not
    // zeroed: the prep kernel gives them beta 0 and decay 1, so their rows and
    // columns of T' are zero, their Delta is exactly 0 (0 times finite values)
    // and they add nothing to the state; their outputs are not stored. Keeping
    // the loaded values raw also keeps the prefetches asynchronous (a select on
    // a loaded value would wait for the load right away).
    // k-slot map of every product here: step 4j + c of a 4-wide group g takes
    // element 16j + 4g + c of the contracted dimension (dims of K / Q, tokens
    // of T', Bm and R), so each 4 lanes of a row read 64 contiguous bytes.
    // K and Q rows of chunk c, dims 16j + 4g .. + 3 (one 16-byte load each)
    auto load_kq_j = [&](int c, int j, float (&kd)[32], float (&qd)[32]) {
        const int t = min(c * kC + tok, rows - 1);
        const float* kr = k + static_cast<int64_t>(t) * qkv_stride + src * kDK + 4 * g;
        const float* qr = q + static_cast<int64_t>(t) * qkv_stride + src * kDK + 4 * g;
        const float4 a = ld4(kr + 16 * j), b = ld4(qr + 16 * j);
        kd[4 * j] = a.x;
        kd[4 * j + 1] = a.y;
        kd[4 * j + 2] = a.z;
        kd[4 * j + 3] = a.w;
        qd[4 * j] = b.x;
        qd[4 * j + 1] = b.y;
        qd[4 * j + 2] = b.z;
        qd[4 * j + 3] = b.w;
    };
    auto load_v = [&](int c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = min(c * kC + tres + r, rows - 1);
            vv[r] = v[static_cast<int64_t>(t) * qkv_stride + static_cast<size_t>(h) * value_dim + j0 + n];
        }
    };
    auto load_gam = [&](int c, float (&g4)[4], float& gl) {
        const float4 gv = ld4(chunk_base(c) + 2 * kC * kC + tres);
        g4[0] = gv.x;
        g4[1] = gv.y;
        g4[2] = gv.z;
        g4[3] = gv.w;
        // gamma_{C-1} through a vector load: its address is wave-uniform, and as
        // a scalar load it would share lgkmcnt with the LDS traffic, so every
        // LDS wait would also wait for it (scalar loads return out of order).
        // lane & (rows >> 31) is 0 (rows > 0) but not known to the compiler to
        // be uniform, which keeps the load on the vector path.
        gl = chunk_base(c)[2 * kC * kC + kC - 1 + (lane & (rows >> 31))];
    };
    // elements 16s + 4g .. 16s + 4g + 3 (s < 4) of a 64-long row: p = row + 4g
    auto load_rows16 = [&](float4 (&dst)[4], const float* p) {
#pragma unroll
        for (int s = 0; s < 4; ++s) dst[s] = ld4(p + 16 * s);
    };
    // the same 16 elements of an LDS row (p = row + 4g), as 4 x 16-byte reads
    auto lds16 = [](float (&dst)[16], const float* p) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float4 t = *reinterpret_cast<const float4*>(p + 16 * s);
            dst[4 * s] = t.x;
            dst[4 * s + 1] = t.y;
            dst[4 * s + 2] = t.z;
            dst[4 * s + 3] = t.w;
        }
    };
    // T' and Bm rows 16wv + n at this lane's k-slot columns; R[C-1] at token tok.
    auto tp_row = [&](int c) { return chunk_base(c) + (16 * wv + n) * kC + 4 * g; };
    auto bm_row = [&](int c) { return chunk_base(c) + kC * kC + (16 * wv + n) * kC + 4 * g; };
    auto rr_tok = [&](int c) { return chunk_base(c)[2 * kC * kC + kC + tok]; };
    // the loop's load order (the wait counts at its head then line up)
#pragma unroll
    for (int j = 0; j < 8; ++j) load_kq_j(0, j, kA, qA);
    load_v(0);
    load_rows16(tpr, tp_row(0));
    load_rows16(bmr, bm_row(0));
    load_gam(0, gm, glast);
    rt = rr_tok(0);

    // Chunk c with its K and Q rows in kc / qc; chunk c + 1's are loaded into
    // kn / qn during c's X and Y products (the loop runs two chunks per pass
    // with the two register sets swapped, so nothing is copied).
    auto chunk_step = [&](int c, float (&kc)[32], float (&qc)[32], float (&kn)[32], float (&qn)[32])
                          __attribute__((always_inline)) {
        const int t0 = c * kC;
        // Inputs of chunk cn are prefetched during this chunk (the last chunk
        // reloads its own; unconditional loads keep the wait counts exact).
        const int cn = min(c + 1, nchunks - 1);

        // S0 as the B operand (rows 16j + 4g + c, column n) and at this wave's
        // rows of the state update's result tiles (32wv + 16mt + 4g + r).
        float sB[32];
        float4 sC[2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 t = *reinterpret_cast<const float4*>(&SlT[n][16 * j + 4 * g]);
            sB[4 * j] = t.x;
            sB[4 * j + 1] = t.y;
            sB[4 * j + 2] = t.z;
            sB[4 * j + 3] = t.w;
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) sC[mt] = *reinterpret_cast<const float4*>(&SlT[n][32 * wv + 16 * mt + 4 * g]);

#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) KsT[16 * j + 4 * g + c][tok] = kc[4 * j + c] * rt;
        v4f_t xa[4], ya[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xa[u] = ya[u] = v4f_t{0.f, 0.f, 0.f, 0.f};
        // The next chunk's 16 row loads go out between the products, two per 8
        // MFMAs: issued in one burst they held the wave ~1000 cycles at a point
        // where the chunk's chain waits on it.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            if ((s & 3) == 0) load_kq_j(cn, s >> 2, kn, qn);
            xa[s & 3] = mfma4(kc[s], sB[s], xa[s & 3]);
            ya[s & 3] = mfma4(qc[s], sB[s], ya[s & 3]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);   // 2 VMEM reads
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);   // 8 MFMAs
        }
        __builtin_amdgcn_sched_barrier(0);
        const v4f_t X = (xa[0] + xa[1]) + (xa[2] + xa[3]);
        const v4f_t Y = (ya[0] + ya[1]) + (ya[2] + ya[3]);
        // gamma and R[C-1] of the next chunk a whole chunk ahead, into their
        // own registers (requested at the end of the chunk they came back
        // ~2000 cycles after the next chunk's Rv needed them)
        load_gam(cn, gm_n, glast_n);
        rt_n = rr_tok(cn);

        // Result rows: tokens 16wv + 4g + r, column n.
        *reinterpret_cast<float4*>(&RvT[n][tres]) =
            make_float4(vv[0] - gm[0] * X[0], vv[1] - gm[1] * X[1], vv[2] - gm[2] * X[2], vv[3] - gm[3] * X[3]);
        load_v(cn);
        __syncthreads();

        // Delta = T' Rv (this wave's 16 rows; K = the chunk's 64 tokens).
        float rb[16];
        lds16(rb, &RvT[n][4 * g]);
        v4f_t D0 = {0.f, 0.f, 0.f, 0.f}, D1 = D0;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            D0 = mfma4(tpr[s].x, rb[4 * s], D0);
            D1 = mfma4(tpr[s].y, rb[4 * s + 1], D1);
            D0 = mfma4(tpr[s].z, rb[4 * s + 2], D0);
            D1 = mfma4(tpr[s].w, rb[4 * s + 3], D1);
        }
        load_rows16(tpr, tp_row(cn));
        *reinterpret_cast<float4*>(&DlT[n][tres]) = make_float4(D0[0] + D1[0], D0[1] + D1[1], D0[2] + D1[2],
                                                                 D0[3] + D1[3]);
        __syncthreads();

        // O = gamma Y + Bm Delta.
        float db[16];   // Delta rows 16s + 4g + c, column n (also the state update's B operands)
        lds16(db, &DlT[n][4 * g]);
        v4f_t O0 = {gm[0] * Y[0], gm[1] * Y[1], gm[2] * Y[2], gm[3] * Y[3]}, O1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            O0 = mfma4(bmr[s].x, db[4 * s], O0);
            O1 = mfma4(bmr[s].y, db[4 * s + 1], O1);
            O0 = mfma4(bmr[s].z, db[4 * s + 2], O0);
            O1 = mfma4(bmr[s].w, db[4 * s + 3], O1);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + tres + r;
            if (t < rows)
                out[static_cast<int64_t>(t) * out_stride + static_cast<size_t>(h) * value_dim + j0 + n] = O0[r] + O1[r];
        }
        load_rows16(bmr, bm_row(cn));

        // S rows 32wv + 16mt + (0..15): gamma_{C-1} S0 + sum_t R[C-1][t] k_t Delta_t
        // (step 4s + c: token 16s + 4g + c).
        v4f_t A0 = {0.f, 0.f, 0.f, 0.f}, A1 = A0;
        const int m0 = 32 * wv + n;
        float ka[16], kb[16];
        lds16(ka, &KsT[m0][4 * g]);
        lds16(kb, &KsT[m0 + 16][4 * g]);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            A0 = mfma4(ka[s], db[s], A0);   // KsT holds R[C-1][t] k_t (the same product)
            A1 = mfma4(kb[s], db[s], A1);
        }
        float4 sn[2];
        sn[0] = make_float4(__builtin_fmaf(glast, sC[0].x, A0[0]), __builtin_fmaf(glast, sC[0].y, A0[1]),
                            __builtin_fmaf(glast, sC[0].z, A0[2]), __builtin_fmaf(glast, sC[0].w, A0[3]));
        sn[1] = make_float4(__builtin_fmaf(glast, sC[1].x, A1[0]), __builtin_fmaf(glast, sC[1].y, A1[1]),
                            __builtin_fmaf(glast, sC[1].z, A1[2]), __builtin_fmaf(glast, sC[1].w, A1[3]));
        // gamma and R[C-1] are dead for this chunk from here on
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            gm[r] = gm_n[r];
        }
        glast = glast_n;
        rt = rt_n;
        __syncthreads();  // every wave is done reading SlT, KsT, DlT of this chunk
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) *reinterpret_cast<float4*>(&SlT[n][32 * wv + 16 * mt + 4 * g]) = sn[mt];
        __syncthreads();
    };
    for (int c = 0; c < nchunks; c += 2) {
        chunk_step(c, kA, qA, kB, qB);
        if (c + 1 < nchunks) chunk_step(c + 1, kB, qB, kA, qA);
    }

    for (int e = threadIdx.x; e < kDK * kNB; e += kThreads)
        Sg[static_cast<size_t>(e / kNB) * value_dim + e % kNB] = SlT[e % kNB][e / kNB];
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

size_t qwen_gdn_recurrent_chunked_workspace_bytes(int rows, int value_heads) {
    if (rows <= 0 || value_heads <= 0) return 0;
    return static_cast<size_t>((rows + kC - 1) / kC) * value_heads * kWsFloats * sizeof(float);
}

int qwen_gdn_recurrent_chunked(float* state, const float* q, const float* k, const float* v, const float* beta,
                               const float* decay, float* out, int rows, int key_heads, int value_heads,
                               int key_dim, int value_dim, int64_t qkv_stride, int64_t out_stride, void* workspace,
                               size_t workspace_bytes, void* stream) {
    // The same limit as the token loop, checked before the path is chosen, so
    // the status does not depend on which path a call's alignment selects.
    QK_REQUIRE(value_dim <= kMaxValueDim, "GDN value dimension exceeds kernel limit");
    const bool chunked = key_dim == kDK && value_dim > 0 && value_dim % kNB == 0 && aligned16(q) && aligned16(k) &&
                         aligned16(workspace) && qkv_stride % 4 == 0 && rows > 0 && key_heads > 0 &&
                         value_heads > 0;
    if (!chunked)  // shapes outside the chunked kernels: the token loop, no workspace
        return qwen_gdn_recurrent_rows(state, q, k, v, beta, decay, out, rows, key_heads, value_heads, key_dim,
                                       value_dim, qkv_stride, out_stride, stream);
    QK_REQUIRE(state && v && beta && decay && out, "gdn_recurrent_chunked: null pointer");
    QK_REQUIRE(rows == 1 || (qkv_stride > 0 && out_stride > 0), "gdn_recurrent_chunked: non-positive row stride");
    const size_t need = qwen_gdn_recurrent_chunked_workspace_bytes(rows, value_heads);
    QK_REQUIRE(workspace_bytes >= need, "gdn_recurrent_chunked: workspace of %zu bytes, %zu needed", workspace_bytes,
               need);
    const hipStream_t s = as_stream(stream);
    const int nchunks = (rows + kC - 1) / kC;
    float* ws = static_cast<float*>(workspace);
    gdn_chunk_prep<<<dim3(nchunks, std::min(key_heads, value_heads)), kThreads, 0, s>>>(q, k, beta, decay, ws, rows, key_heads, value_heads,
                                                                   qkv_stride);
    gdn_chunk_state<<<(value_dim / kNB) * value_heads, kThreads, 0, s>>>(state, q, k, v, ws, out, rows, key_heads,
                                                                         value_heads, value_dim, qkv_stride,
                                                                         out_stride);
    return check_launch("gdn_recurrent_chunked");
}

}  // extern "C"
