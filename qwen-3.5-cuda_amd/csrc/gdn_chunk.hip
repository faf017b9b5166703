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
// Kernel A (one workgroup per (chunk, key head), all chunks in parallel): the
// chunk's K and Q as fp16 pairs (below), K K^T and Q K^T from them once, then
// for each value head that reads this key head the ratios and T as a blocked
// inverse (16 x 16 diagonal blocks by forward substitution, the others as fp32
// MFMA products) -> T', Bm, gamma, R[C-1][.] and the K / Q pairs to the
// caller's workspace.
// Kernel B (one 8-wave workgroup per (value head, 16 state columns), chunks in
// order, the workgroups of one head on one XCD): per SIMD a Q wave computing
// Y = Q S0 and O = gamma Y + Bm Delta for 16 tokens, and a K wave computing
// X = K S0, Delta = T' (V - gamma X) for the same tokens and 32 rows of the state
// update S_C = gamma_{C-1} S0 + K^T (R[C-1] Delta); the K waves hold the
// 128 x 16 state block in registers between chunks (read from / written to the
// state once per call) and publish it to the other waves through LDS.
//
// fp16 pairs. The products with a long sum (K K^T, Q K^T, X and Y over the 128
// key dims, the state update over the chunk's 64 tokens) run on v_mfma_f32_16x16x32_f16:
// it sums 32 terms per lane group where v_mfma_f32_16x16x4f32 sums 4, in ~22
// cycles against ~35 (measured on gfx950), and a SIMD's MFMA time is not hidden
// behind its other work. An fp32 operand x is scaled by 2^e (e chosen per block
// from the block's largest |x| or a bound on it, so that the largest lands in
// [2^14, 2^15)) and held as hi = fp16(x 2^e), lo = fp16(x 2^e - hi); a product is
// hi lo' + lo hi' + hi hi' (fp16 products are exact in fp32), accumulated in
// fp32 and scaled back exactly by ldexp(., -(e + e')). The dropped lo lo' and
// the two roundings are below ~2^-21 of each term, under the fp32 token loop's
// own rounding at these sums; elements below ~2^-38 of their block's scale
// fall into fp16's subnormals and lose their low bits (a scale multiplier
// 2^-(e + e') held as a float, e clamped to keep it normal, lost a strongly
// decayed head's whole state of ~1e-23 this way). The Delta and O products
// (the triangular 16-token blocks) stay fp32.
#include <algorithm>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "gdn_common.hpp"

namespace qk {
namespace {

constexpr int kC = 64;                        // tokens per chunk
constexpr int kDK = 128;                      // key dim of the chunked path
constexpr int kNB = 16;                       // state columns per workgroup (kernel B)
constexpr int kThreads = 256;                 // prep
constexpr int kWalkThreads = 512;             // state walk: two waves per SIMD
constexpr int64_t kMaxWalkStride = 0x7fffffff / (4 * 64);   // floats; 64 rows of 4-byte elements below 2^31 bytes
constexpr int kXcds = 8;                      // gfx950: 8 XCDs, workgroups dealt round-robin
constexpr int kLdA = kC + 4;                  // LDS row stride of the C x C matrices (16-byte rows)
// Per (chunk, value head): T', Bm, gamma, R[C-1][.], then {gamma_{C-1}, eK, eQ, rho}
// (eK, eQ: int bits)
// (rho bounds |R[C-1][t] Delta[t][j]| / max_i |(V - gamma X)[i][j]|).
constexpr int kWsExtra = 2 * kC * kC + 2 * kC;
constexpr size_t kWsFloats = kWsExtra + 4;
// Per (chunk, key head), after all the value-head blocks: fp16 pairs of K and
// Q by token (layout at the prep's stores).
constexpr uint32_t kKRows = 0, kQRows = kC * kDK * 4;
constexpr size_t kKqBytes = 2 * kC * kDK * 4;
constexpr int kKtLd = kDK + 16;               // LDS row of the walk's K copy: 288 bytes (transposed reads without bank conflicts)

typedef float v4f_t __attribute__((ext_vector_type(4)));
typedef unsigned u4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

// D[m][n] += sum over the instruction's 4 k-slots of A[m][k] B[k][n]: lane L
// supplies A[L%16][L/16] and B[L/16][L%16]; D lane L, element r is
// D[4(L/16) + r][L%16].
__device__ __forceinline__ v4f_t mfma4(float a, float b, v4f_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// The same over 32 k-slots: lane L supplies 8 fp16 values, A[L%16][8(L/16) + s]
// and B[8(L/16) + s][L%16] (s < 8); D as above. Only the pairing matters here:
// slot s of lane group g means the same k in both operands.
__device__ __forceinline__ v4f_t mfma16(u4_t a, u4_t b, v4f_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0,
                                                  0);
}

// 2^e puts m (>= 0, finite) in [2^14, 2^15): m = f 2^E with f in [0.5, 1),
// e = 15 - E (fp32 subnormals included); 15 for m = 0.
__device__ __forceinline__ int scale_exp(float m) { return 15 - __builtin_amdgcn_frexp_expf(m); }
// (a, b) 2^e as fp16 pairs: hi rounded to nearest, lo the rest rounded to nearest.
__device__ __forceinline__ void split2(float a, float b, int e, unsigned& hi, unsigned& lo) {
    const f2_t s = {__builtin_amdgcn_ldexpf(a, e), __builtin_amdgcn_ldexpf(b, e)};
    const h2_t h = __builtin_convertvector(s, h2_t);
    const f2_t h32 = __builtin_convertvector(h, f2_t);
    const f2_t r = {s.x - h32.x, s.y - h32.y};
    hi = __builtin_bit_cast(unsigned, h);
    lo = __builtin_bit_cast(unsigned, __builtin_convertvector(r, h2_t));
}
__device__ __forceinline__ void split8(const float* x, int e, u4_t& hi, u4_t& lo) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        unsigned h, l;
        split2(x[2 * p], x[2 * p + 1], e, h, l);
        hi[p] = h;
        lo[p] = l;
    }
}
// T' and Bm are stored in the walk's fragment order, each 64 x 64 matrix as 16
// pieces of 1 KB [row tile][column block s][lane] x 4 floats, lane (n, g)
// holding row 16 tile + n, columns 16s + 4g .. + 3: one wave instruction reads
// one piece. Index (in float4 units) of row 16 tile + 0 at column j.
__host__ __device__ __forceinline__ int frag_index(int tile, int j) {
    return (tile * 4 + (j >> 4)) * 64 + ((j >> 2) & 3) * 16;
}
// max over lanes L, L^16, L^32, L^48 (the four lane groups of a column)
__device__ __forceinline__ float max_groups(float x) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
// max over all 64 lanes
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
    return max_groups(x);
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
                                                           unsigned char* __restrict__ kq, int rows, int key_heads,
                                                           int value_heads, int64_t qkv_stride) {
    // The chunk's K as fp16 pairs while the products run; after them the same
    // storage holds A (strictly lower) and T of the value head in hand.
    __shared__ __align__(16) float kat[2 * kC * kLdA];
    __shared__ __align__(16) float G[kC][kLdA];    // K K^T
    __shared__ __align__(16) float Pm[kC][kLdA];   // Q K^T
    __shared__ __align__(16) float sb[kC], sd[kC];
    __shared__ float smax[2][4];                   // per wave: max |K|, max |Q| over its rows
    __shared__ float stmax[4];                     // per wave: largest |R[C-1][t]| sum_i |T'[t][i]|
    __shared__ float sR[kC];                       // |R[C-1][t]|
    __shared__ float sglast;                       // gamma_{C-1}
    float(*Ab)[kLdA] = reinterpret_cast<float(*)[kLdA]>(kat);
    float(*T)[kLdA] = reinterpret_cast<float(*)[kLdA]>(kat + kC * kLdA);
    const int c = blockIdx.x, src = blockIdx.y;   // chunk, key head
    const int t0 = c * kC;
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int g = lane >> 4, n = lane & 15;
    // src < min(key_heads, value_heads): the blocks are sized per value head
    unsigned char* const kqb = kq + (static_cast<size_t>(c) * value_heads + src) * kKqBytes;
    int eK, eQ;

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
    // dims 32(L/16) .. +31), splits them into fp16 pairs (one scale exponent per
    // chunk tile, from the tile's largest |K| or |Q|) and puts its K pairs in
    // LDS; the products run on v_mfma_f32_16x16x32_f16, hi lo' + lo hi' + hi hi'
    // per k-block of 32 dims (a quarter of the fp32 MFMA time: they were a third
    // of the kernel's). Q K^T tiles (w, nt <= w) stay with wave w (its Q pairs in
    // VGPRs), the K K^T tiles are dealt so that every wave has five tiles.
    {
        const int tok = t0 + 16 * wv + n;
        const int64_t row = static_cast<int64_t>(min(tok, rows - 1)) * qkv_stride + src * kDK;
        float kr[32], qr[32];
        load32(k + row, g, tok < rows, kr);
        load32(q + row, g, tok < rows, qr);
        float mk = 0.0f, mq = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            mk = fmaxf(mk, fabsf(kr[i]));
            mq = fmaxf(mq, fabsf(qr[i]));
        }
        mk = wave_max(mk);
        mq = wave_max(mq);
        if (lane == 0) {
            smax[0][wv] = mk;
            smax[1][wv] = mq;
        }
        __syncthreads();
        eK = scale_exp(fmaxf(fmaxf(smax[0][0], smax[0][1]), fmaxf(smax[0][2], smax[0][3])));
        eQ = scale_exp(fmaxf(fmaxf(smax[1][0], smax[1][1]), fmaxf(smax[1][2], smax[1][3])));
        // K and Q by token (the walk's X and Y operands, and this kernel's) in the
        // order the walk's lanes read them: 1 KB fragments [tile wv][2 kb + (hi, lo)]
        // [lane] x 8 fp16, lane (n, g) = token 16wv + n, slot 4h + c of k-block kb =
        // dim 32kb + 16h + 4g + c, which is this lane's kr[8kb + 4h + c]. One wave
        // instruction then reads 1 KB in one piece (16 rows of 64 bytes cost the
        // CU about twice as long, measured). Padding tokens are zeros.
        u4_t* const KF = reinterpret_cast<u4_t*>(kat);   // [tile][2 kb + (hi, lo)][lane]
        static_assert(4 * 8 * 64 * sizeof(u4_t) <= sizeof(kat), "K pairs fit the A and T storage");
        u4_t qf[8];
        {
            unsigned char* const rk = kqb + kKRows + (wv * 8 * 64 + lane) * 16;
            unsigned char* const rq = kqb + kQRows + (wv * 8 * 64 + lane) * 16;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                u4_t hi, lo;
                split8(kr + 8 * kb, eK, hi, lo);
                *reinterpret_cast<u4_t*>(rk + 2048 * kb) = hi;
                *reinterpret_cast<u4_t*>(rk + 2048 * kb + 1024) = lo;
                KF[(wv * 8 + 2 * kb) * 64 + lane] = hi;
                KF[(wv * 8 + 2 * kb + 1) * 64 + lane] = lo;
                split8(qr + 8 * kb, eQ, qf[2 * kb], qf[2 * kb + 1]);
                *reinterpret_cast<u4_t*>(rq + 2048 * kb) = qf[2 * kb];
                *reinterpret_cast<u4_t*>(rq + 2048 * kb + 1024) = qf[2 * kb + 1];
            }
        }
        __syncthreads();   // every tile's K pairs in LDS
        // The B operand of a tile with column tile nt is K's fragments of that tile
        // (B[k][n] = K[16nt + n][k]: the same lane map as the A fragments).
        auto tile = [&](const u4_t (&a)[8], int mt, int nt, int e, float (*D)[kLdA]) {
            v4f_t acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const u4_t bh = KF[(nt * 8 + 2 * kb) * 64 + lane], bl = KF[(nt * 8 + 2 * kb + 1) * 64 + lane];
                acc[kb] = mfma16(a[2 * kb], bl, acc[kb]);
                acc[kb] = mfma16(a[2 * kb + 1], bh, acc[kb]);
                acc[kb] = mfma16(a[2 * kb], bh, acc[kb]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                D[16 * mt + 4 * g + r][16 * nt + n] =
                    __builtin_amdgcn_ldexpf((acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]), -e);
        };
        for (int nt = 0; nt <= wv; ++nt) tile(qf, wv, nt, eQ + eK, Pm);
        // K K^T tiles (mt, nt), mt >= nt: wave w takes 4 - w of them, A pairs from LDS.
        static constexpr int kTiles[10][2] = {{3, 0}, {3, 1}, {3, 2}, {3, 3}, {2, 0}, {2, 1}, {2, 2}, {1, 0}, {1, 1}, {0, 0}};
        const int first = wv == 0 ? 0 : wv == 1 ? 4 : wv == 2 ? 7 : 9;
        for (int i = first; i < first + 4 - wv; ++i) {
            const int mt = kTiles[i][0], nt = kTiles[i][1];
            u4_t af[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) af[j] = KF[(mt * 8 + j) * 64 + lane];
            tile(af, mt, nt, 2 * eK, G);
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
        // The decays come four at a time from broadcast LDS reads, and the factors
        // outside a lane's range are replaced by 1.0 (exact), so every lane runs
        // the same plain multiplies. (Held as 64 registers for a fully unrolled
        // chain, with its 47 lane masks spilled from SGPRs into VGPR lanes, the
        // prep took 4.6% longer.)
        {
            // The lane index is made opaque per value head so the lane masks of the
            // row loop (t > i, t >= i) and of gamma's unrolled chain (t <= i) are
            // compared where they are used: hoisted out of the value-head loop they
            // were kept in SGPRs spilled to VGPR lanes, a reload per use (4.4% of the
            // prep, no SGPR spills left).
            int i = lane;
            asm volatile("" : "+v"(i));
            const int ta = 16 * wv;
            // the factor up to the wave's first row: d_t for i < t < ta, in order
            float r = 1.0f;
            for (int t4 = 0; t4 < ta; t4 += 4) {   // wave-uniform trip count
                const float4 d4 = *reinterpret_cast<const float4*>(&sd[t4]);
                r *= t4 > i ? d4.x : 1.0f;
                r *= t4 + 1 > i ? d4.y : 1.0f;
                r *= t4 + 2 > i ? d4.z : 1.0f;
                r *= t4 + 3 > i ? d4.w : 1.0f;
            }
            float dv16[16], bv16[16], gv[16], pv[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                dv16[u] = sd[ta + u];
                bv16[u] = sb[ta + u];
                gv[u] = G[ta + u][i];
                pv[u] = Pm[ta + u][i];
            }
            // Bm[t][i] at the walk's fragment position of row t = 16wv + u, column i
            float* const bmi = Bm + frag_index(wv, i) * 4 + (i & 3);
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int t = ta + u;
                if (t > i) r *= dv16[u];
                Ab[t][i] = t > i ? (bv16[u] * gv[u]) * r : 0.0f;
                bmi[4 * u] = t >= i ? pv[u] * r : 0.0f;
            }
            if (wv == 3) {  // R[C-1][i]
                rr[i] = r;
                sR[i] = fabsf(r);
            }
            if (wv == 0) {  // gamma_t = d_0 * ... * d_t in order, lane t
                float gm = 1.0f;
                for (int t4 = 0; t4 < kC; t4 += 4) {
                    const float4 d4 = *reinterpret_cast<const float4*>(&sd[t4]);
                    gm *= t4 <= i ? d4.x : 1.0f;
                    gm *= t4 + 1 <= i ? d4.y : 1.0f;
                    gm *= t4 + 2 <= i ? d4.z : 1.0f;
                    gm *= t4 + 3 <= i ? d4.w : 1.0f;
                }
                gam[lane] = gm;
                if (lane == kC - 1) sglast = gm;
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
        // T' = T diag(beta), zeros above the diagonal; 4 columns per thread
        // (a 16-byte LDS read and store each instead of four 4-byte ones: the
        // recurrence over 4096 tokens 251 -> 245 us).
        // The 16 threads of a row are 16 consecutive lanes: their |T'| sums add
        // within the lane group, and each thread keeps the largest row sum times
        // |R[C-1][t]| it saw (the same token's factors: pairing the largest of each
        // over different tokens overstated the bound by up to ~1e9 for strongly
        // decayed heads, whose R[C-1] Delta then fell into fp16's subnormals).
        float rowmax = 0.0f;
        for (int e = threadIdx.x; e < kC * kC / 4; e += kThreads) {
            const int t = e / (kC / 4), j4 = 4 * (e % (kC / 4));
            const float4 tv = *reinterpret_cast<const float4*>(&T[t][j4]);
            const float4 bv = *reinterpret_cast<const float4*>(&sb[j4]);
            const float4 tp = make_float4(t >= j4 ? tv.x * bv.x : 0.0f, t >= j4 + 1 ? tv.y * bv.y : 0.0f,
                                          t >= j4 + 2 ? tv.z * bv.z : 0.0f, t >= j4 + 3 ? tv.w * bv.w : 0.0f);
            *reinterpret_cast<float4*>(Tp + (frag_index(t >> 4, j4) + (t & 15)) * 4) = tp;
            const float part = (fabsf(tp.x) + fabsf(tp.y)) + (fabsf(tp.z) + fabsf(tp.w));
            rowmax = fmaxf(rowmax, group_sum<16>(part) * sR[t]);
        }
        rowmax = wave_max(rowmax);
        if (lane == 0) stmax[wv] = rowmax;
        __syncthreads();
        // |R[C-1][t] Delta[t][j]| <= |R[C-1][t]| sum_i |T'[t][i]| max_i |(V - gamma X)[i][j]|
        if (threadIdx.x == 0)
            *reinterpret_cast<float4*>(wsc + kWsExtra) =
                make_float4(sglast, __int_as_float(eK), __int_as_float(eQ),
                            fmaxf(fmaxf(stmax[0], stmax[1]), fmaxf(stmax[2], stmax[3])));
    }
}

// ---------------------------------------------------------------- state walk
// Raw buffer access for the walk: a wave-uniform descriptor (base, byte range)
// and a loop-invariant 32-bit lane offset, so a load costs no address
// arithmetic on the vector ALU. A SIMD's vector-ALU and MFMA work do not
// overlap, even from different waves (one wave streaming fp32 MFMAs beside one
// running FMAs takes the sum of their times, measured), so every VALU
// instruction adds to the chunk's time; per-load 64-bit address arithmetic was
// most of the walk's VALU work. Loads at or past the range return 0 and
// stores there are dropped: the padding tokens of a partial last chunk read
// zeros (finite; their beta 0 and decay 1 give them zero rows and columns of
// T' and zero rows of Bm, so they add nothing) and their outputs are not written.
// Descriptor: stride 0 (raw, the range counted in bytes), dword 3 = 0x00020000
// (gfx9 DATA_FORMAT field = 4, 32-bit elements; no swizzle, no index stride).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ u4_t buf_ld4u(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// The 16-byte load is reinterpreted whole: taking its result apart element by
// element compiled to a 4-byte load on this compiler.
__device__ __forceinline__ float4 buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float buf_ld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void buf_st1(float x, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), r, off, 0, 0);
}

// Per-chunk inputs a lane holds, loaded one chunk ahead (two sets, swapped by
// the loop's two chunk steps, so nothing is copied).
struct ChunkIn {
    u4_t a[8];        // K (K waves) or Q (Q waves) by token as fp16 pairs: a[2 kb + (0 hi, 1 lo)]
    float o[4];       // this chunk's outputs (Q waves), stored during the next chunk
};

// One workgroup per (value head, 16 state columns), 8 waves, two per SIMD:
// the K wave of SIMD w (wave w + 4) computes X = K S0 for tokens 16w..16w+15,
// V - gamma X, Delta and state rows 32w..32w+31; the Q wave (wave w) computes
// Y = Q S0 for the same tokens and O. Each SIMD so runs two instruction streams
// whose stalls the other fills. The older wave of a SIMD wins its issue
// arbitration: with the Q waves first, the K waves' LDS writes and loads at the
// start of a chunk run while the Q waves' products hold the matrix pipe (the
// other order measured 5% slower). The role branches hold
// no loads that the other role's code reads, and every path back to the loop
// head issues both chunks' loads, which keeps the compiler's memory-wait counts
// tight (a branch that skipped the second chunk, or one register set loaded at
// different points by the two roles, turned them into full drains).
//
// Operand pairing of the fp16 products (slot s = 4h + r of lane group g):
//   X, Y: k-block kb (32 key dims, the state rows of K wave kb), slot -> key
//         32kb + 16h + 4g + r; the state's fp16 pairs for kb are exactly what
//         lane (n, g) of K wave kb holds (rows 32kb + 16mt + 4g + r, mt = h).
//   state update: k-block kb (32 tokens), slot -> token 32kb + 16h + 4g + r;
//         the R[C-1] Delta pairs are what lane (n, g) of K wave 2kb + h holds.
// So the fp16 pairs of the state and of R[C-1] Delta move through LDS lane to
// same lane. The state update's other operand, K by key, is the K waves' own
// K by token copied to LDS and read back with ds_read_b64_tr_b16 (gfx950's
// transposing LDS read): in each 16-lane group lane j points at 4 consecutive
// key dims of token t_{j/4}, and lane i receives key dim d0 + i of the four
// tokens. A vector-memory instruction costs the CU ~30-60 cycles beside the
// others' (measured; the walk's time follows its count of them), an LDS one ~15.
//
// The gates of a chunk (gamma, R[C-1], the scales) are loaded once per Q wave
// a chunk ahead and shared through LDS.
__global__ __launch_bounds__(kWalkThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_chunk_state(
    float* __restrict__ S, const float* __restrict__ v, const float* __restrict__ ws,
    const unsigned char* __restrict__ kq, float* __restrict__ out, int rows, int key_heads, int value_heads,
    int value_dim, int64_t qkv_stride, int64_t out_stride) {
    __shared__ __align__(16) u4_t SH[4][2][64];           // S0 as fp16 pairs: [32-row slab][hi, lo][lane]
    __shared__ __align__(16) int SE[kNB][4];              // scale exponent e of each (column, slab)
    __shared__ __align__(16) float RvT[kNB][kC + 4];      // V - gamma X, [column][token]
    __shared__ __align__(16) float RvM[kNB][4];           // max |V - gamma X| of each (column, 16-token tile)
    __shared__ __align__(16) float DlT[kNB][kC + 4];      // Delta, [column][token]
    __shared__ __align__(16) u4_t DsH[2][2][64];          // R[C-1] Delta as fp16 pairs: [32-token block][hi, lo][lane]
    __shared__ __align__(16) _Float16 KT[2][kC][kKtLd];   // the chunk's K as fp16 pairs: [hi, lo][token][key]
    __shared__ __align__(16) float GT[2][256];            // by chunk parity: gamma [64], R[C-1] [64], gamma_{C-1}, eK, eQ, rho
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
    const int wid = wave_in_block();
    const int wv = wid & 3;          // token tile (and SIMD)
    const bool qw = wid < 4;         // Q wave
    const int g = lane >> 4, n = lane & 15;
    float* Sg = S + static_cast<size_t>(h) * kDK * value_dim + j0;

    const int nchunks = (rows + kC - 1) / kC;
    const int tres = 16 * wv + 4 * g;   // first of the 4 token rows of this lane's results
    const uint32_t stride4 = static_cast<uint32_t>(qkv_stride) * 4u;
    const uint32_t ostride4 = static_cast<uint32_t>(out_stride) * 4u;
    // Loop-invariant lane byte offsets into the chunk's fp16 block: K or Q by
    // token, this wave's 8 fragments of 1 KB.
    const uint32_t ao = (qw ? kQRows : kKRows) + static_cast<uint32_t>(wv * 8 * 64 + lane) * 16u;
    uint32_t vo[4], oo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        vo[r] = static_cast<uint32_t>(tres + r) * stride4 + 4u * n;
        oo[r] = static_cast<uint32_t>(tres + r) * ostride4 + 4u * n;
    }
    // T' (K waves) or Bm (Q waves): this wave's row tile, one 1 KB piece per column block
    const uint32_t mo = static_cast<uint32_t>((qw ? kC * kC : 0) + (frag_index(wv, 0) + lane) * 4) * 4u;
    // the gates block, 16 bytes per lane (lanes past its 132 floats read zeros)
    const uint32_t go = static_cast<uint32_t>(2 * kC * kC + 4 * lane) * 4u;
    const float* const vsrc = v + static_cast<size_t>(h) * value_dim + j0;
    float* const osrc = out + static_cast<size_t>(h) * value_dim + j0;
    // chunk c's token rows (fewer in a partial last chunk), workspace block and fp16 block
    auto rows_rsrc = [&](const float* base, int c, int64_t stride, uint32_t s4) {
        return buf_rsrc(base + static_cast<int64_t>(c) * kC * stride, static_cast<uint32_t>(min(rows - c * kC, kC)) * s4);
    };
    auto ws_rsrc = [&](int c) {
        return buf_rsrc(ws + (static_cast<size_t>(c) * value_heads + h) * kWsFloats, static_cast<uint32_t>(kWsFloats * 4));
    };
    auto kq_rsrc = [&](int c) {
        return buf_rsrc(kq + (static_cast<size_t>(c) * value_heads + src) * kKqBytes, static_cast<uint32_t>(kKqBytes));
    };
    float vv[4];
    float4 tm[4], bm[4];   // T' rows (K waves), Bm rows (Q waves); each role loads and reads only its own
    float4 gq;             // Q waves: the next chunk's gates, 16 bytes per lane
    float s0[8];           // K waves: the state at rows 32wv + 16mt + 4g + r (s0[4 mt + r]), column n
    ChunkIn inA, inB;
#pragma unroll
    for (int r = 0; r < 4; ++r) inA.o[r] = inB.o[r] = 0.0f;
    auto load_in = [&](int c, ChunkIn& d, int j) {   // operand piece j < 8
        d.a[j] = buf_ld4u(kq_rsrc(c), ao + 1024u * j);
    };
    // Q wave wv publishes lanes 16wv .. 16wv + 15 of the gates it loaded
    auto put_gates = [&](int c) {
        if (g == wv) *reinterpret_cast<float4*>(&GT[c & 1][4 * lane]) = gq;
    };
    // The K wave's state as fp16 pairs for the next products, scaled per
    // (slab, column) by its largest |value| over the slab's 32 rows.
    auto put_state = [&]() {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(s0[i]));
        const int e = scale_exp(max_groups(m));
        u4_t hi, lo;
        split8(s0, e, hi, lo);
        SH[wv][0][lane] = hi;
        SH[wv][1][lane] = lo;
        SE[n][wv] = e;   // the 4 lanes of a column write the same value
    };
    auto load_v = [&](int c) {
        const __amdgpu_buffer_rsrc_t r = rows_rsrc(vsrc, c, qkv_stride, stride4);
#pragma unroll
        for (int i = 0; i < 4; ++i) vv[i] = buf_ld1(r, vo[i]);
    };
    // T' and Bm are zero above their 16 x 16 diagonal blocks: block s > wv is
    // never multiplied, and its load re-reads block wv (the same number of
    // loads on every wave keeps the wait counts uniform).
    auto load_m = [&](int c, float4 (&m)[4]) {
        const __amdgpu_buffer_rsrc_t w = ws_rsrc(c);
#pragma unroll
        for (int s = 0; s < 4; ++s) m[s] = buf_ld4(w, mo + 1024u * min(s, wv));
    };
    // elements 16s + 4g .. 16s + 4g + 3 (s < 4) of a 64-long LDS row (p = row + 4g)
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
    if (!qw) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s0[i] = Sg[static_cast<size_t>(32 * wv + 16 * (i >> 2) + 4 * g + (i & 3)) * value_dim + n];
        put_state();
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) load_in(0, inA, j);
    if (qw) {
        gq = buf_ld4(ws_rsrc(0), go);
        load_m(0, bm);
    } else {
        load_v(0);
        load_m(0, tm);
    }
    // The loop's wait counts are then computed from its own loads only.
    __builtin_amdgcn_s_waitcnt(0);
    if (qw) put_gates(0);
    __syncthreads();   // the state's fp16 pairs, chunk 0's gates

    // Chunk c with its inputs in cur; chunk c + 1's are loaded into nxt (the
    // last chunk reloads its own: unconditional loads keep the wait counts exact).
    auto chunk_step = [&](int c, ChunkIn& cur, ChunkIn& nxt) __attribute__((always_inline)) {
        const int cn = min(c + 1, nchunks - 1);
        // this chunk's gates: gamma and R[C-1] at the lane's 4 result tokens, the scalars
        const float* const gt = GT[c & 1];
        const float4 gm = *reinterpret_cast<const float4*>(gt + tres);
        const float4 rt4 = *reinterpret_cast<const float4*>(gt + kC + tres);
        const float4 ex = *reinterpret_cast<const float4*>(gt + 2 * kC);   // gamma_{C-1}, eK, eQ (int bits), rho
        // S0 as fp16 pairs (the B operand of k-block kb) and its (column, slab) scales
        u4_t bh[4], bl[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            bh[kb] = SH[kb][0][lane];
            bl[kb] = SH[kb][1][lane];
        }
        const int4 se = *reinterpret_cast<const int4*>(&SE[n][0]);
        // X = K S0 (K waves) or Y = Q S0 (Q waves): per slab hi lo' + lo hi' + hi hi',
        // four independent chains; the next chunk's operand loads go out between
        // the products (issued in one burst they held the wave)
        v4f_t xa[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xa[u] = v4f_t{0.f, 0.f, 0.f, 0.f};
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 12; ++s) {
            const int kb = s & 3, p = s >> 2;
            if (s < 8) load_in(cn, nxt, s);
            xa[kb] = mfma16(p == 1 ? cur.a[2 * kb + 1] : cur.a[2 * kb], p == 0 ? bl[kb] : bh[kb], xa[kb]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // 1 VMEM read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_barrier(0);
        // Loads stay where they are issued: without this compiler fence the
        // loads of the loop's first chunk step were sunk below its products to
        // the barrier, and V then counted as the newest load (a full wait).
        asm volatile("" ::: "memory");
        const int ea = __float_as_int(qw ? ex.z : ex.y);   // eQ or eK
        const int s0e = -(ea + se.x), s1e = -(ea + se.y), s2e = -(ea + se.z), s3e = -(ea + se.w);
        v4f_t X;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            X[r] = (__builtin_amdgcn_ldexpf(xa[0][r], s0e) + __builtin_amdgcn_ldexpf(xa[1][r], s1e)) +
                   (__builtin_amdgcn_ldexpf(xa[2][r], s2e) + __builtin_amdgcn_ldexpf(xa[3][r], s3e));
        if (qw) {
            gq = buf_ld4(ws_rsrc(cn), go);
        } else {
            // result rows: tokens 16wv + 4g + r, column n
            float rv[4];
            rv[0] = __builtin_fmaf(-gm.x, X[0], vv[0]);
            rv[1] = __builtin_fmaf(-gm.y, X[1], vv[1]);
            rv[2] = __builtin_fmaf(-gm.z, X[2], vv[2]);
            rv[3] = __builtin_fmaf(-gm.w, X[3], vv[3]);
            *reinterpret_cast<float4*>(&RvT[n][tres]) = make_float4(rv[0], rv[1], rv[2], rv[3]);
            RvM[n][wv] = max_groups(fmaxf(fmaxf(fabsf(rv[0]), fabsf(rv[1])), fmaxf(fabsf(rv[2]), fabsf(rv[3]))));
            load_v(cn);
            // this wave's 16 tokens of K to LDS by token (slot 4h + c of (kb, g) is
            // key 32kb + 16h + 4g + c), for the state update's transposed reads
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int kb = j >> 1, pl = j & 1;
                _Float16* const row = &KT[pl][16 * wv + n][32 * kb + 4 * g];
                *reinterpret_cast<uint2*>(row) = make_uint2(cur.a[j][0], cur.a[j][1]);
                *reinterpret_cast<uint2*>(row + 16) = make_uint2(cur.a[j][2], cur.a[j][3]);
            }
        }
        __syncthreads();
        int eS = 0;   // K waves: eK + eD, the state update's scale exponent
        if (!qw) {
            // Delta = T' Rv (this wave's 16 rows; K = the chunk's tokens up to the diagonal block)
            float rb[16];
            lds16(rb, &RvT[n][4 * g]);
            v4f_t D0 = {0.f, 0.f, 0.f, 0.f}, D1 = D0;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (s <= wv) {
                    D0 = mfma4(tm[s].x, rb[4 * s], D0);
                    D1 = mfma4(tm[s].y, rb[4 * s + 1], D1);
                    D0 = mfma4(tm[s].z, rb[4 * s + 2], D0);
                    D1 = mfma4(tm[s].w, rb[4 * s + 3], D1);
                }
            }
            load_m(cn, tm);
            const v4f_t D = D0 + D1;
            *reinterpret_cast<float4*>(&DlT[n][tres]) = make_float4(D[0], D[1], D[2], D[3]);
            // R[C-1][t] Delta_t, the state update's operand, as fp16 pairs. Its
            // column scale comes from rho max_i |Rv[i][n]| >= max_t |R[C-1][t] Delta[t][n]|,
            // which every K wave computes alike from the four tiles' maxima.
            const float4 rm = *reinterpret_cast<const float4*>(&RvM[n][0]);
            const int eD = scale_exp(ex.w * fmaxf(fmaxf(rm.x, rm.y), fmaxf(rm.z, rm.w)));
            eS = __float_as_int(ex.y) + eD;
            unsigned h01, l01, h23, l23;
            split2(D[0] * rt4.x, D[1] * rt4.y, eD, h01, l01);
            split2(D[2] * rt4.z, D[3] * rt4.w, eD, h23, l23);
            // tokens 16wv + 4g + r: k-block wv / 2, slots 4 (wv & 1) + r
            reinterpret_cast<uint2*>(&DsH[wv >> 1][0][lane])[wv & 1] = make_uint2(h01, h23);
            reinterpret_cast<uint2*>(&DsH[wv >> 1][1][lane])[wv & 1] = make_uint2(l01, l23);
        }
        __syncthreads();
        if (qw) {
            // O = gamma Y + Bm Delta, stored during the next chunk
            float db[16];
            lds16(db, &DlT[n][4 * g]);
            v4f_t O0 = {0.f, 0.f, 0.f, 0.f}, O1 = O0;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (s <= wv) {
                    O0 = mfma4(bm[s].x, db[4 * s], O0);
                    O1 = mfma4(bm[s].y, db[4 * s + 1], O1);
                    O0 = mfma4(bm[s].z, db[4 * s + 2], O0);
                    O1 = mfma4(bm[s].w, db[4 * s + 3], O1);
                }
            }
            load_m(cn, bm);
            put_gates(cn);   // every wave read this chunk's gates before the last two barriers
            const v4f_t O = O0 + O1;
            cur.o[0] = __builtin_fmaf(gm.x, X[0], O[0]);
            cur.o[1] = __builtin_fmaf(gm.y, X[1], O[1]);
            cur.o[2] = __builtin_fmaf(gm.z, X[2], O[2]);
            cur.o[3] = __builtin_fmaf(gm.w, X[3], O[3]);
            // The previous chunk's outputs (none before chunk 0: a zero-range
            // descriptor drops them). Stored a chunk late, their registers stay
            // live: the store's data would otherwise be overwritten right after
            // it by the next chunk's S0 reads, which waits for the store to complete.
            const __amdgpu_buffer_rsrc_t orr =
                c > 0 ? rows_rsrc(osrc, c - 1, out_stride, ostride4) : buf_rsrc(osrc, 0u);
#pragma unroll
            for (int r = 0; r < 4; ++r) buf_st1(nxt.o[r], orr, oo[r]);
        } else {
            // state rows 32wv + 16mt + 4g + r: gamma_{C-1} S0 + sum_t k_t (R[C-1][t] Delta_t),
            // per (mt, 32-token block) hi lo' + lo hi' + hi hi' (four chains)
            u4_t dh[2], dl[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                dh[kb] = DsH[kb][0][lane];
                dl[kb] = DsH[kb][1][lane];
            }
            // K by key, kt[4 mt + 2 kb + plane]: rows 32wv + 16mt + n, slots 4h + r =
            // tokens 32kb + 16h + 4g + r. Lane j = n of group g points at keys
            // 32wv + 16mt + 4 (j & 3) .. + 3 of token 32kb + 16h + 4g + (j >> 2).
            u4_t kt[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int mt = j >> 2, kb = (j >> 1) & 1, pl = j & 1;
                const _Float16* const p = &KT[pl][32 * kb + 4 * g + (n >> 2)][32 * wv + 16 * mt + 4 * (n & 3)];
                typedef short s4_t __attribute__((ext_vector_type(4)));
                typedef __attribute__((address_space(3))) s4_t* lds_s4_t;
                const s4_t t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t)(p));
                const s4_t t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t)(p + 16 * kKtLd));
                const uint2 a0 = __builtin_bit_cast(uint2, t0), a1 = __builtin_bit_cast(uint2, t1);
                kt[j] = u4_t{a0.x, a0.y, a1.x, a1.y};
            }
            v4f_t sa[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) sa[u] = v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int u = 0; u < 4; ++u) {   // u = 2 mt + kb
                    const int kb = u & 1;
                    sa[u] = mfma16(p == 1 ? kt[2 * u + 1] : kt[2 * u], p == 0 ? dl[kb] : dh[kb], sa[u]);
                }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s0[4 * mt + r] = __builtin_fmaf(ex.x, s0[4 * mt + r],
                                                    __builtin_amdgcn_ldexpf(sa[2 * mt][r] + sa[2 * mt + 1][r], -eS));
            // every wave read this chunk's pairs before the last two barriers
            put_state();
        }
        __syncthreads();   // the new state's pairs are visible; RvT, RvM, DlT, DsH are free
    };
    int c = 0;
    for (; c + 1 < nchunks; c += 2) {
        chunk_step(c, inA, inB);
        chunk_step(c + 1, inB, inA);
    }
    if (c < nchunks) chunk_step(c, inA, inB);
    if (qw) {   // the last chunk's outputs
        const __amdgpu_buffer_rsrc_t orr = rows_rsrc(osrc, nchunks - 1, out_stride, ostride4);
        const ChunkIn& last = (nchunks & 1) ? inA : inB;
#pragma unroll
        for (int r = 0; r < 4; ++r) buf_st1(last.o[r], orr, oo[r]);
    }
    if (!qw) {
#pragma unroll
        for (int i = 0; i < 8; ++i) Sg[static_cast<size_t>(32 * wv + 16 * (i >> 2) + 4 * g + (i & 3)) * value_dim + n] = s0[i];
    }
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

size_t qwen_gdn_recurrent_chunked_workspace_bytes(int rows, int value_heads) {
    if (rows <= 0 || value_heads <= 0) return 0;
    // per (chunk, value head) the matrices and gates, then per (chunk, key head
    // read by some value head: fewer than value_heads) the fp16 pairs of K and Q
    return static_cast<size_t>((rows + kC - 1) / kC) * value_heads * (kWsFloats * sizeof(float) + kKqBytes);
}

int qwen_gdn_recurrent_chunked(float* state, const float* q, const float* k, const float* v, const float* beta,
                               const float* decay, float* out, int rows, int key_heads, int value_heads,
                               int key_dim, int value_dim, int64_t qkv_stride, int64_t out_stride, void* workspace,
                               size_t workspace_bytes, void* stream) {
    // The same limit as the token loop, checked before the path is chosen, so
    // the status does not depend on which path a call's alignment selects.
    QK_REQUIRE(value_dim <= kMaxValueDim, "GDN value dimension exceeds kernel limit");
    // The walk addresses a chunk's 64 rows with 32-bit byte offsets and buffer
    // ranges below 2^31: longer row strides take the token loop.
    const bool chunked = key_dim == kDK && value_dim > 0 && value_dim % kNB == 0 && aligned16(q) && aligned16(k) &&
                         aligned16(workspace) && qkv_stride % 4 == 0 && rows > 0 && key_heads > 0 &&
                         value_heads > 0 && qkv_stride <= kMaxWalkStride && out_stride <= kMaxWalkStride;
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
    unsigned char* kq = static_cast<unsigned char*>(workspace) + static_cast<size_t>(nchunks) * value_heads * kWsFloats * sizeof(float);
    gdn_chunk_prep<<<dim3(nchunks, std::min(key_heads, value_heads)), kThreads, 0, s>>>(
        q, k, beta, decay, ws, kq, rows, key_heads, value_heads, qkv_stride);
    // One row: its stride is not used to step between rows, but the walk's
    // buffer range is one stride long, so it must cover the row's q, k, v and out.
    const int64_t row_extent = std::max<int64_t>(static_cast<int64_t>(key_heads) * key_dim,
                                                 static_cast<int64_t>(value_heads) * value_dim);
    const int64_t qs = rows == 1 ? std::max(qkv_stride, row_extent) : qkv_stride;
    const int64_t os = rows == 1 ? std::max(out_stride, row_extent) : out_stride;
    QK_REQUIRE(qs <= kMaxWalkStride && os <= kMaxWalkStride, "gdn_recurrent_chunked: row too long for the chunked walk");
    gdn_chunk_state<<<(value_dim / kNB) * value_heads, kWalkThreads, 0, s>>>(state, v, ws, kq, out, rows, key_heads,
                                                                             value_heads, value_dim, qs, os);
    return check_launch("gdn_recurrent_chunked");
}

}  // extern "C"
