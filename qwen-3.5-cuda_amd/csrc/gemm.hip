// Quantized GEMM for many tokens (prefill) on gfx950:
//   y[t][m] = sum_k W[m][k] * x[t][k],  t < rows, m < M
// with W a K-quant GGML tensor. Reference: the same product is
// matmul_dispatch (src/cuda/matmul_q4.cu:140-167,185-207) called once per
// token; batched, it is a contraction for the matrix cores.
//
// Exact operands in bf16. The quants are small integers (Q4_K 0..15, Q6_K
// q - 32 in -32..31), exact in bf16, so they are the B operand as they are. x
// is split into three bf16 parts x = x1 + x2 + x3 by truncation (x1 keeps the
// top 8 significant bits, x2 the next 8 of the remainder, x3 the rest), each
// exact, so sum_k q x = sum_k q x1 + q x2 + q x3 with exact products and fp32
// accumulation inside the MFMA -- the accuracy of an fp32 dot product at 3
// bf16 MFMAs per product, well above the fp32 MFMA rate. The block scales are
// applied per scale group on the fp32 results:
//   Q4_K (32-element groups): sum (d sc q - dmin m) x = (d sc) P - (dmin m) S
//   Q6_K (16-element groups): sum d sc (q - 32) x      = (d sc) P'
// with P = sum q x, P' = sum (q - 32) x over the group and S = sum x. The
// (d sc) P terms are one fp32 FMA per result and group; the Q4_K min terms of
// a whole block, sum_g (dmin m_g) S_g, are one small fp32 MFMA product per
// block (v_mfma_f32_16x16x4f32: 8 groups = K of 8) into the same
// accumulators, so they cost no VALU per group.
//
// Work: a workgroup owns 64 tokens x 256 weight rows; wave w owns rows
// 64w .. 64w+63 for all 64 tokens. Per 32-element stage the workgroup splits
// x[64 tokens][32] into the three parts in LDS (one pass of 8 values per
// thread; Q4_K also the per-token group sums), double-buffered so that one
// barrier per stage suffices, with the next stage's x and quants loaded while
// the current one is computed. Each wave reads its weight rows' quants and
// scales straight from global memory and turns them into bf16 B operands in
// registers. Q4_K runs 16 x 16 tiles on v_mfma_f32_16x16x32_bf16 (K = one
// 32-element group); Q6_K runs 32 x 32 tiles on v_mfma_f32_32x32x16_bf16
// (K = one 16-element group, full rate).
#include <algorithm>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "ggml_common.hpp"

namespace qk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGemmWaves = 4;
constexpr int kGemmBlock = kGemmWaves * kWave;
constexpr int kGT = 64;            // tokens per workgroup
constexpr int kGR = 256;           // weight rows per workgroup (64 per wave)
constexpr int kGemmMinRows = 16;   // fewer tokens: one GEMV per token
constexpr int kXRow = 40;          // bf16 per staged token row (32 + 8 padding)

typedef uint16_t XStage[3][kGT][kXRow];   // one stage of x: three bf16 parts

// x = x1 + x2 + x3, each a bf16 (the top halves of fp32 values), by truncation.
__device__ __forceinline__ void split3(float x, uint32_t& a, uint32_t& b, uint32_t& c) {
    const uint32_t xb = __float_as_uint(x);
    const float r1 = x - __uint_as_float(xb & 0xffff0000u);
    const uint32_t rb = __float_as_uint(r1);
    const float r2 = r1 - __uint_as_float(rb & 0xffff0000u);
    a = xb >> 16;
    b = rb >> 16;
    c = __float_as_uint(r2) >> 16;
}

// The bf16 (top halves) of two floats in one word, lo in bits 0..15.
__device__ __forceinline__ uint32_t pack_top(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// bf16 of the four bytes of v (small integers), each minus BIAS (exact).
template <int BIAS>
__device__ __forceinline__ void bytes_bf16(uint32_t v, uint32_t& w0, uint32_t& w1) {
    float f[4] = {static_cast<float>(v & 0xff), static_cast<float>((v >> 8) & 0xff),
                  static_cast<float>((v >> 16) & 0xff), static_cast<float>(v >> 24)};
    if constexpr (BIAS != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] -= static_cast<float>(BIAS);
    }
    w0 = pack_top(f[0], f[1]);
    w1 = pack_top(f[2], f[3]);
}

// Q4_K (scale, min) of sub-block sb from the block header hdr (d, dmin,
// scales[12]): scale_min_k4, src/cuda/matmul_q4.cu:18-26. Branch-free in sb.
__device__ __forceinline__ void q4k_scale_min(const uint4& hdr, int sb, uint32_t& sc, uint32_t& m) {
    const int sh = 8 * (sb & 3);
    const uint32_t a = hdr.y >> sh, b = hdr.z >> sh, c = hdr.w >> sh;
    const bool lo = sb < 4;
    sc = lo ? (a & 63) : ((c & 15) | ((a >> 2) & 0x30));
    m = lo ? (b & 63) : (((c >> 4) & 15) | ((b >> 2) & 0x30));
}

// x of one stage for thread (token tok, part): 8 values at k0 + 8 part.
struct XRegs {
    float4 a, b;
};

__device__ __forceinline__ XRegs load_x(const float* __restrict__ xrow, int k0) {
    return XRegs{ld4(xrow + k0), ld4(xrow + k0 + 4)};
}

// Stage the three bf16 parts of a thread's 8 values; returns the sum of the
// token's 32 values of the stage (complete in every lane of the token's quad).
__device__ __forceinline__ float store_x(const XRegs& r, XStage& xs, int tok, int part) {
    const float v[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    uint32_t p[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t a0, b0, c0, a1, b1, c1;
        split3(v[2 * i], a0, b0, c0);
        split3(v[2 * i + 1], a1, b1, c1);
        p[0][i] = a0 | (a1 << 16);
        p[1][i] = b0 | (b1 << 16);
        p[2][i] = c0 | (c1 << 16);
    }
#pragma unroll
    for (int q = 0; q < 3; ++q)
        *reinterpret_cast<uint4*>(&xs[q][tok][8 * part]) = make_uint4(p[q][0], p[q][1], p[q][2], p[q][3]);
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    s += dpp_move<0xB1>(s);   // quad_perm [1,0,3,2]
    s += dpp_move<0x4E>(s);   // quad_perm [2,3,0,1]
    return s;
}

// ------------------------------------------------------------------ Q4_K
// Element i of a block: qs byte 16 + 32(i/64) + i%32, low nibble if i%64 < 32,
// sub-block i/32 (src/cuda/matmul_q4.cu:76-96). Lane (lr, lk) of stage sb
// takes elements 32 sb + 8 lk .. +7: qs bytes 16 + 32(sb/2) + 8 lk .. +7,
// nibble sb%2.
__global__ __launch_bounds__(kGemmBlock) void gemm_q4k(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                       float* __restrict__ y, int T, int M, int K, uint64_t ub0) {
    __shared__ __align__(16) XStage xs[2];
    __shared__ __align__(16) float ssum[2][8][kGT];   // [block parity][sub-block][token]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.y * kGT;
    const int r0 = blockIdx.x * kGR + wv * 64;
    const int nb = K >> 8;
    const int tok = tid >> 2, part = tid & 3;
    const float* xrow = x + static_cast<size_t>(min(t0 + tok, T - 1)) * K + 8 * part;
    const int lr = lane & 15, lk = lane >> 4;
    const uint8_t* wrow[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
        wrow[rt] = w + (ub0 + static_cast<uint64_t>(min(r0 + 16 * rt + lr, M - 1)) * nb) * 144;

    f32x4_t acc[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acc[tt][rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    uint4 hdr[4];
    uint2 qb[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        hdr[rt] = *reinterpret_cast<const uint4*>(wrow[rt]);
        qb[rt] = *reinterpret_cast<const uint2*>(wrow[rt] + 16 + 8 * lk);
    }
    {
        const float s = store_x(load_x(xrow, 0), xs[0], tok, part);
        if (part == 0) ssum[0][0][tok] = s;
    }
    __syncthreads();

    const int stages = K >> 5;
    for (int g = 0; g < stages; ++g) {
        const int sb = g & 7, cur = g & 1;
        const int gn = g + 1;
        const bool more = gn < stages;
        if (sb == 7) {
            // min terms of the block (all 8 group sums are staged): acc[t][row] -=
            // sum_g (dmin m_g)[row] S_g[t], as [16 tokens x 4 groups] x [4 groups x
            // 16 rows] fp32 products, twice.
            const int par = (g >> 3) & 1;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float bm[4];
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    uint32_t sc, mm;
                    q4k_scale_min(hdr[rt], 4 * j + lk, sc, mm);
                    bm[rt] = half_bits(hdr[rt].x >> 16) * static_cast<float>(mm);
                }
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    const float a = -ssum[par][4 * j + lk][16 * tt + lr];
#pragma unroll
                    for (int rt = 0; rt < 4; ++rt)
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bm[rt], acc[tt][rt], 0, 0, 0);
                }
            }
        }
        // this stage's B operands and group scales; then the quants and x of the
        // next stage are loaded into the same registers, in flight during the products
        bf16x8_t B[4];
        float Ag[4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const int shn = 4 * (sb & 1);
            uint32_t e[4];
            bytes_bf16<0>((qb[rt].x >> shn) & 0x0f0f0f0fu, e[0], e[1]);
            bytes_bf16<0>((qb[rt].y >> shn) & 0x0f0f0f0fu, e[2], e[3]);
            __builtin_memcpy(&B[rt], e, 16);
            uint32_t sc, mm;
            q4k_scale_min(hdr[rt], sb, sc, mm);
            Ag[rt] = half_bits(hdr[rt].x & 0xffffu) * static_cast<float>(sc);
        }
        XRegs xn;
        if (more) {
            xn = load_x(xrow, 32 * gn);
            const size_t blk = static_cast<size_t>(gn >> 3) * 144;
            if ((gn & 7) == 0) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) hdr[rt] = *reinterpret_cast<const uint4*>(wrow[rt] + blk);
            }
            if ((gn & 1) == 0) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
                    qb[rt] = *reinterpret_cast<const uint2*>(wrow[rt] + blk + 16 + 32 * ((gn & 7) >> 1) + 8 * lk);
            }
        }
        const XStage& xc = xs[cur];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            bf16x8_t A[3];
#pragma unroll
            for (int q = 0; q < 3; ++q) A[q] = *reinterpret_cast<const bf16x8_t*>(&xc[q][16 * tt + lr][8 * lk]);
            f32x4_t C[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
                C[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], B[rt], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) C[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1], B[rt], C[rt], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) C[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2], B[rt], C[rt], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[tt][rt][r] = __builtin_fmaf(Ag[rt], C[rt][r], acc[tt][rt][r]);
        }
        if (more) {
            const float s = store_x(xn, xs[cur ^ 1], tok, part);
            if (part == 0) ssum[(gn >> 3) & 1][gn & 7][tok] = s;
        }
        __syncthreads();
    }
    // lane L holds C[4 (L/16) + r][L % 16] of tile (tt, rt): token 16 tt + 4 lk + r, row 16 rt + lr
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const int row = r0 + 16 * rt + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + 16 * tt + 4 * lk + r;
                if (t < T && row < M) y[static_cast<size_t>(t) * M + row] = acc[tt][rt][r];
            }
        }
}

// ------------------------------------------------------------------ Q6_K
// 8 bytes at a 2-byte aligned address (gfx950 global loads take any byte
// alignment; Q6_K blocks are 210 bytes).
__device__ __forceinline__ uint2 ldg8_a2(const uint8_t* p) {
    uint2 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 8);
    return v;
}

// Element i of a block (src/cuda/matmul_q4.cu:105-126): ql byte 64(i/128) +
// 32((i%128)/32 & 1) + i%32 (low nibble in quarters 0, 1 of a half, high in
// 2, 3), qh byte 128 + 32(i/128) + i%32 bits 2*quarter, scale byte 192 + i/16,
// d at 208. Stage sg of a block (elements 32 sg ..) is half sg/4, quarter
// sg%4; lane (l32, lh) of step h takes elements 32 sg + 16 h + 8 lh .. +7:
// eight consecutive ql and qh bytes, scale 2 sg + h.
struct Q6Quants {
    uint2 ql[2][2], qh[2][2];   // [row tile][step]
};

__device__ __forceinline__ Q6Quants q6_load(const uint8_t* const (&wrow)[2], int g, int lh) {
    const int sg = g & 7;
    const int off_l = 64 * (sg >> 2) + 32 * (sg & 1) + 8 * lh;
    const int off_h = 128 + 32 * (sg >> 2) + 8 * lh;
    Q6Quants q;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const uint8_t* blk = wrow[rt] + static_cast<size_t>(g >> 3) * 210;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            q.ql[rt][h] = ldg8_a2(blk + off_l + 16 * h);
            q.qh[rt][h] = ldg8_a2(blk + off_h + 16 * h);
        }
    }
    return q;
}

__global__ __launch_bounds__(kGemmBlock, 2) void gemm_q6k(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                          float* __restrict__ y, int T, int M, int K, uint64_t ub0) {
    __shared__ __align__(16) XStage xs[2];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.y * kGT;
    const int r0 = blockIdx.x * kGR + wv * 64;
    const int nb = K >> 8;
    const int tok = tid >> 2, part = tid & 3;
    const float* xrow = x + static_cast<size_t>(min(t0 + tok, T - 1)) * K + 8 * part;
    const int l32 = lane & 31, lh = lane >> 5;
    const uint8_t* wrow[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
        wrow[rt] = w + (ub0 + static_cast<uint64_t>(min(r0 + 32 * rt + l32, M - 1)) * nb) * 210;

    f32x16_t acc[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[tt][rt][i] = 0.f;

    uint4 scl[2];
    float dh[2];
    Q6Quants qc = q6_load(wrow, 0, lh);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        __builtin_memcpy(&scl[rt], __builtin_assume_aligned(wrow[rt] + 192, 2), 16);
        dh[rt] = half_bits(*reinterpret_cast<const uint16_t*>(__builtin_assume_aligned(wrow[rt] + 208, 2)));
    }
    store_x(load_x(xrow, 0), xs[0], tok, part);
    __syncthreads();

    const int stages = K >> 5;
    for (int g = 0; g < stages; ++g) {
        const int sg = g & 7, quarter = sg & 3, cur = g & 1;
        const int gn = g + 1;
        const bool more = gn < stages;
        // this stage's B operands and group scales (both steps); then the next
        // stage's quants, scales and x are loaded into the same registers
        const int nsh = 4 * (quarter >> 1), hsh = 2 * quarter;
        bf16x8_t B[2][2];
        float Ag[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const uint32_t q0 = ((qc.ql[rt][h].x >> nsh) & 0x0f0f0f0fu) | (((qc.qh[rt][h].x >> hsh) & 0x03030303u) << 4);
                const uint32_t q1 = ((qc.ql[rt][h].y >> nsh) & 0x0f0f0f0fu) | (((qc.qh[rt][h].y >> hsh) & 0x03030303u) << 4);
                uint32_t e[4];
                bytes_bf16<32>(q0, e[0], e[1]);
                bytes_bf16<32>(q1, e[2], e[3]);
                __builtin_memcpy(&B[h][rt], e, 16);
                const int si = 2 * sg + h;   // scale byte si of the block
                const uint32_t sw = si < 8 ? (si < 4 ? scl[rt].x : scl[rt].y) : (si < 12 ? scl[rt].z : scl[rt].w);
                Ag[h][rt] = dh[rt] * static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(sw, 8 * (si & 3), 8)));
            }
        XRegs xn;
        if (more) {
            xn = load_x(xrow, 32 * gn);
            qc = q6_load(wrow, gn, lh);
            if ((gn & 7) == 0) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const uint8_t* blk = wrow[rt] + static_cast<size_t>(gn >> 3) * 210;
                    __builtin_memcpy(&scl[rt], __builtin_assume_aligned(blk + 192, 2), 16);
                    dh[rt] = half_bits(*reinterpret_cast<const uint16_t*>(__builtin_assume_aligned(blk + 208, 2)));
                }
            }
        }
        const XStage& xc = xs[cur];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                bf16x8_t A[3];
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    A[q] = *reinterpret_cast<const bf16x8_t*>(&xc[q][32 * tt + l32][16 * h + 8 * lh]);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    f32x16_t C;
#pragma unroll
                    for (int i = 0; i < 16; ++i) C[i] = 0.f;
                    C = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[0], B[h][rt], C, 0, 0, 0);
                    C = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[1], B[h][rt], C, 0, 0, 0);
                    C = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[2], B[h][rt], C, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[tt][rt][i] = __builtin_fmaf(Ag[h][rt], C[i], acc[tt][rt][i]);
                }
            }
        if (more) store_x(xn, xs[cur ^ 1], tok, part);
        __syncthreads();
    }
    // lane L holds C[8 (i/4) + 4 (L/32) + i%4][L % 32] of tile (tt, rt) in register i
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = r0 + 32 * rt + l32;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = t0 + 32 * tt + 8 * (i >> 2) + 4 * lh + (i & 3);
                if (t < T && row < M) y[static_cast<size_t>(t) * M + row] = acc[tt][rt][i];
            }
        }
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_matmul_rows(const void* weight, int type, uint64_t num_elements, const float* x, float* y, int rows, int M,
                     int K, uint64_t element_offset, void* stream) {
    if (!weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    if (M <= 0 || K <= 0 || element_offset > num_elements ||
        static_cast<uint64_t>(M) * static_cast<uint64_t>(K) > num_elements - element_offset)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d)", M, K);
    QK_REQUIRE(rows >= 0, "matmul_rows: negative rows %d", rows);
    if (rows == 0) return ok();
    QK_REQUIRE(x && y, "matmul_rows: null pointer");
    const bool mfma = (type == kQ4_K || type == kQ6_K) && rows >= kGemmMinRows && K % 256 == 0 &&
                      element_offset % 256 == 0 && aligned16(x) && rows <= 65535 * kGT;
    if (!mfma) {   // one GEMV per token (the reference's own loop)
        for (int t = 0; t < rows; ++t) {
            const int rc = qwen_matmul_dispatch(weight, type, num_elements, x + static_cast<size_t>(t) * K,
                                                y + static_cast<size_t>(t) * M, M, K, element_offset, stream);
            if (rc) return rc;
        }
        return ok();
    }
    const dim3 grid(blocks_for(M, kGR), blocks_for(rows, kGT));
    const auto k = type == kQ4_K ? gemm_q4k : gemm_q6k;
    k<<<grid, kGemmBlock, 0, as_stream(stream)>>>(static_cast<const uint8_t*>(weight), x, y, rows, M, K,
                                                  element_offset / 256);
    return check_launch("matmul_rows");
}

}  // extern "C"
