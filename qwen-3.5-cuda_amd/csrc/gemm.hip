// Quantized GEMM for many tokens (prefill) on gfx950:
//   y[t][m] = sum_k W[m][k] * x[t][k],  t < rows, m < M
// with W a K-quant GGML tensor. Reference: the same product is
// matmul_dispatch (src/cuda/matmul_q4.cu:140-167,185-207) called once per
// token; batched, it is a contraction for the matrix cores.
//
// Exact operands in bf16. The quants are small integers (Q4_K 0..15, Q6_K
// 0..63), exact in bf16, so they are the B operand as they are. x is split
// into three bf16 planes x = x1 + x2 + x3 by truncation (x1 keeps the top 8
// significant bits, x2 the next 8 of the remainder, x3 the rest), each exact,
// so sum_k q x = sum_k q x1 + q x2 + q x3 with exact products and fp32
// accumulation inside v_mfma_f32_16x16x32_bf16 / 16x16x16bf16_1k -- the
// accuracy of an fp32 dot product at 3 bf16 MFMAs per product, well above the
// fp32 MFMA rate. The block scales are applied per scale group on the fp32
// results, as the GEMV does:
//   Q4_K (32-element groups):  sum (d sc q - dmin m) x = (d sc) P - (dmin m) S
//   Q6_K (16-element groups):  sum d sc (q - 32) x      = (d sc) (P - 32 S)
// with P = sum q x and S = sum x over the group (one MFMA result per group and
// 16 x 16 tile, S per token from the staged x).
//
// Work: a workgroup owns 64 tokens x 256 weight rows; wave w owns rows
// 64w .. 64w+63 (4 tiles of 16) for all 64 tokens (4 tiles of 16). Per
// 32-element stage the workgroup splits x[64 tokens][32] into the three planes
// in LDS (one pass of 8 values per thread) with the per-token sums, and each
// wave reads its weight rows' quants and scales straight from global memory
// (a row's block is 144 / 210 bytes; the 16 rows of a tile are read by the 16
// lanes of each lane group) and turns them into bf16 B operands in registers.
#include <algorithm>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "ggml_common.hpp"

namespace qk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;
constexpr int kGemmBlock = kGemmWaves * kWave;
constexpr int kGT = 64;        // tokens per workgroup
constexpr int kGR = 256;       // weight rows per workgroup (64 per wave)
constexpr int kGemmMinRows = 16;   // fewer tokens: one GEMV per token
constexpr int kXRow = 40;      // bf16 per staged token row (32 + 8 padding: distinct banks per lane group)

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

// bf16 of a small non-negative integer (exact).
__device__ __forceinline__ uint32_t bf16_int(uint32_t v) { return __float_as_uint(static_cast<float>(v)) >> 16; }

// Q4_K (scale, min) of sub-block sb from the block header hdr (d, dmin,
// scales[12]): scale_min_k4, src/cuda/matmul_q4.cu:18-26.
__device__ __forceinline__ void q4k_scale_min(const uint4& hdr, int sb, uint32_t& sc, uint32_t& m) {
    const int g = sb >> 1;
    const int sh = 16 * (g & 1) + 8 * (sb & 1);
    const uint32_t a = hdr.y >> sh, b = hdr.z >> sh, c = hdr.w >> sh;
    if (g < 2) {
        sc = a & 63;
        m = b & 63;
    } else {
        sc = (c & 15) | ((a >> 2) & 0x30);
        m = ((c >> 4) & 15) | ((b >> 2) & 0x30);
    }
}

// Stage x[t0 .. t0+63][k0 .. k0+31] as three bf16 planes plus the per-token sum
// S of the 32 values, or of each 16-value half (S16). Thread (token tid/4,
// part tid%4) handles 8 values.
template <bool HALVES>
__device__ __forceinline__ void stage_x(const float* __restrict__ xrow, int k0, uint16_t (*xs)[kGT][kXRow],
                                        float* ssum, int tok, int part) {
    const float4 va = ld4(xrow + k0), vb = ld4(xrow + k0 + 4);
    const float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
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
    s += dpp_move<0xB1>(s);                       // parts 0+1 | 2+3: one 16-value half
    if (HALVES) {
        if ((part & 1) == 0) ssum[2 * tok + (part >> 1)] = s;
    } else {
        s += dpp_move<0x4E>(s);                   // all four parts: the 32 values
        if (part == 0) ssum[tok] = s;
    }
}

// A wave's 64 tokens x 64 rows of results: lane L holds C[4 (L/16) + r][L % 16]
// of tile (tt, rt), i.e. token 16 tt + 4 lk + r, row 16 rt + lr.
__device__ __forceinline__ void store_tiles(const f32x4_t (&acc)[4][4], float* __restrict__ y, int T, int M, int t0,
                                            int r0, int lr, int lk) {
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

// Q4_K: one 32-element sub-block per stage, v_mfma_f32_16x16x32_bf16.
__global__ __launch_bounds__(kGemmBlock) void gemm_q4k(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                       float* __restrict__ y, int T, int M, int K, uint64_t ub0) {
    __shared__ __align__(16) uint16_t xs[3][kGT][kXRow];
    __shared__ __align__(16) float ssum[kGT];
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
    const int stages = K >> 5;
    for (int g = 0; g < stages; ++g) {
        const int sb = g & 7;
        const size_t blk = static_cast<size_t>(g >> 3) * 144;
        if (sb == 0) {
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) hdr[rt] = *reinterpret_cast<const uint4*>(wrow[rt] + blk);
        }
        if ((sb & 1) == 0) {
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
                qb[rt] = *reinterpret_cast<const uint2*>(wrow[rt] + blk + 16 + 32 * (sb >> 1) + 8 * lk);
        }
        stage_x<false>(xrow, 32 * g, xs, ssum, tok, part);
        __syncthreads();

        bf16x8_t B[4];
        float Ag[4], Bg[4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const int shn = 4 * (sb & 1);
            const uint32_t lo = qb[rt].x >> shn, hi = qb[rt].y >> shn;
            const uint32_t e[4] = {bf16_int(lo & 15) | (bf16_int((lo >> 8) & 15) << 16),
                                   bf16_int((lo >> 16) & 15) | (bf16_int((lo >> 24) & 15) << 16),
                                   bf16_int(hi & 15) | (bf16_int((hi >> 8) & 15) << 16),
                                   bf16_int((hi >> 16) & 15) | (bf16_int((hi >> 24) & 15) << 16)};
            __builtin_memcpy(&B[rt], e, 16);
            uint32_t sc, mm;
            q4k_scale_min(hdr[rt], sb, sc, mm);
            Ag[rt] = half_bits(hdr[rt].x & 0xffffu) * static_cast<float>(sc);
            Bg[rt] = half_bits(hdr[rt].x >> 16) * static_cast<float>(mm);
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            bf16x8_t A[3];
#pragma unroll
            for (int q = 0; q < 3; ++q) A[q] = *reinterpret_cast<const bf16x8_t*>(&xs[q][16 * tt + lr][8 * lk]);
            const float4 S = *reinterpret_cast<const float4*>(&ssum[16 * tt + 4 * lk]);
            f32x4_t C[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
                C[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], B[rt], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) C[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1], B[rt], C[rt], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) C[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2], B[rt], C[rt], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                acc[tt][rt][0] = __builtin_fmaf(-Bg[rt], S.x, __builtin_fmaf(Ag[rt], C[rt][0], acc[tt][rt][0]));
                acc[tt][rt][1] = __builtin_fmaf(-Bg[rt], S.y, __builtin_fmaf(Ag[rt], C[rt][1], acc[tt][rt][1]));
                acc[tt][rt][2] = __builtin_fmaf(-Bg[rt], S.z, __builtin_fmaf(Ag[rt], C[rt][2], acc[tt][rt][2]));
                acc[tt][rt][3] = __builtin_fmaf(-Bg[rt], S.w, __builtin_fmaf(Ag[rt], C[rt][3], acc[tt][rt][3]));
            }
        }
        __syncthreads();
    }
    store_tiles(acc, y, T, M, t0, r0, lr, lk);
}

// 4 bytes at a 2-byte aligned address (gfx950 global loads take any byte
// alignment; Q6_K blocks are 210 bytes).
__device__ __forceinline__ uint32_t ldg4_a2(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 4);
    return v;
}

// bf16 pair {a, b} of two small non-negative integers (exact).
__device__ __forceinline__ uint32_t bf16_pair(uint32_t a, uint32_t b) { return bf16_int(a) | (bf16_int(b) << 16); }

// Q6_K: 16-element scale groups, so each 32-element stage is two
// v_mfma_f32_16x16x16bf16_1k steps (K = 16, one scale per step). Element i of
// a block (src/cuda/matmul_q4.cu:105-126): ql byte 64(i/128) + 32((i%128)/32
// & 1) + i%32 (low nibble in quarters 0, 1 of a half, high in 2, 3), qh byte
// 128 + 32(i/128) + i%32 bits 2*quarter, scale byte 192 + i/16, d at 208. For
// stage sg of the block (elements 32 sg ..), half sg/4, quarter sg%4, lane
// (lr, lk) of step h takes elements 32 sg + 16 h + 4 lk .. +3: four
// consecutive ql and qh bytes.
__global__ __launch_bounds__(kGemmBlock) void gemm_q6k(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                       float* __restrict__ y, int T, int M, int K, uint64_t ub0) {
    __shared__ __align__(16) uint16_t xs[3][kGT][kXRow];
    __shared__ __align__(16) float ssum[2 * kGT];
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
        wrow[rt] = w + (ub0 + static_cast<uint64_t>(min(r0 + 16 * rt + lr, M - 1)) * nb) * 210;

    f32x4_t acc[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acc[tt][rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint4 scl[4];
    float dh[4];
    const int stages = K >> 5;
    for (int g = 0; g < stages; ++g) {
        const int sg = g & 7, half = sg >> 2, quarter = sg & 3;
        const uint8_t* blk[4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) blk[rt] = wrow[rt] + static_cast<size_t>(g >> 3) * 210;
        if (sg == 0) {
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                __builtin_memcpy(&scl[rt], __builtin_assume_aligned(blk[rt] + 192, 2), 16);
                dh[rt] = half_bits(*reinterpret_cast<const uint16_t*>(__builtin_assume_aligned(blk[rt] + 208, 2)));
            }
        }
        uint32_t ql[4][2], qh[4][2];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                ql[rt][h] = ldg4_a2(blk[rt] + 64 * half + 32 * (quarter & 1) + 16 * h + 4 * lk);
                qh[rt][h] = ldg4_a2(blk[rt] + 128 + 32 * half + 16 * h + 4 * lk);
            }
        stage_x<true>(xrow, 32 * g, xs, ssum, tok, part);
        __syncthreads();

        const int nsh = 4 * (quarter >> 1), hsh = 2 * quarter;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            s16x4_t B[4];
            float Ag[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const uint32_t lo = (ql[rt][h] >> nsh) & 0x0f0f0f0fu;
                const uint32_t hi = ((qh[rt][h] >> hsh) & 0x03030303u) << 4;
                const uint32_t q = lo | hi;
                const uint32_t e[2] = {bf16_pair(q & 63, (q >> 8) & 63), bf16_pair((q >> 16) & 63, q >> 24)};
                __builtin_memcpy(&B[rt], e, 8);
                const uint32_t sw = (2 * sg + h) < 8 ? (sg < 2 ? scl[rt].x : scl[rt].y) : (sg < 6 ? scl[rt].z : scl[rt].w);
                Ag[rt] = dh[rt] * static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(sw, 8 * ((2 * sg + h) & 3), 8)));
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                s16x4_t A[3];
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    A[q] = *reinterpret_cast<const s16x4_t*>(&xs[q][16 * tt + lr][16 * h + 4 * lk]);
                float S[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) S[r] = ssum[2 * (16 * tt + 4 * lk + r) + h];
                f32x4_t C[4];
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
                    C[rt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(A[0], B[rt], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) C[rt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(A[1], B[rt], C[rt], 0, 0, 0);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) C[rt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(A[2], B[rt], C[rt], 0, 0, 0);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[tt][rt][r] = __builtin_fmaf(Ag[rt], __builtin_fmaf(-32.0f, S[r], C[rt][r]), acc[tt][rt][r]);
            }
        }
        __syncthreads();
    }
    store_tiles(acc, y, T, M, t0, r0, lr, lk);
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
