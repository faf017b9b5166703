// Quantized GEMV (matmul_dispatch) on gfx950: y[m] = sum_k W[m][k] * x[k].
//
// Reference semantics: gemv_kernel src/cuda/matmul_q4.cu:140-167 and
// matmul_dispatch :185-207 -- y[m] = sum over k < K of
// dequant(W, element_offset + m*K + k) * x[k], fp32 accumulation, for m < M;
// called for every projection of a decode step (src/layer_attn.cpp:85-87,109,
// src/layer_gdn.cpp:83-86,112, src/layer_moe.cpp:98,131-150, src/model.cpp:216).
// The reference runs one 256-thread block per output row and decodes every
// weight element independently (header and 6-bit scales re-read per element).
//
// The op is bound by the weight bytes read from HBM (x is 8-16 KB and stays in
// L2). Two Q4_K / Q6_K kernels:
//  * large matrices (the LM head): gemv_mfma below -- int8 MFMA on the raw
//    quants against x in exact integer digits, LDS-staged tiles of 16 rows;
//  * everything else: gemv_kquant, whose shorter per-wave latency wins at the
//    per-layer sizes (<= 8192 rows in the model).
// Per-row path (Q4_K, Q6_K): the weight is walked in units of 8 consecutive
// 256-element blocks (2048 elements = 1152 B of Q4_K or 1680 B of Q6_K, both
// multiples of 16 bytes). A row of K = 256*nb elements is nb/8 units when
// 8 | nb; when nb | 8, 8/nb consecutive rows share one unit. A wave owns R
// units at a time: it copies them into its LDS slot with 16-byte non-temporal
// loads (contiguous, fully coalesced), then lane L decodes 32 elements of
// block L/8 of each unit. That lane->element map is the same for every unit,
// so the lane's 32 x values are loaded once and stay in VGPRs across all R
// units. Q4_K rows of whole units skip the LDS copy: lane L loads block L/8's
// 16-byte header and its own 16 qs bytes straight into VGPRs (the lane's x
// values are 128 B against 16 B of quants, so x, not the weights, is most of
// what a CU moves; issuing it first lets each row's decode start when that
// row's loads are back). The dot product runs on the raw quants and the block scale is
// applied once per run of 16 (Q4_K) or 8 (Q6_K) elements:
//   sum((d*sc*q - dmin*m) * x) = (d*sc) * sum(q*x) - (dmin*m) * sum(x)
// which is the reference's sum re-associated (fp32 tolerance, not bit-exact:
// the reference's own order depends on its launch shape).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "ggml_common.hpp"
#include "moe_common.hpp"

namespace qk {
namespace {

constexpr int kGemvWaves = 4;                   // waves per workgroup (fast path)
constexpr int kGemvBlock = kGemvWaves * kWave;
constexpr int kBlock = 256;                     // generic path

template <int TYPE>
struct KQuant;

template <>
struct KQuant<kQ4_K> {
    static constexpr int kBlockBytes = 144;
};

template <>
struct KQuant<kQ6_K> {
    static constexpr int kBlockBytes = 210;
};

// Lane constants of the fast path: which x values the lane multiplies.
//   Q4_K: lane j = L%8 of block L/8 takes qs bytes 16j..16j+15 of the block:
//         low nibbles = elements 64g + 16h + i (sub-block 2g), high nibbles =
//         elements 64g + 32 + 16h + i (sub-block 2g+1), g = j/2, h = j%2.
//   Q6_K: lane j takes elements 128*half + 32*qq + l0 + i, i < 8, for the four
//         quarters qq, half = j/4, l0 = 8*(j%4).
template <int TYPE>
struct LaneX {
    float4 v[8];   // 32 x values, in decode order
    float s[4];    // sums of x per scale run (Q4_K: s[0], s[1]; Q6_K: 32*sum per quarter)
};

// The lane's x values only (Q4_K); lane_x_sums completes the LaneX.
__device__ __forceinline__ void load_lane_x_values(LaneX<kQ4_K>& lx, const float* __restrict__ x, int xb, int j) {
    const float* lo = x + static_cast<size_t>(xb) * 256 + 64 * (j >> 1) + 16 * (j & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lx.v[i] = ld4(lo + 4 * i);
        lx.v[4 + i] = ld4(lo + 32 + 4 * i);
    }
}

__device__ __forceinline__ void lane_x_sums(LaneX<kQ4_K>& lx) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a += (lx.v[i].x + lx.v[i].y) + (lx.v[i].z + lx.v[i].w);
        b += (lx.v[4 + i].x + lx.v[4 + i].y) + (lx.v[4 + i].z + lx.v[4 + i].w);
    }
    lx.s[0] = a;
    lx.s[1] = b;
    lx.s[2] = lx.s[3] = 0.f;
}

template <int TYPE>
__device__ __forceinline__ void load_lane_x(LaneX<TYPE>& lx, const float* __restrict__ x, int xb, int j) {
    if constexpr (TYPE == kQ4_K) {
        load_lane_x_values(lx, x, xb, j);
        lane_x_sums(lx);
    } else {
        const float* base = x + static_cast<size_t>(xb) * 256 + 128 * (j >> 2) + 8 * (j & 3);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            lx.v[2 * qq] = ld4(base + 32 * qq);
            lx.v[2 * qq + 1] = ld4(base + 32 * qq + 4);
        }
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const float4 a = lx.v[2 * qq], b = lx.v[2 * qq + 1];
            lx.s[qq] = 32.0f * (((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)));
        }
    }
}

// v, hidden from the optimiser (no code).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// sum over the 4 bytes of `q` (unsigned) times 4 x values.
__device__ __forceinline__ float dot_u8x4(uint32_t q, float4 xv, float acc) {
    acc = __builtin_fmaf(static_cast<float>(q & 0xffu), xv.x, acc);
    acc = __builtin_fmaf(static_cast<float>((q >> 8) & 0xffu), xv.y, acc);
    acc = __builtin_fmaf(static_cast<float>((q >> 16) & 0xffu), xv.z, acc);
    return __builtin_fmaf(static_cast<float>(q >> 24), xv.w, acc);
}

// Contribution of one Q4_K block to lane j's partial dot product, from the
// block's first 16 bytes (hdr: d, dmin, scales[12]) and its qs bytes
// 16j..16j+15 (q).
__device__ __forceinline__ float block_dot_q4k(uint4 hdr, uint4 q, const LaneX<kQ4_K>& lx, int j) {
    const float d = half_bits(hdr.x & 0xffffu);
    const float dmin = half_bits(hdr.x >> 16);
    // scale_min_k4 (src/cuda/matmul_q4.cu:18-26) for sub-blocks 2g, 2g+1:
    // sub < 4 reads bytes sub, sub+4; sub >= 4 combines byte sub+4 with the
    // top two bits of bytes sub-4 and sub. t = sub % 4 for both pairs.
    const int g = j >> 1;
    const int sh = 16 * (g & 1);                 // byte 2g%4 of each scale word
    const uint32_t a = hdr.y >> sh, b = hdr.z >> sh, c = hdr.w >> sh;
    uint32_t sc0, m0, sc1, m1;
    if (g < 2) {
        sc0 = a & 63;
        sc1 = (a >> 8) & 63;
        m0 = b & 63;
        m1 = (b >> 8) & 63;
    } else {
        sc0 = (c & 15) | ((a >> 2) & 0x30);
        sc1 = ((c >> 8) & 15) | ((a >> 10) & 0x30);
        m0 = ((c >> 4) & 15) | ((b >> 2) & 0x30);
        m1 = ((c >> 12) & 15) | ((b >> 10) & 0x30);
    }
    float lo = 0.f, hi = 0.f;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // opaque: the compiler would otherwise fold each mask into a bit-field
        // extract per byte instead of one AND and four byte conversions.
        lo = dot_u8x4(opaque_u32(w[i] & 0x0f0f0f0fu), lx.v[i], lo);
        hi = dot_u8x4(opaque_u32((w[i] >> 4) & 0x0f0f0f0fu), lx.v[4 + i], hi);
    }
    const float A0 = d * static_cast<float>(sc0), B0 = dmin * static_cast<float>(m0);
    const float A1 = d * static_cast<float>(sc1), B1 = dmin * static_cast<float>(m1);
    return (A0 * lo - B0 * lx.s[0]) + (A1 * hi - B1 * lx.s[1]);
}

// Contribution of one Q6_K block to lane j's partial dot product from the
// lane's bytes of it: ql bytes 64 half + l0 .. + 7 (la0, la1: quarters 0 and 2
// in the low and high nibbles) and 64 half + 32 + l0 .. + 7 (lb0, lb1:
// quarters 1 and 3), qh bytes 128 + 32 half + l0 .. + 7 (h0, h1: 2 bits per
// quarter), scale bytes 192 + 8 half .. + 7 (s0, s1) and the block scale d
// (half = j / 4, l0 = 8 (j % 4)).
__device__ __forceinline__ float q6k_lane_dot(uint32_t la0, uint32_t la1, uint32_t lb0, uint32_t lb1, uint32_t h0,
                                              uint32_t h1, uint32_t s0, uint32_t s1, float d,
                                              const LaneX<kQ6_K>& lx, int j) {
    // scales[8*half + l0/16 + 2*qq]: bytes (l0/16) + {0, 2} of the first word
    // (qq 0, 1) and of the second word (qq 2, 3).
    const int ss = 8 * ((8 * (j & 3)) >> 4);
    const int8_t sc[4] = {static_cast<int8_t>(s0 >> ss), static_cast<int8_t>(s0 >> (ss + 16)),
                          static_cast<int8_t>(s1 >> ss), static_cast<int8_t>(s1 >> (ss + 16))};
    const uint32_t L[4][2] = {{la0 & 0x0f0f0f0fu, la1 & 0x0f0f0f0fu},
                              {lb0 & 0x0f0f0f0fu, lb1 & 0x0f0f0f0fu},
                              {(la0 >> 4) & 0x0f0f0f0fu, (la1 >> 4) & 0x0f0f0f0fu},
                              {(lb0 >> 4) & 0x0f0f0f0fu, (lb1 >> 4) & 0x0f0f0f0fu}};
    float acc = 0.f;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        const uint32_t q0 = L[qq][0] | (((h0 >> (2 * qq)) & 0x03030303u) << 4);
        const uint32_t q1 = L[qq][1] | (((h1 >> (2 * qq)) & 0x03030303u) << 4);
        float t = dot_u8x4(q0, lx.v[2 * qq], 0.f);
        t = dot_u8x4(q1, lx.v[2 * qq + 1], t);
        // sum((q - 32) * x) = sum(q * x) - 32 * sum(x)
        acc = __builtin_fmaf(d * static_cast<float>(sc[qq]), t - lx.s[qq], acc);
    }
    return acc;
}

// Contribution of one block to the lane's partial dot product. `blk` points
// at the block in LDS.
template <int TYPE>
__device__ __forceinline__ float block_dot(const uint8_t* blk, const LaneX<TYPE>& lx, int j) {
    if constexpr (TYPE == kQ4_K) {
        return block_dot_q4k(*reinterpret_cast<const uint4*>(blk), *reinterpret_cast<const uint4*>(blk + 16 + 16 * j),
                             lx, j);
    } else {
        const int half = j >> 2, l0 = 8 * (j & 3);
        const uint8_t* qla = blk + 64 * half + l0;         // quarters 0 (low nibble), 2 (high)
        const uint8_t* qlb = qla + 32;                     // quarters 1, 3
        const uint8_t* qhp = blk + 128 + 32 * half + l0;   // 2 bits per quarter
        return q6k_lane_dot(lds_u32_a2(qla), lds_u32_a2(qla + 4), lds_u32_a2(qlb), lds_u32_a2(qlb + 4),
                            lds_u32_a2(qhp), lds_u32_a2(qhp + 4), lds_u32_a2(blk + 192 + 8 * half),
                            lds_u32_a2(blk + 196 + 8 * half), half_bits(*reinterpret_cast<const uint16_t*>(blk + 208)),
                            lx, j);
    }
}

// Device-side expert selection (MoE): selection slot j (the launch row
// blockIdx.y, or half of it for the gate/up launch) runs selected expert
// idx[j] -- weight rows at element offset idx * stride -- on x + j * x_stride,
// writing y + j * M. An id outside [0, n_experts) gives a NaN row.
// idx == nullptr: a plain GEMV.
struct Experts {
    const int32_t* idx;
    int n_experts;
    uint64_t stride;  // elements between experts (a multiple of 256 on the fast path)
    int64_t x_stride;
};

// Applies the selection of slot j; false if the expert id is invalid (the
// caller writes NaN rows).
__device__ __forceinline__ bool select_expert(const Experts& ex, int j, int M, int64_t& x_off, int64_t& y_off,
                                              uint64_t& element_offset) {
    x_off = y_off = 0;
    if (!ex.idx) return true;
    const int e = ex.idx[j];
    x_off = static_cast<int64_t>(j) * ex.x_stride;
    y_off = static_cast<int64_t>(j) * M;
    if (e < 0 || e >= ex.n_experts) return false;
    element_offset += static_cast<uint64_t>(e) * ex.stride;
    return true;
}

// Output index of GEMV row m. split > 0: the rows are M / (2 split) pairs of
// split-row halves (the fused query | gate projection of attention, one pair
// per head) and the first halves go to y[0, M/2), the second halves to
// y[M/2, M): the layout attn_split_qg produces (src/cuda/attn_kernels.cu:16-24).
__device__ __forceinline__ int64_t out_index(int64_t m, int M, int split) {
    if (split <= 0) return m;
    const int64_t pair = m / (2 * split), r = m - pair * 2 * split;
    return r < split ? pair * split + r : M / 2 + pair * split + (r - split);
}

// Q4_K direct form of gemv_kquant_body: NS (1 or 2) consecutive slices s, s+1
// of R rows from g0 (row = min(g0 + u, groups - 1)), added to acc[u] in slice
// order. Every thread of the workgroup calls it (one barrier). The slices' x
// values (NS x 8 KB) are loaded once per workgroup, 2 NS float4 per thread,
// before the weights, and staged in xs; then each lane loads block L/8's
// 16-byte header and its own 16 qs bytes of every row straight into VGPRs.
// Every wave of every workgroup reads the same x, so the lines holding it are
// the L2's busiest: loaded per wave (8 KB each) x took longer to arrive than
// the weights (measured at 8192 x 2048: ~2 us into a ~3 us wave), loaded per
// workgroup the request count is a quarter.
// x of a GEMV produced in its own launch: the gated per-head RMSNorm of the
// reference's GDN layer, x = ((core * r) * w) * silu(z) per head of 4 LPH
// values (norm_gate_v4<LPH>'s lane groups and arithmetic, so the same bits).
// normed (may be null) receives x from workgroup (0, 0).
struct NormGateX {
    const float* z;
    const float* w;
    float eps;
    float* normed;
};

template <int R, int NS, int MAT = 1, int LPH = 0, int NWV = kGemvWaves>
__device__ __forceinline__ void q4k_direct_slices(const uint8_t* const (&w)[MAT], const float* __restrict__ x,
                                                  float4* xs, float (&acc)[MAT][R], int nb, uint64_t ub0, int g0,
                                                  int groups, int s, int b, int j,
                                                  const NormGateX& ng = NormGateX{}) {
    constexpr int BB = KQuant<kQ4_K>::kBlockBytes;
    constexpr int NX = NS * 512;                    // float4 of x in the NS slices
    constexpr int NTH = NWV * kWave;                // threads of the workgroup
    constexpr int PER = NX / NTH;
    static_assert(PER * NTH == NX, "x staging");
    float4 xt[PER], zt[LPH > 0 ? PER : 1];
    const float* xsl = x + static_cast<size_t>(s) * 2048;
#pragma unroll
    for (int i = 0; i < PER; ++i) xt[i] = ld4(xsl + 4 * (threadIdx.x + i * NTH));
    if constexpr (LPH > 0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) zt[i] = ld4(ng.z + static_cast<size_t>(s) * 2048 + 4 * (threadIdx.x + i * NTH));
    }
    __builtin_amdgcn_sched_barrier(0);   // the x loads first
    uint4 hd[MAT][R][NS], qv[MAT][R][NS];
    // Lane offsets inside a unit (block b's header, its qs bytes 16j..16j+15),
    // the same in every unit; the unit's address is wave-uniform. Every unit
    // read lies inside the tensor: rows are clamped to groups - 1 and every
    // entry point checks the shape (element_offset + M K, or the expert stride)
    // against the tensor on the host. (A per-lane range check here held
    // 64-bit addresses for every row in VGPRs.)
    const uint32_t ho = b * BB, qo = b * BB + 16 + 16 * j;
#pragma unroll
    for (int mt = 0; mt < MAT; ++mt)
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int g = min(g0 + u, groups - 1);
#pragma unroll
            for (int h = 0; h < NS; ++h) {
                const uint8_t* unit = w[mt] + (ub0 + static_cast<uint64_t>(g) * nb + 8 * (s + h)) * BB;
                hd[mt][u][h] = ld16_nt(unit + ho);
                qv[mt][u][h] = ld16_nt(unit + qo);
            }
        }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before the staging
    if constexpr (LPH > 0) {
        // float4 c of the slices is element group c % LPH of head (s * 512 + c) / LPH
        // (s * 512 and i * NTH are multiples of LPH): the LPH lanes of a head
        // are consecutive lanes of one wave, as in norm_gate_v4.
        constexpr int D = 4 * LPH;
        const float4 wv = ld4(ng.w + 4 * (threadIdx.x % LPH));
        const bool first = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const float ss = group_sum<LPH>(sumsq4(xt[i]));
            const float r = rsqrtf(ss / static_cast<float>(D) + ng.eps);
            const float4 sz = silu4(zt[i]);
            float4 o;
            o.x = xt[i].x * r * wv.x * sz.x;
            o.y = xt[i].y * r * wv.y * sz.y;
            o.z = xt[i].z * r * wv.z * sz.z;
            o.w = xt[i].w * r * wv.w * sz.w;
            xt[i] = o;
            if (first && ng.normed) st4(ng.normed + static_cast<size_t>(s) * 2048 + 4 * (threadIdx.x + i * NTH), o);
        }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) xs[threadIdx.x + i * NTH] = xt[i];
    __syncthreads();
    LaneX<kQ4_K> lx[NS];
#pragma unroll
    for (int h = 0; h < NS; ++h) {
        // load_lane_x_values' elements, from the staged copy
        const float4* lo = xs + (h * 2048 + b * 256 + 64 * (j >> 1) + 16 * (j & 1)) / 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lx[h].v[i] = lo[i];
            lx[h].v[4 + i] = lo[8 + i];
        }
        lane_x_sums(lx[h]);
    }
#pragma unroll
    for (int mt = 0; mt < MAT; ++mt)
#pragma unroll
        for (int u = 0; u < R; ++u)
#pragma unroll
            for (int h = 0; h < NS; ++h) acc[mt][u] += block_dot_q4k(hd[mt][u][h], qv[mt][u][h], lx[h], j);
}

// Q6_K direct form (rows of whole units, 8 | nb): the lane map of block_dot
// (lane j of block L/8 takes ql bytes 64 half + l0 .. +7 and +32, qh bytes 128
// + 32 half + l0 .. +7, scale bytes 192 + 8 half .. +7 and d) with every piece
// loaded straight into VGPRs. A 210-byte block starts 2 (b mod 2) bytes past a
// 4-byte boundary of its 16-byte-aligned unit, so each 8-byte piece lies at
// byte 0 or 2 of the 4-byte-aligned 12 bytes around it: one 12-byte load
// (dwordx3, dword alignment) and two v_alignbyte per piece. The 12 bytes stay
// inside the unit (the last piece, block 7's scales, ends the window at the
// unit's byte 1680). x is staged once per workgroup as in q4k_direct_slices.
struct __attribute__((aligned(4))) Q6Piece {
    uint32_t x, y, z;
};
// 8 bytes at byte offset sb (0 or 2) of the 12 bytes w.
__device__ __forceinline__ uint2 q6_piece(Q6Piece w, uint32_t sb) {
    return make_uint2(__builtin_amdgcn_alignbyte(w.y, w.x, sb), __builtin_amdgcn_alignbyte(w.z, w.y, sb));
}

// NS (1 or 2) consecutive slices s, s+1 of R rows from g0 (row = min(g0 + u,
// groups - 1)), added to acc[u] in slice order; every thread of the workgroup
// calls it (one barrier).
template <int R, int NS, int NWV = kGemvWaves>
__device__ __forceinline__ void q6k_direct_slices(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                  float4* xs, float (&acc)[R], int nb, uint64_t ub0, int g0,
                                                  int groups, int s, int b, int j) {
    constexpr int BB = KQuant<kQ6_K>::kBlockBytes;
    constexpr int NX = NS * 512;
    constexpr int NTH = NWV * kWave;
    constexpr int PER = NX / NTH;
    static_assert(PER * NTH == NX, "x staging");
    const int half = j >> 2, l0 = 8 * (j & 3);
    const uint32_t sb = 2 * (b & 1);
    float4 xt[PER];
    const float* xsl = x + static_cast<size_t>(s) * 2048;
#pragma unroll
    for (int i = 0; i < PER; ++i) xt[i] = ld4(xsl + 4 * (threadIdx.x + i * NTH));
    __builtin_amdgcn_sched_barrier(0);   // the x loads first
    Q6Piece pc[R][NS][4];
    uint32_t dh[R][NS];
    // The lane's byte offsets inside a unit (the same in every unit): the four
    // 12-byte windows and d. The unit's address is wave-uniform, so each load is
    // a scalar base plus a 32-bit lane offset.
    const uint32_t blk = b * BB;
    const uint32_t lo[4] = {blk + 64 * half + l0 - sb, blk + 64 * half + 32 + l0 - sb,
                            blk + 128 + 32 * half + l0 - sb, blk + 192 + 8 * half - sb};
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int g = min(g0 + u, groups - 1);
#pragma unroll
        for (int h = 0; h < NS; ++h) {
            // Every unit read lies inside the tensor: rows are clamped to groups - 1
            // and every entry point checks element_offset + M K (or the expert
            // stride) against num_elements on the host.
            const uint8_t* unit = w + (ub0 + static_cast<uint64_t>(g) * nb + 8 * (s + h)) * BB;
#pragma unroll
            for (int q = 0; q < 4; ++q) pc[u][h][q] = *reinterpret_cast<const Q6Piece*>(unit + lo[q]);
            dh[u][h] = *reinterpret_cast<const uint16_t*>(unit + blk + 208);
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before the staging
#pragma unroll
    for (int i = 0; i < PER; ++i) xs[threadIdx.x + i * NTH] = xt[i];
    __syncthreads();
    LaneX<kQ6_K> lx[NS];
#pragma unroll
    for (int h = 0; h < NS; ++h) {
        // load_lane_x<kQ6_K>'s elements, from the staged copy
        const float4* bx = xs + (h * 2048 + b * 256 + 128 * half + l0) / 4;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            lx[h].v[2 * qq] = bx[8 * qq];
            lx[h].v[2 * qq + 1] = bx[8 * qq + 1];
        }
    }
    // every LDS read issued before the first use (one wait, not one per pair)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < NS; ++h) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const float4 a = lx[h].v[2 * qq], c = lx[h].v[2 * qq + 1];
            lx[h].s[qq] = 32.0f * (((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w)));
        }
    }
#pragma unroll
    for (int u = 0; u < R; ++u)
#pragma unroll
        for (int h = 0; h < NS; ++h) {
            const uint2 la = q6_piece(pc[u][h][0], sb), lb = q6_piece(pc[u][h][1], sb);
            const uint2 qh = q6_piece(pc[u][h][2], sb), sc = q6_piece(pc[u][h][3], sb);
            acc[u] += q6k_lane_dot(la.x, la.y, lb.x, lb.y, qh.x, qh.y, sc.x, sc.y, half_bits(dh[u][h]), lx[h], j);
        }
}

// Fast path. Row groups: when 8 | nb, group = one row and unit (row, slice s)
// starts at block ub0 + row*nb + 8s; when nb | 8, group = 8/nb rows (P) and
// unit u starts at block ub0 + 8u. A wave owns groups g0 .. g0+R-1.
template <int TYPE, int R>
__device__ __forceinline__ void gemv_kquant_body(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                 float* __restrict__ y, int M, int nb, uint64_t ub0, int groups,
                                                 uint64_t tensor_bytes, const Experts& ex, int sel,
                                                 int split = 0) {
    constexpr int BB = KQuant<TYPE>::kBlockBytes;
    constexpr int UB = 8 * BB;             // unit bytes
    constexpr int CPU = UB / 16;           // 16-byte chunks per unit
    constexpr int NC = (R * CPU + kWave - 1) / kWave;
    extern __shared__ uint4 gemv_stage[];
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    uint4* slot = gemv_stage + wv * (R * CPU);
    const int g0 = (blockIdx.x * kGemvWaves + wv) * R;
    const int b = lane >> 3, j = lane & 7;
    const bool packed = nb < 8;
    const int S = packed ? 1 : nb >> 3;
    const int P = packed ? 8 / nb : 1;     // rows per unit
    uint64_t eoff = 0;
    int64_t x_off, y_off;
    const bool ok_e = select_expert(ex, sel, M, x_off, y_off, eoff);
    x += x_off;
    y += y_off;
    if (!ok_e) {  // uniform per workgroup: no barrier is reached
        for (int r = g0 * P + lane; r < min((g0 + R) * P, M); r += kWave) y[r] = __builtin_nanf("");
        return;
    }
    ub0 += eoff / 256;

    float acc[R];
#pragma unroll
    for (int u = 0; u < R; ++u) acc[u] = 0.f;

    for (int s = 0; s < S; ++s) {
        LaneX<TYPE> lx;
        load_lane_x<TYPE>(lx, x, packed ? b % nb : 8 * s + b, j);
        uint4 ch[NC];
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            const int u = c / CPU;
            const int k = c - u * CPU;
            const int g = min(g0 + u, groups - 1);
            const uint64_t blk0 = packed ? ub0 + 8 * static_cast<uint64_t>(g)
                                         : ub0 + static_cast<uint64_t>(g) * nb + 8 * s;
            const uint64_t byte = blk0 * BB + 16 * static_cast<uint64_t>(k);
            // Only the tail unit of a packed tensor can reach past its end
            // (rows >= M); those chunks read as zeros and feed no output.
            const bool in = (i < NC - 1 || c < R * CPU) && byte + 16 <= tensor_bytes;
            ch[i] = in ? ld16_nt(w + byte) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            if (i < NC - 1 || c < R * CPU) slot[c] = ch[i];
        }
        __syncthreads();
        const uint8_t* base = reinterpret_cast<const uint8_t*>(slot);
#pragma unroll
        for (int u = 0; u < R; ++u) acc[u] += block_dot<TYPE>(base + u * UB + b * BB, lx, j);
        if (s + 1 < S) __syncthreads();
    }

    if (!packed) {
        float out = 0.f;
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const float t = group_sum<64>(acc[u]);
            if (lane == u) out = t;
        }
        if (lane < R && g0 + lane < M) y[out_index(g0 + lane, M, split)] = out;
    } else {
        // Lanes 8*nb*p .. 8*nb*(p+1)-1 hold row P*g + p.
        const int gl = 8 * nb;
#pragma unroll
        for (int u = 0; u < R; ++u) {
            float t;
            if (gl == 8) t = group_sum<8>(acc[u]);
            else if (gl == 16) t = group_sum<16>(acc[u]);
            else t = group_sum<32>(acc[u]);
            const int row = (g0 + u) * P + lane / gl;
            if (lane % gl == 0 && g0 + u < groups && row < M) y[out_index(row, M, split)] = t;
        }
    }
}

template <int TYPE, int R>
__global__ __launch_bounds__(kGemvBlock) void gemv_kquant(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int nb, uint64_t ub0,
                                                          int groups, uint64_t tensor_bytes, Experts ex) {
    gemv_kquant_body<TYPE, R>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, blockIdx.y);
}

// The Q4_K direct form of gemv_kquant_body for rows of whole units (8 | nb):
// same row groups, expert selection, lane map, block_dot_q4k and summation
// order (so the same bits), with the lane's quants loaded straight into VGPRs
// by q4k_direct_slices, NS (1 or 2, NS | nb / 8) slices at a time. Its own
// kernels, so that the LDS-staged form's registers do not count against it.
// Every exit before the slices is uniform per workgroup (the expert slot is
// blockIdx.y), so every thread that reaches a barrier has company.
template <int R, int NS, int LPH = 0, int NWV = kGemvWaves>
__device__ __forceinline__ void q4k_direct_body(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                float* __restrict__ y, int M, int nb, uint64_t ub0, int groups,
                                                uint64_t tensor_bytes, const Experts& ex, int sel, int split = 0,
                                                const NormGateX& ng = NormGateX{}, int bx = -1) {
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int g0 = ((bx < 0 ? static_cast<int>(blockIdx.x) : bx) * NWV + wv) * R;
    const int b = lane >> 3, j = lane & 7;
    const int S = nb >> 3;
    uint64_t eoff = 0;
    int64_t x_off, y_off;
    const bool ok_e = select_expert(ex, sel, M, x_off, y_off, eoff);
    x += x_off;
    y += y_off;
    if (!ok_e) {
        if (lane < R && g0 + lane < M) y[g0 + lane] = __builtin_nanf("");
        return;
    }
    ub0 += eoff / 256;
    __shared__ float4 xs[NS * 512];
    float acc[1][R];
#pragma unroll
    for (int u = 0; u < R; ++u) acc[0][u] = 0.f;
    const uint8_t* const wm[1] = {w};
    (void)tensor_bytes;
    q4k_direct_slices<R, NS, 1, LPH, NWV>(wm, x, xs, acc, nb, ub0, g0, groups, 0, b, j, ng);
    for (int s = NS; s < S; s += NS) {
        __syncthreads();   // every wave is done with the previous slices' x
        q4k_direct_slices<R, NS, 1, LPH, NWV>(wm, x, xs, acc, nb, ub0, g0, groups, s, b, j, ng);
    }
    float out = 0.f;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const float t = group_sum<64>(acc[0][u]);
        if (lane == u) out = t;
    }
    if (lane < R && g0 + lane < M) y[out_index(g0 + lane, M, split)] = out;
}

// The Q6_K direct form of gemv_kquant_body (rows of whole units): same row
// groups, expert selection, lane map, lane arithmetic (q6k_lane_dot) and
// summation order as the LDS-staged form, so the same bits.
template <int R, int NS>
__device__ __forceinline__ void q6k_direct_body(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                float* __restrict__ y, int M, int nb, uint64_t ub0, int groups,
                                                const Experts& ex, int sel, int split = 0, int bx = -1) {
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int g0 = ((bx < 0 ? static_cast<int>(blockIdx.x) : bx) * kGemvWaves + wv) * R;
    const int b = lane >> 3, j = lane & 7;
    const int S = nb >> 3;
    uint64_t eoff = 0;
    int64_t x_off, y_off;
    const bool ok_e = select_expert(ex, sel, M, x_off, y_off, eoff);
    x += x_off;
    y += y_off;
    if (!ok_e) {   // uniform per workgroup: no barrier is reached
        if (lane < R && g0 + lane < M) y[g0 + lane] = __builtin_nanf("");
        return;
    }
    ub0 += eoff / 256;
    __shared__ float4 xs[NS * 512];
    float acc[R];
#pragma unroll
    for (int u = 0; u < R; ++u) acc[u] = 0.f;
    q6k_direct_slices<R, NS>(w, x, xs, acc, nb, ub0, g0, groups, 0, b, j);
    for (int s = NS; s < S; s += NS) {
        __syncthreads();   // every wave is done with the previous slices' x
        q6k_direct_slices<R, NS>(w, x, xs, acc, nb, ub0, g0, groups, s, b, j);
    }
    float out = 0.f;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const float t = group_sum<64>(acc[u]);
        if (lane == u) out = t;
    }
    if (lane < R && g0 + lane < M) y[out_index(g0 + lane, M, split)] = out;
}

// EX: expert selection (ex.idx set); else a plain GEMV, whose kernel has the
// selection folded away (no scalar loads or branches before the first weight
// load: 3.1 against 2.9 us at 512 x 2048).
template <int R, int NS, bool EX>
__global__ __launch_bounds__(kGemvBlock) void gemv_q6k_direct(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x, float* __restrict__ y,
                                                              int M, int nb, uint64_t ub0, int groups, Experts ex) {
    q6k_direct_body<R, NS>(w, x, y, M, nb, ub0, groups, EX ? ex : Experts{nullptr, 0, 0, 0}, EX ? blockIdx.y : 0);
}

// EX: expert selection (ex.idx set); else a plain GEMV with the selection
// folded away (no scalar loads or branches before the first weight load).
template <int R, int NS, bool EX>
__global__ __launch_bounds__(kGemvBlock) void gemv_q4k_direct(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x, float* __restrict__ y,
                                                              int M, int nb, uint64_t ub0, int groups,
                                                              uint64_t tensor_bytes, Experts ex) {
    q4k_direct_body<R, NS>(w, x, y, M, nb, ub0, groups, tensor_bytes, EX ? ex : Experts{nullptr, 0, 0, 0},
                           EX ? blockIdx.y : 0);
}

// The gated per-head RMSNorm of x (core, heads of 4 LPH) followed by the GEMV
// on its output, one launch: every workgroup normalises the slices of x it
// stages (q4k_direct_slices with a NormGateX), workgroup 0 also writes them out.
// Every workgroup evaluates the norm (and the SiLU of z) for all of x: at
// 2048 x 4096 the launch takes 5.3 us against 4.0 for the GEMV on a ready x
// and 6.3 for the two launches; eight-wave workgroups (half the norm per
// thread, half the workgroups) measured 6.5 us, or 5.3 with one row per wave.
constexpr int kNormGateWaves = kGemvWaves;
template <int R, int NS, int LPH>
__global__ __launch_bounds__(kNormGateWaves * kWave) void gemv_q4k_norm_gate(const uint8_t* __restrict__ w,
                                                                           const float* __restrict__ core,
                                                                           NormGateX ng, float* __restrict__ y, int M,
                                                                           int nb, uint64_t ub0,
                                                                           uint64_t tensor_bytes) {
    q4k_direct_body<R, NS, LPH, kNormGateWaves>(w, core, y, M, nb, ub0, M, tensor_bytes, Experts{nullptr, 0, 0, 0},
                                                0, 0, ng);
}

// The routed experts' gate and up projections of one token in one launch:
// launch rows 0 .. n_sel-1 run the gate tensor, n_sel .. 2 n_sel-1 the up
// tensor, each for selection slot blockIdx.y mod n_sel (uniform per workgroup).
template <int TYPE, int R>
__global__ __launch_bounds__(kGemvBlock) void gemv_kquant_gate_up(const uint8_t* __restrict__ wg,
                                                                  const uint8_t* __restrict__ wu,
                                                                  const float* __restrict__ x, float* __restrict__ yg,
                                                                  float* __restrict__ yu, int M, int nb, int groups,
                                                                  uint64_t tensor_bytes, Experts ex, int n_sel) {
    const bool up = static_cast<int>(blockIdx.y) >= n_sel;
    gemv_kquant_body<TYPE, R>(up ? wu : wg, x, up ? yu : yg, M, nb, 0, groups, tensor_bytes, ex,
                              up ? static_cast<int>(blockIdx.y) - n_sel : static_cast<int>(blockIdx.y));
}

template <int R, int NS>
__global__ __launch_bounds__(kGemvBlock) void gemv_q4k_direct_gate_up(const uint8_t* __restrict__ wg,
                                                                      const uint8_t* __restrict__ wu,
                                                                      const float* __restrict__ x,
                                                                      float* __restrict__ yg, float* __restrict__ yu,
                                                                      int M, int nb, int groups,
                                                                      uint64_t tensor_bytes, Experts ex, int n_sel) {
    const bool up = static_cast<int>(blockIdx.y) >= n_sel;
    q4k_direct_body<R, NS>(up ? wu : wg, x, up ? yu : yg, M, nb, 0, groups, tensor_bytes, ex,
                           up ? static_cast<int>(blockIdx.y) - n_sel : static_cast<int>(blockIdx.y));
}

// The SwiGLU hidden rows of a MoE layer in one launch: h = SiLU(Wg x) * (Wu x)
// for the routed experts (launch rows 0 .. n_sel-1, expert ids on the device)
// and the shared expert (launch row n_sel). A wave takes R rows of both
// tensors -- 2R units staged in LDS, one set of x values for all of them --
// and evaluates each row as the per-row kernel does (same units, lane map and
// reductions) before SiLU(gate) * up, so h has the bits of the two GEMVs
// followed by moe_silu_mul. Rows of 8 | nb blocks (K a multiple of 2048).
//
// VPL > 0: the expert ids come from the router logits instead (routing fused
// in): wave 0 of every routed workgroup runs the top-k of the moe_topk_rows
// kernel (topk_row, the same code, so the same ids and weights) into LDS, and
// workgroup (0, 0) also writes ids and weights out for the later launches. A
// non-finite logit row makes every routed hidden row NaN.
struct PairJob {
    const uint8_t* wg;
    const uint8_t* wu;
    float* h;
    int M;
    Experts ex;     // idx == nullptr: no expert selection
};
struct RouteJob {
    const float* logits;   // n_experts router logits
    int32_t* idx;          // out: the n_sel picks
    float* w;              // out: their softmax weights
};

// The part of a SwiGLU launch before its rows: with VPL > 0 the routing (wave 0
// of every routed workgroup runs the top-k into LDS, workgroup (0, 0) writes the
// ids and weights out), then the expert selection of the workgroup's launch row.
// Sets h (the output rows) and ub (the expert's first block); false (after
// writing NaN rows) when the expert id is invalid. Every decision is uniform per
// workgroup.
template <int R, int VPL>
__device__ __forceinline__ bool swiglu_setup(const PairJob& jb, bool sh, int n_sel, const RouteJob& rt, int lane,
                                             int wv, int g0, float*& h, uint64_t& ub, int by = -1, int bx = -1) {
    if (by < 0) {
        by = static_cast<int>(blockIdx.y);
        bx = static_cast<int>(blockIdx.x);
    }
    Experts ex = jb.ex;
    if constexpr (VPL > 0) {
        __shared__ int32_t sidx[kWave];
        if (!sh) {   // uniform per workgroup
            if (wv == 0) {
                int pi;
                float pw;
                const bool fin = topk_row<VPL>(rt.logits, ex.n_experts, n_sel, pi, pw);
                if (lane < n_sel) sidx[lane] = fin ? pi : -1;
                if (bx == 0 && by == 0) {
                    if (fin && lane < n_sel) {
                        rt.idx[lane] = pi;
                        rt.w[lane] = pw;
                    } else if (!fin && lane == 0) {
                        rt.idx[0] = -1;
                        rt.w[0] = __builtin_nanf("");
                    }
                }
            }
            __syncthreads();
            ex.idx = sidx;
        }
    }
    uint64_t eoff = 0;
    int64_t x_off, y_off;
    const bool ok_e = select_expert(ex, sh ? 0 : by, jb.M, x_off, y_off, eoff);
    h = jb.h + y_off;
    if (!ok_e) {
        if (lane < R && g0 + lane < jb.M) h[g0 + lane] = __builtin_nanf("");
        return false;
    }
    ub = eoff / 256;
    return true;
}

template <int TYPE, int R, int VPL>
__global__ __launch_bounds__(kGemvBlock) void gemv_kquant_swiglu(const float* __restrict__ x, int nb, PairJob routed,
                                                                 PairJob shared, int n_sel, RouteJob rt) {
    constexpr int BB = KQuant<TYPE>::kBlockBytes;
    constexpr int UB = 8 * BB;
    constexpr int CPU = UB / 16;
    constexpr int NC = (2 * R * CPU + kWave - 1) / kWave;
    extern __shared__ uint4 gemv_stage[];
    const bool sh = static_cast<int>(blockIdx.y) == n_sel;
    const PairJob& jb = sh ? shared : routed;
    if (static_cast<int64_t>(blockIdx.x) * kGemvWaves * R >= jb.M) return;   // uniform per workgroup
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    uint4* slot = gemv_stage + wv * (2 * R * CPU);
    const int g0 = (blockIdx.x * kGemvWaves + wv) * R;
    const int b = lane >> 3, j = lane & 7;
    const int S = nb >> 3;
    float* h;
    uint64_t ub;
    if (!swiglu_setup<R, VPL>(jb, sh, n_sel, rt, lane, wv, g0, h, ub)) return;   // uniform per workgroup

    float ag[R], au[R];
#pragma unroll
    for (int u = 0; u < R; ++u) ag[u] = au[u] = 0.f;
    for (int s = 0; s < S; ++s) {
        LaneX<TYPE> lx;
        load_lane_x<TYPE>(lx, x, 8 * s + b, j);
        uint4 ch[NC];
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            const int u = c / CPU;                   // 0 .. R-1 gate, R .. 2R-1 up
            const int k = c - u * CPU;
            const int g = min(g0 + (u < R ? u : u - R), jb.M - 1);
            const uint64_t byte = (ub + static_cast<uint64_t>(g) * nb + 8 * s) * BB + 16 * static_cast<uint64_t>(k);
            const bool in = i < NC - 1 || c < 2 * R * CPU;
            ch[i] = in ? ld16_nt((u < R ? jb.wg : jb.wu) + byte) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            if (i < NC - 1 || c < 2 * R * CPU) slot[c] = ch[i];
        }
        __syncthreads();
        const uint8_t* base = reinterpret_cast<const uint8_t*>(slot);
#pragma unroll
        for (int u = 0; u < R; ++u) {
            ag[u] += block_dot<TYPE>(base + u * UB + b * BB, lx, j);
            au[u] += block_dot<TYPE>(base + (R + u) * UB + b * BB, lx, j);
        }
        if (s + 1 < S) __syncthreads();
    }
    float out = 0.f;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const float tg = group_sum<64>(ag[u]);
        const float tu = group_sum<64>(au[u]);
        if (lane == u) out = silu(tg) * tu;
    }
    if (lane < R && g0 + lane < jb.M) h[g0 + lane] = out;
}

// gemv_kquant_swiglu for Q4_K in the direct form (q4k_direct_slices with the
// gate and up rows of the wave, one staged x for both): same rows, reductions
// and bits.
// One flat grid: workgroups [0, n_sel nr) take the routed slots (nr each),
// the ns after them the shared rows.
template <int R, int NS, int VPL>
__global__ __launch_bounds__(kGemvBlock) void gemv_q4k_direct_swiglu(const float* __restrict__ x, int nb,
                                                                     PairJob routed, PairJob shared, int n_sel,
                                                                     RouteJob rt, int nr) {
    const int fb = static_cast<int>(blockIdx.x);
    const bool sh = fb >= n_sel * nr;
    const int by = sh ? n_sel : fb / nr;
    const int bx = sh ? fb - n_sel * nr : fb - by * nr;
    const PairJob& jb = sh ? shared : routed;
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    const int g0 = (bx * kGemvWaves + wv) * R;
    const int b = lane >> 3, j = lane & 7;
    const int S = nb >> 3;
    float* h;
    uint64_t ub;
    if (!swiglu_setup<R, VPL>(jb, sh, n_sel, rt, lane, wv, g0, h, ub, by, bx)) return;   // uniform per workgroup
    __shared__ float4 xs[NS * 512];
    float acc[2][R];
#pragma unroll
    for (int u = 0; u < R; ++u) acc[0][u] = acc[1][u] = 0.f;
    const uint8_t* const wm[2] = {jb.wg, jb.wu};
    q4k_direct_slices<R, NS, 2>(wm, x, xs, acc, nb, ub, g0, jb.M, 0, b, j);
    for (int s = NS; s < S; s += NS) {
        __syncthreads();   // every wave is done with the previous slices' x
        q4k_direct_slices<R, NS, 2>(wm, x, xs, acc, nb, ub, g0, jb.M, s, b, j);
    }
    float out = 0.f;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const float tg = group_sum<64>(acc[0][u]);
        const float tu = group_sum<64>(acc[1][u]);
        if (lane == u) out = silu(tg) * tu;
    }
    if (lane < R && g0 + lane < jb.M) h[g0 + lane] = out;
}

// Several matrices of one type against the same x (qwen_matmul_dispatch_multi):
// launch row blockIdx.y runs matrix d[blockIdx.y]; the grid is sized for the
// largest, and workgroups past a smaller matrix's rows return at once.
constexpr int kMultiMax = 8;
struct GemvMat {
    const uint8_t* w;
    float* y;
    uint64_t ub0;           // first block of row 0
    uint64_t tensor_bytes;  // bytes of the whole tensor
    int M;
    int groups;
    int split;              // out_index layout (0: y[m] = row m)
};
struct GemvMulti {
    GemvMat d[kMultiMax];
    int start[kMultiMax + 1];   // direct form: workgroups [start[j], start[j+1]) run matrix j
};

template <int TYPE, int R>
__global__ __launch_bounds__(kGemvBlock) void gemv_kquant_multi(const float* __restrict__ x, int nb, GemvMulti mu) {
    const GemvMat& m = mu.d[blockIdx.y];
    if (static_cast<int64_t>(blockIdx.x) * kGemvWaves * R >= m.groups) return;   // uniform per workgroup
    gemv_kquant_body<TYPE, R>(m.w, x, m.y, m.M, nb, m.ub0, m.groups, m.tensor_bytes, Experts{nullptr, 0, 0, 0}, 0,
                              m.split);
}

// One flat grid: workgroup b runs block b - start[j] of matrix j, start[j] <= b <
// start[j+1] (every workgroup has rows; a grid sized for the largest matrix per
// launch row left most of the small matrices' workgroups with nothing to do).
template <int R, int NS>
__global__ __launch_bounds__(kGemvBlock) void gemv_q4k_direct_multi(const float* __restrict__ x, int nb,
                                                                    GemvMulti mu, int n) {
    const int b = static_cast<int>(blockIdx.x);
    int j = 0;
    while (j + 1 < n && mu.start[j + 1] <= b) ++j;   // uniform per workgroup
    const GemvMat& m = mu.d[j];
    q4k_direct_body<R, NS>(m.w, x, m.y, m.M, nb, m.ub0, m.groups, m.tensor_bytes, Experts{nullptr, 0, 0, 0}, 0,
                           m.split, NormGateX{}, b - mu.start[j]);
}

template <int R, int NS>
__global__ __launch_bounds__(kGemvBlock) void gemv_q6k_direct_multi(const float* __restrict__ x, int nb,
                                                                    GemvMulti mu, int n) {
    const int b = static_cast<int>(blockIdx.x);
    int j = 0;
    while (j + 1 < n && mu.start[j + 1] <= b) ++j;   // uniform per workgroup
    const GemvMat& m = mu.d[j];
    q6k_direct_body<R, NS>(m.w, x, m.y, m.M, nb, m.ub0, m.groups, Experts{nullptr, 0, 0, 0}, 0, m.split,
                           b - mu.start[j]);
}

// ------------------------------------------------------------ MoE down + combine
// The rest of a MoE layer's decode step after the SwiGLU hidden rows
// (src/layer_moe.cpp:135-147) in one launch, for routed experts of inter = 512
// (2 blocks per row: rows 4q .. 4q+3 of one expert are one 8-block unit) and
// a shared expert of shared_dim = 2048 * SS. A workgroup owns output rows
// 4q .. 4q+3; wave w
//   * decodes the unit of rows 4q .. 4q+3 of routed expert j = w + 4t (t < KT)
//     against that expert's hidden row;
//   * computes row 4q + w of the shared expert's down projection;
// with the per-row kernel's units, lane map and reductions, so each expert
// output and the shared output have the bits of the separate launches (the
// expert GEMVs, the shared GEMV). Lanes 0..3 of wave 0 then combine
// row 4q + lane in the reference's order (moe_add per expert from a zeroed
// accumulator, then the gated shared add): acc = 0; acc = fma(w_j, e_j, acc)
// for j < k; acc += shared * sigmoid(logit).
constexpr int kDcInter = 512;

template <int TE, int TS, int KT, int SS>
__global__ __launch_bounds__(kGemvBlock) void moe_down_combine_kernel(
        const uint8_t* __restrict__ wd, uint64_t expert_blocks, int n_experts, const int32_t* __restrict__ idx,
        const float* __restrict__ wts, int k, const float* __restrict__ hid, const uint8_t* __restrict__ wsd,
        const float* __restrict__ shid, const float* __restrict__ slogit, float* __restrict__ out) {
    constexpr int BE = KQuant<TE>::kBlockBytes, BS = KQuant<TS>::kBlockBytes;
    constexpr int CE = BE * 8 / 16, CS = BS * 8 / 16;   // 16-byte chunks per unit (72 or 105)
    static_assert(CE > kWave && CE <= 2 * kWave && CS > kWave && CS <= 2 * kWave, "two chunks per lane");
    constexpr int SLOT = KT * CE + SS * CS;
    __shared__ uint4 stage[kGemvWaves][SLOT];
    __shared__ float part[4 * KT][4];
    __shared__ float spart[4];
    const int lane = threadIdx.x & 63, w = wave_in_block();
    const int b = lane >> 3, jj = lane & 7;
    const int q = blockIdx.x;
    const bool tail = lane + kWave < CE;

    // Every unit's bytes requested before the first wait.
    uint4 ce[KT][2], cs[SS][2];
    bool valid[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int j = w + 4 * t;
        const int e = j < k ? idx[j] : 0;
        valid[t] = e >= 0 && e < n_experts;
        const uint8_t* unit = wd + (static_cast<uint64_t>(valid[t] ? e : 0) * expert_blocks + 8 * q) * BE;
        ce[t][0] = ld16_nt(unit + 16 * lane);
        ce[t][1] = tail ? ld16_nt(unit + 16 * (lane + kWave)) : make_uint4(0, 0, 0, 0);
    }
    const int row = 4 * q + w;
#pragma unroll
    for (int s = 0; s < SS; ++s) {
        const uint8_t* unit = wsd + (static_cast<uint64_t>(row) * 8 * SS + 8 * s) * BS;
        cs[s][0] = ld16_nt(unit + 16 * lane);
        cs[s][1] = lane + kWave < CS ? ld16_nt(unit + 16 * (lane + kWave)) : make_uint4(0, 0, 0, 0);
    }
    LaneX<TE> lxe[KT];
    LaneX<TS> lxs[SS];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int j = min(w + 4 * t, k - 1);
        load_lane_x<TE>(lxe[t], hid + static_cast<size_t>(j) * kDcInter, b & 1, jj);
    }
#pragma unroll
    for (int s = 0; s < SS; ++s) load_lane_x<TS>(lxs[s], shid, 8 * s + b, jj);

    uint4* slot = stage[w];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        slot[t * CE + lane] = ce[t][0];
        if (tail) slot[t * CE + kWave + lane] = ce[t][1];
    }
#pragma unroll
    for (int s = 0; s < SS; ++s) {
        slot[KT * CE + s * CS + lane] = cs[s][0];
        if (lane + kWave < CS) slot[KT * CE + s * CS + kWave + lane] = cs[s][1];
    }
    __syncthreads();
    const uint8_t* base = reinterpret_cast<const uint8_t*>(slot);
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        float a = 0.f;
        a += block_dot<TE>(base + t * CE * 16 + b * BE, lxe[t], jj);
        a = group_sum<16>(a);
        const int j = w + 4 * t;
        if (j < k && (lane & 15) == 0) part[j][lane >> 4] = valid[t] ? a : __builtin_nanf("");
    }
    {
        float a = 0.f;
#pragma unroll
        for (int s = 0; s < SS; ++s) a += block_dot<TS>(base + (KT * CE + s * CS) * 16 + b * BS, lxs[s], jj);
        a = group_sum<64>(a);
        if (lane == 0) spart[w] = a;
    }
    __syncthreads();
    if (w == 0 && lane < 4) {
        float acc = 0.f;
        for (int j = 0; j < k; ++j) acc = __builtin_fmaf(wts[j], part[j][lane], acc);
        const float sc = sigmoid(slogit[0]);
        acc += spart[lane] * sc;
        out[4 * q + lane] = acc;
    }
}

// moe_down_combine_kernel for Q4_K routed and shared tensors: the same rows,
// lane map, block_dot_q4k, reductions and combine (so the same bits), with
// every wave's quants loaded straight into VGPRs (144-byte blocks are 16-byte
// aligned: lane L takes block L/8's header and its own 16 qs bytes) and the
// hidden rows the workgroup reads -- routed rows 0 .. 4 KT - 1 (row j clamped to
// k - 1) and the shared row -- loaded once per workgroup, before the weights,
// and staged in LDS (loaded per wave they were 3x the weight bytes, and every
// workgroup reads the same rows).
template <int KT, int SS>
__global__ __launch_bounds__(kGemvBlock) void moe_down_combine_q4k(
        const uint8_t* __restrict__ wd, uint64_t expert_blocks, int n_experts, const int32_t* __restrict__ idx,
        const float* __restrict__ wts, int k, const float* __restrict__ hid, const uint8_t* __restrict__ wsd,
        const float* __restrict__ shid, const float* __restrict__ slogit, float* __restrict__ out) {
    constexpr int BB = KQuant<kQ4_K>::kBlockBytes;
    constexpr int NXR = 4 * KT * (kDcInter / 4);   // float4 of the routed hidden rows
    constexpr int NXS = SS * 512;                  // float4 of the shared hidden row (2048 SS)
    constexpr int PR = NXR / kGemvBlock, PS = NXS / kGemvBlock;
    static_assert(PR * kGemvBlock == NXR && PS * kGemvBlock == NXS, "x staging");
    __shared__ float4 xr[NXR];
    __shared__ float4 xsh[NXS];
    __shared__ float part[4 * KT][4];
    __shared__ float spart[4];
    const int lane = threadIdx.x & 63, w = wave_in_block();
    const int b = lane >> 3, jj = lane & 7;
    const int q = blockIdx.x;

    float4 tr[PR], ts[PS];
#pragma unroll
    for (int i = 0; i < PR; ++i) {
        const int c = threadIdx.x + i * kGemvBlock;
        const int jr = min(c / (kDcInter / 4), k - 1);
        tr[i] = ld4(hid + static_cast<size_t>(jr) * kDcInter + 4 * (c % (kDcInter / 4)));
    }
#pragma unroll
    for (int i = 0; i < PS; ++i) ts[i] = ld4(shid + 4 * (threadIdx.x + i * kGemvBlock));
    __builtin_amdgcn_sched_barrier(0);   // the hidden rows first

    uint4 he[KT], qe[KT], hs[SS], qs[SS];
    bool valid[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int j = w + 4 * t;
        const int e = j < k ? idx[j] : 0;
        valid[t] = e >= 0 && e < n_experts;
        const uint8_t* blk = wd + (static_cast<uint64_t>(valid[t] ? e : 0) * expert_blocks + 8 * q + b) * BB;
        he[t] = ld16_nt(blk);
        qe[t] = ld16_nt(blk + 16 + 16 * jj);
    }
    const int row = 4 * q + w;
#pragma unroll
    for (int s = 0; s < SS; ++s) {
        const uint8_t* blk = wsd + (static_cast<uint64_t>(row) * 8 * SS + 8 * s + b) * BB;
        hs[s] = ld16_nt(blk);
        qs[s] = ld16_nt(blk + 16 + 16 * jj);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before the staging
#pragma unroll
    for (int i = 0; i < PR; ++i) xr[threadIdx.x + i * kGemvBlock] = tr[i];
#pragma unroll
    for (int i = 0; i < PS; ++i) xsh[threadIdx.x + i * kGemvBlock] = ts[i];
    __syncthreads();

    const int xo = 64 * (jj >> 1) + 16 * (jj & 1);   // load_lane_x_values' offsets in a 256-element block
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int j = w + 4 * t;
        LaneX<kQ4_K> lx;
        const float4* lo = xr + (min(j, k - 1) * kDcInter + (b & 1) * 256 + xo) / 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lx.v[i] = lo[i];
            lx.v[4 + i] = lo[8 + i];
        }
        lane_x_sums(lx);
        float a = 0.f;
        a += block_dot_q4k(he[t], qe[t], lx, jj);
        a = group_sum<16>(a);
        if (j < k && (lane & 15) == 0) part[j][lane >> 4] = valid[t] ? a : __builtin_nanf("");
    }
    {
        float a = 0.f;
#pragma unroll
        for (int s = 0; s < SS; ++s) {
            LaneX<kQ4_K> lx;
            const float4* lo = xsh + ((8 * s + b) * 256 + xo) / 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lx.v[i] = lo[i];
                lx.v[4 + i] = lo[8 + i];
            }
            lane_x_sums(lx);
            a += block_dot_q4k(hs[s], qs[s], lx, jj);
        }
        a = group_sum<64>(a);
        if (lane == 0) spart[w] = a;
    }
    __syncthreads();
    if (w == 0 && lane < 4) {
        float acc = 0.f;
        for (int j = 0; j < k; ++j) acc = __builtin_fmaf(wts[j], part[j][lane], acc);
        const float sc = sigmoid(slogit[0]);
        acc += spart[lane] * sc;
        out[4 * q + lane] = acc;
    }
}

__global__ __launch_bounds__(kBlock) void fill_zero(float* __restrict__ p, int n) {
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) p[i] = 0.f;
}

// Generic path (any supported type and shape): one wave per row, element-wise
// decode.
__global__ __launch_bounds__(kBlock) void gemv_any(const uint8_t* __restrict__ w, int type,
                                                   const float* __restrict__ x, float* __restrict__ y, int M, int K,
                                                   uint64_t element_offset, Experts ex, int split) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kBlock / kWave) + wave_in_block();
    if (row >= M) return;
    int64_t x_off, y_off;
    const bool ok_e = select_expert(ex, blockIdx.y, M, x_off, y_off, element_offset);
    x += x_off;
    y += y_off;
    if (!ok_e) {
        if (lane == 0) y[row] = __builtin_nanf("");
        return;
    }
    const uint64_t base = element_offset + static_cast<uint64_t>(row) * K;
    float s = 0.f;
    for (int k = lane; k < K; k += kWave) s = __builtin_fmaf(dequant_elem(w, type, base + k), x[k], s);
    s = group_sum<64>(s);
    if (lane == 0) y[out_index(row, M, split)] = s;
}

// ------------------------------------------------------------------ MFMA path
// Q4_K / Q6_K, K = 256*nb with nb = S*BPW (S in {1, 2, 4} k-slices of BPW in
// 1..4 blocks, so K <= 4096): the dot products run on the matrix cores
// (v_mfma_i32_16x16x64_i8, exact int8 x int8 -> int32).
//
// x is written in integer digits. Over a wave's k-slice, with
// F = 26 - exponent(max |x|), X = rint(x * 2^F) is an integer of at most 27
// bits, split into four signed base-128 digits
//   X = D0*2^21 + D1*2^14 + D2*2^7 + D3,  D1..D3 in [-64, 63], |D0| <= 33.
// The quants are small non-negative integers (Q4_K 0..15, Q6_K 0..63), so a
// tile of 16 weight rows x 64 elements (a chunk) is an int8 B operand taken
// straight from the nibbles, and the A operand holds the digits: A row 4g + i
// is digit i of elements 16g .. 16g+15 of the chunk and zero elsewhere, so
// C[4g+i][n] is the exact integer sum over the 16-element group g of row n,
// digit i. In the 16x16 result layout lane L holds rows 4(L/16)..4(L/16)+3 of
// column L%16: one (weight row n = L%16, group g = L/16) with its four digit
// sums, and that is also the lane that reads row n's quants of group g for B
// (the A and B layouts place element k of the chunk at the same (lane group,
// byte) position, so the product pairs them whatever order the hardware sums
// in). Per lane and chunk:
//   P = sum_i (digit-i sum) * 2^(21-7i)   (the exact integer sum of q*X, one rounding)
//   Q6_K: acc += (d*sc) * (P*2^-F - 32 * sum(X)*2^-F)            (q - 32)
//   Q4_K: acc += (d*sc) * (P*2^-F) - (dmin*m) * sum(X)*2^-F
// with the group sums of X computed once per wave. The only roundings are
// x -> X (|dX| <= 2^-F / 2, at most 2^-26 of the slice's largest |x|), the
// int32 -> fp32 steps and the fp32 sums, so the result matches the
// reference's fp32 dot product to ~1e-7 of the row's sum of |w*x|. A
// non-finite x switches the launch to the per-element form (the reference's
// products).
//
// Work: a workgroup of 4 waves owns 4/S tile slots x S k-slices; wave
// (slot, r) runs tiles_per_slot tiles of 16 rows over blocks
// [r*BPW, (r+1)*BPW). It converts its slice of x once (digits in VGPRs as
// the A operands of all its tiles). Each tile's quantized rows are copied to
// the wave's LDS slot with coalesced 16-byte loads (a block of a row is 14 x
// 16 B for Q6_K -- the last piece overlapping, since 210 B blocks are only
// 2-byte aligned -- or 9 x 16 B for Q4_K; LDS rows padded by 16 B so the
// per-lane reads of 16 rows hit distinct banks); the next tile's loads are in
// flight while the current one is computed. The S partial sums of a row are
// added in k-slice order through LDS at the end (deterministic).
constexpr int kMfmaWaves = 4;
constexpr int kMfmaBlock = kMfmaWaves * kWave;

typedef int v4i_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i_t mfma_i8(v4i_t a, v4i_t b) {
    const v4i_t z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, z, 0, 0, 0);
}

// 16 bytes of global memory at a 2-byte aligned address (gfx950 global loads
// take any byte alignment).
__device__ __forceinline__ uint4 ldg16_a2(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 16);
    return v;
}

// Signed bit field (the builtin's result type is unsigned).
__device__ __forceinline__ int sbfe(uint32_t v, uint32_t off, uint32_t width) {
    return static_cast<int>(__builtin_amdgcn_sbfe(v, off, width));
}

// (a & 0x0f0f0f0f) | (b & 0xf0f0f0f0): low nibbles from a, high from b.
__device__ __forceinline__ uint32_t nibble_merge(uint32_t a, uint32_t b) {
    return (a & 0x0f0f0f0fu) | (b & 0xf0f0f0f0u);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Sum over the four lanes L, L^16, L^32, L^48 (the four groups of a row).
__device__ __forceinline__ float sum_groups(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Per-lane constants of the B decode.
struct Lane {
    int g;            // group: elements 16g .. 16g+15 of each 64-element chunk
    uint32_t hmask;   // Q6_K: the two 2-bit fields of qh this lane's group uses
    int hl, hr;       // Q6_K: shifts that put them at bits 4, 5 (even / odd chunk)
    int ns;           // Q4_K: nibble shift
};

template <int TYPE>
struct MfmaType;

// Q6_K element i: ql byte 64(i/128) + 32((i%128)/32 & 1) + i%32 (low nibble in
// quarters 0, 1, high in 2, 3), qh byte 128 + 32(i/128) + i%32 bits
// 2*quarter, scale byte 192 + 8(i/128) + (i%32)/16 + 2*quarter, d at 208
// (src/cuda/matmul_q4.cu:105-126). For i = 64cb + 16g + p (chunk cb of the
// block) that is ql byte 64(cb/2) + 16g + p, qh byte 128 + 32(cb/2) +
// 16(g%2) + p, quarter 2(cb%2) + g/2, scale byte 192 + 4cb + g. In LDS a block
// is 224 bytes: its bytes 0..207, then bytes 194..209 at 208 (d at 222).
template <>
struct MfmaType<kQ6_K> {
    static constexpr int kBytes = 210;
    static constexpr int kPieces = 14;   // 16-byte pieces per block
    static constexpr int kLast = 194;    // offset of the last (overlapping) piece
    static constexpr float kXs = -32.0f; // q - 32

    // Quants of chunks 2h (low nibbles, qh bits 2(g/2)) and 2h+1 (high nibbles,
    // qh bits 4 + 2(g/2)) as int8 operands: the two qh fields are masked once
    // (bits 6, 7 of each byte end up zero) and moved to bits 4, 5.
    __device__ __forceinline__ static void quants(uint32_t l, uint32_t h, const Lane& ln, int& even, int& odd) {
        const uint32_t hm = h & ln.hmask;
        even = static_cast<int>(nibble_merge(l, hm << ln.hl));
        odd = static_cast<int>(nibble_merge(l >> 4, hm >> ln.hr));
    }

    // One block (LDS bytes at blk) against the digits a[4] of its 4 chunks.
    __device__ __forceinline__ static float block(const uint8_t* blk, const v4i_t* a, const float* xs, float scale,
                                                  const Lane& ln, float acc) {
        const uint4 sc = *reinterpret_cast<const uint4*>(blk + 192);
        const float dh = half_bits(*reinterpret_cast<const uint16_t*>(blk + 222));
        const uint32_t sw[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
        for (int h = 0; h < 2; ++h) {   // chunks 2h, 2h+1 share their ql and qh bytes
            const uint4 ql = *reinterpret_cast<const uint4*>(blk + 64 * h + 16 * ln.g);
            const uint4 qh = *reinterpret_cast<const uint4*>(blk + 128 + 32 * h + 16 * (ln.g & 1));
            const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w}, H[4] = {qh.x, qh.y, qh.z, qh.w};
            int q[2][4];   // [chunk][dword]
#pragma unroll
            for (int j = 0; j < 4; ++j) quants(L[j], H[j], ln, q[0][j], q[1][j]);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int cb = 2 * h + e;
                const v4i_t c = mfma_i8(a[cb], v4i_t{q[e][0], q[e][1], q[e][2], q[e][3]});
                const int t = (c.x * 128 + c.y) * 128 + c.z;   // exact: |t| < 2^30
                const float P = fmaf(static_cast<float>(t), 128.0f, static_cast<float>(c.w));
                const float dsc = dh * static_cast<float>(sbfe(sw[cb], 8 * ln.g, 8));
                acc = fmaf(dsc, fmaf(P, scale, xs[cb]), acc);
            }
        }
        return acc;
    }
};

// Q4_K element i: qs byte 16 + 32(i/64) + i%32, low nibble if i%64 < 32,
// sub-block i/32 with scale_min_k4 (src/cuda/matmul_q4.cu:18-26,76-96); for
// i = 64cb + 16g + p that is qs byte 16 + 32cb + 16(g%2) + p, nibble g/2,
// sub-block 2cb + g/2. In LDS a block is its 144 bytes.
template <>
struct MfmaType<kQ4_K> {
    static constexpr int kBytes = 144;
    static constexpr int kPieces = 9;
    static constexpr int kLast = 128;
    static constexpr float kXs = 1.0f;

    __device__ __forceinline__ static float block(const uint8_t* blk, const v4i_t* a, const float* xs, float scale,
                                                  const Lane& ln, float acc) {
        const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
        uint4 qs[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) qs[cb] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * cb + 16 * (ln.g & 1));
        const float dh = half_bits(hdr.x & 0xffffu), dm = half_bits(hdr.x >> 16);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const uint4 Q = qs[cb];
            const v4i_t b = {static_cast<int>((Q.x >> ln.ns) & 0x0f0f0f0fu), static_cast<int>((Q.y >> ln.ns) & 0x0f0f0f0fu),
                             static_cast<int>((Q.z >> ln.ns) & 0x0f0f0f0fu), static_cast<int>((Q.w >> ln.ns) & 0x0f0f0f0fu)};
            const v4i_t c = mfma_i8(a[cb], b);
            const int t = (c.x * 128 + c.y) * 128 + c.z;
            const float P = fmaf(static_cast<float>(t), 128.0f, static_cast<float>(c.w));
            // byte j%4 (j = 2cb + g/2) of scale words 0..2 (hdr.y, hdr.z, hdr.w) sits at bit bt.
            const uint32_t bt = 16 * (cb & 1) + 8 * (ln.g >> 1);
            uint32_t sc, mn;
            if (cb < 2) {
                sc = __builtin_amdgcn_ubfe(hdr.y, bt, 6);
                mn = __builtin_amdgcn_ubfe(hdr.z, bt, 6);
            } else {
                sc = __builtin_amdgcn_ubfe(hdr.w, bt, 4) | (__builtin_amdgcn_ubfe(hdr.y, bt + 6, 2) << 4);
                mn = __builtin_amdgcn_ubfe(hdr.w, bt + 4, 4) | (__builtin_amdgcn_ubfe(hdr.z, bt + 6, 2) << 4);
            }
            acc = fmaf(dh * static_cast<float>(sc), P * scale, acc);
            acc = fmaf(-(dm * static_cast<float>(mn)), xs[cb], acc);
        }
        return acc;
    }
};

// LDS layout of a wave's slot: 16 rows of BPW blocks of kPieces x 16 bytes,
// each row padded to an odd number of 16-byte units (16 rows at that stride
// start on distinct banks).
template <int TYPE, int BPW>
struct MfmaSlot {
    using T = MfmaType<TYPE>;
    static constexpr int kBlockLds = 16 * T::kPieces;
    static constexpr int kRowLds = BPW * kBlockLds + ((BPW * T::kPieces) % 2 ? 32 : 16);   // odd x 16 B
    static constexpr int kBytes = 16 * kRowLds;
    static constexpr int kLoads = 16 * BPW * T::kPieces;              // 16-byte pieces per tile
    static constexpr int kPerLane = (kLoads + kWave - 1) / kWave;
};

// Occupancy: 4 waves per SIMD (<= 128 VGPRs) for slices of up to 2 blocks.
template <int TYPE, int BPW>
__global__ __launch_bounds__(kMfmaBlock) __attribute__((amdgpu_waves_per_eu(BPW <= 2 ? 4 : 2))) void gemv_mfma(
    const uint8_t* __restrict__ w, int type, const float* __restrict__ x, float* __restrict__ y, int M, int nb,
    uint64_t ub0, int tiles, int S, int maxcnt) {
    using T = MfmaType<TYPE>;
    using Slot = MfmaSlot<TYPE, BPW>;
    constexpr int NC = 4 * BPW;   // chunks per k-slice
    extern __shared__ uint4 mfma_lds[];
    const int lane = threadIdx.x & 63;
    const int wv = wave_in_block();
    uint8_t* slot = reinterpret_cast<uint8_t*>(mfma_lds) + wv * Slot::kBytes;
    float* part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(mfma_lds) + kMfmaWaves * Slot::kBytes);
    const int g = lane >> 4, n = lane & 15;
    const int slots = kMfmaWaves / S;
    const int r = wv % S, sl = wv / S;
    // Slot u of U runs tiles u, u + U, u + 2U, ... (at most maxcnt): at any
    // time the whole grid streams through one region of the matrix, which
    // keeps DRAM pages open (contiguous ranges per slot measured 8% slower).
    const int U = gridDim.x * slots, t0 = blockIdx.x * slots + sl;
    const int cnt = t0 < tiles ? (tiles - 1 - t0) / U + 1 : 0;
    const uint64_t row_bytes = static_cast<uint64_t>(nb) * T::kBytes;

    // This lane's 16-byte pieces of a tile: piece q = lane + 64i is (row,
    // block, piece j) of the tile, packed as row | j << 4 | block << 8.
    uint32_t pc[Slot::kPerLane];
#pragma unroll
    for (int i = 0; i < Slot::kPerLane; ++i) {
        const int q = min(lane + kWave * i, Slot::kLoads - 1);
        const int row = q / (BPW * T::kPieces), rem = q % (BPW * T::kPieces);
        pc[i] = static_cast<uint32_t>(row | (rem % T::kPieces) << 4 | (rem / T::kPieces) << 8);
    }
    const uint8_t* wslice = w + ub0 * T::kBytes + static_cast<uint64_t>(r * BPW) * T::kBytes;
    auto load_tile = [&](uint4 (&v)[Slot::kPerLane], int t) {
#pragma unroll
        for (int i = 0; i < Slot::kPerLane; ++i) {
            const int row = min(t * 16 + static_cast<int>(pc[i] & 15), M - 1);
            const uint32_t off = (pc[i] >> 8) * T::kBytes + min(16 * ((pc[i] >> 4) & 15), static_cast<uint32_t>(T::kLast));
            v[i] = ldg16_a2(wslice + static_cast<uint64_t>(row) * row_bytes + off);
        }
    };
    auto store_tile = [&](const uint4 (&v)[Slot::kPerLane]) {
#pragma unroll
        for (int i = 0; i < Slot::kPerLane; ++i)
            if (i < Slot::kPerLane - 1 || lane + kWave * i < Slot::kLoads)
                *reinterpret_cast<uint4*>(slot + (pc[i] & 15) * Slot::kRowLds + (pc[i] >> 8) * Slot::kBlockLds +
                                          16 * ((pc[i] >> 4) & 15)) = v[i];
    };

    // The first tile's loads go out before x is converted.
    uint4 pre[Slot::kPerLane];
    if (cnt > 0) load_tile(pre, t0);

    // x of this k-slice: element 256*r*BPW + 64c + lane of chunk c < NC.
    const float* xs_base = x + 256 * r * BPW;
    float xv[NC];
    bool fin = true;
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        xv[c] = xs_base[64 * c + lane];
        fin = fin && __builtin_isfinite(xv[c]);
        amax = fmaxf(amax, fabsf(xv[c]));
    }
    const bool nonfinite = __builtin_amdgcn_ballot_w64(!fin) != 0;   // wave-uniform
    amax = wave_max(nonfinite ? 0.0f : amax);
    // amax < 2^e, so |x| * 2^F < 2^26. Slices with amax outside [2^-100, 2^100]
    // take the per-element form too: there 2^-F would leave the normal range
    // or P * 2^-F could overflow before the block scale shrinks it.
    const int e = __builtin_amdgcn_frexp_expf(amax);
    const bool bad = nonfinite || (amax > 0.0f && (e < -100 || e > 100));
    const int F = amax > 0.0f && !bad ? 26 - e : 0;
    const float scale = __builtin_amdgcn_ldexpf(1.0f, -F);
    // Digits through the slot (before any tile is stored there): chunk c as
    // [g][digit][p], 256 bytes; then lane (n, g) reads digit n%4 of group g.
    float xs[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int X = bad ? 0 : static_cast<int>(rintf(__builtin_amdgcn_ldexpf(xv[c], F)));
        const int d3 = sbfe(static_cast<uint32_t>(X), 0, 7);
        const int X1 = (X - d3) >> 7;
        const int d2 = sbfe(static_cast<uint32_t>(X1), 0, 7);
        const int X2 = (X1 - d2) >> 7;
        const int d1 = sbfe(static_cast<uint32_t>(X2), 0, 7);
        const int d0 = (X2 - d1) >> 7;
        uint8_t* dst = slot + c * 256 + g * 64 + n;   // n = element index within group g
        dst[0] = static_cast<uint8_t>(d0);
        dst[16] = static_cast<uint8_t>(d1);
        dst[32] = static_cast<uint8_t>(d2);
        dst[48] = static_cast<uint8_t>(d3);
        // sum of X over group g, the same in all 16 lanes of the group
        xs[c] = T::kXs * (group_sum<16>(static_cast<float>(X)) * scale);
    }
    const bool valid = (n >> 2) == g;
    v4i_t a[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const v4i_t v = *reinterpret_cast<const v4i_t*>(slot + c * 256 + g * 64 + (n & 3) * 16);
        a[c] = valid ? v : v4i_t{0, 0, 0, 0};
    }

    const bool any_bad = __syncthreads_or(bad);
    if (any_bad) {
        // A non-finite x: the per-element form, the reference's fp32 products,
        // full K per row by the k-slice 0 wave of each slot.
        if (r == 0)
            for (int i = 0; i < cnt; ++i)
                for (int row = (t0 + i * U) * 16; row < (t0 + i * U) * 16 + 16 && row < M; ++row) {
                    const uint64_t base = (ub0 + static_cast<uint64_t>(row) * nb) * 256;
                    float s = 0.f;
                    for (int k = lane; k < 256 * nb; k += kWave)
                        s = __builtin_fmaf(dequant_elem(w, type, base + k), x[k], s);
                    s = group_sum<64>(s);
                    if (lane == 0) y[row] = s;
                }
        return;
    }

    Lane ln;
    ln.g = g;
    const int s2 = 2 * (g >> 1);
    ln.hmask = 0x33333333u << s2;
    ln.hl = 4 - s2;
    ln.hr = s2;
    ln.ns = 4 * (g >> 1);

    for (int i = 0; i < cnt; ++i) {
        store_tile(pre);
        if (i + 1 < cnt) load_tile(pre, t0 + (i + 1) * U);
        float acc = 0.f;
#pragma unroll
        for (int bl = 0; bl < BPW; ++bl)
            acc = T::block(slot + n * Slot::kRowLds + bl * Slot::kBlockLds, a + 4 * bl, xs + 4 * bl, scale, ln, acc);
        acc = sum_groups(acc);
        if (S == 1) {
            if (lane < 16 && (t0 + i * U) * 16 + lane < M) y[(t0 + i * U) * 16 + lane] = acc;
        } else if (lane < 16) {
            part[(wv * maxcnt + i) * 16 + lane] = acc;
        }
    }
    if (S > 1) {
        __syncthreads();
        if (r == 0)
            for (int i = 0; i < cnt; ++i) {
                if (lane < 16 && (t0 + i * U) * 16 + lane < M) {
                    float s = part[(wv * maxcnt + i) * 16 + lane];
                    for (int k = 1; k < S; ++k) s += part[((wv + k) * maxcnt + i) * 16 + lane];
                    y[(t0 + i * U) * 16 + lane] = s;
                }
            }
    }
}

// Shapes the MFMA path takes: nb = S * BPW, S in {4, 2, 1}, BPW in 1..4.
inline bool mfma_split(int nb, int& S, int& bpw) {
    for (int s : {4, 2, 1})
        if (nb % s == 0 && nb / s >= 1 && nb / s <= 4) {
            S = s;
            bpw = nb / s;
            return true;
        }
    return false;
}

// Compute units of the current device (cached per device; callers on several
// threads may race to fill an entry, all with the same value).
inline int device_cus() {
    static std::atomic<int> cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cus[dev].load(std::memory_order_relaxed);
    if (!c) {
        int n = 0;
        c = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

constexpr int kMfmaMaxCnt = 32;   // tiles per slot in the LDS partial-sum buffer

template <int TYPE, int BPW>
void launch_mfma_bpw(const uint8_t* w, int type, const float* x, float* y, int M, int nb, uint64_t ub0, int S,
                     hipStream_t s) {
    using Slot = MfmaSlot<TYPE, BPW>;
    const int tiles = (M + 15) / 16;
    const int slots = kMfmaWaves / S;
    const size_t lds_max = static_cast<size_t>(kMfmaWaves) * (Slot::kBytes + kMfmaMaxCnt * 64);
    static const int occ = [&] {
        int n = 0;
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_mfma<TYPE, BPW>, kMfmaBlock, lds_max) ==
                               hipSuccess && n > 0 ? n : 1;
    }();
    // A persistent grid of the workgroups that fit at once (x converted once
    // per workgroup), or more when a slot would need over kMfmaMaxCnt tiles.
    const int64_t resident = static_cast<int64_t>(occ) * device_cus();
    const int64_t gx = std::min<int64_t>(blocks_for(tiles, slots),
                                         std::max<int64_t>(resident, blocks_for(tiles, slots * kMfmaMaxCnt)));
    const int maxcnt = static_cast<int>(blocks_for(tiles, gx * slots));
    const size_t lds = static_cast<size_t>(kMfmaWaves) * (Slot::kBytes + maxcnt * 64);
    gemv_mfma<TYPE, BPW><<<static_cast<unsigned>(gx), kMfmaBlock, lds, s>>>(w, type, x, y, M, nb, ub0, tiles, S, maxcnt);
}

template <int TYPE>
void launch_mfma(const uint8_t* w, int type, const float* x, float* y, int M, int nb, uint64_t ub0, int S, int bpw,
                 hipStream_t s) {
    switch (bpw) {
        case 1: launch_mfma_bpw<TYPE, 1>(w, type, x, y, M, nb, ub0, S, s); break;
        case 2: launch_mfma_bpw<TYPE, 2>(w, type, x, y, M, nb, ub0, S, s); break;
        case 3: launch_mfma_bpw<TYPE, 3>(w, type, x, y, M, nb, ub0, S, s); break;
        default: launch_mfma_bpw<TYPE, 4>(w, type, x, y, M, nb, ub0, S, s); break;
    }
}

// The MFMA path pays a fixed latency per workgroup (converting x, the k-slice
// reduction), so it takes over from the per-row kernel only on large
// matrices: measured crossovers at K = 2048 are ~16K rows for Q6_K and
// between 32K and 248K rows for Q4_K (whose per-row kernel spends fewer VALU
// operations per byte).
inline bool mfma_large(int type, int M) {
    const int tiles = (M + 15) / 16;
    return type == kQ6_K ? tiles >= 1024 : tiles >= 4096;
}

template <int TYPE, int R>
void launch_kquant(const uint8_t* w, const float* x, float* y, int M, int nb, uint64_t ub0, int groups,
                   uint64_t tensor_bytes, const Experts& ex, int n_sel, hipStream_t s) {
    constexpr int CPU = KQuant<TYPE>::kBlockBytes * 8 / 16;
    const int waves = (groups + R - 1) / R;
    const dim3 grid(blocks_for(waves, kGemvWaves), n_sel);
    if (TYPE == kQ4_K && nb >= 8) {   // rows of whole units: the direct form
        const bool two = (nb / 8) % 2 == 0;
        if (ex.idx) {
            if (two)
                gemv_q4k_direct<R, 2, true><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex);
            else
                gemv_q4k_direct<R, 1, true><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex);
        } else {
            if (two)
                gemv_q4k_direct<R, 2, false><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, tensor_bytes,
                                                                         ex);
            else
                gemv_q4k_direct<R, 1, false><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, tensor_bytes,
                                                                         ex);
        }
        return;
    }
    if (TYPE == kQ6_K && nb >= 8) {
        if constexpr (R <= 2) {
            const bool two = (nb / 8) % 2 == 0;
            if (ex.idx) {
                if (two)
                    gemv_q6k_direct<R, 2, true><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, ex);
                else
                    gemv_q6k_direct<R, 1, true><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, ex);
            } else {
                if (two)
                    gemv_q6k_direct<R, 2, false><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, ex);
                else
                    gemv_q6k_direct<R, 1, false><<<grid, kGemvBlock, 0, s>>>(w, x, y, M, nb, ub0, groups, ex);
            }
            return;
        }
    }
    const size_t lds = static_cast<size_t>(kGemvWaves) * R * CPU * 16;
    gemv_kquant<TYPE, R><<<grid, kGemvBlock, lds, s>>>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex);
}

template <int TYPE>
void dispatch_kquant(const uint8_t* w, const float* x, float* y, int M, int nb, uint64_t ub0, int groups,
                     uint64_t tensor_bytes, const Experts& ex, int n_sel, hipStream_t s) {
    // Units per wave: enough waves to fill 256 CUs several times over. More than
    // 4 units per wave measured slower (fewer waves per SIMD to hide latency).
    // Q4_K rows of two or more units (K >= 4096) load all of a row's units at
    // once: 2 rows per wave from 4096 units (measured at 2048 x 4096: 3.8 us
    // against 4.3 with 1 row per wave).
    const int64_t all = static_cast<int64_t>(groups) * n_sel;
    const bool multi_unit = TYPE == kQ4_K && nb >= 16;
    if (TYPE == kQ6_K && nb >= 8) {   // the direct form: 2 rows per wave from 8192 rows (measured at 8192 x 2048)
        if (all >= 2 * 4096)
            launch_kquant<TYPE, 2>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
        else
            launch_kquant<TYPE, 1>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
        return;
    }
    if (all >= 4 * 4096)
        launch_kquant<TYPE, 4>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
    else if (all >= 2 * 4096 || (multi_unit && all * (nb / 8) >= 4096))
        launch_kquant<TYPE, 2>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
    else
        launch_kquant<TYPE, 1>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
}

// One GEMV (ex.idx == nullptr, n_sel == 1) or n_sel expert GEMVs of one launch.
// The caller has validated the shapes against the tensor.
int launch_gemv(const uint8_t* w, int type, uint64_t num_elements, const float* x, float* y, int M, int K,
                uint64_t element_offset, const Experts& ex, int n_sel, hipStream_t s, const char* what) {
    const bool kquant = type == kQ4_K || type == kQ6_K;
    const int nb = K / 256;
    const uint64_t tensor_bytes = (num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
    const bool shape_ok = K % 256 == 0 && (nb % 8 == 0 || 8 % nb == 0) && element_offset % 256 == 0 &&
                          num_elements % 256 == 0 && tensor_bytes % 16 == 0 && (!ex.idx || ex.stride % 256 == 0);
    // Units start 16-byte aligned: always for 144-byte blocks, every 8 blocks for 210.
    const bool aligned = aligned16(w) && aligned16(x) && (!ex.idx || ex.x_stride % 4 == 0) &&
                         (type == kQ4_K || ((element_offset / 256) % 8 == 0 && (!ex.idx || (ex.stride / 256) % 8 == 0)));
    int S = 0, bpw = 0;
    const bool mfma_ok = kquant && !ex.idx && K % 256 == 0 && mfma_split(nb, S, bpw) && element_offset % 256 == 0 &&
                         mfma_large(type, M);
    if (mfma_ok) {
        if (type == kQ4_K)
            launch_mfma<kQ4_K>(w, type, x, y, M, nb, element_offset / 256, S, bpw, s);
        else
            launch_mfma<kQ6_K>(w, type, x, y, M, nb, element_offset / 256, S, bpw, s);
    } else if (kquant && shape_ok && aligned) {
        const uint64_t ub0 = element_offset / 256;
        const int groups = nb >= 8 ? M : (M + 8 / nb - 1) / (8 / nb);
        if (type == kQ4_K)
            dispatch_kquant<kQ4_K>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
        else
            dispatch_kquant<kQ6_K>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
    } else {
        gemv_any<<<dim3(blocks_for(M, kBlock / kWave), n_sel), kBlock, 0, s>>>(w, type, x, y, M, K, element_offset,
                                                                             ex, 0);
    }
    return check_launch(what);
}


// Whether a plain GEMV of this matrix takes the per-row kernel (the same
// conditions as launch_gemv without expert selection). A split output layout
// (out_index) takes it whenever the shape allows, large or not.
bool kquant_rowpath(const uint8_t* w, int type, uint64_t num_elements, const float* x, int M, int K,
                    uint64_t element_offset, bool split = false) {
    if (type != kQ4_K && type != kQ6_K) return false;
    const int nb = K / 256;
    const uint64_t tensor_bytes = (num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
    int S = 0, bpw = 0;
    if (!split && K % 256 == 0 && mfma_split(nb, S, bpw) && element_offset % 256 == 0 && mfma_large(type, M))
        return false;
    const bool shape_ok = K % 256 == 0 && (nb % 8 == 0 || 8 % nb == 0) && element_offset % 256 == 0 &&
                          num_elements % 256 == 0 && tensor_bytes % 16 == 0;
    const bool aligned = aligned16(w) && aligned16(x) && (type == kQ4_K || (element_offset / 256) % 8 == 0);
    return shape_ok && aligned;
}

template <int TYPE, int R>
void launch_multi_r(const GemvMulti& mu, int n, const float* x, int nb, hipStream_t s) {
    constexpr int CPU = KQuant<TYPE>::kBlockBytes * 8 / 16;
    int64_t gx = 1;
    for (int j = 0; j < n; ++j) gx = std::max<int64_t>(gx, blocks_for((mu.d[j].groups + R - 1) / R, kGemvWaves));
    const dim3 grid(static_cast<unsigned>(gx), n);
    if (TYPE == kQ4_K && nb >= 8) {   // rows of whole units: the direct form, one flat grid
        GemvMulti mf = mu;
        mf.start[0] = 0;
        for (int j = 0; j < n; ++j)
            mf.start[j + 1] = mf.start[j] + static_cast<int>(blocks_for((mu.d[j].groups + R - 1) / R, kGemvWaves));
        if ((nb / 8) % 2 == 0)
            gemv_q4k_direct_multi<R, 2><<<mf.start[n], kGemvBlock, 0, s>>>(x, nb, mf, n);
        else
            gemv_q4k_direct_multi<R, 1><<<mf.start[n], kGemvBlock, 0, s>>>(x, nb, mf, n);
        return;
    }
    if (TYPE == kQ6_K && nb >= 8) {
        if constexpr (R <= 2) {
            GemvMulti mf = mu;
            mf.start[0] = 0;
            for (int j = 0; j < n; ++j)
                mf.start[j + 1] =
                    mf.start[j] + static_cast<int>(blocks_for((mu.d[j].groups + R - 1) / R, kGemvWaves));
            if ((nb / 8) % 2 == 0)
                gemv_q6k_direct_multi<R, 2><<<mf.start[n], kGemvBlock, 0, s>>>(x, nb, mf, n);
            else
                gemv_q6k_direct_multi<R, 1><<<mf.start[n], kGemvBlock, 0, s>>>(x, nb, mf, n);
            return;
        }
    }
    const size_t lds = static_cast<size_t>(kGemvWaves) * R * CPU * 16;
    gemv_kquant_multi<TYPE, R><<<grid, kGemvBlock, lds, s>>>(x, nb, mu);
}

// Up to kMultiMax matrices of one K-quant type, each on the per-row path.
template <int TYPE>
void launch_multi(const GemvMulti& mu, int n, const float* x, int nb, hipStream_t s) {
    int64_t all = 0;   // units per wave as dispatch_kquant picks them, over all matrices
    for (int j = 0; j < n; ++j) all += mu.d[j].groups;
    if (TYPE == kQ6_K && nb >= 8)   // the direct form: at most 2 rows per wave
        all = std::min<int64_t>(all, 4 * 4096 - 1);
    if (all >= 4 * 4096)
        launch_multi_r<TYPE, 4>(mu, n, x, nb, s);
    else if (all >= 2 * 4096)
        launch_multi_r<TYPE, 2>(mu, n, x, nb, s);
    else
        launch_multi_r<TYPE, 1>(mu, n, x, nb, s);
}

template <int TYPE, int R>
void launch_gate_up_r(const uint8_t* wg, const uint8_t* wu, const float* x, float* yg, float* yu, int M, int nb,
                      int groups, uint64_t tensor_bytes, const Experts& ex, int n_sel, hipStream_t s) {
    constexpr int CPU = KQuant<TYPE>::kBlockBytes * 8 / 16;
    const int waves = (groups + R - 1) / R;
    const dim3 grid(blocks_for(waves, kGemvWaves), 2 * n_sel);
    if (TYPE == kQ4_K && nb >= 8) {   // rows of whole units: the direct form
        if ((nb / 8) % 2 == 0)
            gemv_q4k_direct_gate_up<R, 2><<<grid, kGemvBlock, 0, s>>>(wg, wu, x, yg, yu, M, nb, groups,
                                                                       tensor_bytes, ex, n_sel);
        else
            gemv_q4k_direct_gate_up<R, 1><<<grid, kGemvBlock, 0, s>>>(wg, wu, x, yg, yu, M, nb, groups,
                                                                       tensor_bytes, ex, n_sel);
        return;
    }
    const size_t lds = static_cast<size_t>(kGemvWaves) * R * CPU * 16;
    gemv_kquant_gate_up<TYPE, R><<<grid, kGemvBlock, lds, s>>>(wg, wu, x, yg, yu, M, nb, groups, tensor_bytes, ex,
                                                              n_sel);
}

// Units per wave as dispatch_kquant picks them for the 2 n_sel matrices.
template <int TYPE>
void launch_gate_up(const uint8_t* wg, const uint8_t* wu, const float* x, float* yg, float* yu, int M, int nb,
                    int groups, uint64_t tensor_bytes, const Experts& ex, int n_sel, hipStream_t s) {
    const int64_t all = static_cast<int64_t>(groups) * 2 * n_sel;
    if (all >= 4 * 4096)
        launch_gate_up_r<TYPE, 4>(wg, wu, x, yg, yu, M, nb, groups, tensor_bytes, ex, n_sel, s);
    else if (all >= 2 * 4096)
        launch_gate_up_r<TYPE, 2>(wg, wu, x, yg, yu, M, nb, groups, tensor_bytes, ex, n_sel, s);
    else
        launch_gate_up_r<TYPE, 1>(wg, wu, x, yg, yu, M, nb, groups, tensor_bytes, ex, n_sel, s);
}

struct DownCombine {
    const uint8_t* wd;
    uint64_t expert_blocks;
    int n_experts;
    const int32_t* idx;
    const float* wts;
    int k;
    const float* hid;
    const uint8_t* wsd;
    const float *shid, *slogit;
    float* out;
    int d_model;
};

template <int TE, int TS, int KT, int SS>
void launch_dc(const DownCombine& a, hipStream_t s) {
    if (TE == kQ4_K && TS == kQ4_K) {
        moe_down_combine_q4k<KT, SS><<<a.d_model / 4, kGemvBlock, 0, s>>>(
            a.wd, a.expert_blocks, a.n_experts, a.idx, a.wts, a.k, a.hid, a.wsd, a.shid, a.slogit, a.out);
        return;
    }
    moe_down_combine_kernel<TE, TS, KT, SS><<<a.d_model / 4, kGemvBlock, 0, s>>>(
        a.wd, a.expert_blocks, a.n_experts, a.idx, a.wts, a.k, a.hid, a.wsd, a.shid, a.slogit, a.out);
}

template <int TE, int TS>
void launch_dc_t(const DownCombine& a, int ss, hipStream_t s) {
    if (a.k <= 4)
        ss == 1 ? launch_dc<TE, TS, 1, 1>(a, s) : launch_dc<TE, TS, 1, 2>(a, s);
    else
        ss == 1 ? launch_dc<TE, TS, 2, 1>(a, s) : launch_dc<TE, TS, 2, 2>(a, s);
}

void launch_down_combine(const DownCombine& a, int te, int ts, int ss, hipStream_t s) {
    if (te == kQ4_K)
        ts == kQ4_K ? launch_dc_t<kQ4_K, kQ4_K>(a, ss, s) : launch_dc_t<kQ4_K, kQ6_K>(a, ss, s);
    else
        ts == kQ4_K ? launch_dc_t<kQ6_K, kQ4_K>(a, ss, s) : launch_dc_t<kQ6_K, kQ6_K>(a, ss, s);
}

inline size_t align16(size_t n) { return (n + 15) / 16 * 16; }

template <int TYPE, int R, int VPL>
void launch_swiglu_r(const float* x, int nb, const PairJob& routed, const PairJob& shared, int n_sel,
                     const RouteJob& rt, hipStream_t s) {
    constexpr int CPU = KQuant<TYPE>::kBlockBytes * 8 / 16;
    const int rows = std::max(n_sel > 0 ? routed.M : 0, shared.M);
    const int rows_y = n_sel + (shared.M > 0 ? 1 : 0);
    const dim3 grid(blocks_for((rows + R - 1) / R, kGemvWaves), rows_y);
    if (TYPE == kQ4_K) {   // rows of whole units (8 | nb here): the direct form, one flat grid
        const int nr = n_sel > 0 ? static_cast<int>(blocks_for((routed.M + R - 1) / R, kGemvWaves)) : 0;
        const int ns = shared.M > 0 ? static_cast<int>(blocks_for((shared.M + R - 1) / R, kGemvWaves)) : 0;
        const unsigned flat = static_cast<unsigned>(n_sel * nr + ns);
        if ((nb / 8) % 2 == 0)
            gemv_q4k_direct_swiglu<R, 2, VPL><<<flat, kGemvBlock, 0, s>>>(x, nb, routed, shared, n_sel, rt, nr);
        else
            gemv_q4k_direct_swiglu<R, 1, VPL><<<flat, kGemvBlock, 0, s>>>(x, nb, routed, shared, n_sel, rt, nr);
        return;
    }
    const size_t lds = static_cast<size_t>(kGemvWaves) * 2 * R * CPU * 16;
    gemv_kquant_swiglu<TYPE, R, VPL><<<grid, kGemvBlock, lds, s>>>(x, nb, routed, shared, n_sel, rt);
}

template <int TYPE, int VPL>
void launch_swiglu_v(const float* x, int nb, const PairJob& routed, const PairJob& shared, int n_sel,
                     const RouteJob& rt, hipStream_t s) {
    const int64_t rows = static_cast<int64_t>(n_sel) * routed.M + shared.M;
    if (rows >= 8192)
        launch_swiglu_r<TYPE, 2, VPL>(x, nb, routed, shared, n_sel, rt, s);
    else
        launch_swiglu_r<TYPE, 1, VPL>(x, nb, routed, shared, n_sel, rt, s);
}

// One launch for the routed rows (n_sel > 0) and / or the shared rows
// (shared.M > 0); with rt.logits set, the routing of the routed rows too
// (vpl = logits per lane of the top-k, 1, 2 or 4).
template <int TYPE>
void launch_swiglu(const float* x, int nb, const PairJob& routed, const PairJob& shared, int n_sel,
                   const RouteJob& rt, int vpl, hipStream_t s) {
    if (!rt.logits) launch_swiglu_v<TYPE, 0>(x, nb, routed, shared, n_sel, rt, s);
    else if (vpl == 1) launch_swiglu_v<TYPE, 1>(x, nb, routed, shared, n_sel, rt, s);
    else if (vpl == 2) launch_swiglu_v<TYPE, 2>(x, nb, routed, shared, n_sel, rt, s);
    else launch_swiglu_v<TYPE, 4>(x, nb, routed, shared, n_sel, rt, s);
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_matmul_type_supported(int type) { return type_supported(type) ? 1 : 0; }

// Validation mirrors src/cuda/matmul_q4.cu:187-195.
int qwen_matmul_dispatch(const void* weight, int type, uint64_t num_elements, const float* x, float* y, int M, int K,
                         uint64_t element_offset, void* stream) {
    if (!weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    if (M <= 0 || K <= 0 || element_offset > num_elements ||
        static_cast<uint64_t>(M) * static_cast<uint64_t>(K) > num_elements - element_offset)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d)", M, K);
    QK_REQUIRE(x && y, "matmul_dispatch: null pointer");
    return launch_gemv(static_cast<const uint8_t*>(weight), type, num_elements, x, y, M, K, element_offset,
                       Experts{nullptr, 0, 0, 0}, 1, as_stream(stream), "matmul_dispatch");
}

// qwen_gdn_norm_gate + qwen_matmul_dispatch in one launch when the shape allows
// (see the header); validation as the two calls.
int qwen_gdn_norm_gate_matmul(const float* x, const float* z, const float* norm_weight, float* normed, int heads,
                              int dim, float eps, const void* weight, int type, uint64_t num_elements, float* y,
                              int M, uint64_t element_offset, void* stream) {
    QK_REQUIRE(heads > 0 && dim > 0, "gdn_norm_gate_matmul: bad heads %d / dim %d", heads, dim);
    QK_REQUIRE(x && z && norm_weight && normed, "gdn_norm_gate_matmul: null pointer");
    const int64_t K64 = static_cast<int64_t>(heads) * dim;
    QK_REQUIRE(K64 <= (int64_t{1} << 30), "gdn_norm_gate_matmul: %lld inputs", static_cast<long long>(K64));
    const int K = static_cast<int>(K64);
    if (!weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    if (M <= 0 || element_offset > num_elements ||
        static_cast<uint64_t>(M) * static_cast<uint64_t>(K) > num_elements - element_offset)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d)", M, K);
    QK_REQUIRE(y, "gdn_norm_gate_matmul: null pointer");
    const auto* w = static_cast<const uint8_t*>(weight);
    const int lph = dim == 64 ? 16 : dim == 128 ? 32 : dim == 256 ? 64 : 0;
    const bool one = type == kQ4_K && lph && K % 2048 == 0 && aligned16(z) && aligned16(norm_weight) &&
                     aligned16(normed) && kquant_rowpath(w, type, num_elements, x, M, K, element_offset);
    if (!one) {
        const int rc = qwen_gdn_norm_gate(x, z, norm_weight, normed, heads, dim, eps, stream);
        return rc ? rc : qwen_matmul_dispatch(weight, type, num_elements, normed, y, M, K, element_offset, stream);
    }
    const hipStream_t s = as_stream(stream);
    const int nb = K / 256;
    const uint64_t tensor_bytes = (num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
    const uint64_t ub0 = element_offset / 256;
    const NormGateX ng{z, norm_weight, eps, normed};
    // rows per wave as dispatch_kquant picks them for this matrix
    const int R = M >= 4 * 4096 ? 4 : (M >= 2 * 4096 || (nb >= 16 && static_cast<int64_t>(M) * (nb / 8) >= 4096)) ? 2 : 1;
    const bool two = (nb / 8) % 2 == 0;
    auto go = [&](auto r_c, auto ns_c, auto lph_c) {
        constexpr int RR = decltype(r_c)::value, NS = decltype(ns_c)::value, L = decltype(lph_c)::value;
        gemv_q4k_norm_gate<RR, NS, L><<<blocks_for((M + RR - 1) / RR, kNormGateWaves), kNormGateWaves * kWave, 0,
                                        s>>>(w, x, ng, y, M, nb, ub0, tensor_bytes);
    };
    auto by_lph = [&](auto r_c, auto ns_c) {
        if (lph == 16) go(r_c, ns_c, std::integral_constant<int, 16>{});
        else if (lph == 32) go(r_c, ns_c, std::integral_constant<int, 32>{});
        else go(r_c, ns_c, std::integral_constant<int, 64>{});
    };
    auto by_ns = [&](auto r_c) {
        if (two) by_lph(r_c, std::integral_constant<int, 2>{});
        else by_lph(r_c, std::integral_constant<int, 1>{});
    };
    if (R == 4) by_ns(std::integral_constant<int, 4>{});
    else if (R == 2) by_ns(std::integral_constant<int, 2>{});
    else by_ns(std::integral_constant<int, 1>{});
    return check_launch("gdn_norm_gate_matmul");
}

int qwen_moe_expert_matmul(const void* weight, int type, uint64_t num_elements, uint64_t expert_stride, int n_experts,
                           const int32_t* idx, int n_sel, const float* x, int64_t x_stride, float* y, int M, int K,
                           void* stream) {
    if (!weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    QK_REQUIRE(n_sel >= 0 && n_experts > 0 && x_stride >= 0, "moe_expert_matmul: bad n_sel %d / n_experts %d",
               n_sel, n_experts);
    if (M <= 0 || K <= 0 || static_cast<uint64_t>(M) * static_cast<uint64_t>(K) > expert_stride ||
        expert_stride > num_elements / static_cast<uint64_t>(n_experts))
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d, %d experts)", M, K, n_experts);
    if (n_sel == 0) return ok();
    QK_REQUIRE(idx && x && y, "moe_expert_matmul: null pointer");
    QK_REQUIRE(n_sel <= 65535, "moe_expert_matmul: n_sel %d too large", n_sel);
    return launch_gemv(static_cast<const uint8_t*>(weight), type, num_elements, x, y, M, K, 0,
                       Experts{idx, n_experts, expert_stride, x_stride}, n_sel, as_stream(stream),
                       "moe_expert_matmul");
}


int qwen_moe_expert_gate_up(const void* w_gate, const void* w_up, int type, uint64_t num_elements,
                            uint64_t expert_stride, int n_experts, const int32_t* idx, int n_sel, const float* x,
                            float* gate_out, float* up_out, int M, int K, void* stream) {
    if (!w_gate || !w_up) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    QK_REQUIRE(n_sel >= 0 && n_experts > 0, "moe_expert_gate_up: bad n_sel %d / n_experts %d", n_sel, n_experts);
    if (M <= 0 || K <= 0 || static_cast<uint64_t>(M) * static_cast<uint64_t>(K) > expert_stride ||
        expert_stride > num_elements / static_cast<uint64_t>(n_experts))
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d, %d experts)", M, K, n_experts);
    if (n_sel == 0) return ok();
    QK_REQUIRE(idx && x && gate_out && up_out, "moe_expert_gate_up: null pointer");
    QK_REQUIRE(n_sel <= 32767, "moe_expert_gate_up: n_sel %d too large", n_sel);
    const hipStream_t s = as_stream(stream);
    const auto* wg = static_cast<const uint8_t*>(w_gate);
    const auto* wu = static_cast<const uint8_t*>(w_up);
    const Experts ex{idx, n_experts, expert_stride, 0};
    const int nb = K / 256;
    const uint64_t tensor_bytes = (num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
    // The per-row kernel's conditions (launch_gemv, expert form) for both tensors.
    const bool rowpath = (type == kQ4_K || type == kQ6_K) && K % 256 == 0 && (nb % 8 == 0 || 8 % nb == 0) &&
                         num_elements % 256 == 0 && tensor_bytes % 16 == 0 && expert_stride % 256 == 0 &&
                         aligned16(wg) && aligned16(wu) && aligned16(x) &&
                         (type == kQ4_K || (expert_stride / 256) % 8 == 0);
    if (!rowpath) {
        const int rc = launch_gemv(wg, type, num_elements, x, gate_out, M, K, 0, ex, n_sel, s, "moe_expert_gate_up");
        if (rc) return rc;
        return launch_gemv(wu, type, num_elements, x, up_out, M, K, 0, ex, n_sel, s, "moe_expert_gate_up");
    }
    const int groups = nb >= 8 ? M : (M + 8 / nb - 1) / (8 / nb);
    if (type == kQ4_K)
        launch_gate_up<kQ4_K>(wg, wu, x, gate_out, up_out, M, nb, groups, tensor_bytes, ex, n_sel, s);
    else
        launch_gate_up<kQ6_K>(wg, wu, x, gate_out, up_out, M, nb, groups, tensor_bytes, ex, n_sel, s);
    return check_launch("moe_expert_gate_up");
}

size_t qwen_moe_expert_swiglu_workspace_bytes(int n_sel, int inter, int shared_dim) {
    if (n_sel < 0 || inter < 0 || shared_dim < 0) return 0;
    return 2 * align16(sizeof(float) * (n_sel * static_cast<size_t>(inter) + shared_dim));
}

namespace {
// The per-row pair kernel's conditions for one gate / up pair of tensors.
bool swiglu_rowpath(const uint8_t* wg, const uint8_t* wu, int type, uint64_t num_elements, uint64_t expert_stride,
                    const float* x, int K) {
    const int nb = K / 256;
    const uint64_t tensor_bytes = (num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
    return (type == kQ4_K || type == kQ6_K) && K % 2048 == 0 && num_elements % 256 == 0 && tensor_bytes % 16 == 0 &&
           expert_stride % 2048 == 0 && aligned16(wg) && aligned16(wu) && aligned16(x) && nb >= 8;
}
}  // namespace

namespace {
// qwen_moe_expert_swiglu, and with `logits` set qwen_moe_route_swiglu: the ids
// (and weights) then come from the router logits and are written to idx / w.
int expert_swiglu(const void* w_gate, const void* w_up, int type, uint64_t num_elements, uint64_t expert_stride,
                  int n_experts, const float* logits, int32_t* idx, float* w, int n_sel, int inter,
                  const void* w_shared_gate, const void* w_shared_up, int shared_type, uint64_t shared_elements,
                  int shared_dim, const float* x, int K, float* hidden, float* shared_hidden, void* workspace,
                  size_t workspace_bytes, void* stream, const char* what) {
    const bool has_shared = w_shared_gate || w_shared_up;
    if (!w_gate || !w_up || (has_shared && (!w_shared_gate || !w_shared_up)))
        return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    if (has_shared && !type_supported(shared_type))
        return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", shared_type);
    QK_REQUIRE(n_sel >= 0 && n_sel <= 32767 && n_experts > 0, "%s: bad n_sel %d / n_experts %d", what, n_sel,
               n_experts);
    if (logits)
        QK_REQUIRE(n_sel > 0 && n_sel <= n_experts && n_sel <= kWave && n_experts <= 4 * kWave,
                   "%s: need 0 < k <= min(n, 64) and n <= %d (n=%d, k=%d)", what, 4 * kWave, n_experts, n_sel);
    if (inter <= 0 || K <= 0 || static_cast<uint64_t>(inter) * static_cast<uint64_t>(K) > expert_stride ||
        expert_stride > num_elements / static_cast<uint64_t>(n_experts))
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d, %d experts)", inter, K,
                    n_experts);
    if (has_shared && (shared_dim <= 0 || static_cast<uint64_t>(shared_dim) * static_cast<uint64_t>(K) > shared_elements))
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d)", shared_dim, K);
    const int sdim = has_shared ? shared_dim : 0;
    QK_REQUIRE(x && (n_sel == 0 || (idx && hidden)) && (!has_shared || shared_hidden) && (!logits || w),
               "%s: null pointer", what);
    const size_t need = qwen_moe_expert_swiglu_workspace_bytes(n_sel, inter, sdim);
    QK_REQUIRE(workspace || need == 0, "%s: null workspace", what);
    QK_REQUIRE(workspace_bytes >= need, "%s: workspace of %zu bytes, need %zu", what, workspace_bytes, need);
    const hipStream_t s = as_stream(stream);
    const auto* wg = static_cast<const uint8_t*>(w_gate);
    const auto* wu = static_cast<const uint8_t*>(w_up);
    const auto* wsg = static_cast<const uint8_t*>(w_shared_gate);
    const auto* wsu = static_cast<const uint8_t*>(w_shared_up);
    const Experts ex{idx, n_experts, expert_stride, 0};
    const Experts none{nullptr, 0, 0, 0};
    const bool r_fast = n_sel > 0 && swiglu_rowpath(wg, wu, type, num_elements, expert_stride, x, K);
    const bool s_fast = has_shared && swiglu_rowpath(wsg, wsu, shared_type, shared_elements, 2048, x, K);
    const PairJob routed{wg, wu, hidden, inter, ex};
    const PairJob shared{wsg, wsu, shared_hidden, sdim, none};
    const PairJob off{nullptr, nullptr, nullptr, 0, none};
    const int nb = K / 256;
    const int vpl = (n_experts + kWave - 1) / kWave;
    int rc = 0;
    // Routing without the fused kernel: the top-k launch first.
    if (logits && !r_fast) rc = qwen_moe_topk_rows(logits, idx, w, 1, n_experts, n_sel, stream);
    if (rc) return rc;
    const RouteJob rt{logits && r_fast ? logits : nullptr, idx, w};
    const RouteJob no_rt{nullptr, nullptr, nullptr};
    auto launch = [&](int t, const PairJob& r, const PairJob& sj, int n, const RouteJob& rj) {
        if (t == kQ4_K) launch_swiglu<kQ4_K>(x, nb, r, sj, n, rj, vpl, s);
        else launch_swiglu<kQ6_K>(x, nb, r, sj, n, rj, vpl, s);
    };
    if (r_fast && s_fast && type == shared_type) {
        launch(type, routed, shared, n_sel, rt);
    } else {
        if (r_fast) launch(type, routed, off, n_sel, rt);
        if (s_fast) launch(shared_type, off, shared, 0, no_rt);
    }
    rc = check_launch(what);
    // Other shapes: the two GEMVs into the workspace, then SiLU x up.
    auto* gbuf = static_cast<float*>(workspace);
    auto* ubuf = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + need / 2);
    const size_t nr = static_cast<size_t>(n_sel) * inter;
    if (!rc && n_sel > 0 && !r_fast) {
        rc = launch_gemv(wg, type, num_elements, x, gbuf, inter, K, 0, ex, n_sel, s, what);
        if (!rc) rc = launch_gemv(wu, type, num_elements, x, ubuf, inter, K, 0, ex, n_sel, s, what);
        if (!rc) rc = qwen_moe_silu_mul(gbuf, ubuf, hidden, static_cast<int>(nr), stream);
    }
    if (!rc && has_shared && !s_fast) {
        rc = launch_gemv(wsg, shared_type, shared_elements, x, gbuf + nr, sdim, K, 0, none, 1, s, what);
        if (!rc) rc = launch_gemv(wsu, shared_type, shared_elements, x, ubuf + nr, sdim, K, 0, none, 1, s, what);
        if (!rc) rc = qwen_moe_silu_mul(gbuf + nr, ubuf + nr, shared_hidden, sdim, stream);
    }
    return rc;
}
}  // namespace

int qwen_moe_expert_swiglu(const void* w_gate, const void* w_up, int type, uint64_t num_elements,
                           uint64_t expert_stride, int n_experts, const int32_t* idx, int n_sel, int inter,
                           const void* w_shared_gate, const void* w_shared_up, int shared_type,
                           uint64_t shared_elements, int shared_dim, const float* x, int K, float* hidden,
                           float* shared_hidden, void* workspace, size_t workspace_bytes, void* stream) {
    return expert_swiglu(w_gate, w_up, type, num_elements, expert_stride, n_experts, nullptr,
                         const_cast<int32_t*>(idx), nullptr, n_sel, inter, w_shared_gate, w_shared_up, shared_type,
                         shared_elements, shared_dim, x, K, hidden, shared_hidden, workspace, workspace_bytes, stream,
                         "moe_expert_swiglu");
}

int qwen_moe_route_swiglu(const float* logits, int32_t* idx, float* weights, int k, const void* w_gate,
                          const void* w_up, int type, uint64_t num_elements, uint64_t expert_stride, int n_experts,
                          int inter, const void* w_shared_gate, const void* w_shared_up, int shared_type,
                          uint64_t shared_elements, int shared_dim, const float* x, int K, float* hidden,
                          float* shared_hidden, void* workspace, size_t workspace_bytes, void* stream) {
    QK_REQUIRE(logits, "moe_route_swiglu: null pointer");
    return expert_swiglu(w_gate, w_up, type, num_elements, expert_stride, n_experts, logits, idx, weights, k, inter,
                         w_shared_gate, w_shared_up, shared_type, shared_elements, shared_dim, x, K, hidden,
                         shared_hidden, workspace, workspace_bytes, stream, "moe_route_swiglu");
}

size_t qwen_moe_down_combine_workspace_bytes(int n_sel, int d_model) {
    if (n_sel < 0 || d_model < 0) return 0;
    const size_t f = sizeof(float);
    return align16(f * n_sel * static_cast<size_t>(d_model)) + align16(f * d_model);
}

int qwen_moe_down_combine(const void* w_down, int down_type, uint64_t down_elements, uint64_t expert_stride,
                          int n_experts, const int32_t* idx, const float* weights, int n_sel, const float* hidden,
                          int inter, const void* w_shared_down, int shared_type, uint64_t shared_elements,
                          const float* shared_hidden, int shared_dim, const float* shared_logit, float* out,
                          int d_model, void* workspace, size_t workspace_bytes, void* stream) {
    if (!w_down || !w_shared_down) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(down_type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", down_type);
    if (!type_supported(shared_type))
        return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", shared_type);
    QK_REQUIRE(n_sel > 0 && n_sel <= 64 && n_experts > 0, "moe_down_combine: bad n_sel %d / n_experts %d", n_sel,
               n_experts);
    if (d_model <= 0 || inter <= 0 ||
        static_cast<uint64_t>(d_model) * static_cast<uint64_t>(inter) > expert_stride ||
        expert_stride > down_elements / static_cast<uint64_t>(n_experts))
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d, %d experts)", d_model, inter,
                    n_experts);
    if (shared_dim <= 0 || static_cast<uint64_t>(d_model) * static_cast<uint64_t>(shared_dim) > shared_elements)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d)", d_model, shared_dim);
    QK_REQUIRE(idx && weights && hidden && shared_hidden && shared_logit && out && workspace,
               "moe_down_combine: null pointer");
    const size_t need = qwen_moe_down_combine_workspace_bytes(n_sel, d_model);
    QK_REQUIRE(workspace_bytes >= need, "moe_down_combine: workspace of %zu bytes, need %zu", workspace_bytes, need);
    const hipStream_t s = as_stream(stream);
    const auto* wd = static_cast<const uint8_t*>(w_down);
    const auto* wsd = static_cast<const uint8_t*>(w_shared_down);
    const auto kq = [](int t) { return t == kQ4_K || t == kQ6_K; };
    const bool fused = kq(down_type) && kq(shared_type) && inter == kDcInter && shared_dim % 2048 == 0 &&
                       shared_dim <= 4096 && d_model % 4 == 0 && n_sel <= 8 && expert_stride % 2048 == 0 &&
                       aligned16(wd) && aligned16(wsd) && aligned16(hidden) && aligned16(shared_hidden);
    if (fused) {
        const DownCombine a{wd, expert_stride / 256, n_experts, idx, weights, n_sel, hidden, wsd, shared_hidden,
                            shared_logit, out, d_model};
        launch_down_combine(a, down_type, shared_type, shared_dim / 2048, s);
        return check_launch("moe_down_combine");
    }
    // Other shapes: the same steps as separate launches through the workspace.
    auto* eo = static_cast<float*>(workspace);
    auto* so = reinterpret_cast<float*>(reinterpret_cast<char*>(eo) + align16(4 * n_sel * static_cast<size_t>(d_model)));
    int rc = launch_gemv(wd, down_type, down_elements, hidden, eo, d_model, inter, 0,
                         Experts{idx, n_experts, expert_stride, inter}, n_sel, s, "moe_down_combine");
    if (!rc)
        rc = launch_gemv(wsd, shared_type, shared_elements, shared_hidden, so, d_model, shared_dim, 0,
                         Experts{nullptr, 0, 0, 0}, 1, s, "moe_down_combine");
    if (rc) return rc;
    fill_zero<<<blocks_for(d_model, kBlock), kBlock, 0, s>>>(out, d_model);
    rc = check_launch("moe_down_combine");
    if (!rc) rc = qwen_moe_weighted_sum_rows(out, eo, weights, 1, n_sel, d_model, stream);
    if (!rc) rc = qwen_moe_shared_add_rows(out, so, shared_logit, 1, d_model, stream);
    return rc;
}

int qwen_matmul_dispatch_multi(const qwen_gemv_desc* descs, int n, const float* x, int K, void* stream) {
    QK_REQUIRE(n >= 0 && n <= 64, "matmul_dispatch_multi: n = %d outside [0, 64]", n);
    if (n == 0) return ok();
    QK_REQUIRE(descs && x, "matmul_dispatch_multi: null pointer");
    // Validate everything first (qwen_matmul_dispatch's checks, in its order).
    for (int j = 0; j < n; ++j) {
        const qwen_gemv_desc& e = descs[j];
        if (!e.weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "descriptor %d: tensor is not loaded", j);
        if (!type_supported(e.type))
            return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "descriptor %d: unsupported GGML type %d", j, e.type);
        if (e.M <= 0 || K <= 0 || e.element_offset > e.num_elements ||
            static_cast<uint64_t>(e.M) * static_cast<uint64_t>(K) > e.num_elements - e.element_offset)
            return fail(QWEN_STATUS_OUT_OF_RANGE, "descriptor %d: GEMV shape exceeds tensor (M=%d, K=%d)", j, e.M, K);
        QK_REQUIRE(e.y, "matmul_dispatch_multi: descriptor %d has a null output", j);
        QK_REQUIRE(e.split >= 0 && (e.split == 0 || e.M % (2 * e.split) == 0),
                   "matmul_dispatch_multi: descriptor %d: split %d does not pair the %d rows", j, e.split, e.M);
    }
    const hipStream_t s = as_stream(stream);
    const int nb = K / 256;
    for (const int type : {static_cast<int>(kQ4_K), static_cast<int>(kQ6_K)}) {
        GemvMulti mu{};
        int m = 0;
        for (int j = 0; j < n; ++j) {
            const qwen_gemv_desc& e = descs[j];
            const auto* w = static_cast<const uint8_t*>(e.weight);
            if (e.type != type || !kquant_rowpath(w, e.type, e.num_elements, x, e.M, K, e.element_offset, e.split > 0))
                continue;
            GemvMat& g = mu.d[m++];
            g.w = w;
            g.y = e.y;
            g.ub0 = e.element_offset / 256;
            g.tensor_bytes = (e.num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
            g.M = e.M;
            g.groups = nb >= 8 ? e.M : (e.M + 8 / nb - 1) / (8 / nb);
            g.split = e.split;
            if (m == kMultiMax) {
                if (type == kQ4_K) launch_multi<kQ4_K>(mu, m, x, nb, s);
                else launch_multi<kQ6_K>(mu, m, x, nb, s);
                m = 0;
            }
        }
        if (m > 0) {
            if (type == kQ4_K) launch_multi<kQ4_K>(mu, m, x, nb, s);
            else launch_multi<kQ6_K>(mu, m, x, nb, s);
        }
        const int st = check_launch("matmul_dispatch_multi");
        if (st) return st;
    }
    // Everything else: the single-matrix kernels.
    for (int j = 0; j < n; ++j) {
        const qwen_gemv_desc& e = descs[j];
        const auto* w = static_cast<const uint8_t*>(e.weight);
        if ((e.type == kQ4_K || e.type == kQ6_K) &&
            kquant_rowpath(w, e.type, e.num_elements, x, e.M, K, e.element_offset, e.split > 0))
            continue;
        if (e.split > 0) {   // the generic kernel writes the split layout itself
            gemv_any<<<dim3(blocks_for(e.M, kBlock / kWave), 1), kBlock, 0, s>>>(w, e.type, x, e.y, e.M, K,
                                                                                e.element_offset,
                                                                                Experts{nullptr, 0, 0, 0}, e.split);
            const int st = check_launch("matmul_dispatch_multi");
            if (st) return st;
            continue;
        }
        const int st = launch_gemv(w, e.type, e.num_elements, x, e.y, e.M, K, e.element_offset,
                                   Experts{nullptr, 0, 0, 0}, 1, s, "matmul_dispatch_multi");
        if (st) return st;
    }
    return ok();
}

}  // extern "C"
