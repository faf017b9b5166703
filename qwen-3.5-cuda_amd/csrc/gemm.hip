// Quantized GEMM for many tokens (prefill) on gfx950:
//   y[t][m] = sum_k W[m][k] * x[t][k],  t < rows, m < M
// with W a K-quant GGML tensor. Reference: the same product is
// matmul_dispatch (src/cuda/matmul_q4.cu:140-167,185-207) called once per
// token; batched, it is a contraction for the matrix cores.
//
// Exact fp16 operands. A prep kernel scales each token row by a power of two,
// v = x * 2^e with max |v| in [2^14, 2^15), and splits it into two fp16 parts
// v = h + l (h = fp16(v), l = fp16(v - h)): |v - h - l| <= 2^-22 |v| (or
// 2^-25 absolute for the smallest values), so the products below carry an
// fp32 dot product's accuracy. The weights enter as exact small integers:
//   Q4_K: B = q * sc (q 0..15, sc 0..63: at most 945, exact in fp16), so the
//         MFMA accumulator sums a whole 256-element block across its eight
//         scale groups, and per block
//         y += d * P_block - dmin * sum_g m_g S_g        (P = sum (q sc) v)
//         with S_g the group sums of v; the min terms are one fp16 MFMA per
//         tile and block (v_mfma_f32_16x16x16_f16, k = 8 groups x 2 parts):
//         m_g exact, S_g 2^-5 split into two fp16 parts like x (22 bits).
//   Q6_K: B = q - 32 (exact); the signed 8-bit scales do not fit in the fp16
//         operand, so per 16-element group y += (d sc) P_g (one FMA).
// The result is scaled back by 2^-e (exact). Products of fp16 values are exact
// in the MFMA's fp32 accumulation, so the roundings are those of an fp32 sum.
//
// fp16 operands are built with v_perm / v_pk_add_f16 only: bytes b < 1024
// placed under 0x64 give the fp16 1024 + b, and one packed fp16 add of -1024
// (Q4_K after the integer q * sc, Q6_K -1056 for q - 32) leaves the exact
// value. The perm pairs bytes (0, 2) and (1, 3) of a word, so the prep kernel
// stores x in that order within each 4 consecutive elements (0, 2, 1, 3);
// A and B then agree slot by slot.
//
// Work, per 32-element stage (one barrier per stage): a workgroup of 8 waves
// owns 128 tokens x 256 weight rows, wave w rows 64 (w % 4) .. +63 of token half
// w / 4, and the next stage's B operands are decoded (each wave pair splitting
// the work, through LDS) while the current stage's products run. Q4_K: 16 x 16
// tiles on v_mfma_f32_16x16x32_f16, operands through an LDS ring filled three
// stages ahead by global -> LDS loads. Q6_K: 32 x 32 tiles on
// v_mfma_f32_32x32x16_f16 (K = one 16-element scale group), x staged through
// LDS from registers, quant bytes and scales per half-block through LDS. The
// kernels' own comments have the details.
#include <algorithm>
#include <cfloat>
#include <type_traits>
#include <utility>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "ggml_common.hpp"

namespace qk {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGR = 256;           // weight rows per workgroup (64 per wave)
constexpr int kGemmMinRows = 16;   // fewer tokens: one GEMV per token
constexpr int kGemmMaxRows = 65535 * 128;   // token blocks of 128 in grid.y
constexpr int kXRow = 40;          // halves per staged token row (32 + 8 padding)

// Matrices of one launch (all of one K-quant type, one x): workgroup column
// blockIdx.x in [start[j], start[j+1]) works on rows (blockIdx.x - start[j]) * kGR ..
// of matrix j.
constexpr int kGemmJobs = 8;
struct GemmJobs {
    const uint8_t* w[kGemmJobs];
    float* y[kGemmJobs];
    uint64_t ub0[kGemmJobs];   // first block of row 0
    int M[kGemmJobs];
    int start[kGemmJobs + 1];
    int n;
};

struct GemmJob {
    const uint8_t* w;
    float* y;
    uint64_t ub0;
    int M, mb;
};

__device__ __forceinline__ GemmJob gemm_job(const GemmJobs& jobs) {
    const int bx = static_cast<int>(blockIdx.x);
    int j = 0;
    while (j + 1 < jobs.n && bx >= jobs.start[j + 1]) ++j;
    return GemmJob{jobs.w[j], jobs.y[j], jobs.ub0[j], jobs.M[j], bx - jobs.start[j]};
}

// Workspace: per token the exponent e, the group sums of v per 32 elements and
// the fp16 parts [T][K/32][2][32].
inline size_t ws_align(size_t b) { return (b + 255) & ~size_t{255}; }
inline size_t ws_exp_bytes(int T) { return ws_align(4 * static_cast<size_t>(T)); }
inline size_t ws_sum_bytes(int T, int K) { return ws_align(4 * static_cast<size_t>(T) * (K / 32)); }
inline size_t ws_bytes(int T, int K) { return ws_exp_bytes(T) + ws_sum_bytes(T, K) + 4 * static_cast<size_t>(T) * K; }

__device__ __forceinline__ float wave_max_abs(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ uint32_t half_bits_of(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// The two fp16 parts of v (element order 0, 2, 1, 3) and the sums of v per 32
// elements, for the 4 values of lane `lane` at k (k = 4 lane + 256 i).
__device__ __forceinline__ void prep_store(const float4 v4, int e, int k, int lane, size_t t, int nst,
                                           float* __restrict__ sx, uint16_t* __restrict__ xp) {
    const float v[4] = {ldexpf(v4.x, e), ldexpf(v4.y, e), ldexpf(v4.z, e), ldexpf(v4.w, e)};
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const _Float16 hh = static_cast<_Float16>(v[i]);
        h[i] = __builtin_bit_cast(uint16_t, hh);
        l[i] = half_bits_of(v[i] - static_cast<float>(hh));
    }
    uint16_t* dst = xp + (t * nst + (k >> 5)) * 64 + (k & 31);
    *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[2] << 16), h[1] | (h[3] << 16));
    *reinterpret_cast<uint2*>(dst + 32) = make_uint2(l[0] | (l[2] << 16), l[1] | (l[3] << 16));
    float s = (v[0] + v[1]) + (v[2] + v[3]);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if ((lane & 7) == 0) sx[t * nst + (k >> 5)] = s;
}

// Exponent slot of a token row holding an infinity: the fp16 split cannot carry
// it (h = inf, l = inf - inf = NaN would turn the whole output row into NaN),
// so the GEMM evaluates that row's outputs per element instead.
constexpr int kRowNonFinite = 0x7fffffff;

// e for a row whose largest |x| is m (NaN is ignored by the max; a NaN row's
// outputs are NaN either way): zero rows unscaled, rows with an infinity marked.
__device__ __forceinline__ int prep_exponent(float m) {
    if (!(m <= FLT_MAX)) return kRowNonFinite;
    int e = 0;
    if (m > 0.f) {
        int em;
        frexpf(m, &em);   // m in [2^(em-1), 2^em)
        e = 15 - em;
    }
    return e;
}

// y for (token row x, weight row at element `base`) when x holds an infinity:
// the reference's per-element fp32 products and sum (src/cuda/matmul_q4.cu:
// 140-167), so inf * w, 0 * inf = NaN and +inf + -inf = NaN give the same
// pattern of infinities and NaNs as its GEMV.
__device__ float row_dot_per_element(const uint8_t* __restrict__ w, int type, uint64_t base,
                                     const float* __restrict__ x, int K) {
    float s = 0.f;
    for (int k = 0; k < K; ++k) s = __builtin_fmaf(dequant_elem(w, type, base + k), x[k], s);
    return s;
}

__device__ __forceinline__ float max_abs4(float m, const float4& v) {
    return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}

// One wave per token: e, the two fp16 parts of x * 2^e (element order 0, 2, 1, 3
// within each 4) and the sums of x * 2^e per 32 elements. K % 256 == 0. NIT > 0:
// K == 256 NIT, the row is held in registers (read once); NIT == 0: any K, read twice.
template <int NIT>
__global__ __launch_bounds__(256) void gemm_prep_x(const float* __restrict__ x, int* __restrict__ ex,
                                                   float* __restrict__ sx, uint16_t* __restrict__ xp, int T, int K) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= T) return;   // the whole wave
    const float* row = x + static_cast<size_t>(t) * K;
    const int nst = K >> 5;
    float m = 0.f;
    if constexpr (NIT > 0) {
        float4 v[NIT];
#pragma unroll
        for (int i = 0; i < NIT; ++i) {
            v[i] = ld4(row + 4 * lane + 256 * i);
            m = max_abs4(m, v[i]);
        }
        const int e = prep_exponent(wave_max_abs(m));
        if (lane == 0) ex[t] = e;
        const int es = e == kRowNonFinite ? 0 : e;   // a marked row's parts are not used
#pragma unroll
        for (int i = 0; i < NIT; ++i) prep_store(v[i], es, 4 * lane + 256 * i, lane, t, nst, sx, xp);
    } else {
        for (int k = 4 * lane; k < K; k += 256) m = max_abs4(m, ld4(row + k));
        const int e = prep_exponent(wave_max_abs(m));
        if (lane == 0) ex[t] = e;
        const int es = e == kRowNonFinite ? 0 : e;
        for (int k = 4 * lane; k < K; k += 256) prep_store(ld4(row + k), es, k, lane, t, nst, sx, xp);
    }
}

// A thread's share of one stage of x: 32 bytes (part p: fp16 part p/2, halves
// 16 (p%2) .. +15 of its token's 32).
struct XRegs {
    uint4 a, b;
};

__device__ __forceinline__ XRegs load_x(const uint16_t* __restrict__ src) {
    return XRegs{ld16(src), ld16(src + 8)};
}

// Bytes (0, 2) and (1, 3) of n placed under `hi` (byte values 0 or 0x64).
__device__ __forceinline__ uint32_t bytes02(uint32_t hi, uint32_t n) { return __builtin_amdgcn_perm(hi, n, 0x04020400u); }
__device__ __forceinline__ uint32_t bytes13(uint32_t hi, uint32_t n) { return __builtin_amdgcn_perm(hi, n, 0x04030401u); }

__device__ __forceinline__ uint32_t hadd2(uint32_t w, _Float16 c) {
    const f16x2_t r = __builtin_bit_cast(f16x2_t, w) + f16x2_t{c, c};
    return __builtin_bit_cast(uint32_t, r);
}

// fp16 q * sc of four quants (bytes of n, each < 16), sc < 64: two words in
// the order (0, 2), (1, 3).
__device__ __forceinline__ void q4_operand(uint32_t n, uint32_t sc, uint32_t& w02, uint32_t& w13) {
    w02 = hadd2(__umul24(bytes02(0, n), sc) + 0x64006400u, static_cast<_Float16>(-1024.0f));
    w13 = hadd2(__umul24(bytes13(0, n), sc) + 0x64006400u, static_cast<_Float16>(-1024.0f));
}

// fp16 q - 32 of four 6-bit quants (bytes of q): two words in the order (0, 2), (1, 3).
__device__ __forceinline__ void q6_operand(uint32_t q, uint32_t& w02, uint32_t& w13) {
    w02 = hadd2(bytes02(0x64646464u, q), static_cast<_Float16>(-1056.0f));
    w13 = hadd2(bytes13(0x64646464u, q), static_cast<_Float16>(-1056.0f));
}

// ------------------------------------------------------------------ Q4_K
// Element i of a block: qs byte 16 + 32(i/64) + i%32, low nibble if i%64 < 32,
// sub-block i/32 (src/cuda/matmul_q4.cu:76-96). Lane (lr, lk) of stage sb
// takes elements 32 sb + 8 lk .. +7: qs bytes 16 + 32(sb/2) + 8 lk .. +7,
// nibble sb%2.
//
// A workgroup (8 waves, one per CU) owns 128 tokens x 256 weight rows; wave w
// owns rows 64 (w % 4) .. +63 for tokens 64 (w / 4) .. +63. Its operands come
// through an LDS ring filled by global_load_lds_dwordx4 (no VGPRs, no LDS store
// instructions) kQ4Dist stages ahead: x per stage, the quant bytes per pair of
// stages (both nibbles), the headers and group sums per block. While stage g's
// products run, waves w and w + 4 (same rows) each decode two of the four row
// tiles of stage g + 1's B operands into an LDS slot that both read after the
// stage's barrier, so the decode's VALU work hides under the matrix cores.
constexpr int kQ4Waves = 8;
constexpr int kQ4Block = kQ4Waves * kWave;
constexpr int kQ4T = 128;                   // tokens per workgroup
constexpr int kQ4Dist = 3;                  // ring distance (stages)
constexpr int kQ4XSlots = 4;                // x slots (one stage each)
constexpr int kQ4QSlots = 2;                // quant slots (one pair of stages each)
typedef uint16_t Q4XSlot[2][kQ4T][32];      // one stage of x: [fp16 part][token][k], 16-byte chunks swizzled
typedef uint8_t Q4QSlot[kGR][32];           // one pair's quant bytes
typedef uint8_t Q4HSlot[kGR][16];           // one block's headers (d, dmin, scales)
typedef float Q4SSlot[kQ4T][8];             // one block's group sums
typedef f16x8_t Q4BSlot[4][4][kWave];       // B operands: [row group][row tile][lane]

template <int S>
using IC = std::integral_constant<int, S>;

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(IC<I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// A value the compiler may not fold into its users (keeps v_fmac_f32 from
// becoming v_fma_mix_f32, which issues at half the rate).
__device__ __forceinline__ float opaque(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// 16 bytes per lane global -> LDS (m0 + 16 lane). As inline assembly the
// compiler neither counts these loads nor waits for them; the kernel waits on
// its own vmcnt (only stricter for the compiler's own loads, of which the main
// loop has none).
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// This wave's loads in ring group j: 2 (x) + 1 (a pair's quant bytes, even j) +
// 2 (headers and group sums, a block's first stage).
__host__ __device__ constexpr int q4_group_loads(int j) {
    return 2 + ((j & 1) == 0 ? 1 : 0) + ((j & 7) == 0 ? 2 : 0);
}

__global__ __launch_bounds__(kQ4Block, 1) void gemm_q4k(const GemmJobs jobs, const int* __restrict__ ex,
                                                         const float* __restrict__ sx, const uint16_t* __restrict__ xp,
                                                         const float* __restrict__ x, int T, int K) {
    __shared__ __align__(16) Q4XSlot xr[kQ4XSlots];
    __shared__ __align__(16) Q4QSlot qr[kQ4QSlots];
    __shared__ __align__(16) Q4HSlot hr[2];
    __shared__ __align__(16) Q4SSlot sr[2];
    __shared__ __align__(16) Q4BSlot bs[2];
    const GemmJob job = gemm_job(jobs);
    const uint8_t* __restrict__ w = job.w;
    float* __restrict__ y = job.y;
    const int M = job.M;
    const uint64_t ub0 = job.ub0;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int rg = wv & 3, th = wv >> 2;                       // row group, token half
    const int t0w = blockIdx.y * kQ4T;                         // the workgroup's first token
    const int tw = t0w + 64 * th;                              // this wave's first token
    const int rw0 = job.mb * kGR;                              // the workgroup's first row
    const int r0 = rw0 + 64 * rg;                              // this wave's first row
    const int nb = K >> 8, nst = K >> 5;
    const int lr = lane & 15, lk = lane >> 4;
    const uint8_t* wbase = w + ub0 * 144;
    const uint8_t* xpb = reinterpret_cast<const uint8_t*>(xp);
    // Ring loads of a wave (byte offsets; stage and block offsets go into the
    // scalar base). x: part wv / 4, tokens 32 (wv % 4) + 16 i + lane / 4 (i < 2);
    // the lane at chunk c of its token's 64 bytes loads chunk c ^ ((token / 4) % 4),
    // which spreads the A reads over the LDS banks. Quant bytes: rows 32 wv + lane / 2.
    // Headers: rows 64 (wv % 4) + lane; group sums: tokens 32 (wv % 4) + lane / 2
    // (waves 4-7 repeat 0-3: the same bytes to the same place).
    const int xtk0 = 32 * (wv & 3);
    auto xoff = [&](int i) {
        const int tk = xtk0 + 16 * i + (lane >> 2);
        const int ch = (lane & 3) ^ ((tk >> 2) & 3);
        return 2u * (static_cast<uint32_t>(min(t0w + tk, T - 1)) * static_cast<uint32_t>(nst) * 64u + 32u * (wv >> 2) + 8u * ch);
    };
    const uint32_t qo = static_cast<uint32_t>(min(rw0 + 32 * wv + (lane >> 1), M - 1)) * static_cast<uint32_t>(nb) * 144u + 16u +
                        16u * (lane & 1);
    const uint32_t ho = static_cast<uint32_t>(min(r0 + lane, M - 1)) * static_cast<uint32_t>(nb) * 144u;
    const uint32_t so = 4u * (static_cast<uint32_t>(min(t0w + 32 * rg + (lane >> 1), T - 1)) * static_cast<uint32_t>(nst) +
                              4u * (lane & 1));
    auto lds_addr = [](const void* l) {
        return __builtin_amdgcn_readfirstlane(
            static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const void __attribute__((address_space(3)))*)(l))));
    };
    const uint32_t xr_a = lds_addr(&xr[0][0][0][0]), qr_a = lds_addr(&qr[0][0][0]), hr_a = lds_addr(&hr[0][0][0]),
                   sr_a = lds_addr(&sr[0][0][0]);
    // ring group gs, in 4 parts: x (2 halves), the pair's quant bytes (even gs),
    // the block's headers and group sums (its first stage)
    auto issue_part = [&](int gs, int part) {
        if (part < 2) {
            dma16(xoff(part), xpb + static_cast<size_t>(gs) * 128,
                  xr_a + static_cast<uint32_t>(gs % kQ4XSlots) * sizeof(Q4XSlot) + ((wv >> 2) * kQ4T + xtk0 + 16 * part) * 64u);
        } else if (part == 2) {
            if ((gs & 1) == 0)
                dma16(qo, wbase + static_cast<size_t>(gs >> 3) * 144 + 32 * ((gs & 7) >> 1),
                      qr_a + static_cast<uint32_t>((gs >> 1) % kQ4QSlots) * sizeof(Q4QSlot) + 32u * wv * 32u);
        } else if ((gs & 7) == 0) {
            const uint32_t hb = (gs >> 3) & 1;
            dma16(ho, wbase + static_cast<size_t>(gs >> 3) * 144, hr_a + hb * sizeof(Q4HSlot) + 64u * rg * 16u);
            dma16(so, sx + gs, sr_a + hb * sizeof(Q4SSlot) + 32u * rg * 32u);
        }
    };
    // B operand of row tile rt of stage gs (scale group SB of its block)
    auto decode_rt = [&](auto sbI, int gs, int rt) {
        constexpr int SB = decltype(sbI)::value;
        const int qs = (gs >> 1) % kQ4QSlots, hb = (gs >> 3) & 1;
        const uint32_t* hw = reinterpret_cast<const uint32_t*>(&hr[hb][64 * rg + 16 * rt + lr][0]);
        uint32_t sc;   // scale_min_k4 (src/cuda/matmul_q4.cu:18-26), scale part
        if constexpr (SB < 4)
            sc = (hw[1] >> (8 * SB)) & 63u;
        else
            sc = ((hw[3] >> (8 * (SB - 4))) & 15u) | (((hw[1] >> (8 * (SB - 4) + 6)) & 3u) << 4);
        const uint2 qb = *reinterpret_cast<const uint2*>(&qr[qs][64 * rg + 16 * rt + lr][8 * lk]);
        const uint32_t n0 = ((SB & 1) ? (qb.x >> 4) : qb.x) & 0x0f0f0f0fu;
        const uint32_t n1 = ((SB & 1) ? (qb.y >> 4) : qb.y) & 0x0f0f0f0fu;
        uint32_t e[4];
        q4_operand(n0, sc, e[0], e[1]);
        q4_operand(n1, sc, e[2], e[3]);
        f16x8_t r;
        __builtin_memcpy(&r, e, 16);
        return r;
    };
    auto wait_ring = [](int n) {   // at most n of this wave's ring loads in flight
        switch (n) {
            case 2: wait_vm<2>(); break;
            case 3: wait_vm<3>(); break;
            case 5: wait_vm<5>(); break;
            default: wait_vm<0>(); break;
        }
    };
    auto barrier = []() {   // LDS stores (the B slot) complete; the ring's loads stay in flight
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    f32x4_t acc[4][4], C[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acc[tt][rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // groups 0 .. kQ4Dist - 1 (nst >= 8); groups 0 and 1 complete
    {
        int pend = 0;
        for (int gs = 0; gs < kQ4Dist; ++gs) {
#pragma unroll
            for (int part = 0; part < 4; ++part) issue_part(gs, part);
            if (gs >= 2) pend += q4_group_loads(gs);
        }
        wait_ring(pend);
    }
    barrier();
#pragma unroll
    for (int i = 0; i < 2; ++i) bs[0][rg][2 * th + i][lane] = decode_rt(IC<0>{}, 0, 2 * th + i);
    barrier();

    // the A operand of lane (lr, lk): token 16 tt + lr, k 8 lk .. + 7 = chunk lk ^ ((lr / 4) % 4)
    const int ach = 8 * (lk ^ ((lr >> 2) & 3));
    // the min-term operand of lane (lr, lk): groups 2 lk, 2 lk + 1
    const bool mlo = lk < 2;
    const uint32_t msh = 16u * (lk & 1);
    for (int b = 0; b < nb; ++b) {
        const int g0 = 8 * b;
        static_for<8>([&](auto sI) {
            constexpr int S = decltype(sI)::value;
            const int g = g0 + S;
            const bool iss = g + kQ4Dist < nst;
            const bool dec = g + 1 < nst;
            f16x8_t B[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) B[rt] = bs[S & 1][rg][rt][lane];
            // the block's epilogue operands (last stage): d, -32 dmin and m_g
            float dsc[4], dmn5[4];
            f16x4_t Bm[4];
            if constexpr (S == 7) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    const uint4 h = *reinterpret_cast<const uint4*>(&hr[b & 1][64 * rg + 16 * rt + lr][0]);
                    const uint32_t z = h.z, wq = h.w;
                    const uint32_t l0 = (z >> msh) & 63u, l1 = (z >> (msh + 8)) & 63u;
                    const uint32_t h0 = ((wq >> (msh + 4)) & 15u) | (((z >> (msh + 6)) & 3u) << 4);
                    const uint32_t h1 = ((wq >> (msh + 12)) & 15u) | (((z >> (msh + 14)) & 3u) << 4);
                    const uint32_t m0 = mlo ? l0 : h0, m1 = mlo ? l1 : h1;
                    // fp16 1024 + m (bits 0x6400 | m) minus 1024: the exact small integers
                    const uint32_t pk = hadd2(((m1 << 16) | m0) + 0x64006400u, static_cast<_Float16>(-1024.0f));
                    const f16x2_t p2 = __builtin_bit_cast(f16x2_t, pk);
                    Bm[rt] = f16x4_t{p2[0], p2[0], p2[1], p2[1]};
                    dsc[rt] = opaque(half_bits(h.x & 0xffffu));
                    dmn5[rt] = opaque(-32.0f * half_bits(h.x >> 16));
                }
            }
            const Q4XSlot& xc = xr[g % kQ4XSlots];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                if (iss) issue_part(g + kQ4Dist, tt);
                if (dec && (tt & 1)) {
                    const int rt = 2 * th + (tt >> 1);
                    bs[(S + 1) & 1][rg][rt][lane] = decode_rt(IC<(S + 1) & 7>{}, g + 1, rt);
                }
                f16x8_t A[2];
#pragma unroll
                for (int p = 0; p < 2; ++p) A[p] = *reinterpret_cast<const f16x8_t*>(&xc[p][64 * th + 16 * tt + lr][ach]);
                // a block's first stage starts its sums from zero
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
                    C[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], B[rt], S == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : C[tt][rt], 0, 0, 0);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) C[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1], B[rt], C[tt][rt], 0, 0, 0);
                if constexpr (S == 7) {
                    // token tile tt of the block is complete: acc += d P_block - 32 dmin P_min with
                    // P_min = sum_g m_g (S_g 2^-5) as one [16 tokens x 16] x [16 x 16 rows] fp16
                    // product, k = (group 2 lk + i / 2, part i % 2): the two fp16 parts of S 2^-5
                    // (|S| < 2^20) against m_g twice
                    const float2 v = *reinterpret_cast<const float2*>(&sr[b & 1][64 * th + 16 * tt + lr][2 * lk]);
                    const float s0 = v.x * 0.03125f, s1 = v.y * 0.03125f;
                    const _Float16 a0 = static_cast<_Float16>(s0), a1 = static_cast<_Float16>(s1);
                    const f16x4_t As = f16x4_t{a0, static_cast<_Float16>(s0 - static_cast<float>(a0)), a1,
                                               static_cast<_Float16>(s1 - static_cast<float>(a1))};
#pragma unroll
                    for (int rt = 0; rt < 4; ++rt) {
                        const f32x4_t pm = __builtin_amdgcn_mfma_f32_16x16x16f16(As, Bm[rt], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[tt][rt][r] = __builtin_fmaf(dsc[rt], C[tt][rt][r], acc[tt][rt][r]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[tt][rt][r] = __builtin_fmaf(dmn5[rt], pm[r], acc[tt][rt][r]);
                    }
                }
            }
            // group g + 2 (the next stage's decode) complete; group g + 3 may stay in flight
            wait_ring(g + 3 < nst ? q4_group_loads((S + 3) & 7) : 0);
            barrier();
        });
    }
    // lane L holds C[4 (L/16) + r][L % 16] of tile (tt, rt): token 16 tt + 4 lk + r, row 16 rt + lr
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = tw + 16 * tt + 4 * lk + r;
            if (t >= T) continue;
            const int et = ex[t];
            if (et == kRowNonFinite) {
                for (int rt = 0; rt < 4; ++rt) {
                    const int row = r0 + 16 * rt + lr;
                    if (row < M)
                        y[static_cast<size_t>(t) * M + row] = row_dot_per_element(
                            w, kQ4_K, (ub0 + static_cast<uint64_t>(row) * nb) * 256, x + static_cast<size_t>(t) * K, K);
                }
                continue;
            }
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const int row = r0 + 16 * rt + lr;
                if (row < M) y[static_cast<size_t>(t) * M + row] = ldexpf(acc[tt][rt][r], -et);
            }
        }
}

// ------------------------------------------------------------------ Q6_K
// Element i of a block (src/cuda/matmul_q4.cu:105-126): ql byte 64(i/128) +
// 32((i%128)/32 & 1) + i%32 (low nibble in quarters 0, 1 of a half, high in
// 2, 3), qh byte 128 + 32(i/128) + i%32 bits 2*quarter, scale byte 192 + i/16,
// d at 208. Stage sg of a block (elements 32 sg ..) is half sg/4, quarter
// sg%4; lane (l32, lh) of step h takes elements 32 sg + 16 h + 8 lh .. +7:
// eight consecutive ql and qh bytes, scale 2 sg + h.
//
// A workgroup (8 waves, one per CU) owns 128 tokens x 256 weight rows; wave w
// owns rows 64 (w % 4) .. +63 for tokens 64 (w / 4) .. +63 (2 x 2 tiles of
// 32 x 32 on v_mfma_f32_32x32x16_f16, k = one 16-element scale group, so each
// group's product is scaled by d * sc in fp32 before it joins the sums). x goes
// through LDS from registers (the next stage loaded while the current one
// computes). The quant bytes and scales of a half-block (4 stages: 64 ql
// bytes, both nibbles; 32 qh bytes; the 16 scales and d) are staged per row in
// LDS with coalesced 16-byte loads four stages ahead; waves w and w + 4 (same
// rows) split the next stage's B decode (wave w / 4 takes step h = w / 4) into
// an LDS slot both read after the stage's barrier.
constexpr int kQ6Waves = 8;
constexpr int kQ6Block = kQ6Waves * kWave;
constexpr int kQ6T = 128;                    // tokens per workgroup
typedef uint16_t Q6XStage[2][kQ6T][kXRow];   // one stage of x: the two fp16 parts
typedef f16x8_t Q6BSlot[4][2][2][kWave];     // B operands: [row group][step h][row tile][lane]
// One half-block of a row: ql bytes 64 half .. +63 | qh bytes 128 + 32 half .. +31 |
// scales (block bytes 192..207) | block bytes 194..209 (d in the last two) | pad (row
// stride 36 dwords spreads a wave's 32 rows over the LDS banks)
typedef uint8_t Q6WSlot[kGR][144];

// 16 bytes at a 2-byte aligned address (gfx950 global loads take any byte
// alignment; Q6_K blocks are 210 bytes).
__device__ __forceinline__ uint4 ldg16_a2(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 2), 16);
    return v;
}

__global__ __launch_bounds__(kQ6Block, 1) void gemm_q6k(const GemmJobs jobs, const int* __restrict__ ex,
                                                         const uint16_t* __restrict__ xp, const float* __restrict__ x,
                                                         int T, int K) {
    __shared__ __align__(16) Q6XStage xs[2];
    __shared__ __align__(16) Q6BSlot bs[2];
    __shared__ __align__(16) Q6WSlot wsl[2];
    const GemmJob job = gemm_job(jobs);
    const uint8_t* __restrict__ w = job.w;
    float* __restrict__ y = job.y;
    const int M = job.M;
    const uint64_t ub0 = job.ub0;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int rg = wv & 3, th = wv >> 2;                       // row group, token half (= decode step)
    const int t0w = blockIdx.y * kQ6T;
    const int tw = t0w + 64 * th;
    const int rw0 = job.mb * kGR;
    const int r0 = rw0 + 64 * rg;
    const int nb = K >> 8, nst = K >> 5, nhb = nst >> 2;
    const int tok = tid >> 2, part = tid & 3;
    const uint16_t* xsrc = xp + static_cast<size_t>(min(t0w + tok, T - 1)) * nst * 64 + 32 * (part >> 1) + 16 * (part & 1);
    const int l32 = lane & 31, lh = lane >> 5;
    auto store_xs = [&](const XRegs& r, Q6XStage& d) {
        uint16_t* p = &d[part >> 1][tok][16 * (part & 1)];
        st16(p, r.a);
        st16(p + 8, r.b);
    };
    // half-block j of every row: thread tid loads 16-byte pieces tid + 512 i (i < 4)
    // of the 2048 (row c / 8, piece c % 8: ql 0-3, qh 4-5, scales 6, d 7)
    uint4 wst[4];
    auto wstage_load = [&](int j) {
        const int half = j & 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 512 * i;
            const int row = c >> 3, piece = c & 7;
            const uint8_t* blk = w + (ub0 + static_cast<uint64_t>(min(rw0 + row, M - 1)) * nb + (j >> 1)) * 210;
            const int off = piece < 4 ? 64 * half + 16 * piece
                                      : piece < 6 ? 128 + 32 * half + 16 * (piece - 4) : 192 + 2 * (piece - 6);
            wst[i] = ldg16_a2(blk + off);
        }
    };
    auto wstage_store = [&](int j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 512 * i;
            *reinterpret_cast<uint4*>(&wsl[j & 1][c >> 3][16 * (c & 7)]) = wst[i];
        }
    };
    // this wave's share of stage g's B operands (step h = th, both row tiles): q - 32
    auto decode = [&](int g) {
        const int sg = g & 7, quarter = sg & 3;
        const int nsh = 4 * (quarter >> 1), hsh = 2 * quarter;
        const Q6WSlot& sl = wsl[(g >> 2) & 1];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = 64 * rg + 32 * rt + l32;
            const uint2 ql = *reinterpret_cast<const uint2*>(&sl[row][32 * (quarter & 1) + 16 * th + 8 * lh]);
            const uint2 qh = *reinterpret_cast<const uint2*>(&sl[row][64 + 16 * th + 8 * lh]);
            const uint32_t q0 = ((ql.x >> nsh) & 0x0f0f0f0fu) | (((qh.x >> hsh) & 0x03030303u) << 4);
            const uint32_t q1 = ((ql.y >> nsh) & 0x0f0f0f0fu) | (((qh.y >> hsh) & 0x03030303u) << 4);
            uint32_t e[4];
            q6_operand(q0, e[0], e[1]);
            q6_operand(q1, e[2], e[3]);
            f16x8_t r;
            __builtin_memcpy(&r, e, 16);
            bs[g & 1][rg][th][rt][lane] = r;
        }
    };
    auto barrier = []() {   // LDS stores complete, then the workgroup meets
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[tt][rt][i] = 0.f;

    wstage_load(0);
    wstage_store(0);
    if (nhb > 1) {   // K >= 256: nhb >= 2
        wstage_load(1);
        wstage_store(1);
    }
    store_xs(load_x(xsrc), xs[0]);
    barrier();
    decode(0);
    barrier();

    for (int g = 0; g < nst; ++g) {
        const int sg = g & 7, cur = g & 1;
        const int gn = g + 1;
        const bool more = gn < nst;
        // d * sc of this stage's two groups for the lane's two rows
        float Ag[2][2];
        {
            const Q6WSlot& sl = wsl[(g >> 2) & 1];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const int row = 64 * rg + 32 * rt + l32;
                const uint32_t sp = *reinterpret_cast<const uint16_t*>(&sl[row][96 + 2 * sg]);   // scales 2 sg, 2 sg + 1
                const float d = half_bits(*reinterpret_cast<const uint16_t*>(&sl[row][126]));
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    Ag[h][rt] = d * static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(sp, 8 * h, 8)));
            }
        }
        XRegs xn;
        if (more) xn = load_x(xsrc + static_cast<size_t>(gn) * 64);
        // half-block k + 1 (loaded at half-block k - 1's first stage) goes into k - 1's
        // slot at half-block k's first stage (k - 1's decodes and scale reads ended with
        // the previous barrier); then half-block k + 2 is loaded
        const int jh = g >> 2;
        if ((g & 3) == 0) {
            if (jh >= 1 && jh + 1 < nhb) wstage_store(jh + 1);
            if (jh + 2 < nhb) wstage_load(jh + 2);
        }
        f16x8_t B[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) B[h][rt] = bs[cur][rg][h][rt][lane];
        if (more) decode(gn);
        const Q6XStage& xc = xs[cur];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                f16x8_t A[2];
#pragma unroll
                for (int p = 0; p < 2; ++p)
                    A[p] = *reinterpret_cast<const f16x8_t*>(&xc[p][64 * th + 32 * tt + l32][16 * h + 8 * lh]);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    f32x16_t Cq;
#pragma unroll
                    for (int i = 0; i < 16; ++i) Cq[i] = 0.f;
                    Cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[h][rt], Cq, 0, 0, 0);
                    Cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[h][rt], Cq, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[tt][rt][i] = __builtin_fmaf(Ag[h][rt], Cq[i], acc[tt][rt][i]);
                }
            }
        if (more) store_xs(xn, xs[cur ^ 1]);
        barrier();
    }
    // lane L holds C[8 (i/4) + 4 (L/32) + i%4][L % 32] of tile (tt, rt) in register i
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int t = tw + 32 * tt + 8 * (i >> 2) + 4 * lh + (i & 3);
            if (t >= T) continue;
            const int et = ex[t];
            if (et == kRowNonFinite) {
                for (int rt = 0; rt < 2; ++rt) {
                    const int row = r0 + 32 * rt + l32;
                    if (row < M)
                        y[static_cast<size_t>(t) * M + row] = row_dot_per_element(
                            w, kQ6_K, (ub0 + static_cast<uint64_t>(row) * nb) * 256, x + static_cast<size_t>(t) * K, K);
                }
                continue;
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const int row = r0 + 32 * rt + l32;
                if (row < M) y[static_cast<size_t>(t) * M + row] = ldexpf(acc[tt][rt][i], -et);
            }
        }
}

// The Q4_K kernel's ring loads address x's fp16 parts and the weight rows with
// 32-bit byte offsets.
bool gemm_rows_ok(int rows, int K, const float* x) {
    return rows >= kGemmMinRows && K % 256 == 0 && aligned16(x) && rows <= kGemmMaxRows &&
           4 * static_cast<uint64_t>(rows) * static_cast<uint64_t>(K) < (uint64_t{1} << 32);
}

bool gemm_job_ok(int type, uint64_t element_offset, int M, int K) {
    if (element_offset % 256 != 0) return false;
    if (type == kQ6_K) return true;
    return type == kQ4_K && static_cast<uint64_t>(M) * static_cast<uint64_t>(K / 256) * 144 < (uint64_t{1} << 32);
}

struct Prepared {
    const int* ex;
    const float* sx;
    const uint16_t* xp;
    const float* x;   // the token rows themselves (rows holding an infinity)
};

// Checks the workspace and launches the prep kernel.
int prepare_x(const float* x, int rows, int K, void* workspace, size_t workspace_bytes, hipStream_t s, Prepared& p) {
    const size_t need = ws_bytes(rows, K);
    QK_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
               "matmul_rows: workspace of %zu bytes (16-byte aligned) needed, got %zu", need,
               workspace ? workspace_bytes : size_t{0});
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    int* ex = reinterpret_cast<int*>(ws);
    float* sx = reinterpret_cast<float*>(ws + ws_exp_bytes(rows));
    uint16_t* xp = reinterpret_cast<uint16_t*>(ws + ws_exp_bytes(rows) + ws_sum_bytes(rows, K));
    const unsigned grid = blocks_for(rows, 4);
    switch (K) {
        case 512: gemm_prep_x<2><<<grid, 256, 0, s>>>(x, ex, sx, xp, rows, K); break;
        case 1024: gemm_prep_x<4><<<grid, 256, 0, s>>>(x, ex, sx, xp, rows, K); break;
        case 2048: gemm_prep_x<8><<<grid, 256, 0, s>>>(x, ex, sx, xp, rows, K); break;
        case 4096: gemm_prep_x<16><<<grid, 256, 0, s>>>(x, ex, sx, xp, rows, K); break;
        default: gemm_prep_x<0><<<grid, 256, 0, s>>>(x, ex, sx, xp, rows, K); break;
    }
    p = Prepared{ex, sx, xp, x};
    return check_launch("matmul_rows prep");
}

void launch_gemm(int type, const GemmJobs& jobs, const Prepared& p, int rows, int K, hipStream_t s) {
    if (type == kQ4_K)
        gemm_q4k<<<dim3(jobs.start[jobs.n], blocks_for(rows, kQ4T)), kQ4Block, 0, s>>>(jobs, p.ex, p.sx, p.xp, p.x, rows, K);
    else
        gemm_q6k<<<dim3(jobs.start[jobs.n], blocks_for(rows, kQ6T)), kQ6Block, 0, s>>>(jobs, p.ex, p.xp, p.x, rows, K);
}

// One GEMV per token (the reference's own loop).
int per_token(const void* weight, int type, uint64_t num_elements, const float* x, float* y, int rows, int M, int K,
              uint64_t element_offset, void* stream) {
    for (int t = 0; t < rows; ++t) {
        const int rc = qwen_matmul_dispatch(weight, type, num_elements, x + static_cast<size_t>(t) * K,
                                            y + static_cast<size_t>(t) * M, M, K, element_offset, stream);
        if (rc) return rc;
    }
    return ok();
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

size_t qwen_matmul_rows_workspace_bytes(int rows, int K) {
    if (rows < kGemmMinRows || K <= 0 || K % 256 != 0) return 0;
    return ws_bytes(rows, K);
}

int qwen_matmul_rows(const void* weight, int type, uint64_t num_elements, const float* x, float* y, int rows, int M,
                     int K, uint64_t element_offset, void* workspace, size_t workspace_bytes, void* stream) {
    if (!weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "tensor is not loaded");
    if (!type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "unsupported GGML type %d", type);
    if (M <= 0 || K <= 0 || element_offset > num_elements ||
        static_cast<uint64_t>(M) * static_cast<uint64_t>(K) > num_elements - element_offset)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "GEMV shape exceeds tensor (M=%d, K=%d)", M, K);
    QK_REQUIRE(rows >= 0, "matmul_rows: negative rows %d", rows);
    if (rows == 0) return ok();
    QK_REQUIRE(x && y, "matmul_rows: null pointer");
    if (!gemm_rows_ok(rows, K, x) || !gemm_job_ok(type, element_offset, M, K))
        return per_token(weight, type, num_elements, x, y, rows, M, K, element_offset, stream);
    const hipStream_t s = as_stream(stream);
    Prepared p;
    if (const int rc = prepare_x(x, rows, K, workspace, workspace_bytes, s, p)) return rc;
    GemmJobs jobs{};
    jobs.w[0] = static_cast<const uint8_t*>(weight);
    jobs.y[0] = y;
    jobs.ub0[0] = element_offset / 256;
    jobs.M[0] = M;
    jobs.start[0] = 0;
    jobs.start[1] = static_cast<int>(blocks_for(M, kGR));
    jobs.n = 1;
    launch_gemm(type, jobs, p, rows, K, s);
    return check_launch("matmul_rows");
}

int qwen_matmul_rows_multi(const qwen_gemv_desc* descs, int n, const float* x, int rows, int K, void* workspace,
                           size_t workspace_bytes, void* stream) {
    QK_REQUIRE(n >= 0 && n <= 64, "matmul_rows_multi: n = %d outside [0, 64]", n);
    if (n == 0) return ok();
    QK_REQUIRE(descs, "matmul_rows_multi: null descriptors");
    for (int j = 0; j < n; ++j) {
        const qwen_gemv_desc& e = descs[j];
        if (!e.weight) return fail(QWEN_STATUS_INVALID_ARGUMENT, "descriptor %d: tensor is not loaded", j);
        if (!type_supported(e.type))
            return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "descriptor %d: unsupported GGML type %d", j, e.type);
        if (e.M <= 0 || K <= 0 || e.element_offset > e.num_elements ||
            static_cast<uint64_t>(e.M) * static_cast<uint64_t>(K) > e.num_elements - e.element_offset)
            return fail(QWEN_STATUS_OUT_OF_RANGE, "descriptor %d: GEMV shape exceeds tensor (M=%d, K=%d)", j, e.M, K);
        QK_REQUIRE(e.split == 0, "matmul_rows_multi: descriptor %d: split rows are not supported", j);
        QK_REQUIRE(e.y, "matmul_rows_multi: descriptor %d has a null output", j);
    }
    QK_REQUIRE(rows >= 0, "matmul_rows_multi: negative rows %d", rows);
    if (rows == 0) return ok();
    QK_REQUIRE(x, "matmul_rows_multi: null x");
    const bool gemm = gemm_rows_ok(rows, K, x);
    const hipStream_t s = as_stream(stream);
    Prepared p{};
    bool prepared = false;
    for (const int type : {static_cast<int>(kQ4_K), static_cast<int>(kQ6_K)}) {
        GemmJobs jobs{};
        auto flush = [&]() {
            if (jobs.n == 0) return;
            launch_gemm(type, jobs, p, rows, K, s);
            jobs.n = 0;
        };
        for (int j = 0; gemm && j < n; ++j) {
            const qwen_gemv_desc& e = descs[j];
            if (e.type != type || !gemm_job_ok(e.type, e.element_offset, e.M, K)) continue;
            if (!prepared) {
                if (const int rc = prepare_x(x, rows, K, workspace, workspace_bytes, s, p)) return rc;
                prepared = true;
            }
            const int k = jobs.n;
            jobs.w[k] = static_cast<const uint8_t*>(e.weight);
            jobs.y[k] = e.y;
            jobs.ub0[k] = e.element_offset / 256;
            jobs.M[k] = e.M;
            if (k == 0) jobs.start[0] = 0;
            jobs.start[k + 1] = jobs.start[k] + static_cast<int>(blocks_for(e.M, kGR));
            jobs.n = k + 1;
            if (jobs.n == kGemmJobs) flush();
        }
        flush();
    }
    if (prepared)
        if (const int rc = check_launch("matmul_rows_multi")) return rc;
    for (int j = 0; j < n; ++j) {   // the rest: one GEMV per token
        const qwen_gemv_desc& e = descs[j];
        if (gemm && gemm_job_ok(e.type, e.element_offset, e.M, K)) continue;
        if (const int rc = per_token(e.weight, e.type, e.num_elements, x, e.y, rows, e.M, K, e.element_offset, stream))
            return rc;
    }
    return ok();
}

}  // extern "C"
