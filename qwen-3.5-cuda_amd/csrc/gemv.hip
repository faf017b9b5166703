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
// L2). Fast path (Q4_K, Q6_K): the weight is walked in units of 8 consecutive
// 256-element blocks (2048 elements = 1152 B of Q4_K or 1680 B of Q6_K, both
// multiples of 16 bytes). A row of K = 256*nb elements is nb/8 units when
// 8 | nb; when nb | 8, 8/nb consecutive rows share one unit. A wave owns R
// units at a time: it copies them into its LDS slot with 16-byte non-temporal
// loads (contiguous, fully coalesced), then lane L decodes 32 elements of
// block L/8 of each unit. That lane->element map is the same for every unit,
// so the lane's 32 x values are loaded once and stay in VGPRs across all R
// units. The dot product runs on the raw quants and the block scale is
// applied once per run of 16 (Q4_K) or 8 (Q6_K) elements:
//   sum((d*sc*q - dmin*m) * x) = (d*sc) * sum(q*x) - (dmin*m) * sum(x)
// which is the reference's sum re-associated (fp32 tolerance, not bit-exact:
// the reference's own order depends on its launch shape).
#include <algorithm>
#include <type_traits>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "ggml_common.hpp"

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

template <int TYPE>
__device__ __forceinline__ void load_lane_x(LaneX<TYPE>& lx, const float* __restrict__ x, int xb, int j) {
    const float* xblk = x + static_cast<size_t>(xb) * 256;
    if constexpr (TYPE == kQ4_K) {
        const float* lo = xblk + 64 * (j >> 1) + 16 * (j & 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lx.v[i] = ld4(lo + 4 * i);
            lx.v[4 + i] = ld4(lo + 32 + 4 * i);
        }
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a += (lx.v[i].x + lx.v[i].y) + (lx.v[i].z + lx.v[i].w);
            b += (lx.v[4 + i].x + lx.v[4 + i].y) + (lx.v[4 + i].z + lx.v[4 + i].w);
        }
        lx.s[0] = a;
        lx.s[1] = b;
        lx.s[2] = lx.s[3] = 0.f;
    } else {
        const float* base = xblk + 128 * (j >> 2) + 8 * (j & 3);
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

// sum over the 4 bytes of `q` (unsigned) times 4 x values.
__device__ __forceinline__ float dot_u8x4(uint32_t q, float4 xv, float acc) {
    acc = __builtin_fmaf(static_cast<float>(q & 0xffu), xv.x, acc);
    acc = __builtin_fmaf(static_cast<float>((q >> 8) & 0xffu), xv.y, acc);
    acc = __builtin_fmaf(static_cast<float>((q >> 16) & 0xffu), xv.z, acc);
    return __builtin_fmaf(static_cast<float>(q >> 24), xv.w, acc);
}

// Contribution of one block to the lane's partial dot product. `blk` points
// at the block in LDS.
template <int TYPE>
__device__ __forceinline__ float block_dot(const uint8_t* blk, const LaneX<TYPE>& lx, int j) {
    if constexpr (TYPE == kQ4_K) {
        const uint4 hdr = *reinterpret_cast<const uint4*>(blk);                // d, dmin, scales[12]
        const uint4 q = *reinterpret_cast<const uint4*>(blk + 16 + 16 * j);   // qs bytes 16j..16j+15
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
            lo = dot_u8x4(w[i] & 0x0f0f0f0fu, lx.v[i], lo);
            hi = dot_u8x4((w[i] >> 4) & 0x0f0f0f0fu, lx.v[4 + i], hi);
        }
        const float A0 = d * static_cast<float>(sc0), B0 = dmin * static_cast<float>(m0);
        const float A1 = d * static_cast<float>(sc1), B1 = dmin * static_cast<float>(m1);
        return (A0 * lo - B0 * lx.s[0]) + (A1 * hi - B1 * lx.s[1]);
    } else {
        const int half = j >> 2, l0 = 8 * (j & 3);
        const uint8_t* qla = blk + 64 * half + l0;         // quarters 0 (low nibble), 2 (high)
        const uint8_t* qlb = qla + 32;                     // quarters 1, 3
        const uint8_t* qhp = blk + 128 + 32 * half + l0;   // 2 bits per quarter
        const uint32_t la0 = lds_u32_a2(qla), la1 = lds_u32_a2(qla + 4);
        const uint32_t lb0 = lds_u32_a2(qlb), lb1 = lds_u32_a2(qlb + 4);
        const uint32_t h0 = lds_u32_a2(qhp), h1 = lds_u32_a2(qhp + 4);
        // scales[8*half + l0/16 + 2*qq]: bytes (l0/16) + {0, 2} of the first
        // word (qq 0, 1) and of the second word (qq 2, 3).
        const uint32_t s0 = lds_u32_a2(blk + 192 + 8 * half), s1 = lds_u32_a2(blk + 196 + 8 * half);
        const int ss = 8 * (l0 >> 4);
        const float d = half_bits(*reinterpret_cast<const uint16_t*>(blk + 208));
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
}

// Device-side expert selection (MoE): launch row blockIdx.y runs selected
// expert idx[blockIdx.y] -- weight rows at element offset idx * stride -- on
// x + blockIdx.y * x_stride, writing y + blockIdx.y * M. An id outside
// [0, n_experts) gives a NaN row. idx == nullptr: a plain GEMV.
struct Experts {
    const int32_t* idx;
    int n_experts;
    uint64_t stride;  // elements between experts (a multiple of 256 on the fast path)
    int64_t x_stride;
};

// Applies the selection of launch row blockIdx.y; false if the expert id is
// invalid (the caller writes NaN rows).
__device__ __forceinline__ bool select_expert(const Experts& ex, int M, int64_t& x_off, int64_t& y_off,
                                              uint64_t& element_offset) {
    x_off = y_off = 0;
    if (!ex.idx) return true;
    const int j = blockIdx.y;
    const int e = ex.idx[j];
    x_off = static_cast<int64_t>(j) * ex.x_stride;
    y_off = static_cast<int64_t>(j) * M;
    if (e < 0 || e >= ex.n_experts) return false;
    element_offset += static_cast<uint64_t>(e) * ex.stride;
    return true;
}

// Fast path. Row groups: when 8 | nb, group = one row and unit (row, slice s)
// starts at block ub0 + row*nb + 8s; when nb | 8, group = 8/nb rows (P) and
// unit u starts at block ub0 + 8u. A wave owns groups g0 .. g0+R-1.
template <int TYPE, int R>
__global__ __launch_bounds__(kGemvBlock) void gemv_kquant(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int nb, uint64_t ub0,
                                                          int groups, uint64_t tensor_bytes, Experts ex) {
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
    const bool ok_e = select_expert(ex, M, x_off, y_off, eoff);
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
        if (lane < R && g0 + lane < M) y[g0 + lane] = out;
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
            if (lane % gl == 0 && g0 + u < groups && row < M) y[row] = t;
        }
    }
}

// Generic path (any supported type and shape): one wave per row, element-wise
// decode.
__global__ __launch_bounds__(kBlock) void gemv_any(const uint8_t* __restrict__ w, int type,
                                                   const float* __restrict__ x, float* __restrict__ y, int M, int K,
                                                   uint64_t element_offset, Experts ex) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kBlock / kWave) + wave_in_block();
    if (row >= M) return;
    int64_t x_off, y_off;
    const bool ok_e = select_expert(ex, M, x_off, y_off, element_offset);
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
    if (lane == 0) y[row] = s;
}

template <int TYPE, int R>
void launch_kquant(const uint8_t* w, const float* x, float* y, int M, int nb, uint64_t ub0, int groups,
                   uint64_t tensor_bytes, const Experts& ex, int n_sel, hipStream_t s) {
    constexpr int CPU = KQuant<TYPE>::kBlockBytes * 8 / 16;
    const size_t lds = static_cast<size_t>(kGemvWaves) * R * CPU * 16;
    const int waves = (groups + R - 1) / R;
    gemv_kquant<TYPE, R><<<dim3(blocks_for(waves, kGemvWaves), n_sel), kGemvBlock, lds, s>>>(
        w, x, y, M, nb, ub0, groups, tensor_bytes, ex);
}

template <int TYPE>
void dispatch_kquant(const uint8_t* w, const float* x, float* y, int M, int nb, uint64_t ub0, int groups,
                     uint64_t tensor_bytes, const Experts& ex, int n_sel, hipStream_t s) {
    // Units per wave: enough waves to fill 256 CUs several times over. More than
    // 4 units per wave measured slower (fewer waves per SIMD to hide latency).
    const int64_t all = static_cast<int64_t>(groups) * n_sel;
    if (all >= 4 * 4096)
        launch_kquant<TYPE, 4>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
    else if (all >= 2 * 4096)
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
    if (kquant && shape_ok && aligned) {
        const uint64_t ub0 = element_offset / 256;
        const int groups = nb >= 8 ? M : (M + 8 / nb - 1) / (8 / nb);
        if (type == kQ4_K)
            dispatch_kquant<kQ4_K>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
        else
            dispatch_kquant<kQ6_K>(w, x, y, M, nb, ub0, groups, tensor_bytes, ex, n_sel, s);
    } else {
        gemv_any<<<dim3(blocks_for(M, kBlock / kWave), n_sel), kBlock, 0, s>>>(w, type, x, y, M, K, element_offset,
                                                                             ex);
    }
    return check_launch(what);
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

}  // extern "C"
