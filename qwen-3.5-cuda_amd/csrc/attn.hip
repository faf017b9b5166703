// Attention front end on gfx950: per-head RMSNorm fused with split-half partial
// RoPE for Q and K, in place.
//
// Reference semantics: head_norm_kernel (src/cuda/attn_kernels.cu:34-63,
// x = x * (r * w)) followed by rope_kernel (src/cuda/rope.cu:9-29,
// theta = pos / powf(base, 2i/rd)), called as src/layer_attn.cpp:91-96.
//
// Mapping: a head of head_dim = 4*LPH floats is held by LPH lanes as one float4
// each. The sum of squares is a DPP group reduction; the RoPE partner of dims
// (i..i+3) sits half/4 lanes away. Each lane group evaluates the sincos values
// of its own head's (position, pair) once and hands them to the lanes that need
// them, instead of every rotary lane recomputing them. The production shape
// (head_dim 256, rope_dim 64) has its own form: three heads of one token per
// wave, one set of angles for the three, cross-lane moves by DPP and permlane
// swaps only (qk_norm_rope_grouped).
//
// The inverse-frequency denominators powf(theta, 2i/rd) are computed on the host
// (double pow, rounded once) and passed as kernel arguments: a one-ulp change in
// a denominator moves cos/sin by up to ~6e-5 at pos 511, theta 1e7, so the
// device must divide by exactly the value the host oracle uses. The division
// pos / den is IEEE (correctly rounded) and sincosf is the accurate ocml form.
#include <algorithm>
#include <cmath>

#include "attn_common.hpp"
#include "capi_common.hpp"
#include "device_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;

// ------------------------------------------------------------ vector kernel
// Any head_dim of 64, 128 or 256 floats (LPH = 16, 32, 64 lanes per head): the
// RoPE partner and the angles move through ds_bpermute.
template <int LPH, bool NORM, bool ROPE>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_v4(float* __restrict__ q, float* __restrict__ k,
                                                          const float* __restrict__ qw, const float* __restrict__ kw,
                                                          const int32_t* __restrict__ pos, int pos0, int rows,
                                                          int q_heads, int k_heads, int rope_dim, RopeDen den,
                                                          float eps) {
    constexpr int HPW = kWave / LPH;  // heads per wave
    constexpr int HD = 4 * LPH;
    const int lane = threadIdx.x & 63;
    const int lg = lane % LPH;
    const int gbase = lane - lg;
    // 32-bit index math (the host checks rows * heads < 2^31); the wave index is
    // made explicitly uniform so that, with one head per wave, the head and
    // position arithmetic and the position load stay scalar.
    const int hpr = q_heads + k_heads;
    const int total = rows * hpr;
    const int wave = static_cast<int>(blockIdx.x) * (kBlock / kWave) + wave_in_block();
    if (wave * HPW >= total) return;  // wave-uniform
    const int slot = wave * HPW + (HPW > 1 ? lane / LPH : 0);  // wave-uniform when HPW == 1
    const bool active = slot < total;
    const int sl = active ? slot : total - 1;  // clamped: loads never branch
    const int t = sl / hpr;
    const int h = sl - t * hpr;
    float* p = (h < q_heads) ? q + (static_cast<size_t>(t) * q_heads + h) * HD
                             : k + (static_cast<size_t>(t) * k_heads + (h - q_heads)) * HD;
    const float* wt = (h < q_heads) ? qw : kw;
    const int half = rope_dim >> 1;

    // Issue order matters (vector loads return in order): the denominators
    // first, then the row and its weights, then the angle math, which only
    // waits for the denominators and so overlaps the row's flight. The
    // position is a scalar load when a wave holds one head.
    float fp = 0.f, dn0 = 1.f, dn1 = 1.f;
    if constexpr (ROPE) {
        fp = static_cast<float>(pos ? pos[t] : pos0 + t);
        dn0 = den.den[min(lg, kMaxDen - 1)];
        dn1 = den.den[min(lg + LPH, kMaxDen - 1)];
    }
    float4 v = ld4_nt(p + 4 * lg);
    const float4 wv = NORM ? ld4(wt + 4 * lg) : make_float4(1.f, 1.f, 1.f, 1.f);

    // Rotation angles of this group's head (pairs lg and lg + LPH).
    float c0 = 1.f, s0 = 0.f, c1 = 1.f, s1 = 0.f;
    if constexpr (ROPE) {
        if (lg < half) sincosf(fp / dn0, &s0, &c0);
        if (lg + LPH < half) sincosf(fp / dn1, &s1, &c1);
    }

    if constexpr (NORM) {
        const float ss = group_sum<LPH>(sumsq4(v));
        const float r = rsqrtf(ss / static_cast<float>(HD) + eps);
        v.x = v.x * (r * wv.x);
        v.y = v.y * (r * wv.y);
        v.z = v.z * (r * wv.z);
        v.w = v.w * (r * wv.w);
    }

    if constexpr (ROPE) {
        const int d0 = 4 * lg;
        const bool first = d0 < half;                 // dims i..i+3, partner i+half
        const bool second = !first && d0 < rope_dim;  // dims i+half.., partner i
        const int plg = first ? lg + (half >> 2) : (second ? lg - (half >> 2) : lg);
        const int src = gbase + plg;
        float4 pv;
        pv.x = lane_fetch(v.x, src);
        pv.y = lane_fetch(v.y, src);
        pv.z = lane_fetch(v.z, src);
        pv.w = lane_fetch(v.w, src);

        const int i0 = first ? d0 : (second ? d0 - half : 0);  // pair index of .x
        float cs[4], sn[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int from = gbase + ((i0 + j) % LPH);
            cs[j] = lane_fetch(c0, from);
            sn[j] = lane_fetch(s0, from);
        }
        if (half > LPH) {  // wave-uniform: only when rope_dim > head_dim / 2
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = i0 + j;
                const int from = gbase + (i % LPH);
                const float cb = lane_fetch(c1, from), sb = lane_fetch(s1, from);
                if (i >= LPH) {
                    cs[j] = cb;
                    sn[j] = sb;
                }
            }
        }
        const float a[4] = {v.x, v.y, v.z, v.w};
        const float b[4] = {pv.x, pv.y, pv.z, pv.w};
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (first)
                o[j] = a[j] * cs[j] - b[j] * sn[j];  // x[i]      = a c - b s
            else if (second)
                o[j] = a[j] * cs[j] + b[j] * sn[j];  // x[i+half] = b c + a s (a here is x[i+half])
            else
                o[j] = a[j];
        }
        v = make_float4(o[0], o[1], o[2], o[3]);
    }
    if (active) st4_nt(p + 4 * lg, v);
}

// ------------------------------------------------------------ grouped heads
// The production shape (head_dim 256, rope_dim 64) with HPW heads of one token
// per wave: every lane holds one float4 of each head, all HPW row loads are in
// flight together, and the token's rotation angles are evaluated once for the
// HPW heads. Every value the rotation needs moves through VALU cross-lane ops
// instead of ds_bpermute: lane 16r + m evaluates the angle of pair
// 4*(m % 8) + r, so rotary lane m (m < 16) finds its four pairs at lanes m,
// m+16, m+32, m+48 (gathered with v_permlane16_swap / v_permlane32_swap), and
// its partner 8 lanes away in the same 16-lane row (DPP row_ror:8). Head h of a
// token is Q head h for h < q_heads, else K head h - q_heads; a group may hold
// both. At C2 (16 + 2 heads, 18.9 MB in place) three heads per wave in
// 192-thread workgroups measured 4.5 us against 5.5 us for one head per wave
// (launch shapes swept on the MI355X): more bytes in flight per wave and 3
// waves per SIMD, all resident at once.
constexpr int kGroupHeads = 3;
constexpr int kGroupBlock = 192;


// POS: positions from the array `pos`, else pos0 + t.
template <int HPW, bool NORM, bool POS>
__global__ __launch_bounds__(kGroupBlock) void qk_norm_rope_grouped(float* __restrict__ q, float* __restrict__ k,
                                                                   const float* __restrict__ qw,
                                                                   const float* __restrict__ kw,
                                                                   const int32_t* __restrict__ pos, int pos0, int rows,
                                                                   int q_heads, int k_heads, RopeDen den, float eps) {
    const int lane = threadIdx.x & 63;
    const int hpr = q_heads + k_heads;
    const int gpt = (hpr + HPW - 1) / HPW;  // head groups per token
    const int wave = static_cast<int>(blockIdx.x) * (kGroupBlock / kWave) + wave_in_block();
    if (wave >= rows * gpt) return;  // wave-uniform (the host checks rows * gpt < 2^31)
    const int t = wave / gpt;
    const int h0 = (wave - t * gpt) * HPW;
    // Issue order: the position (a scalar load) and the denominator, then the
    // rows and weights, then the angle math, which waits only for the first two.
    // No load sits behind a branch, so the scalar argument loads are not
    // serialised behind waits.
    const float fp = static_cast<float>(POS ? pos[t] : pos0 + t);
    const float dn0 = rope256_den(den, lane);
    float4 v[HPW];
    float* ptr[HPW];
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
        const int h = min(h0 + j, hpr - 1);  // clamped: loads never branch
        ptr[j] = (h < q_heads) ? q + (static_cast<size_t>(t) * q_heads + h) * 256
                               : k + (static_cast<size_t>(t) * k_heads + (h - q_heads)) * 256;
        v[j] = ld4_nt(ptr[j] + 4 * lane);
    }
    float4 wq = make_float4(1.f, 1.f, 1.f, 1.f), wk = wq;
    if constexpr (NORM) {
        // a tensor with no heads may come without weights: read the other's
        wq = ld4((q_heads > 0 ? qw : kw) + 4 * lane);
        wk = ld4((k_heads > 0 ? kw : qw) + 4 * lane);
    }
    const Rope256 rp = rope256_angles(fp, dn0);
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
        const int h = h0 + j;
        const float4 wv = (min(h, hpr - 1) < q_heads) ? wq : wk;
        const float4 o = norm_rope256<NORM>(v[j], wv, rp, eps, lane);
        if (h < hpr) st4_nt(ptr[j] + 4 * lane, o);  // wave-uniform
    }
}

// ------------------------------------------------------------ generic kernels
// Any head_dim / alignment: one block per head, in place.
__global__ __launch_bounds__(kBlock) void head_norm_any(float* __restrict__ x, const float* __restrict__ w, int dim,
                                                        float eps) {
    __shared__ float lds[kBlock / kWave];
    float* p = x + static_cast<size_t>(blockIdx.x) * dim;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kBlock) ss += p[i] * p[i];
    ss = group_sum<kWave>(ss);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    const float r = rsqrtf(ss / static_cast<float>(dim) + eps);
    for (int i = threadIdx.x; i < dim; i += kBlock) p[i] = p[i] * (r * w[i]);
}

// Pairs [lo, lo + count) of every head; one block per (row, head).
__global__ __launch_bounds__(kMaxDen) void rope_any(float* __restrict__ x, const int32_t* __restrict__ pos, int pos0,
                                                    int heads, int head_dim, int rope_dim, RopeDen den, int lo,
                                                    int count) {
    const int i = threadIdx.x;
    if (i >= count) return;
    const int t = blockIdx.x / heads;
    const int pp = pos ? pos[t] : pos0 + t;
    float* p = x + static_cast<size_t>(blockIdx.x) * head_dim;
    const int half = rope_dim >> 1;
    float s, c;
    sincosf(static_cast<float>(pp) / den.den[i], &s, &c);
    const float a = p[lo + i];
    const float b = p[lo + i + half];
    p[lo + i] = a * c - b * s;
    p[lo + i + half] = b * c + a * s;
}

// -------------------------------------------------------------- launcher
template <bool NORM, bool ROPE>
void launch_vec(int lph, float* q, float* k, const float* qw, const float* kw, const int32_t* pos, int pos0, int rows,
                int qh, int kh, int rope_dim, const RopeDen& den, float eps, hipStream_t s) {
    const int64_t heads = static_cast<int64_t>(rows) * (qh + kh);
    const int hpw = kWave / lph;
    const int64_t waves = (heads + hpw - 1) / hpw;
    const dim3 grid(blocks_for(waves, kBlock / kWave)), block(kBlock);
    if (lph == 64 && ROPE && rope_dim == 64) {
        const int64_t gwaves = static_cast<int64_t>(rows) * ((qh + kh + kGroupHeads - 1) / kGroupHeads);
        const unsigned ggrid = blocks_for(gwaves, kGroupBlock / kWave);
        if (pos)
            qk_norm_rope_grouped<kGroupHeads, NORM, true><<<ggrid, kGroupBlock, 0, s>>>(q, k, qw, kw, pos, pos0, rows,
                                                                                       qh, kh, den, eps);
        else
            qk_norm_rope_grouped<kGroupHeads, NORM, false><<<ggrid, kGroupBlock, 0, s>>>(q, k, qw, kw, pos, pos0, rows,
                                                                                        qh, kh, den, eps);
    } else if (lph == 64)
        qk_norm_rope_v4<64, NORM, ROPE><<<grid, block, 0, s>>>(q, k, qw, kw, pos, pos0, rows, qh, kh, rope_dim,
                                                                     den, eps);
    else if (lph == 32)
        qk_norm_rope_v4<32, NORM, ROPE><<<grid, block, 0, s>>>(q, k, qw, kw, pos, pos0, rows, qh, kh, rope_dim,
                                                                     den, eps);
    else
        qk_norm_rope_v4<16, NORM, ROPE><<<grid, block, 0, s>>>(q, k, qw, kw, pos, pos0, rows, qh, kh, rope_dim,
                                                                     den, eps);
}

// Common path of the three entry points. Pointers of a tensor with 0 heads are
// ignored.
int qk_norm_rope(float* q, float* k, const float* qw, const float* kw, const int32_t* pos, int pos0, int rows, int qh,
                 int kh, int head_dim, int rope_dim, float theta, float eps, bool norm, hipStream_t s,
                 const char* what) {
    const bool rope = rope_dim > 0;
    const int lph = head_dim / 4;
    bool vec = head_dim % 4 == 0 && (lph == 16 || lph == 32 || lph == 64) && (!rope || rope_dim % 8 == 0);
    if (qh > 0) vec = vec && aligned16(q) && (!norm || aligned16(qw));
    if (kh > 0) vec = vec && aligned16(k) && (!norm || aligned16(kw));
    if (vec) {
        const RopeDen den = rope ? make_den(0, rope_dim / 2, rope_dim, theta) : RopeDen{};
        if (norm && rope)
            launch_vec<true, true>(lph, q, k, qw, kw, pos, pos0, rows, qh, kh, rope_dim, den, eps, s);
        else if (norm)
            launch_vec<true, false>(lph, q, k, qw, kw, pos, pos0, rows, qh, kh, rope_dim, den, eps, s);
        else
            launch_vec<false, true>(lph, q, k, qw, kw, pos, pos0, rows, qh, kh, rope_dim, den, eps, s);
        return check_launch(what);
    }
    // Generic path: norm pass, then the rotation in chunks of kMaxDen pairs.
    if (norm) {
        if (qh > 0) head_norm_any<<<static_cast<unsigned>(rows) * qh, kBlock, 0, s>>>(q, qw, head_dim, eps);
        if (kh > 0) head_norm_any<<<static_cast<unsigned>(rows) * kh, kBlock, 0, s>>>(k, kw, head_dim, eps);
    }
    if (rope) {
        const int half = rope_dim / 2;
        for (int lo = 0; lo < half; lo += kMaxDen) {
            const int count = std::min(kMaxDen, half - lo);
            const RopeDen den = make_den(lo, count, rope_dim, theta);
            if (qh > 0)
                rope_any<<<static_cast<unsigned>(rows) * qh, kMaxDen, 0, s>>>(q, pos, pos0, qh, head_dim, rope_dim,
                                                                            den, lo, count);
            if (kh > 0)
                rope_any<<<static_cast<unsigned>(rows) * kh, kMaxDen, 0, s>>>(k, pos, pos0, kh, head_dim, rope_dim,
                                                                            den, lo, count);
        }
    }
    return check_launch(what);
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_attn_head_norm(float* x, const float* weight, int heads, int dim, float eps, void* stream) {
    QK_REQUIRE(heads >= 0 && dim >= 0, "attn_head_norm: negative size (heads=%d, dim=%d)", heads, dim);
    if (heads == 0 || dim == 0) return ok();
    QK_REQUIRE(x && weight, "attn_head_norm: null pointer");
    return qk_norm_rope(x, nullptr, weight, nullptr, nullptr, 0, 1, heads, 0, dim, 0, 1.0f, eps, true,
                        as_stream(stream), "attn_head_norm");
}

// Validation mirrors src/cuda/rope.cu:33-43.
int qwen_rope_forward(float* x, int pos, int heads, int head_dim, int rope_dim, float theta, void* stream) {
    if (!x || pos < 0 || heads <= 0 || head_dim <= 0 || rope_dim <= 0 || rope_dim > head_dim || (rope_dim & 1) ||
        (rope_dim / 2 > 1024) || !(theta > 0.0f)) {
        return fail(QWEN_STATUS_INVALID_ARGUMENT, "invalid RoPE arguments");
    }
    return qk_norm_rope(x, nullptr, nullptr, nullptr, nullptr, pos, 1, heads, 0, head_dim, rope_dim, theta, 0.f, false,
                        as_stream(stream), "rope_forward");
}

int qwen_attn_qk_norm_rope_rows(float* q, float* k, const float* q_weight, const float* k_weight, const int32_t* pos,
                                int pos0, int rows, int q_heads, int k_heads, int head_dim, int rope_dim, float theta,
                                float eps, void* stream) {
    QK_REQUIRE(rows >= 0 && q_heads >= 0 && k_heads >= 0, "attn_qk_norm_rope: negative size");
    QK_REQUIRE(head_dim > 0, "attn_qk_norm_rope: head_dim %d must be positive", head_dim);
    QK_REQUIRE(rope_dim >= 0 && rope_dim <= head_dim && (rope_dim & 1) == 0 && rope_dim / 2 <= 1024,
               "attn_qk_norm_rope: rope_dim %d invalid for head_dim %d", rope_dim, head_dim);
    QK_REQUIRE(rope_dim == 0 || theta > 0.0f, "attn_qk_norm_rope: theta must be positive");
    QK_REQUIRE(pos != nullptr || pos0 >= 0, "attn_qk_norm_rope: negative pos0 %d", pos0);
    QK_REQUIRE(static_cast<int64_t>(rows) * (static_cast<int64_t>(q_heads) + k_heads) < (int64_t{1} << 31),
               "attn_qk_norm_rope: rows x heads exceeds 2^31");
    if (rows == 0 || q_heads + k_heads == 0) return ok();
    QK_REQUIRE(q_heads == 0 || (q && q_weight), "attn_qk_norm_rope: null q or q_weight");
    QK_REQUIRE(k_heads == 0 || (k && k_weight), "attn_qk_norm_rope: null k or k_weight");
    return qk_norm_rope(q, k, q_weight, k_weight, pos, pos0, rows, q_heads, k_heads, head_dim, rope_dim, theta, eps,
                        true, as_stream(stream), "attn_qk_norm_rope");
}

}  // extern "C"
