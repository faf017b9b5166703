// MoE expert activations on gfx950: SwiGLU h = silu(g) * u (fp32 and bf16
// storage), the sigmoid-gated shared expert, and the shared-expert accumulate.
//
// Reference semantics: silu_mul_kernel (src/cuda/moe.cu:61-67) and shared_kernel
// (src/cuda/moe.cu:90-96, out += x * sigmoid(gate[0])). The reference runs one
// launch per expert per token with 4-byte accesses; here a launch covers every
// token and expert (and, in swiglu_routed_shared, the shared expert as well),
// each thread moves 16-byte vectors and keeps U vectors in flight, and the bf16
// forms do the math in fp32 with one round-to-nearest-even at the store.
#include <algorithm>

#include "capi_common.hpp"
#include "device_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;
// 16-byte chunks of each input in flight per thread: best of 1/2/4/8 at C3b's
// 100 MB, and at C3c's 12.6 MB (4.0 us, against 4.2 us with one).
constexpr int kUnroll = 2;

// ------------------------------------------------------------ bf16 SwiGLU
// Eight bf16 pairs (one 16-byte chunk of g and of u) -> eight bf16 outputs,
// h = (silu(g) * u) [* scale], fp32 math, one rounding per output.
template <bool SCALED>
__device__ __forceinline__ uint4 swiglu8(uint4 g, uint4 u, float scale) {
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
    float s[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        s[2 * k] = bf16_lo(gw[k]);
        s[2 * k + 1] = bf16_hi(gw[k]);
    }
    silu_n<8>(s);
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float lo = s[2 * k] * bf16_lo(uw[k]);
        float hi = s[2 * k + 1] * bf16_hi(uw[k]);
        if (SCALED) {
            lo *= scale;
            hi *= scale;
        }
        o[k] = pack_bf16(lo, hi);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// Chunk i = 8 bf16 (16 bytes). Block b covers chunks b*kUnroll*kBlock + k*kBlock
// + threadIdx.x, k < kUnroll, so each load instruction of a wave reads 1 KB of
// contiguous memory. Every block but the last takes the unconditional path: all
// 2*kUnroll streaming loads are issued before any math. SCALED: the shared
// expert's rows x dim layout with one logit per row (dim % 8 == 0, so a chunk
// never straddles two rows).
template <int U, bool SCALED>
__device__ __forceinline__ void swiglu_block(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                             const float* __restrict__ logits, uint16_t* __restrict__ h, int64_t n8,
                                             int dim8, unsigned block) {
    const int64_t first = static_cast<int64_t>(block) * U * kBlock + threadIdx.x;
    uint4 gv[U], uv[U];
    float sc[U];
    if (static_cast<int64_t>(block + 1) * U * kBlock <= n8) {  // block-uniform
#pragma unroll
        for (int k = 0; k < U; ++k) {
            if (SCALED) sc[k] = logits[static_cast<int>(first + k * kBlock) / dim8];  // n8 < 2^31 (host check)
            gv[k] = ld16_nt(g + 8 * (first + k * kBlock));
            uv[k] = ld16_nt(u + 8 * (first + k * kBlock));
        }
        // Every load is issued before any math: without this fence the
        // scheduler hoists the first sigmoid above the later loads, and each
        // output then waits for two memory round trips instead of one.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < U; ++k)
            st16_nt(h + 8 * (first + k * kBlock), swiglu8<SCALED>(gv[k], uv[k], SCALED ? sigmoid(sc[k]) : 1.0f));
    } else {
        for (int k = 0; k < U; ++k) {
            const int64_t i = first + k * kBlock;
            if (i < n8)
                st16_nt(h + 8 * i, swiglu8<SCALED>(ld16_nt(g + 8 * i), ld16_nt(u + 8 * i),
                                                   SCALED ? sigmoid(logits[i / dim8]) : 1.0f));
        }
    }
}

template <int U, bool SCALED>
__global__ __launch_bounds__(kBlock) void swiglu_bf16_v8(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                         const float* __restrict__ logits, uint16_t* __restrict__ h,
                                                         int64_t n8, int dim8) {
    swiglu_block<U, SCALED>(g, u, logits, h, n8, dim8, blockIdx.x);
}

// One part of the routed + shared launch: n8 chunks of 8 bf16 from `blocks`
// workgroups.
struct SwigluPart {
    const uint16_t* g;
    const uint16_t* u;
    const float* logits;   // shared part only
    uint16_t* h;
    int64_t n8;
    int dim8;
    unsigned blocks;
};

// The MoE layer's two SwiGLUs in one grid: workgroups [0, routed.blocks) take
// the routed experts' rows, the rest the shared expert's rows with their
// sigmoid gate. Each workgroup runs exactly the code of the separate launches,
// so the outputs equal them bit for bit; one launch drains once where two
// would each pay their own ramp and tail.
__global__ __launch_bounds__(kBlock) void swiglu_routed_shared_v8(const SwigluPart routed, const SwigluPart shared) {
    if (blockIdx.x < routed.blocks)  // block-uniform
        swiglu_block<kUnroll, false>(routed.g, routed.u, nullptr, routed.h, routed.n8, 1, blockIdx.x);
    else
        swiglu_block<kUnroll, true>(shared.g, shared.u, shared.logits, shared.h, shared.n8, shared.dim8,
                                    blockIdx.x - routed.blocks);
}

__device__ __forceinline__ float bf16_at(const uint16_t* p) { return __uint_as_float(static_cast<uint32_t>(*p) << 16); }

__global__ __launch_bounds__(kBlock) void swiglu_bf16_any(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                          const float* __restrict__ logits, uint16_t* __restrict__ h,
                                                          int64_t n, int dim) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        float v = silu(bf16_at(g + i)) * bf16_at(u + i);
        if (logits) v *= sigmoid(logits[i / dim]);
        h[i] = static_cast<uint16_t>(pack_bf16(v, 0.f) & 0xffffu);
    }
}

// ------------------------------------------------------------ fp32 forms
__global__ __launch_bounds__(kBlock) void silu_mul_v4(const float* __restrict__ g, const float* __restrict__ u,
                                                      float* __restrict__ h, int64_t n4) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n4;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        const float4 a = ld4_nt(g + 4 * i);
        const float4 b = ld4_nt(u + 4 * i);
        const float4 s = silu4(a);
        st4_nt(h + 4 * i, make_float4(s.x * b.x, s.y * b.y, s.z * b.z, s.w * b.w));
    }
}

__global__ __launch_bounds__(kBlock) void silu_mul_any(const float* __restrict__ g, const float* __restrict__ u,
                                                       float* __restrict__ h, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        h[i] = silu(g[i]) * u[i];
}

// accum[t, i] += x[t, i] * sigmoid(gate[t]); one block row-strip per row.
__global__ __launch_bounds__(kBlock) void shared_add_rows(float* __restrict__ accum, const float* __restrict__ x,
                                                          const float* __restrict__ gate, int dim) {
    const float sc = sigmoid(gate[blockIdx.y]);
    const size_t base = static_cast<size_t>(blockIdx.y) * dim;
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < dim; i += gridDim.x * kBlock)
        accum[base + i] += x[base + i] * sc;
}

unsigned stride_grid(int64_t items) { return static_cast<unsigned>(std::min<int64_t>(blocks_for(items, kBlock), 8192)); }

// The 16-byte-vector kernels apply: whole chunks (and whole chunks per row when
// a logit scales each row), 16-byte aligned pointers, chunk indices in int32.
bool swiglu_vec_ok(const uint16_t* g, const uint16_t* u, const float* logits, const uint16_t* h, int64_t n, int dim) {
    return n % 8 == 0 && n / 8 < (int64_t{1} << 31) && (!logits || dim % 8 == 0) && aligned16(g) && aligned16(u) &&
           aligned16(h);
}

int swiglu_common(const uint16_t* g, const uint16_t* u, const float* logits, uint16_t* h, int64_t n, int dim,
                  hipStream_t s, const char* what) {
    if (swiglu_vec_ok(g, u, logits, h, n, dim)) {
        const int64_t n8 = n / 8;
        const unsigned grid = blocks_for(n8, static_cast<int64_t>(kUnroll) * kBlock);
        if (logits)
            swiglu_bf16_v8<kUnroll, true><<<grid, kBlock, 0, s>>>(g, u, logits, h, n8, dim / 8);
        else
            swiglu_bf16_v8<kUnroll, false><<<grid, kBlock, 0, s>>>(g, u, nullptr, h, n8, 1);
    } else {
        swiglu_bf16_any<<<stride_grid(n), kBlock, 0, s>>>(g, u, logits, h, n, dim);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n, void* stream) {
    QK_REQUIRE(n >= 0, "swiglu_bf16: negative size");
    if (n == 0) return ok();
    QK_REQUIRE(gate && up && hidden, "swiglu_bf16: null pointer");
    return swiglu_common(gate, up, nullptr, hidden, n, 1, as_stream(stream), "swiglu_bf16");
}

int qwen_shared_swiglu_sigmoid_rows_bf16(const uint16_t* gate, const uint16_t* up, const float* logits,
                                         uint16_t* hidden, int rows, int dim, void* stream) {
    QK_REQUIRE(rows >= 0 && dim >= 0, "shared_swiglu_sigmoid: negative size");
    if (rows == 0 || dim == 0) return ok();
    QK_REQUIRE(gate && up && logits && hidden, "shared_swiglu_sigmoid: null pointer");
    return swiglu_common(gate, up, logits, hidden, static_cast<int64_t>(rows) * dim, dim, as_stream(stream),
                         "shared_swiglu_sigmoid");
}

int qwen_swiglu_routed_shared_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* hidden, int64_t n,
                                   const uint16_t* shared_gate, const uint16_t* shared_up, const float* logits,
                                   uint16_t* shared_hidden, int rows, int dim, void* stream) {
    QK_REQUIRE(n >= 0 && rows >= 0 && dim >= 0, "swiglu_routed_shared: negative size");
    const int64_t ns = static_cast<int64_t>(rows) * dim;
    QK_REQUIRE(n == 0 || (gate && up && hidden), "swiglu_routed_shared: null routed pointer");
    QK_REQUIRE(ns == 0 || (shared_gate && shared_up && logits && shared_hidden),
               "swiglu_routed_shared: null shared pointer");
    const hipStream_t s = as_stream(stream);
    if (n > 0 && ns > 0 && swiglu_vec_ok(gate, up, nullptr, hidden, n, 1) &&
        swiglu_vec_ok(shared_gate, shared_up, logits, shared_hidden, ns, dim)) {
        const int64_t per = static_cast<int64_t>(kUnroll) * kBlock;
        const SwigluPart r{gate, up, nullptr, hidden, n / 8, 1, blocks_for(n / 8, per)};
        const SwigluPart sh{shared_gate, shared_up, logits, shared_hidden, ns / 8, dim / 8, blocks_for(ns / 8, per)};
        QK_REQUIRE(static_cast<uint64_t>(r.blocks) + sh.blocks <= 0x7fffffffu,
                   "swiglu_routed_shared: %lld + %lld elements exceed one launch", static_cast<long long>(n),
                   static_cast<long long>(ns));
        swiglu_routed_shared_v8<<<r.blocks + sh.blocks, kBlock, 0, s>>>(r, sh);
        return check_launch("swiglu_routed_shared");
    }
    // shapes or pointers outside the vector kernel: the two separate launches
    if (n > 0)
        if (const int rc = swiglu_common(gate, up, nullptr, hidden, n, 1, s, "swiglu_routed_shared")) return rc;
    if (ns > 0) return swiglu_common(shared_gate, shared_up, logits, shared_hidden, ns, dim, s, "swiglu_routed_shared");
    return ok();
}

int qwen_moe_silu_mul(const float* gate, const float* up, float* hidden, int n, void* stream) {
    QK_REQUIRE(n >= 0, "moe_silu_mul: negative size");
    if (n == 0) return ok();
    QK_REQUIRE(gate && up && hidden, "moe_silu_mul: null pointer");
    hipStream_t s = as_stream(stream);
    if (n % 4 == 0 && aligned16(gate) && aligned16(up) && aligned16(hidden))
        silu_mul_v4<<<stride_grid(n / 4), kBlock, 0, s>>>(gate, up, hidden, n / 4);
    else
        silu_mul_any<<<stride_grid(n), kBlock, 0, s>>>(gate, up, hidden, n);
    return check_launch("moe_silu_mul");
}

int qwen_moe_shared_add_rows(float* accum, const float* shared_out, const float* gate, int rows, int n, void* stream) {
    QK_REQUIRE(rows >= 0 && n >= 0, "moe_shared_add: negative size");
    if (rows == 0 || n == 0) return ok();
    QK_REQUIRE(accum && shared_out && gate, "moe_shared_add: null pointer");
    QK_REQUIRE(rows <= 65535, "moe_shared_add: %d rows exceed one launch (65535)", rows);
    const dim3 grid(std::min<unsigned>(blocks_for(n, kBlock), 64u), static_cast<unsigned>(rows));
    shared_add_rows<<<grid, kBlock, 0, as_stream(stream)>>>(accum, shared_out, gate, n);
    return check_launch("moe_shared_add");
}

int qwen_moe_shared_add(float* accum, const float* shared_out, const float* gate, int n, void* stream) {
    return qwen_moe_shared_add_rows(accum, shared_out, gate, 1, n, stream);
}

}  // extern "C"
