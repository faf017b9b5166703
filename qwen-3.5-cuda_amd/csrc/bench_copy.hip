// Measurement reference for bench.py and the traffic calibration: a plain
// 16-byte-vector device copy with the same streaming pattern as the fused
// kernels (8 vectors in flight per thread, nontemporal loads and stores, an
// unconditional path for every block but the last). It is the practical HBM
// ceiling the fused kernels are compared with, and the kernel whose
// FETCH_SIZE / WRITE_SIZE counters calibrate bytes per counter unit; and the
// copy forms of the small-size sweep (qwen_bench_copy_form). Built into
// libqwen35_benchutil.so, not into the kernel library.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 8;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kBlock) void copy16(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                 int64_t n) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * kUnroll * kBlock + threadIdx.x;
    if (static_cast<int64_t>(blockIdx.x + 1) * kUnroll * kBlock <= n) {
        u32x4_t v[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) v[k] = __builtin_nontemporal_load(src + first + k * kBlock);
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) __builtin_nontemporal_store(v[k], dst + first + k * kBlock);
    } else {
        for (int k = 0; k < kUnroll; ++k) {
            const int64_t i = first + k * kBlock;
            if (i < n) dst[i] = src[i];
        }
    }
}

// Copy forms for the small-size sweep (bench.py --copy-sweep): block b copies
// super-chunks b, b + gridDim.x, ... of U x blockDim.x vectors, so a grid of
// ceil(n / (U * blockDim.x)) blocks is the one-shot form and a smaller grid the
// persistent (grid-stride) form. NT: nontemporal loads and stores.
// (No __restrict__: the in-place form passes src == dst.)
template <int U, bool NT>
__global__ __launch_bounds__(1024) void copy_form(const u32x4_t* src, u32x4_t* dst, int64_t n) {
    const int64_t per = static_cast<int64_t>(U) * blockDim.x;
    for (int64_t sc = blockIdx.x; sc * per < n; sc += gridDim.x) {
        const int64_t first = sc * per + threadIdx.x;
        if ((sc + 1) * per <= n) {
            u32x4_t v[U];
#pragma unroll
            for (int k = 0; k < U; ++k)
                v[k] = NT ? __builtin_nontemporal_load(src + first + k * blockDim.x) : src[first + k * blockDim.x];
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (NT)
                    __builtin_nontemporal_store(v[k], dst + first + k * blockDim.x);
                else
                    dst[first + k * blockDim.x] = v[k];
            }
        } else {
            for (int k = 0; k < U; ++k) {
                const int64_t i = first + k * blockDim.x;
                if (i < n) dst[i] = src[i];
            }
        }
    }
}

template <bool NT>
void launch_form(int unroll, unsigned grid, unsigned block, const u32x4_t* src, u32x4_t* dst, int64_t n,
                 hipStream_t s) {
    switch (unroll) {
        case 1: copy_form<1, NT><<<grid, block, 0, s>>>(src, dst, n); break;
        case 2: copy_form<2, NT><<<grid, block, 0, s>>>(src, dst, n); break;
        case 4: copy_form<4, NT><<<grid, block, 0, s>>>(src, dst, n); break;
        case 8: copy_form<8, NT><<<grid, block, 0, s>>>(src, dst, n); break;
        default: copy_form<16, NT><<<grid, block, 0, s>>>(src, dst, n); break;
    }
}

}  // namespace

extern "C" {

// A copy form of the sweep: `unroll` vectors of 16 bytes per thread per
// super-chunk (1, 2, 4, 8 or 16), `block` threads per workgroup (a multiple of
// 64, at most 1024), `grid_cap` workgroups at most (0: one-shot grid), `nt`
// nontemporal accesses. src == dst copies in place (read and write the same
// lines, as an in-place kernel does). Returns 0, or 1 on a bad argument /
// launch error.
int qwen_bench_copy_form(const void* src, void* dst, int64_t bytes, int unroll, int block, int grid_cap, int nt,
                         void* stream) {
    if (!src || !dst || bytes < 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15) ||
        (reinterpret_cast<uintptr_t>(dst) & 15) || block <= 0 || block > 1024 || block % 64 || grid_cap < 0 ||
        (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16))
        return 1;
    const int64_t n = bytes / 16;
    if (n == 0) return 0;
    const int64_t per = static_cast<int64_t>(unroll) * block;
    int64_t grid = (n + per - 1) / per;
    if (grid_cap > 0 && grid > grid_cap) grid = grid_cap;
    if (grid > 0x7fffffff) return 1;
    const auto s = reinterpret_cast<hipStream_t>(stream);
    const auto* in = static_cast<const u32x4_t*>(src);
    auto* out = static_cast<u32x4_t*>(dst);
    if (nt)
        launch_form<true>(unroll, static_cast<unsigned>(grid), static_cast<unsigned>(block), in, out, n, s);
    else
        launch_form<false>(unroll, static_cast<unsigned>(grid), static_cast<unsigned>(block), in, out, n, s);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// dst[0:bytes] = src[0:bytes]; bytes must be a multiple of 16 and both
// pointers 16-byte aligned. Returns 0, or 1 on a bad argument / launch error.
int qwen_bench_copy(const void* src, void* dst, int64_t bytes, void* stream) {
    if (!src || !dst || bytes < 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15) ||
        (reinterpret_cast<uintptr_t>(dst) & 15))
        return 1;
    const int64_t n = bytes / 16;
    if (n == 0) return 0;
    const unsigned grid = static_cast<unsigned>((n + kUnroll * kBlock - 1) / (kUnroll * kBlock));
    copy16<<<grid, kBlock, 0, reinterpret_cast<hipStream_t>(stream)>>>(static_cast<const u32x4_t*>(src),
                                                                       static_cast<u32x4_t*>(dst), n);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
