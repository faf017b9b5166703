// Measurement reference for bench.py and the traffic calibration: a plain
// 16-byte-vector device copy with the same streaming pattern as the fused
// kernels (8 vectors in flight per thread, nontemporal loads and stores, an
// unconditional path for every block but the last). It is the practical HBM
// ceiling the fused kernels are compared with, and the kernel whose
// FETCH_SIZE / WRITE_SIZE counters calibrate bytes per counter unit. Built
// into libqwen35_benchutil.so, not into the kernel library.
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

}  // namespace

extern "C" {

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
