// GGML block formats shared by the dequant-gather and the quantized GEMV:
// type codes, block sizes and the per-element decode of the 9 supported types.
//
// Reference: include/quantized.hpp:12-105 (GgmlType, block sizes),
// src/cuda/matmul_q4.cu:13-26 (fp16_at, scale_min_k4) and :30-129 (dequant).
#pragma once

#include <cstdint>

#include "device_common.hpp"

namespace qk {
namespace {

enum : int {
    kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kBF16 = 30
};

inline bool type_supported(int t) {
    return t == kF32 || t == kF16 || t == kBF16 || t == kQ4_0 || t == kQ5_0 || t == kQ8_0 || t == kQ4_K ||
           t == kQ5_K || t == kQ6_K;
}

// Bytes per block (include/quantized.hpp:72-95).
inline int block_bytes(int t) {
    switch (t) {
        case kF32: return 4;
        case kF16: case kBF16: return 2;
        case kQ4_0: return 18;
        case kQ5_0: return 22;
        case kQ8_0: return 34;
        case kQ4_K: return 144;
        case kQ5_K: return 176;
        case kQ6_K: return 210;
        default: return 0;
    }
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ float fp16_at(const uint8_t* p) { return half_bits(p[0] | (p[1] << 8)); }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// Byte i (0..11) of three packed words.
__device__ __forceinline__ uint32_t byte12(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = (i < 4) ? s0 : (i < 8) ? s1 : s2;
    return byte_of(w, i & 3);
}

// -------------------------------------------------------------- generic decode
// One element of a GGML tensor; the formulas of src/cuda/matmul_q4.cu:30-129.
__device__ inline float dequant_elem(const uint8_t* __restrict__ data, int type, uint64_t index) {
    switch (type) {
        case kF32: return reinterpret_cast<const float*>(data)[index];
        case kF16: return half_bits(reinterpret_cast<const uint16_t*>(data)[index]);
        case kBF16: return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(data)[index]) << 16);
        case kQ8_0: {
            const uint8_t* b = data + (index / 32) * 34;
            return fp16_at(b) * static_cast<float>(static_cast<int8_t>(b[2 + index % 32]));
        }
        case kQ4_0: {
            const uint8_t* b = data + (index / 32) * 18;
            const int i = static_cast<int>(index % 32);
            const int q = (i < 16) ? (b[2 + i] & 15) : (b[2 + i - 16] >> 4);
            return fp16_at(b) * static_cast<float>(q - 8);
        }
        case kQ5_0: {
            const uint8_t* b = data + (index / 32) * 22;
            const int i = static_cast<int>(index % 32);
            const uint32_t qh = b[2] | (b[3] << 8) | (b[4] << 16) | (static_cast<uint32_t>(b[5]) << 24);
            const int j = i & 15;
            const int high = (i < 16) ? ((qh >> j) & 1) : ((qh >> (j + 16)) & 1);
            const int low = (i < 16) ? (b[6 + j] & 15) : (b[6 + j] >> 4);
            return fp16_at(b) * static_cast<float>((low | (high << 4)) - 16);
        }
        case kQ4_K:
        case kQ5_K: {
            const uint8_t* b = data + (index / 256) * (type == kQ4_K ? 144 : 176);
            const int i = static_cast<int>(index % 256);
            const float d = fp16_at(b);
            const float dmin = fp16_at(b + 2);
            const uint8_t* s = b + 4;
            const int j = i / 32;
            int sc, mn;
            if (j < 4) {
                sc = s[j] & 63;
                mn = s[j + 4] & 63;
            } else {
                sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
                mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
            }
            const int g = i / 64, in64 = i % 64, l = in64 & 31;
            int v;
            if (type == kQ4_K) {
                const uint8_t q = b[16 + g * 32 + l];
                v = (in64 < 32) ? (q & 15) : (q >> 4);
            } else {
                const uint8_t q = b[48 + g * 32 + l];
                const uint8_t mask = static_cast<uint8_t>(1u << (2 * g + (in64 >= 32)));
                v = ((in64 < 32) ? (q & 15) : (q >> 4)) + ((b[16 + l] & mask) ? 16 : 0);
            }
            return d * static_cast<float>(sc) * static_cast<float>(v) - dmin * static_cast<float>(mn);
        }
        case kQ6_K: {
            const uint8_t* b = data + (index / 256) * 210;
            const int i = static_cast<int>(index % 256);
            const int half = i / 128, r = i % 128, l = r & 31, quarter = r / 32;
            const uint8_t qlb = b[half * 64 + (quarter & 1) * 32 + l];
            const int lo = (quarter < 2) ? (qlb & 15) : (qlb >> 4);
            const int hi = (b[128 + half * 32 + l] >> (2 * quarter)) & 3;
            const int8_t sc = static_cast<int8_t>(b[192 + half * 8 + l / 16 + 2 * quarter]);
            return fp16_at(b + 208) * static_cast<float>(sc) * static_cast<float>((lo | (hi << 4)) - 32);
        }
        default: return 0.0f;
    }
}

// Unsigned 32-bit little-endian word at a 2-byte aligned LDS address.
__device__ __forceinline__ uint32_t lds_u32_a2(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
}

}  // namespace
}  // namespace qk
