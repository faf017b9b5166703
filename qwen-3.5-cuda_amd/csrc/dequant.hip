// GGML dequant-gather on gfx950 (token-embedding lookup of a quantized table).
//
// Reference semantics: dequant() in src/cuda/matmul_q4.cu:30-129 (per-element
// decode of 9 GGML types, fp16_at :13-16, scale_min_k4 :18-26), row_kernel
// :169-173 and dequantize_row :209-227 (element index = row * cols + i), called
// once per token at src/model.cpp:190. The reference decodes every element
// independently, re-reading the block header and re-unpacking the 6-bit scales
// for each of the 256 elements, with byte loads.
//
// Fast paths (Q4_K, Q6_K, rows of whole 256-element blocks): one wave per id.
// The wave copies the id's quantized row into LDS with 16-byte loads (1152 B
// for a Q4_K row of 2048, 1680 B for Q6_K -- whole-row coalesced reads), then
// lane L decodes elements 4L..4L+3 of every block and writes them as one
// float4, so each store instruction of the wave writes 1 KB of contiguous
// output. Every product in these formats is exact in fp32 (fp16 has 11
// significant bits, sub-scales 6-8, quants 4-6), so the result is bit-identical
// to the reference formula; the float association (d * sc) * q is kept because
// it fixes the sign of zero.
#include <algorithm>

#include "capi_common.hpp"
#include "device_common.hpp"
#include "ggml_common.hpp"

namespace qk {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxStageBytes = 16384;  // LDS staging per wave (fast paths)

// out[t*cols + i] = element (id_t * cols + i); ids NULL means id_t = fixed_row.
__global__ __launch_bounds__(kBlock) void gather_any(const uint8_t* __restrict__ data, int type,
                                                     const int32_t* __restrict__ ids, int fixed_row, int n_ids,
                                                     int64_t vocab_rows, int cols, float* __restrict__ out) {
    const int64_t n = static_cast<int64_t>(n_ids) * cols;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < n;
         e += static_cast<int64_t>(gridDim.x) * kBlock) {
        const int64_t t = e / cols;
        const int i = static_cast<int>(e - t * cols);
        const int64_t id = ids ? ids[t] : fixed_row;
        out[e] = (id >= 0 && id < vocab_rows)
                     ? dequant_elem(data, type, static_cast<uint64_t>(id) * cols + i)
                     : __builtin_nanf("");
    }
}

// -------------------------------------------------------------- fast paths
// Copies the quantized row of `id` into this wave's LDS slot; returns the byte
// offset of the row inside the slot (the copy starts at a 16-byte boundary).
__device__ __forceinline__ int stage_row(const uint8_t* __restrict__ table, int64_t id, int row_bytes, uint4* slot,
                                         int lane) {
    const uint64_t start = static_cast<uint64_t>(id) * row_bytes;
    const uint64_t a = start & ~static_cast<uint64_t>(15);
    const int off = static_cast<int>(start - a);
    const int chunks = (off + row_bytes + 15) >> 4;
    const uint4* src = reinterpret_cast<const uint4*>(table + a);
    for (int j = lane; j < chunks; j += kWave) slot[j] = ld16_nt(src + j);
    return off;
}

__device__ __forceinline__ void fill_nan(float* orow, int nb, int lane) {
    const float q = __builtin_nanf("");
    for (int k = 0; k < nb; ++k) st4_nt(orow + k * 256 + 4 * lane, make_float4(q, q, q, q));
}

// Q4_K: 144-byte blocks = d, dmin (fp16), scales[12], qs[128]. Rows are whole
// blocks, so every block starts 16-byte aligned inside the slot.
__global__ __launch_bounds__(kBlock) void gather_q4k(const uint8_t* __restrict__ table, const int32_t* __restrict__ ids,
                                                     int fixed_row, int n_ids, int64_t vocab_rows, int nb,
                                                     int slot_chunks, float* __restrict__ out) {
    extern __shared__ uint4 stage[];
    const int lane = threadIdx.x & 63;
    const int w = wave_in_block();
    const int t = blockIdx.x * kWavesPerBlock + w;
    const bool live = t < n_ids;  // wave-uniform
    const int64_t id = live ? (ids ? ids[t] : fixed_row) : 0;
    const bool valid = live && id >= 0 && id < vocab_rows;
    uint4* slot = stage + w * slot_chunks;
    if (valid) stage_row(table, id, nb * 144, slot, lane);
    __syncthreads();
    if (!live) return;
    float* orow = out + static_cast<size_t>(t) * nb * 256;
    if (!valid) {
        fill_nan(orow, nb, lane);
        return;
    }
    const uint8_t* row = reinterpret_cast<const uint8_t*>(slot);
    const int sub = lane >> 3;                        // 32-element sub-block of elements 4L..4L+3
    const int qoff = 16 + (lane >> 4) * 32 + 4 * (lane & 7);
    const int shift = (lane & 8) ? 4 : 0;             // high nibble for the second 32 of each 64
    for (int k = 0; k < nb; ++k) {
        const uint8_t* b = row + k * 144;
        const uint4 hdr = *reinterpret_cast<const uint4*>(b);
        const uint32_t qw = *reinterpret_cast<const uint32_t*>(b + qoff);
        const float d = half_bits(hdr.x & 0xffffu);
        const float dmin = half_bits(hdr.x >> 16);
        uint32_t sc, mn;
        if (sub < 4) {
            sc = byte12(hdr.y, hdr.z, hdr.w, sub) & 63;
            mn = byte12(hdr.y, hdr.z, hdr.w, sub + 4) & 63;
        } else {
            const uint32_t hi = byte12(hdr.y, hdr.z, hdr.w, sub + 4);
            sc = (hi & 0x0f) | ((byte12(hdr.y, hdr.z, hdr.w, sub - 4) >> 6) << 4);
            mn = (hi >> 4) | ((byte12(hdr.y, hdr.z, hdr.w, sub) >> 6) << 4);
        }
        const float A = d * static_cast<float>(sc);   // d * sc
        const float B = dmin * static_cast<float>(mn);
        const uint32_t nib = (qw >> shift) & 0x0f0f0f0fu;
        float4 o;
        o.x = A * static_cast<float>(byte_of(nib, 0)) - B;
        o.y = A * static_cast<float>(byte_of(nib, 1)) - B;
        o.z = A * static_cast<float>(byte_of(nib, 2)) - B;
        o.w = A * static_cast<float>(byte_of(nib, 3)) - B;
        st4_nt(orow + k * 256 + 4 * lane, o);
    }
}

// Q6_K: 210-byte blocks = ql[128], qh[64], scales int8[16], d fp16. Blocks sit
// at 2-byte alignment, so the decoder reads LDS in 16-bit pieces.
__global__ __launch_bounds__(kBlock) void gather_q6k(const uint8_t* __restrict__ table, const int32_t* __restrict__ ids,
                                                     int fixed_row, int n_ids, int64_t vocab_rows, int nb,
                                                     int slot_chunks, float* __restrict__ out) {
    extern __shared__ uint4 stage[];
    const int lane = threadIdx.x & 63;
    const int w = wave_in_block();
    const int t = blockIdx.x * kWavesPerBlock + w;
    const bool live = t < n_ids;
    const int64_t id = live ? (ids ? ids[t] : fixed_row) : 0;
    const bool valid = live && id >= 0 && id < vocab_rows;
    uint4* slot = stage + w * slot_chunks;
    int off = 0;
    if (valid) off = stage_row(table, id, nb * 210, slot, lane);
    __syncthreads();
    if (!live) return;
    float* orow = out + static_cast<size_t>(t) * nb * 256;
    if (!valid) {
        fill_nan(orow, nb, lane);
        return;
    }
    const uint8_t* row = reinterpret_cast<const uint8_t*>(slot) + off;
    const int half = lane >> 5;
    const int quarter = (lane >> 3) & 3;
    const int l = 4 * (lane & 7);
    const int ql_off = half * 64 + (quarter & 1) * 32 + l;
    const int qh_off = 128 + half * 32 + l;
    const int sc_off = 192 + half * 8 + (l >> 4) + 2 * quarter;
    const int lo_shift = (quarter >= 2) ? 4 : 0;
    const int hi_shift = 2 * quarter;
    for (int k = 0; k < nb; ++k) {
        const uint8_t* b = row + k * 210;
        const uint32_t ql = (lds_u32_a2(b + ql_off) >> lo_shift) & 0x0f0f0f0fu;
        const uint32_t qh = (lds_u32_a2(b + qh_off) >> hi_shift) & 0x03030303u;
        const uint32_t q = ql | (qh << 4);
        const float d = half_bits(*reinterpret_cast<const uint16_t*>(b + 208));
        const float A = d * static_cast<float>(static_cast<int8_t>(b[sc_off]));  // d * sc
        float4 o;
        o.x = A * static_cast<float>(static_cast<int>(byte_of(q, 0)) - 32);
        o.y = A * static_cast<float>(static_cast<int>(byte_of(q, 1)) - 32);
        o.z = A * static_cast<float>(static_cast<int>(byte_of(q, 2)) - 32);
        o.w = A * static_cast<float>(static_cast<int>(byte_of(q, 3)) - 32);
        st4_nt(orow + k * 256 + 4 * lane, o);
    }
}

// Launch helper shared by the gather and single-row entry points.
int launch_gather(const void* table, int type, uint64_t num_elements, const int32_t* ids, int fixed_row, int n_ids,
                  int cols, float* out, hipStream_t s, const char* what) {
    const uint8_t* data = static_cast<const uint8_t*>(table);
    const int64_t vocab_rows = static_cast<int64_t>(num_elements / static_cast<uint64_t>(cols));
    const bool kquant = type == kQ4_K || type == kQ6_K;
    const int nb = cols / 256;
    const int row_bytes = nb * block_bytes(type);
    // The staging copy reads whole 16-byte chunks, so the rows it can touch
    // must end inside a tensor whose byte size is a multiple of 16.
    const uint64_t tensor_bytes = (num_elements / 256) * static_cast<uint64_t>(block_bytes(type));
    const bool fast = kquant && cols % 256 == 0 && num_elements % 256 == 0 && tensor_bytes % 16 == 0 &&
                      aligned16(table) && aligned16(out) && row_bytes + 32 <= kMaxStageBytes;
    if (fast) {
        const int slot_chunks = (row_bytes + 15) / 16 + 1;
        const size_t lds = static_cast<size_t>(slot_chunks) * 16 * kWavesPerBlock;
        const unsigned grid = blocks_for(n_ids, kWavesPerBlock);
        if (type == kQ4_K)
            gather_q4k<<<grid, kBlock, lds, s>>>(data, ids, fixed_row, n_ids, vocab_rows, nb, slot_chunks, out);
        else
            gather_q6k<<<grid, kBlock, lds, s>>>(data, ids, fixed_row, n_ids, vocab_rows, nb, slot_chunks, out);
    } else {
        const int64_t n = static_cast<int64_t>(n_ids) * cols;
        const unsigned grid = static_cast<unsigned>(std::min<int64_t>(blocks_for(n, kBlock), 8192));
        gather_any<<<grid, kBlock, 0, s>>>(data, type, ids, fixed_row, n_ids, vocab_rows, cols, out);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace qk

using namespace qk;

extern "C" {

int qwen_type_supported(int type) { return type_supported(type) ? 1 : 0; }

// Validation mirrors src/cuda/matmul_q4.cu:210-217.
int qwen_dequantize_row(const void* data, int type, uint64_t num_elements, float* out, int row, int cols,
                        void* stream) {
    if (!data || !type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "cannot dequantize tensor");
    const uint64_t start = static_cast<uint64_t>(static_cast<int64_t>(row)) * static_cast<uint64_t>(cols);
    if (row < 0 || cols <= 0 || start + static_cast<uint64_t>(cols) > num_elements)
        return fail(QWEN_STATUS_OUT_OF_RANGE, "row is outside tensor");
    QK_REQUIRE(out, "dequantize_row: null output");
    // Row `row` of a tensor viewed as rows of `cols` elements: the gather with a
    // single host-side id. (row + 1) * cols <= num_elements, so row is in range.
    return launch_gather(data, type, num_elements, nullptr, row, 1, cols, out, as_stream(stream), "dequantize_row");
}

int qwen_dequant_gather_rows(const void* table, int type, uint64_t num_elements, const int32_t* ids, int n_ids,
                             int cols, float* out, void* stream) {
    if (!table || !type_supported(type)) return fail(QWEN_STATUS_UNSUPPORTED_TYPE, "cannot dequantize tensor");
    QK_REQUIRE(n_ids >= 0 && cols > 0, "dequant_gather: bad n_ids %d / cols %d", n_ids, cols);
    if (n_ids == 0) return ok();
    QK_REQUIRE(ids && out, "dequant_gather: null pointer");
    return launch_gather(table, type, num_elements, ids, 0, n_ids, cols, out, as_stream(stream), "dequant_gather");
}

}  // extern "C"
