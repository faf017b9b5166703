// GGML tensor descriptor and block-size tables.
//
// Interface kept identical to include/quantized.hpp of the reference
// (sahan974/qwen-3.5-cuda, :12-105): the enum values are the GGUF type ids and
// QuantTensor keeps the reference's member order, because the loader fills it and
// dequantize_row() receives it by const reference. The helper functions are
// re-implemented from the GGML block formats.
#ifndef QWEN35_QUANTIZED_HPP
#define QWEN35_QUANTIZED_HPP

#include <cstdint>
#include <limits>
#include <string>
#include <vector>

namespace qwen {

enum class GgmlType : uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 6,
    Q5_1 = 7,
    Q8_0 = 8,
    Q8_1 = 9,
    Q2_K = 10,
    Q3_K = 11,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
    Q8_K = 15,
    IQ2_XXS = 16,
    IQ2_XS = 17,
    IQ3_XXS = 18,
    I8 = 24,
    I16 = 25,
    I32 = 26,
    F64 = 28,
    BF16 = 30,
    COUNT
};

struct QuantTensor {
    std::string name;
    GgmlType type;
    std::vector<int64_t> shape;
    uint64_t num_elements;
    uint64_t size_bytes;
    uint64_t offset;              // offset of the tensor in the GGUF payload
    void* device_ptr = nullptr;   // device memory holding the blocks
};

namespace detail {
struct BlockFormat {
    uint64_t elems;  // elements per block (0 = unknown type)
    uint64_t bytes;  // bytes per block
};

inline BlockFormat block_format(GgmlType type) {
    switch (type) {
        case GgmlType::F32: case GgmlType::I32: return {1, 4};
        case GgmlType::F16: case GgmlType::BF16: case GgmlType::I16: return {1, 2};
        case GgmlType::I8: return {1, 1};
        case GgmlType::Q4_0: return {32, 2 + 16};
        case GgmlType::Q4_1: return {32, 2 + 2 + 16};
        case GgmlType::Q5_0: return {32, 2 + 4 + 16};
        case GgmlType::Q5_1: return {32, 2 + 2 + 4 + 16};
        case GgmlType::Q8_0: return {32, 2 + 32};
        case GgmlType::Q8_1: return {32, 4 + 32};
        case GgmlType::Q2_K: return {256, 16 + 64 + 2 + 2};  // GGML block_q2_K; the reference table says 82
        case GgmlType::Q3_K: return {256, 32 + 64 + 12 + 2};
        case GgmlType::Q4_K: return {256, 2 + 2 + 12 + 128};
        case GgmlType::Q5_K: return {256, 2 + 2 + 12 + 32 + 128};
        case GgmlType::Q6_K: return {256, 128 + 64 + 16 + 2};
        case GgmlType::Q8_K: return {256, 4 + 256 + 32};
        default: return {0, 0};
    }
}
}  // namespace detail

// Elements per block (0 for types without a block layout here).
inline uint64_t ggml_type_block_size(GgmlType type) { return detail::block_format(type).elems; }

// Bytes per block (0 for types without a block layout here).
inline uint64_t ggml_type_size(GgmlType type) { return detail::block_format(type).bytes; }

// Bytes of a tensor of num_elements, or 0 if the count is not whole blocks or overflows.
inline uint64_t calculate_tensor_bytes(GgmlType type, uint64_t num_elements) {
    const detail::BlockFormat f = detail::block_format(type);
    if (f.elems == 0 || f.bytes == 0 || num_elements % f.elems != 0) return 0;
    const uint64_t blocks = num_elements / f.elems;
    if (blocks > std::numeric_limits<uint64_t>::max() / f.bytes) return 0;
    return blocks * f.bytes;
}

}  // namespace qwen

#endif  // QWEN35_QUANTIZED_HPP
