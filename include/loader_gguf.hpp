// GGUF model-file loader: the reference's qwen::GgufLoader interface
// (include/loader_gguf.hpp:11-115 of sahan974/qwen-3.5-cuda) over this
// library's own parser and device upload (csrc/gguf.cpp).
//
// Kept alike, because callers compile against it: the class and method names,
// their signatures and defaults, GgufMetadataValueType (GGUF's on-disk type
// ids), the metadata accessors' parsing rules (std::stoi / std::stod with the
// default on failure) and which failures return false and which throw
// std::runtime_error. Different: the file is parsed from a read-only mapping,
// and load_tensors_to_gpu() places all tensors in one device arena filled
// through pinned double-buffered staging with asynchronous copies.
#ifndef QWEN35_LOADER_GGUF_HPP
#define QWEN35_LOADER_GGUF_HPP

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "quantized.hpp"

namespace qwen {

// GGUF metadata value types (the GGUF file format's ids).
enum class GgufMetadataValueType : uint32_t {
    UINT8 = 0,
    INT8 = 1,
    UINT16 = 2,
    INT16 = 3,
    UINT32 = 4,
    INT32 = 5,
    FLOAT32 = 6,
    BOOL = 7,
    STRING = 8,
    ARRAY = 9,
    UINT64 = 10,
    INT64 = 11,
    FLOAT64 = 12,
};

class GgufLoader {
public:
    GgufLoader() = default;
    ~GgufLoader();
    GgufLoader(const GgufLoader&) = delete;
    GgufLoader& operator=(const GgufLoader&) = delete;

    // Parses header, metadata and tensor infos. false: the file cannot be
    // opened or is not GGUF; throws std::runtime_error on malformed content.
    bool open(const std::string& filepath);

    // If base_layer_count is non-negative, tensors belonging to blk.N with
    // N >= base_layer_count stay on disk (device_ptr nullptr). false if the
    // device arena cannot be allocated or the file cannot be read (nothing
    // stays loaded then).
    bool load_tensors_to_gpu(int base_layer_count = -1);
    // Same, with the copies enqueued on `stream` (synchronised before return).
    bool load_tensors_to_gpu(int base_layer_count, hipStream_t stream);

    void unload_gpu();
    void close();

    uint32_t version() const { return version_; }
    uint64_t tensor_count() const { return tensor_count_; }
    uint64_t metadata_count() const { return metadata_count_; }
    uint64_t total_vram_bytes() const { return total_vram_bytes_; }
    uint64_t payload_offset() const { return payload_offset_; }

    const std::vector<QuantTensor>& tensors() const { return tensors_; }
    const std::unordered_map<std::string, std::string>& metadata() const { return metadata_str_; }
    // Metadata keys in file order.
    const std::vector<std::string>& metadata_keys() const { return key_order_; }

    const std::vector<std::string>* get_meta_array(const std::string& key) const {
        auto it = metadata_arrays_.find(key);
        return it == metadata_arrays_.end() ? nullptr : &it->second;
    }

    const QuantTensor* get_tensor(const std::string& name) const {
        auto it = tensor_index_.find(name);
        return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
    }

    int get_meta_int(const std::string& key, int default_val = 0) const {
        auto it = metadata_str_.find(key);
        if (it == metadata_str_.end()) return default_val;
        try {
            return std::stoi(it->second);
        } catch (...) {
            return default_val;
        }
    }

    double get_meta_float(const std::string& key, double default_val = 0.0) const {
        auto it = metadata_str_.find(key);
        if (it == metadata_str_.end()) return default_val;
        try {
            return std::stod(it->second);
        } catch (...) {
            return default_val;
        }
    }

    std::string get_meta_string(const std::string& key, const std::string& default_val = {}) const {
        auto it = metadata_str_.find(key);
        return it == metadata_str_.end() ? default_val : it->second;
    }

    void print_summary() const;

    // Why the last load_tensors_to_gpu() returned false ("" after a success).
    const std::string& load_error() const { return load_error_; }
    bool load_out_of_memory() const { return load_oom_; }

private:
    std::string filepath_;
    uint32_t version_ = 0;
    uint64_t tensor_count_ = 0;
    uint64_t metadata_count_ = 0;
    uint64_t payload_offset_ = 0;
    uint64_t total_vram_bytes_ = 0;
    std::vector<QuantTensor> tensors_;
    std::unordered_map<std::string, size_t> tensor_index_;
    std::unordered_map<std::string, std::string> metadata_str_;
    std::unordered_map<std::string, std::vector<std::string>> metadata_arrays_;
    std::vector<std::string> key_order_;
    void* arena_ = nullptr;   // device memory of every loaded tensor
    std::string load_error_;
    bool load_oom_ = false;
};

// Index N of a tensor named "blk.N.*", else -1 (ref: src/loader_gguf.cpp:28-45).
int tensor_block_index(const std::string& name);

}  // namespace qwen

#endif  // QWEN35_LOADER_GGUF_HPP
