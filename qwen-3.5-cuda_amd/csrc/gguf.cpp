// GGUF model-file loader (host side): qwen::GgufLoader and its C ABI.
//
// Reference behaviour followed (src/loader_gguf.cpp): GGUF v2/v3 only; 64-bit
// string and array lengths; scalar metadata kept as text (std::to_string for
// numbers, "true"/"false", strings verbatim) and arrays as vectors of that
// text (:155-175, :80-101); general.alignment (default 32, a power of two)
// fixes the payload start; each tensor's byte range must be aligned, inside
// the file and disjoint from the others (:270-306); the same limits and
// messages for malformed files (:17-26, :61-78, :196-266).
//
// Design: the file is parsed from a read-only mapping with a bounds-checked
// cursor (no per-field stream reads). The upload places all selected tensors
// in one device allocation (256-byte aligned slots) and streams the file in
// file order through two pinned staging buffers: while the copies of one
// buffer run on the stream, several host threads fill the other from the
// mapping, so disk / page-cache reads overlap the PCIe transfers.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <thread>
#include <unordered_set>

#include "capi_common.hpp"
#include "loader_gguf.hpp"
#include "qwen35_gguf.h"

namespace qwen {
namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;   // "GGUF" as a little-endian u32
constexpr uint64_t kArenaAlign = 256;
constexpr size_t kStageBytes = size_t{64} << 20;

// Read-only mapping of a whole file.
class Mapping {
public:
    ~Mapping() {
        if (data_) munmap(const_cast<uint8_t*>(data_), size_);
        if (fd_ >= 0) ::close(fd_);
    }
    bool map(const std::string& path) {
        fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd_ < 0) return false;
        struct stat st {};
        if (fstat(fd_, &st) != 0 || st.st_size < 0) return false;
        size_ = static_cast<size_t>(st.st_size);
        if (size_ == 0) return true;
        void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (p == MAP_FAILED) return false;
        data_ = static_cast<const uint8_t*>(p);
        return true;
    }
    void advise_sequential() const {
        if (fd_ >= 0) (void)posix_fadvise(fd_, 0, 0, POSIX_FADV_SEQUENTIAL);
    }
    const uint8_t* data() const { return data_; }
    int fd() const { return fd_; }
    size_t size() const { return size_; }

private:
    int fd_ = -1;
    const uint8_t* data_ = nullptr;
    size_t size_ = 0;
};

// Bounds-checked little-endian reader over the mapping.
class Cursor {
public:
    Cursor(const uint8_t* d, size_t n) : d_(d), n_(n) {}

    template <typename T>
    T get(const char* what) {
        if (n_ - pos_ < sizeof(T)) throw std::runtime_error(std::string("truncated GGUF while reading ") + what);
        T v;
        std::memcpy(&v, d_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }

    std::string str() {
        const uint64_t len = get<uint64_t>("string length");
        if (len > (uint64_t{1} << 32)) throw std::runtime_error("unreasonable GGUF string length");
        if (n_ - pos_ < len) throw std::runtime_error("truncated GGUF string");
        std::string s(reinterpret_cast<const char*>(d_ + pos_), static_cast<size_t>(len));
        pos_ += static_cast<size_t>(len);
        return s;
    }

    size_t pos() const { return pos_; }

private:
    const uint8_t* d_;
    size_t n_;
    size_t pos_ = 0;
};

using VT = GgufMetadataValueType;

std::string scalar_text(Cursor& c, uint32_t raw) {
    switch (static_cast<VT>(raw)) {
        case VT::UINT8: return std::to_string(c.get<uint8_t>("uint8 metadata"));
        case VT::INT8: return std::to_string(c.get<int8_t>("int8 metadata"));
        case VT::BOOL: return c.get<uint8_t>("bool metadata") ? "true" : "false";
        case VT::UINT16: return std::to_string(c.get<uint16_t>("uint16 metadata"));
        case VT::INT16: return std::to_string(c.get<int16_t>("int16 metadata"));
        case VT::UINT32: return std::to_string(c.get<uint32_t>("uint32 metadata"));
        case VT::INT32: return std::to_string(c.get<int32_t>("int32 metadata"));
        case VT::FLOAT32: return std::to_string(c.get<float>("float32 metadata"));
        case VT::UINT64: return std::to_string(c.get<uint64_t>("uint64 metadata"));
        case VT::INT64: return std::to_string(c.get<int64_t>("int64 metadata"));
        case VT::FLOAT64: return std::to_string(c.get<double>("float64 metadata"));
        case VT::STRING: return c.str();
        case VT::ARRAY: throw std::runtime_error("array metadata must be read with read_metadata_array");
        default: throw std::runtime_error("Unknown GGUF metadata value type");
    }
}

std::vector<std::string> array_text(Cursor& c) {
    const uint32_t raw = c.get<uint32_t>("array element type");
    const uint64_t count = c.get<uint64_t>("array length");
    if (count > (uint64_t{1} << 32)) throw std::runtime_error("invalid GGUF metadata array");
    if (static_cast<VT>(raw) == VT::ARRAY) throw std::runtime_error("nested GGUF arrays are unsupported");
    std::vector<std::string> out;
    out.reserve(static_cast<size_t>(std::min<uint64_t>(count, 1 << 20)));
    for (uint64_t i = 0; i < count; ++i) out.push_back(scalar_text(c, raw));
    return out;
}

uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// pread of n bytes at file offset `off` into dst, split over up to `threads`
// host threads (this is where the tensor data is read from the file). Returns
// false when the file ends before n bytes or a read fails: a file cut short
// while it is being loaded ends in an error, as the reference's fin.read does
// (src/loader_gguf.cpp:357-361), never in a read past the end of a mapping.
bool parallel_read(int fd, void* dst, uint64_t off, size_t n, unsigned threads) {
    auto read_all = [fd](uint8_t* d, uint64_t o, size_t len) {
        while (len > 0) {
            const ssize_t r = ::pread(fd, d, len, static_cast<off_t>(o));
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) return false;
            d += r;
            o += static_cast<uint64_t>(r);
            len -= static_cast<size_t>(r);
        }
        return true;
    };
    constexpr size_t kMinPerThread = size_t{4} << 20;
    const unsigned t = static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>(threads, n / kMinPerThread)));
    uint8_t* d = static_cast<uint8_t*>(dst);
    if (t <= 1) return read_all(d, off, n);
    std::vector<std::thread> pool;
    std::vector<char> good(t, 0);
    const size_t part = (n + t - 1) / t;
    for (unsigned i = 0; i < t; ++i) {
        const size_t b = i * part, e = std::min(n, b + part);
        if (b < e)
            pool.emplace_back([&, i, b, e] { good[i] = read_all(d + b, off + b, e - b); });
        else
            good[i] = 1;
    }
    for (auto& th : pool) th.join();
    return std::all_of(good.begin(), good.end(), [](char g) { return g != 0; });
}

}  // namespace

int tensor_block_index(const std::string& name) {
    if (name.compare(0, 4, "blk.") != 0) return -1;
    const size_t dot = name.find('.', 4);
    if (dot == std::string::npos || dot == 4) return -1;
    int64_t v = 0;
    for (size_t i = 4; i < dot; ++i) {
        const char ch = name[i];
        if (ch < '0' || ch > '9') return -1;
        v = v * 10 + (ch - '0');
        if (v > std::numeric_limits<int>::max()) return -1;
    }
    return static_cast<int>(v);
}

GgufLoader::~GgufLoader() { close(); }

void GgufLoader::close() {
    unload_gpu();
    filepath_.clear();
    version_ = 0;
    tensor_count_ = metadata_count_ = payload_offset_ = 0;
    tensors_.clear();
    tensor_index_.clear();
    metadata_str_.clear();
    metadata_arrays_.clear();
    key_order_.clear();
}

bool GgufLoader::open(const std::string& filepath) {
    close();
    Mapping m;
    if (!m.map(filepath)) return false;
    Cursor c(m.data(), m.size());
    if (c.get<uint32_t>("magic") != kGgufMagic) return false;

    const uint32_t version = c.get<uint32_t>("version");
    if (version != 2 && version != 3) throw std::runtime_error("unsupported GGUF version " + std::to_string(version));
    const uint64_t n_tensors = c.get<uint64_t>("tensor count");
    const uint64_t n_meta = c.get<uint64_t>("metadata count");
    if (n_tensors > (uint64_t{1} << 24) || n_meta > (uint64_t{1} << 24))
        throw std::runtime_error("unreasonable GGUF header counts");

    std::unordered_map<std::string, std::string> meta;
    std::unordered_map<std::string, std::vector<std::string>> arrays;
    std::vector<std::string> keys;
    keys.reserve(static_cast<size_t>(n_meta));
    for (uint64_t i = 0; i < n_meta; ++i) {
        std::string key = c.str();
        if (meta.count(key) || arrays.count(key)) throw std::runtime_error("duplicate GGUF metadata key: " + key);
        const uint32_t vt = c.get<uint32_t>("metadata value type");
        if (static_cast<VT>(vt) == VT::ARRAY)
            arrays.emplace(key, array_text(c));
        else
            meta.emplace(key, scalar_text(c, vt));
        keys.push_back(std::move(key));
    }

    std::vector<QuantTensor> tensors;
    std::unordered_map<std::string, size_t> index;
    tensors.reserve(static_cast<size_t>(n_tensors));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        QuantTensor t;
        t.name = c.str();
        if (index.count(t.name)) throw std::runtime_error("duplicate GGUF tensor name: " + t.name);
        const uint32_t nd = c.get<uint32_t>("tensor dimension count");
        if (nd == 0 || nd > 4) throw std::runtime_error("invalid dimensions for tensor " + t.name);
        t.shape.resize(nd);
        t.num_elements = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const int64_t e = c.get<int64_t>("tensor dimension");
            if (e <= 0 || t.num_elements > std::numeric_limits<uint64_t>::max() / static_cast<uint64_t>(e))
                throw std::runtime_error("invalid or overflowing shape for tensor " + t.name);
            t.shape[d] = e;
            t.num_elements *= static_cast<uint64_t>(e);
        }
        const uint32_t raw_type = c.get<uint32_t>("tensor type");
        t.type = static_cast<GgmlType>(raw_type);
        t.offset = c.get<uint64_t>("tensor offset");
        t.size_bytes = calculate_tensor_bytes(t.type, t.num_elements);
        if (t.size_bytes == 0)
            throw std::runtime_error("unsupported or malformed tensor '" + t.name + "' (GGML type " +
                                     std::to_string(raw_type) + ")");
        const uint64_t block = ggml_type_block_size(t.type);
        if (block > 1 && static_cast<uint64_t>(t.shape[0]) % block != 0)
            throw std::runtime_error("quantized row width is not block-aligned for tensor " + t.name);
        index.emplace(t.name, tensors.size());
        tensors.push_back(std::move(t));
    }

    // Alignment as the reference reads it: the metadata text through std::stoi,
    // 32 when absent or unparsable.
    int align_i = 32;
    if (auto it = meta.find("general.alignment"); it != meta.end()) {
        try {
            align_i = std::stoi(it->second);
        } catch (...) {
            align_i = 32;
        }
    }
    const uint64_t alignment = static_cast<uint64_t>(align_i);
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) throw std::runtime_error("invalid GGUF alignment");
    const uint64_t payload = round_up(c.pos(), alignment);
    const uint64_t file_size = m.size();

    struct Span {
        uint64_t begin, end;
        const std::string* name;
    };
    std::vector<Span> spans;
    spans.reserve(tensors.size());
    for (const auto& t : tensors) {
        if (t.offset % alignment != 0 || t.offset > std::numeric_limits<uint64_t>::max() - payload ||
            payload + t.offset > file_size || t.size_bytes > file_size - (payload + t.offset))
            throw std::runtime_error("invalid data range for tensor " + t.name);
        spans.push_back({payload + t.offset, payload + t.offset + t.size_bytes, &t.name});
    }
    std::sort(spans.begin(), spans.end(), [](const Span& a, const Span& b) { return a.begin < b.begin; });
    for (size_t i = 1; i < spans.size(); ++i)
        if (spans[i].begin < spans[i - 1].end)
            throw std::runtime_error("overlapping GGUF tensors: " + *spans[i - 1].name + " and " + *spans[i].name);

    filepath_ = filepath;
    version_ = version;
    tensor_count_ = n_tensors;
    metadata_count_ = n_meta;
    payload_offset_ = payload;
    tensors_ = std::move(tensors);
    tensor_index_ = std::move(index);
    metadata_str_ = std::move(meta);
    metadata_arrays_ = std::move(arrays);
    key_order_ = std::move(keys);
    return true;
}

void GgufLoader::unload_gpu() {
    if (arena_) {
        (void)hipFree(arena_);
        arena_ = nullptr;
    }
    for (auto& t : tensors_) t.device_ptr = nullptr;
    total_vram_bytes_ = 0;
}

bool GgufLoader::load_tensors_to_gpu(int base_layer_count) { return load_tensors_to_gpu(base_layer_count, nullptr); }

bool GgufLoader::load_tensors_to_gpu(int base_layer_count, hipStream_t stream) {
    unload_gpu();
    load_error_.clear();
    load_oom_ = false;
    auto fail = [&](const std::string& why, bool oom) {
        load_error_ = why;
        load_oom_ = oom;
        return false;
    };
    if (filepath_.empty()) return fail("no GGUF file is open", false);
    Mapping m;
    if (!m.map(filepath_) || m.size() < payload_offset_) return fail("cannot re-read GGUF file " + filepath_, false);

    // Selected tensors in file order, each at a 256-byte aligned arena offset.
    std::vector<size_t> sel;
    for (size_t i = 0; i < tensors_.size(); ++i) {
        const int blk = tensor_block_index(tensors_[i].name);
        if (base_layer_count < 0 || blk < 0 || blk < base_layer_count) sel.push_back(i);
    }
    std::sort(sel.begin(), sel.end(), [&](size_t a, size_t b) { return tensors_[a].offset < tensors_[b].offset; });
    // The file may have changed since open(): every selected tensor must still
    // lie inside it, checked here before any device call; the reference's read
    // fails instead ("Error reading binary tensor data", src/loader_gguf.cpp:
    // 355-360). The data itself is read with pread (parallel_read), so a file
    // cut short after this check still ends in that error.
    const uint64_t avail = m.size() - payload_offset_;
    for (size_t i : sel) {
        const QuantTensor& t = tensors_[i];
        if (t.offset > avail || t.size_bytes > avail - t.offset)
            return fail("cannot re-read GGUF file " + filepath_ + ": tensor '" + t.name + "' lies past its end", false);
    }
    std::vector<uint64_t> slot(sel.size());
    uint64_t arena_bytes = 0, data_bytes = 0;
    for (size_t k = 0; k < sel.size(); ++k) {
        slot[k] = round_up(arena_bytes, kArenaAlign);
        arena_bytes = slot[k] + tensors_[sel[k]].size_bytes;
        data_bytes += tensors_[sel[k]].size_bytes;
    }
    if (sel.empty()) return true;
    if (hipMalloc(&arena_, arena_bytes) != hipSuccess) {
        (void)hipGetLastError();
        arena_ = nullptr;
        return fail("device allocation of " + std::to_string(arena_bytes) + " bytes for " + std::to_string(sel.size()) +
                        " tensors failed", true);
    }

    hipStream_t s = stream;
    bool own_stream = false;
    if (!s) {
        if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
            (void)hipGetLastError();
            unload_gpu();
            return fail("cannot create a stream for the upload", false);
        }
        own_stream = true;
    }
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool ok = true;
    std::string short_read;   // tensor whose data the file no longer holds
    for (int b = 0; b < 2 && ok; ++b)
        ok = hipHostMalloc(&stage[b], kStageBytes, hipHostMallocDefault) == hipSuccess &&
             hipEventCreateWithFlags(&done[b], hipEventDisableTiming) == hipSuccess;

    if (ok) {
        m.advise_sequential();
        const unsigned threads = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
        uint8_t* arena = static_cast<uint8_t*>(arena_);
        int b = 0;
        size_t fill = 0;
        bool in_flight[2] = {false, false};
        for (size_t k = 0; k < sel.size() && ok; ++k) {
            const QuantTensor& t = tensors_[sel[k]];
            const uint64_t src = payload_offset_ + t.offset;
            uint64_t done_bytes = 0;
            while (done_bytes < t.size_bytes && ok) {
                const size_t n = static_cast<size_t>(std::min<uint64_t>(t.size_bytes - done_bytes, kStageBytes - fill));
                uint8_t* dst = static_cast<uint8_t*>(stage[b]) + fill;
                if (!parallel_read(m.fd(), dst, src + done_bytes, n, threads)) {
                    short_read = t.name;
                    ok = false;
                    break;
                }
                ok = hipMemcpyAsync(arena + slot[k] + done_bytes, dst, n, hipMemcpyHostToDevice, s) == hipSuccess;
                fill += n;
                done_bytes += n;
                if (fill == kStageBytes && ok) {
                    // Hand buffer b to the stream; refill the other once its copies are done.
                    ok = hipEventRecord(done[b], s) == hipSuccess;
                    in_flight[b] = true;
                    b ^= 1;
                    fill = 0;
                    if (ok && in_flight[b]) ok = hipEventSynchronize(done[b]) == hipSuccess;
                    in_flight[b] = false;
                }
            }
        }
        // Also on failure: copies already enqueued read the staging buffers and
        // write the arena, so they must finish before either is freed.
        const bool synced = hipStreamSynchronize(s) == hipSuccess;
        ok = ok && synced;
    } else {
        // No pinned staging (pinned memory exhausted): reads into a pageable
        // buffer and synchronous copies, as the reference uploads.
        (void)hipGetLastError();
        std::vector<uint8_t> bounce;
        try {
            bounce.resize(kStageBytes);
            ok = true;
        } catch (const std::bad_alloc&) {
            ok = false;
        }
        uint8_t* arena = static_cast<uint8_t*>(arena_);
        const unsigned threads = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
        for (size_t k = 0; k < sel.size() && ok; ++k) {
            const QuantTensor& t = tensors_[sel[k]];
            for (uint64_t done_bytes = 0; done_bytes < t.size_bytes && ok;) {
                const size_t n = static_cast<size_t>(std::min<uint64_t>(t.size_bytes - done_bytes, kStageBytes));
                if (!parallel_read(m.fd(), bounce.data(), payload_offset_ + t.offset + done_bytes, n, threads)) {
                    short_read = t.name;
                    ok = false;
                    break;
                }
                ok = hipMemcpy(arena + slot[k] + done_bytes, bounce.data(), n, hipMemcpyHostToDevice) == hipSuccess;
                done_bytes += n;
            }
        }
    }
    for (int b = 0; b < 2; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (stage[b]) (void)hipHostFree(stage[b]);
    }
    if (own_stream) (void)hipStreamDestroy(s);
    if (!ok) {
        const hipError_t err = hipGetLastError();
        unload_gpu();
        if (!short_read.empty())
            return fail("cannot re-read GGUF file " + filepath_ + ": error reading binary tensor data for '" +
                            short_read + "'",
                        false);
        return fail(std::string("tensor upload failed: ") + hipGetErrorString(err), false);
    }
    for (size_t k = 0; k < sel.size(); ++k) tensors_[sel[k]].device_ptr = static_cast<uint8_t*>(arena_) + slot[k];
    total_vram_bytes_ = data_bytes;
    return true;
}

void GgufLoader::print_summary() const {
    std::cout << "--- GGUF Header Summary ---\n"
              << "File: " << filepath_ << "\n"
              << "GGUF Version: " << version_ << "\n"
              << "Tensor Count: " << tensor_count_ << "\n"
              << "Metadata KV Count: " << metadata_count_ << "\n\nAll Metadata Entries:\n";
    for (const auto& key : key_order_) {
        auto it = metadata_str_.find(key);
        if (it == metadata_str_.end()) continue;
        if (it->second.size() > 120)
            std::cout << "  " << key << " = [... " << it->second.size() << " chars ...]\n";
        else
            std::cout << "  " << key << " = " << it->second << "\n";
    }
    std::cout.flush();
}

}  // namespace qwen

// ------------------------------------------------------------------ C ABI
struct qwen_gguf {
    qwen::GgufLoader loader;
};

extern "C" {

int qwen_gguf_open(const char* path, qwen_gguf** out) {
    QK_REQUIRE(path && out, "qwen_gguf_open: null pointer");
    *out = nullptr;
    auto g = std::make_unique<qwen_gguf>();
    try {
        if (!g->loader.open(path)) return qk::fail(QWEN_STATUS_IO_ERROR, "cannot open GGUF file %s", path);
    } catch (const std::exception& e) {
        return qk::fail(QWEN_STATUS_MALFORMED, "%s", e.what());
    }
    *out = g.release();
    return qk::ok();
}

int qwen_gguf_close(qwen_gguf* g) {
    delete g;
    return qk::ok();
}

int qwen_gguf_get_info(const qwen_gguf* g, qwen_gguf_info* info) {
    QK_REQUIRE(g && info, "qwen_gguf_get_info: null pointer");
    info->version = g->loader.version();
    info->tensor_count = g->loader.tensor_count();
    info->metadata_count = g->loader.metadata_count();
    info->payload_offset = g->loader.payload_offset();
    info->device_bytes = g->loader.total_vram_bytes();
    return qk::ok();
}

int qwen_gguf_get_tensor(const qwen_gguf* g, uint64_t index, qwen_gguf_tensor* out) {
    QK_REQUIRE(g && out, "qwen_gguf_get_tensor: null pointer");
    const auto& ts = g->loader.tensors();
    if (index >= ts.size())
        return qk::fail(QWEN_STATUS_OUT_OF_RANGE, "tensor index %llu of %zu", static_cast<unsigned long long>(index),
                        ts.size());
    const qwen::QuantTensor& t = ts[index];
    out->name = t.name.c_str();
    out->type = static_cast<uint32_t>(t.type);
    out->n_dims = static_cast<uint32_t>(t.shape.size());
    for (int d = 0; d < 4; ++d) out->shape[d] = d < static_cast<int>(t.shape.size()) ? t.shape[d] : 1;
    out->num_elements = t.num_elements;
    out->size_bytes = t.size_bytes;
    out->offset = t.offset;
    out->device_ptr = t.device_ptr;
    return qk::ok();
}

int qwen_gguf_find_tensor(const qwen_gguf* g, const char* name, int64_t* index) {
    QK_REQUIRE(g && name && index, "qwen_gguf_find_tensor: null pointer");
    const qwen::QuantTensor* t = g->loader.get_tensor(name);
    *index = t ? static_cast<int64_t>(t - g->loader.tensors().data()) : -1;
    return qk::ok();
}

int qwen_gguf_get_meta(const qwen_gguf* g, const char* key, const char** value) {
    QK_REQUIRE(g && key && value, "qwen_gguf_get_meta: null pointer");
    const auto& m = g->loader.metadata();
    auto it = m.find(key);
    *value = it == m.end() ? nullptr : it->second.c_str();
    return qk::ok();
}

int qwen_gguf_get_meta_array_size(const qwen_gguf* g, const char* key, int64_t* count) {
    QK_REQUIRE(g && key && count, "qwen_gguf_get_meta_array_size: null pointer");
    const auto* a = g->loader.get_meta_array(key);
    *count = a ? static_cast<int64_t>(a->size()) : -1;
    return qk::ok();
}

int qwen_gguf_get_meta_array_item(const qwen_gguf* g, const char* key, uint64_t index, const char** value) {
    QK_REQUIRE(g && key && value, "qwen_gguf_get_meta_array_item: null pointer");
    const auto* a = g->loader.get_meta_array(key);
    if (!a) return qk::fail(QWEN_STATUS_OUT_OF_RANGE, "no array metadata '%s'", key);
    if (index >= a->size())
        return qk::fail(QWEN_STATUS_OUT_OF_RANGE, "index %llu of array '%s' (%zu items)",
                        static_cast<unsigned long long>(index), key, a->size());
    *value = (*a)[index].c_str();
    return qk::ok();
}

int qwen_gguf_get_meta_key(const qwen_gguf* g, uint64_t index, const char** key, int* is_array) {
    QK_REQUIRE(g && key && is_array, "qwen_gguf_get_meta_key: null pointer");
    const auto& keys = g->loader.metadata_keys();
    if (index >= keys.size())
        return qk::fail(QWEN_STATUS_OUT_OF_RANGE, "metadata index %llu of %zu", static_cast<unsigned long long>(index),
                        keys.size());
    *key = keys[index].c_str();
    *is_array = g->loader.get_meta_array(keys[index]) ? 1 : 0;
    return qk::ok();
}

int qwen_gguf_load(qwen_gguf* g, int base_layer_count, void* stream) {
    QK_REQUIRE(g, "qwen_gguf_load: null handle");
    if (g->loader.load_tensors_to_gpu(base_layer_count, qk::as_stream(stream))) return qk::ok();
    return qk::fail(g->loader.load_out_of_memory() ? QWEN_STATUS_OUT_OF_MEMORY : QWEN_STATUS_IO_ERROR, "%s",
                    g->loader.load_error().c_str());
}

int qwen_gguf_unload(qwen_gguf* g) {
    QK_REQUIRE(g, "qwen_gguf_unload: null handle");
    g->loader.unload_gpu();
    return qk::ok();
}

}  // extern "C"
