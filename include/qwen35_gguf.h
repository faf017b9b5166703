/*
 * qwen35_gguf.h -- C ABI of the GGUF model-file loader.
 *
 * Parses a GGUF v2/v3 file (header, metadata, tensor infos), validates every
 * tensor's byte range, and uploads the tensors to device memory. Unlike the
 * kernel entry points of qwen35_hip.h these functions do host I/O, allocate
 * (one device arena per loaded file, pinned staging buffers while uploading)
 * and synchronise; they are not meant for a decode loop. They return a
 * qwen_status and never throw; qwen_last_error() holds the message, with the
 * reference's wording where the reference throws.
 *
 * ref: include/loader_gguf.hpp:34-115 (class GgufLoader), src/loader_gguf.cpp:13-381.
 * The C++ drop-in class qwen::GgufLoader (loader_gguf.hpp) has the reference's
 * public interface over the same implementation.
 */
#ifndef QWEN35_GGUF_H
#define QWEN35_GGUF_H

#include <stdint.h>

#include "qwen35_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque handle of an open GGUF file. */
typedef struct qwen_gguf qwen_gguf;

typedef struct qwen_gguf_info {
    uint32_t version;        /* 2 or 3 */
    uint64_t tensor_count;
    uint64_t metadata_count;
    uint64_t payload_offset; /* file offset of the tensor data (aligned) */
    uint64_t device_bytes;   /* sum of the loaded tensors' sizes (0 if none) */
} qwen_gguf_info;

typedef struct qwen_gguf_tensor {
    const char* name;      /* valid until qwen_gguf_close */
    uint32_t type;         /* GGML type id (include/quantized.hpp GgmlType) */
    uint32_t n_dims;       /* 1..4 */
    int64_t shape[4];      /* GGUF order: shape[0] is the row width */
    uint64_t num_elements;
    uint64_t size_bytes;
    uint64_t offset;       /* from the start of the payload */
    void* device_ptr;      /* NULL unless loaded */
} qwen_gguf_tensor;

/* Opens and parses `path`. *out receives the handle on success.
 * QWEN_STATUS_IO_ERROR: the file cannot be opened or is not GGUF (bad magic)
 * -- the cases where the reference's open() returns false.
 * QWEN_STATUS_MALFORMED: everything the reference rejects by throwing
 * (unsupported version, truncation, bad counts or dimensions, duplicate keys
 * or tensor names, unsupported tensor types, misaligned or overlapping data).
 * ref: src/loader_gguf.cpp:178-309 (GgufLoader::open) */
int qwen_gguf_open(const char* path, qwen_gguf** out);

/* Frees the device arena and the handle (NULL is a no-op).
 * ref: src/loader_gguf.cpp:48-57 (close) */
int qwen_gguf_close(qwen_gguf* g);

int qwen_gguf_get_info(const qwen_gguf* g, qwen_gguf_info* info);

/* Tensor `index` (< tensor_count, file order) -> QWEN_STATUS_OUT_OF_RANGE otherwise. */
int qwen_gguf_get_tensor(const qwen_gguf* g, uint64_t index, qwen_gguf_tensor* out);

/* *index = position of the tensor called `name`, or -1.
 * ref: include/loader_gguf.hpp:60-65 (get_tensor) */
int qwen_gguf_find_tensor(const qwen_gguf* g, const char* name, int64_t* index);

/* Scalar metadata as the reference stores it (integers in decimal, floats as
 * std::to_string, bools "true"/"false", strings verbatim); *value = NULL if
 * the key is absent or holds an array. ref: src/loader_gguf.cpp:155-175 */
int qwen_gguf_get_meta(const qwen_gguf* g, const char* key, const char** value);

/* Array metadata: *count = number of elements, or -1 if `key` is not an array.
 * ref: include/loader_gguf.hpp:55-58 (get_meta_array), src/loader_gguf.cpp:80-101 */
int qwen_gguf_get_meta_array_size(const qwen_gguf* g, const char* key, int64_t* count);
int qwen_gguf_get_meta_array_item(const qwen_gguf* g, const char* key, uint64_t index, const char** value);

/* Metadata key `index` in file order (< metadata_count); *is_array = 1 for arrays. */
int qwen_gguf_get_meta_key(const qwen_gguf* g, uint64_t index, const char** key, int* is_array);

/* Uploads the tensors to device memory (one arena, 256-byte aligned tensors).
 * base_layer_count >= 0 leaves tensors "blk.N.*" with N >= base_layer_count
 * on disk (device_ptr NULL), as the reference does for Qwen3.5's MTP blocks.
 * Reads the file through pinned double-buffered staging with the copies
 * enqueued on `stream` (NULL: an internal non-blocking stream) and
 * synchronises before returning; if pinned memory cannot be allocated it
 * falls back to synchronous copies from the mapped file.
 * QWEN_STATUS_OUT_OF_MEMORY if the arena cannot be allocated,
 * QWEN_STATUS_IO_ERROR if the file cannot be re-read or a copy fails; either
 * way nothing stays loaded.
 * ref: src/loader_gguf.cpp:322-381 (load_tensors_to_gpu) */
int qwen_gguf_load(qwen_gguf* g, int base_layer_count, void* stream);

/* Frees the device arena (device_ptr -> NULL). ref: src/loader_gguf.cpp:312-320 */
int qwen_gguf_unload(qwen_gguf* g);

#ifdef __cplusplus
}
#endif

#endif /* QWEN35_GGUF_H */
