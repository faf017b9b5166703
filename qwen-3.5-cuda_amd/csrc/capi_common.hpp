// Host-side plumbing shared by the C entry points: status codes, the per-thread
// error message, argument checks and the post-launch check.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>

#include "qwen35_hip.h"

namespace qk {

// Records a printf-style message for the calling thread and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the calling thread's message and returns QWEN_STATUS_OK.
int ok();

// QWEN_STATUS_LAUNCH_FAILED with the runtime's message if the last launch on
// this thread was rejected, else ok().
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Number of blocks for `items` work items at `per_block` per block.
inline unsigned blocks_for(int64_t items, int64_t per_block) {
    return static_cast<unsigned>((items + per_block - 1) / per_block);
}

}  // namespace qk

#define QK_REQUIRE(cond, ...)                                          \
    do {                                                               \
        if (!(cond)) return ::qk::fail(QWEN_STATUS_INVALID_ARGUMENT, __VA_ARGS__); \
    } while (0)
