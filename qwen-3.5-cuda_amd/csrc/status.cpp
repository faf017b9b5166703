// Status codes and the per-thread error message of the C ABI.
#include <cstdio>
#include <cstring>

#include "capi_common.hpp"

namespace qk {
namespace {
thread_local char g_message[512] = "";
}  // namespace

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_message, sizeof(g_message), fmt, ap);
    va_end(ap);
    return status;
}

int ok() {
    g_message[0] = '\0';
    return QWEN_STATUS_OK;
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return fail(QWEN_STATUS_LAUNCH_FAILED, "%s: launch failed: %s", what, hipGetErrorString(err));
    }
    return ok();
}

}  // namespace qk

extern "C" {

int qwen_abi_version(void) { return 2; }

const char* qwen_last_error(void) { return qk::g_message; }

const char* qwen_status_name(int status) {
    switch (status) {
        case QWEN_STATUS_OK: return "QWEN_STATUS_OK";
        case QWEN_STATUS_INVALID_ARGUMENT: return "QWEN_STATUS_INVALID_ARGUMENT";
        case QWEN_STATUS_UNSUPPORTED_TYPE: return "QWEN_STATUS_UNSUPPORTED_TYPE";
        case QWEN_STATUS_OUT_OF_RANGE: return "QWEN_STATUS_OUT_OF_RANGE";
        case QWEN_STATUS_LAUNCH_FAILED: return "QWEN_STATUS_LAUNCH_FAILED";
        case QWEN_STATUS_IO_ERROR: return "QWEN_STATUS_IO_ERROR";
        case QWEN_STATUS_MALFORMED: return "QWEN_STATUS_MALFORMED";
        case QWEN_STATUS_OUT_OF_MEMORY: return "QWEN_STATUS_OUT_OF_MEMORY";
        default: return "QWEN_STATUS_UNKNOWN";
    }
}

}  // extern "C"
