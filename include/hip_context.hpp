// HIP stream context and error check for host code that drives the kernels of
// libqwen35_hip.so the way the reference's layers drive theirs.
//
// Replaces, for a caller ported to HIP, what the reference's layer headers take
// from include/cuda_utils.hpp:30-87 (each of include/layer_attn.hpp:4,
// layer_gdn.hpp:5, layer_moe.hpp:5 and model.hpp:5 includes it):
//   CUDA_CHECK(call)        -> QWEN_HIP_CHECK(call): throws std::runtime_error
//                              ("HIP Error: <hipGetErrorString>") after printing
//                              the file and line, as CUDA_CHECK does
//   qwen::CudaContext       -> qwen::HipContext: owns one stream created with
//                              hipStreamCreate; stream(), synchronize()
// The reference's context also creates a cuBLAS handle (handle(),
// cuda_utils.hpp:53-57) that no reference code calls; it has no counterpart
// here. Header-only; the library itself does not use it.
#ifndef QWEN35_HIP_CONTEXT_HPP
#define QWEN35_HIP_CONTEXT_HPP

#include <hip/hip_runtime.h>

#include <iostream>
#include <stdexcept>
#include <string>

#define QWEN_HIP_CHECK(call)                                                                                 \
    do {                                                                                                     \
        const hipError_t qwen_hip_err_ = (call);                                                             \
        if (qwen_hip_err_ != hipSuccess) {                                                                   \
            std::cerr << "HIP Error at " << __FILE__ << ":" << __LINE__ << " - "                             \
                      << hipGetErrorString(qwen_hip_err_) << std::endl;                                      \
            throw std::runtime_error("HIP Error: " + std::string(hipGetErrorString(qwen_hip_err_)));         \
        }                                                                                                    \
    } while (0)

namespace qwen {

class HipContext {
public:
    HipContext() { QWEN_HIP_CHECK(hipStreamCreate(&stream_)); }
    ~HipContext() {
        if (stream_) (void)hipStreamDestroy(stream_);
    }
    HipContext(const HipContext&) = delete;
    HipContext& operator=(const HipContext&) = delete;

    hipStream_t stream() const { return stream_; }
    void synchronize() const { QWEN_HIP_CHECK(hipStreamSynchronize(stream_)); }

private:
    hipStream_t stream_ = nullptr;
};

}  // namespace qwen

#endif  // QWEN35_HIP_CONTEXT_HPP
