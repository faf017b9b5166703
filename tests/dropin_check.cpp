// Drop-in check: compiles the way the reference's layer code does — against
// ops.hpp / rope.hpp / gdn.hpp / matmul_q4.hpp plus the layers' own forward
// declarations (src/layer_attn.cpp:11, src/layer_moe.cpp:10,12, here with
// hipStream_t) — and repeats the reference's host-side checks of the in-scope
// kernels (tests/kernel_tests.cu: dequant layouts :116-223, RMSNorm :301-325,
// RoPE :327-359) through the namespace-qwen API.
//
//   dropin_check --cpu   exception paths only (no device needed)
//   dropin_check --gpu   the numeric checks on the default HIP device
// Exit status 0 = all checks passed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <unistd.h>
#include <stdexcept>
#include <string>
#include <vector>

#include "gdn.hpp"
#include "loader_gguf.hpp"
#include "matmul_q4.hpp"
#include "ops.hpp"
#include "rope.hpp"

namespace qwen {
// The reference layers declare these themselves instead of including a header.
void attn_head_norm(float* x, const float* weight, int heads, int dim, float eps, hipStream_t stream);
void moe_silu_mul(const float* gate, const float* up, float* hidden, int dim, hipStream_t stream);
void moe_shared_add(float* accum, const float* shared_out, const float* sgate, int dim, hipStream_t stream);
}  // namespace qwen

namespace {

int g_failures = 0;

void expect(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) ++g_failures;
}

template <class F>
void expect_throw(F&& f, const std::string& message, const std::string& what) {
    try {
        f();
        expect(false, what + " (no exception)");
    } catch (const std::runtime_error& e) {
        expect(message == e.what(), what + " -> \"" + e.what() + "\"");
    }
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <class T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    hip_ok(hipMalloc(&d, h.size() * sizeof(T)), "hipMalloc");
    hip_ok(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    return d;
}

template <class T>
std::vector<T> to_host(const T* d, size_t n) {
    std::vector<T> h(n);
    hip_ok(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return h;
}

float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    float e = 0.f;
    for (size_t i = 0; i < a.size(); ++i) e = std::fmax(e, std::fabs(a[i] - b[i]));
    return e;
}

// ------------------------------------------------------------------ CPU checks

// ------------------------------------------------------------------ GGUF
// A small GGUF v3 file: a few metadata kinds and a Q4_K "token_embd.weight"
// [256 x 4] of known blocks (d = 1, dmin = 0, scale 1, quant = element % 16)
// plus blk.0 / blk.1 norm weights, so the loader can be driven the way the
// reference's main.cpp / model.cpp / tokenizer.cpp drive it.
struct GgufBytes {
    std::vector<uint8_t> b;
    template <class T>
    void put(T v) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
        b.insert(b.end(), p, p + sizeof(T));
    }
    void str(const std::string& s) {
        put<uint64_t>(s.size());
        b.insert(b.end(), s.begin(), s.end());
    }
    void pad(size_t a) {
        while (b.size() % a) b.push_back(0);
    }
};

std::vector<uint8_t> q4k_known_block() {
    std::vector<uint8_t> blk(144, 0);
    blk[0] = 0x00;
    blk[1] = 0x3c;   // d = 1.0 (fp16), dmin = 0
    for (int j = 0; j < 4; ++j) blk[4 + j] = 1;   // sub-blocks 0..3: scale 1, min 0
    for (int j = 8; j < 12; ++j) blk[4 + j] = 1;  // sub-blocks 4..7: low nibbles of bytes 8..11
    for (int i = 0; i < 128; ++i) blk[16 + i] = static_cast<uint8_t>((i % 16) | ((i % 16) << 4));
    return blk;
}

std::string write_gguf(uint32_t version) {
    GgufBytes f;
    f.put<uint32_t>(0x46554747u);
    f.put<uint32_t>(version);
    f.put<uint64_t>(3);   // tensors
    f.put<uint64_t>(4);   // metadata
    f.str("general.architecture");
    f.put<uint32_t>(8);
    f.str("qwen35moe");
    f.str("qwen35moe.full_attention_interval");
    f.put<uint32_t>(4);
    f.put<uint32_t>(4);
    f.str("qwen35moe.rope.freq_base");
    f.put<uint32_t>(6);
    f.put<float>(10000000.0f);
    f.str("tokenizer.ggml.tokens");
    f.put<uint32_t>(9);
    f.put<uint32_t>(8);
    f.put<uint64_t>(2);
    f.str("hello");
    f.str("world");
    const char* names[3] = {"token_embd.weight", "blk.0.attn_norm.weight", "blk.1.attn_norm.weight"};
    uint64_t off = 0;
    for (int i = 0; i < 3; ++i) {
        f.str(names[i]);
        if (i == 0) {
            f.put<uint32_t>(2);
            f.put<int64_t>(256);
            f.put<int64_t>(4);
            f.put<uint32_t>(12);   // Q4_K
        } else {
            f.put<uint32_t>(1);
            f.put<int64_t>(8);
            f.put<uint32_t>(0);    // F32
        }
        f.put<uint64_t>(off);
        off += i == 0 ? 4 * 144 : 32;
    }
    f.pad(32);
    const std::vector<uint8_t> blk = q4k_known_block();
    for (int r = 0; r < 4; ++r) f.b.insert(f.b.end(), blk.begin(), blk.end());
    for (int i = 0; i < 16; ++i) f.put<float>(1.0f + i);
    const std::string path = "/tmp/qwen35_dropin_" + std::to_string(version) + "_" + std::to_string(getpid()) + ".gguf";
    FILE* fp = std::fopen(path.c_str(), "wb");
    if (!fp) throw std::runtime_error("cannot write " + path);
    std::fwrite(f.b.data(), 1, f.b.size(), fp);
    std::fclose(fp);
    return path;
}

void gguf_cpu_checks() {
    qwen::GgufLoader l;
    expect(!l.open("/nonexistent/model.gguf"), "GgufLoader::open missing file returns false");
    const std::string p = write_gguf(3);
    expect(l.open(p), "GgufLoader::open");
    expect(l.version() == 3 && l.tensor_count() == 3 && l.metadata_count() == 4, "GGUF header counts");
    expect(l.get_meta_string("general.architecture") == "qwen35moe", "get_meta_string");
    expect(l.get_meta_int("qwen35moe.full_attention_interval", 1) == 4, "get_meta_int");
    expect(l.get_meta_float("qwen35moe.rope.freq_base", 0) == 10000000.0, "get_meta_float");
    expect(l.get_meta_int("absent.key", -7) == -7 && l.get_meta_int("general.architecture", 5) == 5,
           "get_meta_int default and unparsable text");
    const auto* tokens = l.get_meta_array("tokenizer.ggml.tokens");
    expect(tokens && tokens->size() == 2 && (*tokens)[1] == "world", "get_meta_array");
    const qwen::QuantTensor* emb = l.get_tensor("token_embd.weight");
    expect(emb && emb->type == qwen::GgmlType::Q4_K && emb->shape.size() == 2 && emb->shape[0] == 256 &&
               emb->shape[1] == 4 && emb->num_elements == 1024 && emb->size_bytes == 576 && !emb->device_ptr,
           "get_tensor token_embd.weight");
    expect(!l.get_tensor("output.weight") && l.tensors().size() == 3 && l.total_vram_bytes() == 0, "tensors()");
    expect(qwen::tensor_block_index("blk.12.ffn_up.weight") == 12 && qwen::tensor_block_index("token_embd.weight") == -1 &&
               qwen::tensor_block_index("blk..x") == -1 && qwen::tensor_block_index("blk.1a.x") == -1,
           "tensor_block_index");
    std::remove(p.c_str());
    const std::string p1 = write_gguf(1);
    expect_throw([&] { l.open(p1); }, "unsupported GGUF version 1", "GgufLoader::open version 1 throws");
    std::remove(p1.c_str());
}

void gguf_gpu_checks() {
    qwen::GgufLoader l;
    const std::string p = write_gguf(3);
    expect(l.open(p) && l.load_tensors_to_gpu(1), "load_tensors_to_gpu(base_layer_count = 1)");
    const qwen::QuantTensor* emb = l.get_tensor("token_embd.weight");
    expect(emb->device_ptr && l.get_tensor("blk.0.attn_norm.weight")->device_ptr &&
               !l.get_tensor("blk.1.attn_norm.weight")->device_ptr && l.total_vram_bytes() == 576 + 32,
           "blk.1 stays on disk");
    // src/model.cpp:190: the embedding row of a token straight from the loaded table
    float* d_out = nullptr;
    hip_ok(hipMalloc(&d_out, 256 * sizeof(float)), "hipMalloc");
    qwen::dequantize_row(*emb, d_out, 3, 256);
    std::vector<float> out(256);
    hip_ok(hipMemcpy(out.data(), d_out, 256 * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    bool ok = true;
    for (int i = 0; i < 256; ++i) ok = ok && out[i] == static_cast<float>(i % 16);
    expect(ok, "dequantize_row of a loaded GGUF table");
    (void)hipFree(d_out);
    l.unload_gpu();
    expect(!l.get_tensor("token_embd.weight")->device_ptr && l.total_vram_bytes() == 0, "unload_gpu");
    std::remove(p.c_str());
}

void cpu_checks() {
    gguf_cpu_checks();
    std::vector<float> dummy(16);
    expect_throw([&] { qwen::rope_forward(nullptr, 3, 2, 8, 4, 100.f); }, "invalid RoPE arguments", "rope null");
    expect_throw([&] { qwen::rope_forward(dummy.data(), 3, 2, 8, 3, 100.f); }, "invalid RoPE arguments", "rope odd");
    expect_throw([&] { qwen::rope_forward(dummy.data(), 3, 2, 8, 10, 100.f); }, "invalid RoPE arguments",
                 "rope rd > hd");
    expect_throw([&] { qwen::rope_forward(dummy.data(), -1, 2, 8, 4, 100.f); }, "invalid RoPE arguments",
                 "rope pos < 0");
    expect_throw([&] { qwen::rope_forward(dummy.data(), 3, 2, 8, 4, 0.f); }, "invalid RoPE arguments",
                 "rope theta 0");

    qwen::QuantTensor t;
    t.name = "token_embd.weight";
    t.type = qwen::GgmlType::Q4_1;  // no dequant path, as in the reference
    t.num_elements = 512;
    t.device_ptr = dummy.data();
    expect_throw([&] { qwen::dequantize_row(t, dummy.data(), 0, 256); }, "cannot dequantize tensor 'token_embd.weight'",
                 "dequantize_row unsupported type");
    t.type = qwen::GgmlType::Q4_K;
    t.device_ptr = nullptr;
    expect_throw([&] { qwen::dequantize_row(t, dummy.data(), 0, 256); }, "cannot dequantize tensor 'token_embd.weight'",
                 "dequantize_row unloaded tensor");
    t.device_ptr = dummy.data();
    expect_throw([&] { qwen::dequantize_row(t, dummy.data(), 2, 256); }, "row is outside tensor 'token_embd.weight'",
                 "dequantize_row row past the end");
    expect_throw([&] { qwen::dequantize_row(t, dummy.data(), -1, 256); }, "row is outside tensor 'token_embd.weight'",
                 "dequantize_row negative row");
    expect(qwen::matmul_type_supported(qwen::GgmlType::Q6_K) && !qwen::matmul_type_supported(qwen::GgmlType::Q2_K),
           "matmul_type_supported");

    // matmul_dispatch validation, in the reference's order (src/cuda/matmul_q4.cu:187-195)
    qwen::QuantTensor wq;
    wq.name = "blk.0.attn_q.weight";
    wq.type = qwen::GgmlType::Q4_K;
    wq.num_elements = 4 * 512;
    wq.device_ptr = nullptr;
    expect_throw([&] { qwen::matmul_dispatch(wq, dummy.data(), dummy.data(), 4, 512); },
                 "tensor 'blk.0.attn_q.weight' is not loaded", "matmul_dispatch unloaded tensor");
    wq.device_ptr = dummy.data();
    wq.type = qwen::GgmlType::Q4_1;
    expect_throw([&] { qwen::matmul_dispatch(wq, dummy.data(), dummy.data(), 4, 512); },
                 "unsupported GGML type for tensor 'blk.0.attn_q.weight'", "matmul_dispatch unsupported type");
    wq.type = qwen::GgmlType::Q4_K;
    expect_throw([&] { qwen::matmul_dispatch(wq, dummy.data(), dummy.data(), 5, 512); },
                 "GEMV shape exceeds tensor 'blk.0.attn_q.weight'", "matmul_dispatch rows past the end");
    expect_throw([&] { qwen::matmul_dispatch(wq, dummy.data(), dummy.data(), 2, 512, nullptr, 1024 + 256); },
                 "GEMV shape exceeds tensor 'blk.0.attn_q.weight'", "matmul_dispatch offset past the end");
    expect_throw([&] { qwen::matmul_dispatch(wq, dummy.data(), dummy.data(), 0, 512); },
                 "GEMV shape exceeds tensor 'blk.0.attn_q.weight'", "matmul_dispatch M = 0");
    // the fused MoE entry points name the tensor the reference's separate calls would
    qwen::QuantTensor wg = wq, wu = wq, wd = wq, wsd = wq;
    wg.name = "blk.0.ffn_gate_exps.weight";
    wu.name = "blk.0.ffn_up_exps.weight";
    wd.name = "blk.0.ffn_down_exps.weight";
    wsd.name = "blk.0.ffn_down_shexp.weight";
    wg.num_elements = wu.num_elements = wd.num_elements = 4 * 2 * 512;    // 4 experts of 2 x 512
    wsd.num_elements = 2 * 512;
    wu.device_ptr = nullptr;
    const int32_t* no_ids = nullptr;
    expect_throw([&] { qwen::moe_expert_gate_up(wg, wu, 1024, 4, no_ids, 2, dummy.data(), dummy.data(), dummy.data(),
                                                2, 512); },
                 "tensor 'blk.0.ffn_up_exps.weight' is not loaded", "moe_expert_gate_up unloaded up tensor");
    wu.device_ptr = dummy.data();
    expect_throw([&] { qwen::moe_expert_gate_up(wg, wu, 1024, 4, no_ids, 2, dummy.data(), dummy.data(), dummy.data(),
                                                3, 512); },
                 "GEMV shape exceeds tensor 'blk.0.ffn_gate_exps.weight'", "moe_expert_gate_up rows past the expert");
    wsd.device_ptr = nullptr;
    expect_throw([&] { qwen::moe_down_combine(wd, 1024, 4, no_ids, dummy.data(), 2, dummy.data(), 512, wsd,
                                              dummy.data(), 512, dummy.data(), dummy.data(), 2, dummy.data(),
                                              1 << 20); },
                 "tensor 'blk.0.ffn_down_shexp.weight' is not loaded", "moe_down_combine unloaded shared tensor");
    wsd.device_ptr = dummy.data();
    expect_throw([&] { qwen::moe_down_combine(wd, 1024, 4, no_ids, dummy.data(), 2, dummy.data(), 512, wsd,
                                              dummy.data(), 1024, dummy.data(), dummy.data(), 2, dummy.data(),
                                              1 << 20); },
                 "GEMV shape exceeds tensor 'blk.0.ffn_down_shexp.weight'", "moe_down_combine shared rows past the end");
    expect_throw([&] { qwen::moe_down_combine(wd, 1024, 4, no_ids, dummy.data(), 2, dummy.data(), 1024, wsd,
                                              dummy.data(), 512, dummy.data(), dummy.data(), 2, dummy.data(),
                                              1 << 20); },
                 "GEMV shape exceeds tensor 'blk.0.ffn_down_exps.weight'", "moe_down_combine expert rows past the end");
    qwen::QuantTensor wsg = wq, wsu = wq;
    wsg.name = "blk.0.ffn_gate_shexp.weight";
    wsu.name = "blk.0.ffn_up_shexp.weight";
    wsg.num_elements = wsu.num_elements = 2 * 512;
    wsu.device_ptr = nullptr;
    expect_throw([&] { qwen::moe_expert_swiglu(wg, wu, 1024, 4, no_ids, 2, 2, &wsg, &wsu, 2, dummy.data(), 512,
                                               dummy.data(), dummy.data(), dummy.data(), 1 << 20); },
                 "tensor 'blk.0.ffn_up_shexp.weight' is not loaded", "moe_expert_swiglu unloaded shared up");
    wsu.device_ptr = dummy.data();
    expect_throw([&] { qwen::moe_expert_swiglu(wg, wu, 1024, 4, no_ids, 2, 3, &wsg, &wsu, 2, dummy.data(), 512,
                                               dummy.data(), dummy.data(), dummy.data(), 1 << 20); },
                 "GEMV shape exceeds tensor 'blk.0.ffn_gate_exps.weight'", "moe_expert_swiglu routed rows past the end");
    expect_throw([&] { qwen::moe_expert_swiglu(wg, wu, 1024, 4, no_ids, 2, 2, &wsg, &wsu, 3, dummy.data(), 512,
                                               dummy.data(), dummy.data(), dummy.data(), 1 << 20); },
                 "GEMV shape exceeds tensor 'blk.0.ffn_gate_shexp.weight'", "moe_expert_swiglu shared rows past the end");
    expect(qwen::calculate_tensor_bytes(qwen::GgmlType::Q4_K, 2048) == 8 * 144 &&
               qwen::calculate_tensor_bytes(qwen::GgmlType::Q6_K, 100) == 0,
           "calculate_tensor_bytes");
    // zero-size calls are no-ops and never touch the device
    qwen::rmsnorm_forward(nullptr, nullptr, nullptr, 0);
    qwen::residual_add(nullptr, nullptr, nullptr, 0);
    expect(true, "zero-size calls return");
}

// ------------------------------------------------------------------ GPU checks
// Block fixtures: the byte patterns of tests/kernel_tests.cu:116-223, expected
// values by the test's own closed forms (d = 1, dmin = 0.5).
void half_one(std::vector<uint8_t>& b, size_t off) {
    b[off] = 0x00;
    b[off + 1] = 0x3c;
}

void scale_min(int j, const uint8_t* s, int& d, int& m) {
    if (j < 4) {
        d = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        d = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

void check_block(qwen::GgmlType type, const char* name, const std::vector<uint8_t>& raw,
                 const std::vector<float>& expected) {
    qwen::QuantTensor t;
    t.name = name;
    t.type = type;
    t.num_elements = expected.size();
    t.size_bytes = raw.size();
    t.device_ptr = to_device(raw);
    float* out = nullptr;
    hip_ok(hipMalloc(&out, expected.size() * sizeof(float)), "hipMalloc");
    qwen::dequantize_row(t, out, 0, static_cast<int>(expected.size()));
    const std::vector<float> got = to_host(out, expected.size());
    expect(max_abs_diff(got, expected) < 1e-6f, std::string("dequantize_row ") + name + " fixture");
    // matmul_dispatch over the same block as one row: x = 1, 2, 1, 2, ... gives
    // y = sum(w) + sum(w at odd k).
    std::vector<float> x(expected.size());
    double ref = 0.0, mag = 0.0;
    for (size_t k = 0; k < x.size(); ++k) {
        x[k] = (k & 1) ? 2.0f : 1.0f;
        ref += static_cast<double>(expected[k]) * x[k];
        mag += std::fabs(static_cast<double>(expected[k]) * x[k]);
    }
    float* dx = to_device(x);
    qwen::matmul_dispatch(t, dx, out, 1, static_cast<int>(x.size()));
    const float y = to_host(out, 1)[0];
    expect(std::fabs(y - ref) <= 1e-5 * mag, std::string("matmul_dispatch ") + name + " fixture row");
    (void)hipFree(dx);
    (void)hipFree(out);
    (void)hipFree(t.device_ptr);
}

void gpu_checks() {
    gguf_gpu_checks();
    const uint8_t packed[12] = {0xc1, 0x82, 0x43, 0x04, 0x85, 0x46, 0x07, 0xc8, 0x91, 0x2a, 0xb3, 0x4c};
    {  // Q4_K
        std::vector<uint8_t> b(144);
        half_one(b, 0);
        b[3] = 0x38;
        std::memcpy(&b[4], packed, 12);
        for (int j = 0; j < 128; ++j) b[16 + j] = static_cast<uint8_t>(((j * 11 + 5) & 15) << 4 | ((j * 3 + 1) & 15));
        std::vector<float> r(256);
        for (int i = 0; i < 256; ++i) {
            int sc, mn;
            scale_min(i / 32, &b[4], sc, mn);
            const uint8_t q = b[16 + (i / 64) * 32 + i % 32];
            r[i] = static_cast<float>(sc * ((i % 64) < 32 ? (q & 15) : (q >> 4))) - 0.5f * mn;
        }
        check_block(qwen::GgmlType::Q4_K, "Q4_K", b, r);
    }
    {  // Q6_K
        std::vector<uint8_t> b(210);
        for (int j = 0; j < 128; ++j) b[j] = static_cast<uint8_t>(j * 29 + 7);
        for (int j = 0; j < 64; ++j) b[128 + j] = static_cast<uint8_t>(j * 43 + 19);
        for (int j = 0; j < 16; ++j) b[192 + j] = static_cast<uint8_t>(static_cast<int8_t>(j * 9 - 61));
        half_one(b, 208);
        std::vector<float> r(256);
        for (int i = 0; i < 256; ++i) {
            const int half = i / 128, rr = i % 128, lane = rr & 31, quarter = rr / 32;
            const uint8_t qlb = b[half * 64 + (quarter & 1) * 32 + lane];
            const int lo = quarter < 2 ? (qlb & 15) : (qlb >> 4);
            const int hi = (b[128 + half * 32 + lane] >> (2 * quarter)) & 3;
            r[i] = static_cast<float>(static_cast<int8_t>(b[192 + half * 8 + lane / 16 + 2 * quarter]) *
                                      ((lo | (hi << 4)) - 32));
        }
        check_block(qwen::GgmlType::Q6_K, "Q6_K", b, r);
    }
    {  // Q8_0
        std::vector<uint8_t> b(34);
        half_one(b, 0);
        std::vector<float> r(32);
        for (int j = 0; j < 32; ++j) {
            const int8_t v = static_cast<int8_t>(j * 7 - 101);
            b[2 + j] = static_cast<uint8_t>(v);
            r[j] = v;
        }
        check_block(qwen::GgmlType::Q8_0, "Q8_0", b, r);
    }
    {  // RMSNorm closed form, tests/kernel_tests.cu:301-325
        const std::vector<float> x = {3.f, 4.f}, w = {2.f, .5f};
        const float r = 1.f / std::sqrt(12.5f + 1e-6f);
        float *dx = to_device(x), *dw = to_device(w), *dy = nullptr;
        hip_ok(hipMalloc(&dy, 2 * sizeof(float)), "hipMalloc");
        qwen::rmsnorm_forward(dx, dw, dy, 2, 1e-6f);
        expect(max_abs_diff(to_host(dy, 2), {x[0] * r * w[0], x[1] * r * w[1]}) < 1e-5f, "rmsnorm_forward fixture");
        (void)hipFree(dx);
        (void)hipFree(dw);
        (void)hipFree(dy);
    }
    {  // RoPE fixture, tests/kernel_tests.cu:327-359
        const int heads = 2, hd = 8, rd = 4, pos = 3;
        const float base = 100.f;
        std::vector<float> x(heads * hd);
        for (size_t i = 0; i < x.size(); ++i) x[i] = .125f * static_cast<float>(i + 1);
        std::vector<float> e = x;
        for (int h = 0; h < heads; ++h)
            for (int i = 0; i < rd / 2; ++i) {
                const float th = pos / std::pow(base, 2.f * i / rd);
                const float c = std::cos(th), s = std::sin(th);
                const float a = x[h * hd + i], b = x[h * hd + i + rd / 2];
                e[h * hd + i] = a * c - b * s;
                e[h * hd + i + rd / 2] = b * c + a * s;
            }
        float* d = to_device(x);
        qwen::rope_forward(d, pos, heads, hd, rd, base);
        expect(max_abs_diff(to_host(d, x.size()), e) < 2e-6f, "rope_forward fixture");
        (void)hipFree(d);
    }
    {  // attn_head_norm + moe_silu_mul + moe_shared_add + gdn_conv_step through the layer declarations
        std::vector<float> x(2 * 256), w(256, 1.f);
        for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * static_cast<float>(i)) * 2.f;
        float *dx = to_device(x), *dw = to_device(w);
        qwen::attn_head_norm(dx, dw, 2, 256, 1e-6f, nullptr);
        const std::vector<float> y = to_host(dx, x.size());
        double ms = 0;
        for (int i = 0; i < 256; ++i) ms += static_cast<double>(y[i]) * y[i];
        expect(std::fabs(ms / 256 - 1.0) < 1e-4, "attn_head_norm unit rms");
        std::vector<float> g = {0.f, 1.f, -2.f, 30.f}, u = {5.f, 2.f, 1.f, 0.5f};
        float *dg = to_device(g), *du = to_device(u), *dh = nullptr;
        hip_ok(hipMalloc(&dh, 4 * sizeof(float)), "hipMalloc");
        qwen::moe_silu_mul(dg, du, dh, 4, nullptr);
        const std::vector<float> h = to_host(dh, 4);
        bool ok = true;
        for (int i = 0; i < 4; ++i) {
            const float ref = g[i] / (1.f + std::exp(-g[i])) * u[i];
            ok = ok && std::fabs(h[i] - ref) <= 1e-5f * std::fmax(1.f, std::fabs(ref));
        }
        expect(ok, "moe_silu_mul");
        std::vector<float> acc = {1.f, 2.f, 3.f, 4.f}, gate = {0.f};
        float *da = to_device(acc), *dgt = to_device(gate);
        qwen::moe_shared_add(da, dg, dgt, 4, nullptr);  // sigmoid(0) = 1/2
        const std::vector<float> a2 = to_host(da, 4);
        expect(a2[0] == 1.f && a2[1] == 2.5f && a2[2] == 2.f && a2[3] == 19.f, "moe_shared_add");
        // conv step with one-hot taps on the newest input: y = silu(x), history shifts
        const int C = 8;
        std::vector<float> cx(C), cw(C * 4, 0.f), hist(C * 3);
        for (int c = 0; c < C; ++c) {
            cx[c] = 0.5f * c - 1.f;
            cw[c * 4 + 3] = 1.f;
            for (int j = 0; j < 3; ++j) hist[c * 3 + j] = 10.f * c + j;
        }
        float *dcx = to_device(cx), *dcw = to_device(cw), *dhist = to_device(hist), *dcy = nullptr;
        hip_ok(hipMalloc(&dcy, C * sizeof(float)), "hipMalloc");
        qwen::gdn_conv_step(dcx, dcw, dhist, dcy, C, 4, nullptr);
        const std::vector<float> cy = to_host(dcy, C), h2 = to_host(dhist, C * 3);
        ok = true;
        for (int c = 0; c < C; ++c) {
            const float ref = cx[c] / (1.f + std::exp(-cx[c]));
            ok = ok && std::fabs(cy[c] - ref) <= 1e-5f * std::fmax(1.f, std::fabs(ref));
            ok = ok && h2[c * 3] == hist[c * 3 + 1] && h2[c * 3 + 1] == hist[c * 3 + 2] && h2[c * 3 + 2] == cx[c];
        }
        expect(ok, "gdn_conv_step one-hot taps and history shift");
        for (float* p : {dx, dw, dg, du, dh, da, dgt, dcx, dcw, dhist, dcy}) (void)hipFree(p);
    }
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

}  // namespace

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    try {
        cpu_checks();
        if (gpu) gpu_checks();
    } catch (const std::exception& e) {
        std::printf("FAIL unexpected exception: %s\n", e.what());
        return 2;
    }
    std::printf("%s: %d failure(s)\n", gpu ? "cpu+gpu checks" : "cpu checks", g_failures);
    return g_failures == 0 ? 0 : 1;
}
