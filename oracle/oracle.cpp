// CPU oracle for the fused per-layer kernels -- TEST INFRASTRUCTURE ONLY.
//
// Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
// never by the product library. Each function restates one reference kernel
// (sahan974/qwen-3.5-cuda, paths relative to its root) with that kernel's float
// association. The build uses -ffp-contract=off so that the host compiler never
// fuses a multiply and an add behind the restatement's back; the one place where
// the reference relies on nvcc's default multiply-add contraction (the GDN conv
// accumulation) calls fmaf explicitly.
//
// Math functions: the reference calls CUDA's expf / rsqrtf / cosf / sinf. The
// oracle evaluates each in double precision and rounds to float once, so its
// value is within one float ulp of the exact function value. (Built with
// ORACLE_FP32_MATH, as liboracle_fp32.so, the same source evaluates them and the
// sums of squares in float instead: that build is only the timed CPU baseline.)
// Sums of squares: the reference's order is fixed by its launch shape (strided
// per-thread partials, then a shuffle tree). The oracle accumulates the exact
// squares in double and rounds the total once, which is closer to the exact sum
// than any fp32 order; kernels are compared against it with a tolerance.

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

namespace {

inline float bits_to_f32(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline uint32_t f32_to_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

// Split [0, n) into contiguous chunks, one per thread, each thread taking at
// least kMinItemsPerThread items (a thread costs tens of microseconds to start).
constexpr int64_t kMinItemsPerThread = 16;

void parallel_for(int64_t n, int threads, const std::function<void(int64_t, int64_t)>& fn) {
    const int64_t t = std::min<int64_t>(threads, n / kMinItemsPerThread);
    if (t <= 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(static_cast<size_t>(t));
    for (int64_t k = 0; k < t; ++k) {
        const int64_t lo = n * k / t;
        const int64_t hi = n * (k + 1) / t;
        pool.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto& th : pool) th.join();
}

#ifdef ORACLE_FP32_MATH
// The CPU-baseline build (liboracle_fp32.so, timed by bench.py, never the
// checker): float math as the reference's host-side checks write it
// (tests/kernel_tests.cu:305-308: 1.f / std::sqrt(float), float products) --
// the C library's float expf / sqrtf / cosf / sinf, and squares summed in one
// float accumulator in index order.
inline float sum_squares(const float* x, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += x[i] * x[i];
    return s;
}

inline float exp_f(float x) { return std::exp(x); }
inline float rsqrt_f(float x) { return 1.0f / std::sqrt(x); }
inline float cos_f(float x) { return std::cos(x); }
inline float sin_f(float x) { return std::sin(x); }
#else
// Sum of squares of n floats: exact squares accumulated in double, rounded once.
inline float sum_squares(const float* x, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += static_cast<double>(x[i]) * static_cast<double>(x[i]);
    return static_cast<float>(s);
}

inline float exp_f(float x) { return static_cast<float>(std::exp(static_cast<double>(x))); }
inline float rsqrt_f(float x) { return static_cast<float>(1.0 / std::sqrt(static_cast<double>(x))); }
inline float cos_f(float x) { return static_cast<float>(std::cos(static_cast<double>(x))); }
inline float sin_f(float x) { return static_cast<float>(std::sin(static_cast<double>(x))); }
#endif

}  // namespace

extern "C" {

// ---------------------------------------------------------------- helpers

// silu(x) = x / (1 + expf(-x))            -- src/cuda/ops.cu:9-11, moe.cu:63
float or_silu(float x) { return x / (1.0f + exp_f(-x)); }

// sigmoid(g) = 1 / (1 + expf(-g))         -- src/cuda/moe.cu:94, gdn.cu:93
float or_sigmoid(float x) { return 1.0f / (1.0f + exp_f(-x)); }

// rsqrtf(x), evaluated exactly and rounded once.
float or_rsqrt(float x) { return rsqrt_f(x); }

// IEEE binary16 -> binary32, exact (subnormals included); NaNs stay NaN with
// the quiet bit set.                     -- src/cuda/matmul_q4.cu:13-16
float or_half_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1f;
    const uint32_t man = h & 0x3ff;
    if (exp == 0) {
        const float mag = std::ldexp(static_cast<float>(man), -24);
        return sign ? -mag : mag;
    }
    if (exp == 31) {
        return bits_to_f32(sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0u));
    }
    return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

float or_bf16_to_float(uint16_t b) { return bits_to_f32(static_cast<uint32_t>(b) << 16); }

// binary32 -> bf16, round to nearest even; NaN -> quiet NaN with the same sign.
uint16_t or_float_to_bf16(float f) {
    uint32_t u = f32_to_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// 6-bit (scale, min) pair j of a K-quant block's 12 packed bytes.
//                                         -- src/cuda/matmul_q4.cu:18-26
void or_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = static_cast<uint8_t>((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = static_cast<uint8_t>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static inline float fp16_at(const uint8_t* p) {
    return or_half_to_float(static_cast<uint16_t>(p[0] | (p[1] << 8)));
}

// Element `index` of a GGML tensor of `type`.  -- src/cuda/matmul_q4.cu:30-129
float or_dequant(const uint8_t* data, int type, uint64_t index) {
    switch (type) {
        case 0: {  // F32
            float v;
            std::memcpy(&v, data + index * 4, 4);
            return v;
        }
        case 1:  // F16
            return fp16_at(data + index * 2);
        case 30:  // BF16
            return or_bf16_to_float(static_cast<uint16_t>(data[index * 2] | (data[index * 2 + 1] << 8)));
        case 8: {  // Q8_0: 34-byte blocks of 32
            const uint8_t* b = data + (index / 32) * 34;
            return fp16_at(b) * static_cast<float>(static_cast<int8_t>(b[2 + index % 32]));
        }
        case 2: {  // Q4_0: 18-byte blocks of 32
            const uint8_t* b = data + (index / 32) * 18;
            const int i = static_cast<int>(index % 32);
            const int q = (i < 16) ? (b[2 + i] & 15) : (b[2 + i - 16] >> 4);
            return fp16_at(b) * static_cast<float>(q - 8);
        }
        case 6: {  // Q5_0: 22-byte blocks of 32
            const uint8_t* b = data + (index / 32) * 22;
            const int i = static_cast<int>(index % 32);
            const uint32_t qh = static_cast<uint32_t>(b[2]) | (static_cast<uint32_t>(b[3]) << 8) |
                                (static_cast<uint32_t>(b[4]) << 16) | (static_cast<uint32_t>(b[5]) << 24);
            const int j = i & 15;
            const int high = (i < 16) ? ((qh >> j) & 1) : ((qh >> (j + 16)) & 1);
            const int low = (i < 16) ? (b[6 + j] & 15) : (b[6 + j] >> 4);
            return fp16_at(b) * static_cast<float>((low | (high << 4)) - 16);
        }
        case 12:
        case 13: {  // Q4_K (144 B) / Q5_K (176 B), blocks of 256
            const int block_bytes = (type == 12) ? 144 : 176;
            const uint8_t* b = data + (index / 256) * block_bytes;
            const int i = static_cast<int>(index % 256);
            const float d = fp16_at(b);
            const float dmin = fp16_at(b + 2);
            uint8_t sc, mn;
            or_scale_min_k4(i / 32, b + 4, &sc, &mn);
            const int group64 = i / 64;
            const int in64 = i % 64;
            const int lane = in64 & 31;
            int value;
            if (type == 12) {
                const uint8_t q = b[16 + group64 * 32 + lane];
                value = (in64 < 32) ? (q & 15) : (q >> 4);
            } else {
                const uint8_t q = b[48 + group64 * 32 + lane];
                const uint8_t mask = static_cast<uint8_t>(1u << (2 * group64 + (in64 >= 32)));
                value = ((in64 < 32) ? (q & 15) : (q >> 4)) + ((b[16 + lane] & mask) ? 16 : 0);
            }
            // ((d * sc) * q) - (dmin * m), left to right as in matmul_q4.cu:95,101
            return d * static_cast<float>(sc) * static_cast<float>(value) - dmin * static_cast<float>(mn);
        }
        case 14: {  // Q6_K: 210-byte blocks of 256
            const uint8_t* b = data + (index / 256) * 210;
            const int i = static_cast<int>(index % 256);
            const uint8_t* ql = b;
            const uint8_t* qh = b + 128;
            const int8_t* scales = reinterpret_cast<const int8_t*>(b + 192);
            const int half = i / 128;
            const int r = i % 128;
            const int lane = r & 31;
            const int quarter = r / 32;
            const uint8_t lo = (quarter == 0)   ? (ql[half * 64 + lane] & 15)
                               : (quarter == 1) ? (ql[half * 64 + 32 + lane] & 15)
                               : (quarter == 2) ? (ql[half * 64 + lane] >> 4)
                                                : (ql[half * 64 + 32 + lane] >> 4);
            const uint8_t hi = (qh[half * 32 + lane] >> (2 * quarter)) & 3;
            const int si = half * 8 + (lane / 16) + 2 * quarter;
            // (d * sc) * (q - 32): the association fixes the sign of zero (matmul_q4.cu:125)
            return fp16_at(b + 208) * static_cast<float>(scales[si]) *
                   static_cast<float>(static_cast<int>(lo | (hi << 4)) - 32);
        }
        default:
            return 0.0f;
    }
}

int or_type_supported(int t) {
    return t == 0 || t == 1 || t == 30 || t == 2 || t == 6 || t == 8 || t == 12 || t == 13 || t == 14;
}

// ---------------------------------------------------------------- ops.hpp

// out = (x * r) * w,  r = rsqrtf(sum(x^2)/N + eps)   -- src/cuda/ops.cu:25-65
void or_rmsnorm_rows(const float* x, const float* w, float* out, int rows, int n, float eps,
                     int threads) {
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            const float* xr = x + t * n;
            float* o = out + t * n;
            const float r = or_rsqrt(sum_squares(xr, n) / static_cast<float>(n) + eps);
            for (int i = 0; i < n; ++i) o[i] = xr[i] * r * w[i];
        }
    });
}

// out = ((x * r) * w) * silu(gate)                   -- src/cuda/ops.cu:68-109
void or_rmsnorm_gated_rows(const float* x, const float* gate, const float* w, float* out, int rows,
                           int n, float eps, int threads) {
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            const float* xr = x + t * n;
            const float* g = gate + t * n;
            float* o = out + t * n;
            const float r = or_rsqrt(sum_squares(xr, n) / static_cast<float>(n) + eps);
            for (int i = 0; i < n; ++i) o[i] = xr[i] * r * w[i] * or_silu(g[i]);
        }
    });
}

// out = x1 + x2                                      -- src/cuda/ops.cu:115-125
void or_residual_add(const float* x1, const float* x2, float* out, int64_t size) {
    for (int64_t i = 0; i < size; ++i) out[i] = x1[i] + x2[i];
}

// out[t] = table[ids[t]] (fp32 rows)                 -- src/cuda/ops.cu:128-138
void or_encoder_rows(const int32_t* ids, int n_ids, const float* table, float* out, int d_model) {
    for (int t = 0; t < n_ids; ++t)
        std::memcpy(out + static_cast<int64_t>(t) * d_model,
                    table + static_cast<int64_t>(ids[t]) * d_model, sizeof(float) * d_model);
}

// resid = x + branch; normed = rmsnorm(resid) * w     -- src/model.cpp:205,208
void or_residual_rmsnorm_rows_f32(const float* x, const float* branch, const float* w, float* resid,
                                  float* normed, int rows, int n, float eps, int threads) {
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            float* rr = resid + t * n;
            for (int i = 0; i < n; ++i) rr[i] = x[t * n + i] + branch[t * n + i];
            const float r = or_rsqrt(sum_squares(rr, n) / static_cast<float>(n) + eps);
            for (int i = 0; i < n; ++i) normed[t * n + i] = rr[i] * r * w[i];
        }
    });
}

// bf16 storage: the sum is rounded to bf16 (what the residual stream stores) and
// the norm reads the stored value back, exactly as residual_add followed by
// rmsnorm_forward on bf16 buffers would.
void or_residual_rmsnorm_rows_bf16(const uint16_t* x, const uint16_t* branch, const float* w,
                                   uint16_t* resid, uint16_t* normed, int rows, int n, float eps,
                                   int threads) {
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        std::vector<float> rs(static_cast<size_t>(n));
        for (int64_t t = lo; t < hi; ++t) {
            for (int i = 0; i < n; ++i) {
                const uint16_t s = or_float_to_bf16(or_bf16_to_float(x[t * n + i]) +
                                                    or_bf16_to_float(branch[t * n + i]));
                resid[t * n + i] = s;
                rs[static_cast<size_t>(i)] = or_bf16_to_float(s);
            }
            const float r = or_rsqrt(sum_squares(rs.data(), n) / static_cast<float>(n) + eps);
            for (int i = 0; i < n; ++i) normed[t * n + i] = or_float_to_bf16(rs[static_cast<size_t>(i)] * r * w[i]);
        }
    });
}

// ---------------------------------------------------------------- attention

// Per-head RMSNorm in place: x = x * (r * w)          -- src/cuda/attn_kernels.cu:34-63
static void head_norm(float* x, const float* w, int dim, float eps) {
    const float r = or_rsqrt(sum_squares(x, dim) / static_cast<float>(dim) + eps);
    for (int i = 0; i < dim; ++i) x[i] *= r * w[i];
}

void or_head_norm_rows(float* x, const float* w, int rows, int heads, int dim, float eps, int threads) {
    parallel_for(static_cast<int64_t>(rows) * heads, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t h = lo; h < hi; ++h) head_norm(x + h * dim, w, dim, eps);
    });
}

// powf(base, (2.0f * i) / rd), exponent formed in float as in src/cuda/rope.cu:19
// and tests/kernel_tests.cu:338; the power is evaluated in double and rounded once.
float or_rope_den(int i, int rope_dim, float theta) {
    const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(rope_dim);
    return static_cast<float>(std::pow(static_cast<double>(theta), static_cast<double>(e)));
}

// Split-half rotation of the first rope_dim dims of one head.  -- src/cuda/rope.cu:9-29
static void rope_head(float* p, int pos, int rope_dim, const float* den) {
    const int half = rope_dim / 2;
    for (int i = 0; i < half; ++i) {
        const float th = static_cast<float>(pos) / den[i];
        const float c = cos_f(th);
        const float s = sin_f(th);
        const float a = p[i];
        const float b = p[i + half];
        p[i] = a * c - b * s;
        p[i + half] = b * c + a * s;
    }
}

void or_rope_rows(float* x, const int32_t* pos, int pos0, int rows, int heads, int head_dim, int rope_dim,
                  float theta, int threads) {
    std::vector<float> den(static_cast<size_t>(rope_dim / 2));
    for (int i = 0; i < rope_dim / 2; ++i) den[static_cast<size_t>(i)] = or_rope_den(i, rope_dim, theta);
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            const int p = pos ? pos[t] : pos0 + static_cast<int>(t);
            for (int h = 0; h < heads; ++h) rope_head(x + (t * heads + h) * head_dim, p, rope_dim, den.data());
        }
    });
}

// attn_head_norm(q), attn_head_norm(k), rope(q), rope(k)  -- src/layer_attn.cpp:91-96
void or_qk_norm_rope_rows(float* q, float* k, const float* qw, const float* kw, const int32_t* pos, int pos0,
                          int rows, int q_heads, int k_heads, int head_dim, int rope_dim, float theta,
                          float eps, int threads) {
    std::vector<float> den(static_cast<size_t>(rope_dim / 2));
    for (int i = 0; i < rope_dim / 2; ++i) den[static_cast<size_t>(i)] = or_rope_den(i, rope_dim, theta);
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            const int p = pos ? pos[t] : pos0 + static_cast<int>(t);
            for (int h = 0; h < q_heads; ++h) {
                float* hp = q + (t * q_heads + h) * head_dim;
                head_norm(hp, qw, head_dim, eps);
                if (rope_dim > 0) rope_head(hp, p, rope_dim, den.data());
            }
            for (int h = 0; h < k_heads; ++h) {
                float* hp = k + (t * k_heads + h) * head_dim;
                head_norm(hp, kw, head_dim, eps);
                if (rope_dim > 0) rope_head(hp, p, rope_dim, den.data());
            }
        }
    });
}

// ---------------------------------------------------------------- Gated DeltaNet

// `rows` sequential gdn_conv_step calls.              -- src/cuda/gdn.cu:9-27
// sum += hist*w is contracted to a fused multiply-add by nvcc's default
// (--fmad=true); fmaf restates that.
void or_conv_rows(const float* x, const float* w, const float* hist_in, float* hist_out, float* y, int rows,
                  int channels, int kernel, int threads) {
    const int hk = kernel - 1;
    // Input s of channel c: x row s, or for s < 0 the carried history (entry
    // hk + s holds x[s]), so every output row depends only on inputs and the
    // rows can be split across threads; the per-element fmaf order is the
    // reference's sliding window, oldest first.
    auto xin = [&](int64_t s, int64_t c) -> float {
        return s >= 0 ? x[s * channels + c] : hist_in[c * hk + (hk + s)];
    };
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t)
            for (int64_t c = 0; c < channels; ++c) {
                const float* wc = w + c * kernel;
                float sum = 0.0f;
                for (int j = 0; j < hk; ++j) sum = std::fmaf(xin(t - hk + j, c), wc[j], sum);
                sum = std::fmaf(x[t * channels + c], wc[kernel - 1], sum);
                y[t * channels + c] = or_silu(sum);
            }
    });
    for (int64_t c = 0; c < channels; ++c)
        for (int j = 0; j < hk; ++j) hist_out[c * hk + j] = xin(static_cast<int64_t>(rows) - hk + j, c);
}

// Per-head L2 norm of q and k in place; q also scaled by rsqrtf(dim). eps is
// added to the sum of squares, not the mean.        -- src/cuda/gdn.cu:36-81
void or_qk_l2_rows(float* q, float* k, int64_t row_stride, int rows, int heads, int dim, float eps,
                   int threads) {
    const float scale = or_rsqrt(static_cast<float>(dim));
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            for (int h = 0; h < heads; ++h) {
                float* qh = q + t * row_stride + static_cast<int64_t>(h) * dim;
                float* kh = k + t * row_stride + static_cast<int64_t>(h) * dim;
                const float rq = or_rsqrt(sum_squares(qh, dim) + eps);
                const float rk = or_rsqrt(sum_squares(kh, dim) + eps);
                for (int i = 0; i < dim; ++i) {
                    qh[i] *= rq * scale;
                    kh[i] *= rk;
                }
            }
        }
    });
}

// gdn_conv_step then gdn_qk_normalize on the q and k channel ranges.
//                                                    -- src/layer_gdn.cpp:89-97
void or_gdn_frontend_rows(const float* x, const float* w, const float* hist_in, float* hist_out, float* y,
                          int rows, int channels, int kernel, int k_heads, int key_dim, float eps,
                          int threads) {
    or_conv_rows(x, w, hist_in, hist_out, y, rows, channels, kernel, threads);
    if (k_heads > 0)
        or_qk_l2_rows(y, y + static_cast<int64_t>(k_heads) * key_dim, channels, rows, k_heads, key_dim, eps,
                      threads);
}

// out = ((x * r) * w) * silu(z), r = rsqrtf(sum(x^2)/d + eps)  -- src/cuda/gdn.cu:176-210
void or_norm_gate_rows(const float* x, const float* z, const float* w, float* out, int rows, int heads,
                       int dim, float eps, int threads) {
    parallel_for(static_cast<int64_t>(rows) * heads, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t h = lo; h < hi; ++h) {
            const float* xh = x + h * dim;
            const float* zh = z + h * dim;
            float* o = out + h * dim;
            const float r = or_rsqrt(sum_squares(xh, dim) / static_cast<float>(dim) + eps);
            for (int i = 0; i < dim; ++i) o[i] = xh[i] * r * w[i] * or_silu(zh[i]);
        }
    });
}

// beta = sigmoid(b); decay = expf(a * softplus(alpha + dt))  -- src/cuda/gdn.cu:90-99
void or_gdn_gate_values(const float* b, const float* alpha, const float* a, const float* dt, float* beta,
                        float* decay, int n) {
    for (int i = 0; i < n; ++i) {
        beta[i] = or_sigmoid(b[i]);
        const float x = alpha[i] + dt[i];
        const float sp =
            (x > 20.0f) ? x : static_cast<float>(std::log1p(static_cast<double>(exp_f(x))));
        decay[i] = exp_f(a[i] * sp);
    }
}

// Delta-rule state update and readout, restated as the reference's own host
// check does (tests/kernel_tests.cu:237-257)          -- src/cuda/gdn.cu:108-151
void or_gdn_recurrent_step(float* state, const float* q, const float* k, const float* v, const float* beta,
                           const float* decay, float* out, int key_heads, int value_heads, int key_dim,
                           int value_dim) {
    for (int h = 0; h < value_heads; ++h) {
        const int src = h % key_heads;
        float* S = state + static_cast<int64_t>(h) * key_dim * value_dim;
        for (int j = 0; j < value_dim; ++j) {
            float mem = 0.0f;
            for (int i = 0; i < key_dim; ++i) {
                float& cell = S[static_cast<int64_t>(i) * value_dim + j];
                cell *= decay[h];
                mem += k[src * key_dim + i] * cell;
            }
            const float delta = (v[h * value_dim + j] - mem) * beta[h];
            for (int i = 0; i < key_dim; ++i) S[static_cast<int64_t>(i) * value_dim + j] += k[src * key_dim + i] * delta;
            float o = 0.0f;
            for (int i = 0; i < key_dim; ++i) o += q[src * key_dim + i] * S[static_cast<int64_t>(i) * value_dim + j];
            out[h * value_dim + j] = o;
        }
    }
}

// T consecutive recurrent steps (the reference calls gdn_recurrent_step once
// per token, src/layer_gdn.cpp:100-106): token t reads q, k, v at
// t * qkv_stride, beta / decay at t * value_heads, writes out at t * out_stride.
void or_gdn_recurrent_rows(float* state, const float* q, const float* k, const float* v, const float* beta,
                           const float* decay, float* out, int rows, int key_heads, int value_heads, int key_dim,
                           int value_dim, int64_t qkv_stride, int64_t out_stride) {
    for (int t = 0; t < rows; ++t)
        or_gdn_recurrent_step(state, q + t * qkv_stride, k + t * qkv_stride, v + t * qkv_stride,
                              beta + static_cast<int64_t>(t) * value_heads, decay + static_cast<int64_t>(t) * value_heads,
                              out + t * out_stride, key_heads, value_heads, key_dim, value_dim);
}

// ---------------------------------------------------------------- attention core (decode)

// q[h][j] = in[h][j], g[h][j] = in[h][d + j] (rows of 2d)  -- src/cuda/attn_kernels.cu:16-31
void or_attn_split_qg(const float* in, float* q, float* g, int heads, int dim) {
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t j = 0; j < dim; ++j) {
            q[h * dim + j] = in[h * 2 * dim + j];
            g[h * dim + j] = in[h * 2 * dim + dim + j];
        }
}

// scores[h][t] = (q_h . k_t) * rsqrt(D), t <= pos, kv head h / (H / Hkv)
//                                                     -- src/cuda/attn_kernels.cu:72-96
void or_attn_scores(const float* q, const float* k_cache, float* scores, int heads, int kv_heads, int dim, int pos) {
    const int group = heads / kv_heads;
    const float scale = or_rsqrt(static_cast<float>(dim));
    for (int64_t h = 0; h < heads; ++h) {
        const int64_t kv = h / group;
        for (int64_t t = 0; t <= pos; ++t) {
            double sum = 0.0;
            const float* kt = k_cache + (t * kv_heads + kv) * dim;
            for (int i = 0; i < dim; ++i) sum += static_cast<double>(q[h * dim + i]) * kt[i];
            scores[h * (pos + 1) + t] = static_cast<float>(sum) * scale;
        }
    }
}

// Row softmax: r = expf(r - max) / sum               -- src/cuda/attn_kernels.cu:99-158
void or_attn_softmax(float* scores, int heads, int n) {
    for (int64_t h = 0; h < heads; ++h) {
        float* r = scores + h * n;
        float m = -INFINITY;
        for (int i = 0; i < n; ++i) m = std::fmax(m, r[i]);
        double sum = 0.0;
        for (int i = 0; i < n; ++i) {
            r[i] = exp_f(r[i] - m);
            sum += r[i];
        }
        const float fs = static_cast<float>(sum);
        for (int i = 0; i < n; ++i) r[i] /= fs;
    }
}

// out[h][j] = sum_t s[h][t] * v[t][kv][j]            -- src/cuda/attn_kernels.cu:162-181
void or_attn_values(const float* scores, const float* v_cache, float* out, int heads, int kv_heads, int dim, int pos) {
    const int group = heads / kv_heads;
    for (int64_t h = 0; h < heads; ++h) {
        const int64_t kv = h / group;
        for (int64_t j = 0; j < dim; ++j) {
            double z = 0.0;
            for (int64_t t = 0; t <= pos; ++t)
                z += static_cast<double>(scores[h * (pos + 1) + t]) * v_cache[(t * kv_heads + kv) * dim + j];
            out[h * dim + j] = static_cast<float>(z);
        }
    }
}

// out = x / (1 + expf(-g))                            -- src/cuda/attn_kernels.cu:185-195
void or_attn_sigmoid_gate(const float* x, const float* g, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] / (1.0f + exp_f(-g[i]));
}

// The decode sequence of src/layer_attn.cpp:103-108 after the cache store:
// scores, softmax over pos + 1 keys, values, then the sigmoid gate when gate
// is non-null. scratch holds heads * (pos + 1) floats.
void or_attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* gate, float* out,
                    float* scratch, int heads, int kv_heads, int dim, int pos) {
    or_attn_scores(q, k_cache, scratch, heads, kv_heads, dim, pos);
    or_attn_softmax(scratch, heads, pos + 1);
    or_attn_values(scratch, v_cache, out, heads, kv_heads, dim, pos);
    if (gate) or_attn_sigmoid_gate(out, gate, out, static_cast<int64_t>(heads) * dim);
}

// ---------------------------------------------------------------- MoE routing

// Top-k of n router logits by repeated selection (strictly greater wins, so
// ties go to the lowest index), then a softmax over the k picks; a non-finite
// logit gives idx[0] = -1, w[0] = NaN and leaves the rest untouched.
//                                                     -- src/cuda/moe.cu:7-51
void or_moe_topk(const float* x, int32_t* idx, float* w, int n, int k) {
    for (int i = 0; i < n; ++i)
        if (!std::isfinite(x[i])) {
            idx[0] = -1;
            w[0] = NAN;
            return;
        }
    for (int j = 0; j < k; ++j) {
        float best = -INFINITY;
        int bi = -1;
        for (int i = 0; i < n; ++i) {
            bool used = false;
            for (int p = 0; p < j; ++p) used |= (idx[p] == i);
            if (!used && x[i] > best) {
                best = x[i];
                bi = i;
            }
        }
        idx[j] = bi;
        w[j] = best;
    }
    float mx = w[0];
    for (int j = 1; j < k; ++j) mx = std::fmax(mx, w[j]);
    double sum = 0.0;
    for (int j = 0; j < k; ++j) {
        w[j] = exp_f(w[j] - mx);
        sum += w[j];
    }
    const float fs = static_cast<float>(sum);
    for (int j = 0; j < k; ++j) w[j] /= fs;
}

void or_moe_topk_rows(const float* x, int32_t* idx, float* w, int rows, int n, int k) {
    for (int64_t t = 0; t < rows; ++t) or_moe_topk(x + t * n, idx + t * k, w + t * k, n, k);
}

// out += a * x                                        -- src/cuda/moe.cu:76-86
// (one fused multiply-add, as nvcc contracts `out[i] += a * x[i]`)
void or_moe_add(float* out, const float* x, float a, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = std::fma(a, x[i], out[i]);
}

// out[t] += sum_j w[t][j] * y[t][j]: the layer's k moe_add calls per token
// (src/layer_moe.cpp:127-142) with the weights read from device memory.
void or_moe_weighted_sum_rows(float* out, const float* y, const float* w, int rows, int k, int dim) {
    for (int64_t t = 0; t < rows; ++t)
        for (int j = 0; j < k; ++j) or_moe_add(out + t * dim, y + (t * k + j) * dim, w[t * k + j], dim);
}

// y[j] = W[idx[j] * expert_stride ...] x[j * x_stride ...]: matmul_dispatch of
// each selected expert (src/layer_moe.cpp:131-138, element offset
// e * stride). An id outside [0, n_experts) gives a NaN row.
void or_moe_expert_gemv(const uint8_t* w, int type, const int32_t* idx, int n_sel, int n_experts,
                        uint64_t expert_stride, const float* x, int64_t x_stride, float* y, int M, int K) {
    for (int j = 0; j < n_sel; ++j) {
        float* yj = y + static_cast<int64_t>(j) * M;
        if (idx[j] < 0 || idx[j] >= n_experts) {
            for (int m = 0; m < M; ++m) yj[m] = NAN;
            continue;
        }
        or_gemv(w, type, x + j * x_stride, yj, M, K, static_cast<uint64_t>(idx[j]) * expert_stride, 1);
    }
}

// ---------------------------------------------------------------- MoE activations

// h = silu(g) * u                                    -- src/cuda/moe.cu:61-67
void or_silu_mul_f32(const float* g, const float* u, float* h, int64_t n, int threads) {
    parallel_for(n, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) h[i] = or_silu(g[i]) * u[i];
    });
}

// bf16 storage, fp32 math, one rounding at the store.
void or_swiglu_bf16(const uint16_t* g, const uint16_t* u, uint16_t* h, int64_t n, int threads) {
    parallel_for(n, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i)
            h[i] = or_float_to_bf16(or_silu(or_bf16_to_float(g[i])) * or_bf16_to_float(u[i]));
    });
}

// Shared expert: h = (silu(g) * u) * sigmoid(logit[t]). The reference applies the
// sigmoid after the down projection (src/cuda/moe.cu:90-96, layer_moe.cpp:153);
// by linearity the same scale can be applied to the SwiGLU rows instead.
void or_shared_swiglu_sigmoid_bf16(const uint16_t* g, const uint16_t* u, const float* logits, uint16_t* h,
                                   int rows, int dim, int threads) {
    parallel_for(rows, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            const float s = or_sigmoid(logits[t]);
            for (int64_t i = t * dim; i < (t + 1) * dim; ++i)
                h[i] = or_float_to_bf16(or_silu(or_bf16_to_float(g[i])) * or_bf16_to_float(u[i]) * s);
        }
    });
}

// accum += x * sigmoid(gate[t]) per row              -- src/cuda/moe.cu:90-96
void or_shared_add_rows(float* accum, const float* x, const float* gate, int rows, int dim) {
    for (int64_t t = 0; t < rows; ++t) {
        const float s = or_sigmoid(gate[t]);
        for (int64_t i = t * dim; i < (t + 1) * dim; ++i) accum[i] += x[i] * s;
    }
}

// ---------------------------------------------------------------- dequant gather

// out[t] = dequantize_row(table, ids[t], cols)       -- src/cuda/matmul_q4.cu:169-173,209-227
void or_dequant_gather(const uint8_t* table, int type, const int32_t* ids, int n_ids, int cols, float* out,
                       int threads) {
    parallel_for(n_ids, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t t = lo; t < hi; ++t) {
            const uint64_t start = static_cast<uint64_t>(ids[t]) * static_cast<uint64_t>(cols);
            for (int i = 0; i < cols; ++i) out[t * cols + i] = or_dequant(table, type, start + static_cast<uint64_t>(i));
        }
    });
}

void or_dequant_span(const uint8_t* data, int type, uint64_t start, int count, float* out) {
    for (int i = 0; i < count; ++i) out[i] = or_dequant(data, type, start + static_cast<uint64_t>(i));
}

// ---------------------------------------------------------------- quantized GEMV

// y[m] = sum_k dequant(W, element_offset + m*K + k) * x[k], m < M
//                                                    -- src/cuda/matmul_q4.cu:140-167,185-207
// The reference sums fp32 products in an order fixed by its launch shape
// (256 strided partial sums, then a shuffle tree); the oracle takes every
// product exactly (a float times a float fits a double), sums in double and
// rounds once.
void or_gemv(const uint8_t* w, int type, const float* x, float* y, int M, int K, uint64_t element_offset,
             int threads) {
    parallel_for(M, threads, [&](int64_t lo, int64_t hi) {
        for (int64_t m = lo; m < hi; ++m) {
            const uint64_t base = element_offset + static_cast<uint64_t>(m) * static_cast<uint64_t>(K);
            double s = 0.0;
            for (int k = 0; k < K; ++k)
                s += static_cast<double>(or_dequant(w, type, base + static_cast<uint64_t>(k))) *
                     static_cast<double>(x[k]);
            y[m] = static_cast<float>(s);
        }
    });
}

}  // extern "C"
