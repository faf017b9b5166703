/*
 * CPU oracle for the fused per-layer kernels -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or as the timed CPU baseline). The
 * product library (qwen-3.5-cuda_amd) never links, loads or calls it.
 *
 * Every function is a scalar restatement of one reference kernel, with the
 * reference's float association; each cites the reference file:line it follows
 * (paths are relative to the sahan974/qwen-3.5-cuda tree). Where the reference
 * leaves a choice to the parallel schedule (the order of a sum of squares), the
 * oracle sums in double and rounds once; where the reference calls a CUDA math
 * function (expf, rsqrtf, cosf, sinf) the oracle evaluates the function in
 * double and rounds to float once, which is within one float ulp of the exact
 * value.
 *
 * Parity pins (what checks this restatement independently of its own formulas)
 * are listed per function in tests/test_oracle.py and in the repository's design
 * notes. No function here is left unpinned.
 *
 * Storage conventions: fp32 is IEEE binary32, bf16 is the top 16 bits of a
 * binary32 (uint16_t), fp16 is IEEE binary16 (uint16_t). Threads: `threads` <= 1
 * runs on the calling thread; larger values split rows over std::threads (used
 * only for the CPU baseline timing).
 */
#ifndef QWEN35_ORACLE_H
#define QWEN35_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers exposed for tests ---- */
float or_silu(float x);                 /* src/cuda/ops.cu:9-11            */
float or_sigmoid(float x);              /* src/cuda/moe.cu:94              */
float or_rsqrt(float x);                /* CUDA rsqrtf, exact-then-rounded */
float or_half_to_float(uint16_t h);     /* src/cuda/matmul_q4.cu:13-16     */
float or_bf16_to_float(uint16_t b);
uint16_t or_float_to_bf16(float f);     /* round to nearest even            */
void or_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m); /* matmul_q4.cu:18-26 */
float or_dequant(const uint8_t* data, int type, uint64_t index);         /* matmul_q4.cu:30-129 */

/* ---- ops.hpp ---- */
void or_rmsnorm_rows(const float* x, const float* w, float* out, int rows, int n,
                     float eps, int threads);                            /* ops.cu:25-65   */
void or_rmsnorm_gated_rows(const float* x, const float* gate, const float* w, float* out,
                           int rows, int n, float eps, int threads);     /* ops.cu:68-109  */
void or_residual_add(const float* x1, const float* x2, float* out, int64_t size); /* ops.cu:115-125 */
void or_encoder_rows(const int32_t* ids, int n_ids, const float* table, float* out,
                     int d_model);                                       /* ops.cu:128-138 */
/* residual_add followed by rmsnorm_forward on the stored sum (model.cpp:205,208) */
void or_residual_rmsnorm_rows_f32(const float* x, const float* branch, const float* w,
                                  float* resid, float* normed, int rows, int n, float eps,
                                  int threads);
void or_residual_rmsnorm_rows_bf16(const uint16_t* x, const uint16_t* branch, const float* w,
                                   uint16_t* resid, uint16_t* normed, int rows, int n,
                                   float eps, int threads);

/* ---- attention: head norm + partial RoPE ---- */
void or_head_norm_rows(float* x, const float* w, int rows, int heads, int dim, float eps,
                       int threads);                                     /* attn_kernels.cu:34-63 */
float or_rope_den(int i, int rope_dim, float theta);                     /* rope.cu:19, kernel_tests.cu:338 */
void or_rope_rows(float* x, const int32_t* pos, int pos0, int rows, int heads, int head_dim,
                  int rope_dim, float theta, int threads);               /* rope.cu:9-29 */
void or_qk_norm_rope_rows(float* q, float* k, const float* qw, const float* kw,
                          const int32_t* pos, int pos0, int rows, int q_heads, int k_heads,
                          int head_dim, int rope_dim, float theta, float eps, int threads);

/* ---- Gated DeltaNet ---- */
void or_conv_rows(const float* x, const float* w, const float* hist_in, float* hist_out,
                  float* y, int rows, int channels, int kernel, int threads); /* gdn.cu:9-27 */
void or_qk_l2_rows(float* q, float* k, int64_t row_stride, int rows, int heads, int dim,
                   float eps, int threads);                               /* gdn.cu:36-81 */
void or_gdn_frontend_rows(const float* x, const float* w, const float* hist_in,
                          float* hist_out, float* y, int rows, int channels, int kernel,
                          int k_heads, int key_dim, float eps, int threads);
void or_norm_gate_rows(const float* x, const float* z, const float* w, float* out, int rows,
                       int heads, int dim, float eps, int threads);      /* gdn.cu:176-210 */
void or_gdn_gate_values(const float* b, const float* alpha, const float* a, const float* dt,
                        float* beta, float* decay, int n);               /* gdn.cu:90-99 */
void or_gdn_recurrent_step(float* state, const float* q, const float* k, const float* v,
                           const float* beta, const float* decay, float* out, int key_heads,
                           int value_heads, int key_dim, int value_dim); /* gdn.cu:108-151 */
void or_gdn_recurrent_rows(float* state, const float* q, const float* k, const float* v,
                           const float* beta, const float* decay, float* out, int rows,
                           int key_heads, int value_heads, int key_dim, int value_dim,
                           int64_t qkv_stride, int64_t out_stride);  /* layer_gdn.cpp:100-106 */

/* ---- attention core (decode) ---- */
void or_attn_split_qg(const float* in, float* q, float* g, int heads, int dim);  /* attn_kernels.cu:16-31 */
void or_attn_scores(const float* q, const float* k_cache, float* scores, int heads, int kv_heads,
                    int dim, int pos);                                  /* attn_kernels.cu:72-96 */
void or_attn_softmax(float* scores, int heads, int n);                  /* attn_kernels.cu:99-158 */
void or_attn_values(const float* scores, const float* v_cache, float* out, int heads, int kv_heads,
                    int dim, int pos);                                  /* attn_kernels.cu:162-181 */
void or_attn_sigmoid_gate(const float* x, const float* g, float* out, int64_t n); /* :185-195 */
void or_attn_decode(const float* q, const float* k_cache, const float* v_cache, const float* gate,
                    float* out, float* scratch, int heads, int kv_heads, int dim,
                    int pos);                                           /* layer_attn.cpp:99-108 */

/* ---- MoE routing ---- */
void or_moe_topk(const float* x, int32_t* idx, float* w, int n, int k);   /* moe.cu:7-51 */
void or_moe_topk_rows(const float* x, int32_t* idx, float* w, int rows, int n, int k);
void or_moe_add(float* out, const float* x, float a, int64_t n);          /* moe.cu:76-86 */
void or_moe_weighted_sum_rows(float* out, const float* y, const float* w, int rows, int k,
                              int dim);                                  /* layer_moe.cpp:127-142 */
void or_moe_expert_gemv(const uint8_t* w, int type, const int32_t* idx, int n_sel, int n_experts,
                        uint64_t expert_stride, const float* x, int64_t x_stride, float* y, int M,
                        int K);                                          /* layer_moe.cpp:131-138 */

/* ---- MoE activations ---- */
void or_silu_mul_f32(const float* g, const float* u, float* h, int64_t n, int threads); /* moe.cu:61-67 */
void or_swiglu_bf16(const uint16_t* g, const uint16_t* u, uint16_t* h, int64_t n, int threads);
void or_shared_swiglu_sigmoid_bf16(const uint16_t* g, const uint16_t* u, const float* logits,
                                   uint16_t* h, int rows, int dim, int threads);
void or_shared_add_rows(float* accum, const float* x, const float* gate, int rows, int dim); /* moe.cu:90-96 */

/* ---- quantized embedding gather ---- */
int or_type_supported(int type);                                          /* matmul_q4.cu:179-183 */
void or_dequant_gather(const uint8_t* table, int type, const int32_t* ids, int n_ids,
                       int cols, float* out, int threads);                /* matmul_q4.cu:169-173,209-227 */
void or_dequant_span(const uint8_t* data, int type, uint64_t start, int count, float* out);

/* ---- quantized GEMV ---- */
void or_gemv(const uint8_t* w, int type, const float* x, float* y, int M, int K,
             uint64_t element_offset, int threads);             /* matmul_q4.cu:140-167,185-207 */

#ifdef __cplusplus
}
#endif

#endif /* QWEN35_ORACLE_H */
