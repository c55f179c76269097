/*
 * cbq_oracle.h - CPU restatement of cuBlade's quantization numerics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels in cublade_amd/csrc. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product path never calls it.
 *
 * Dtype codes match include/cublade_quant.h: 0 = fp32, 1 = fp16, 2 = bf16.
 * 16-bit floating-point tensors are passed as their raw uint16 bit patterns;
 * FP8 E4M3 (OCP "e4m3fn") codes are passed as raw uint8.
 */
#ifndef CBQ_ORACLE_H
#define CBQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar conversions (bit-level, round-to-nearest-even) */
float    cbo_f16_to_f32(uint16_t h);
float    cbo_bf16_to_f32(uint16_t h);
float    cbo_e4m3_to_f32(uint8_t b);
uint16_t cbo_f32_to_f16(float f);
uint16_t cbo_f32_to_bf16(float f);
uint8_t  cbo_f32_to_e4m3_satfinite(float f);
int8_t   cbo_round_clamp_int8(float v);

/* element-wise helpers over arrays (for exhaustive tests) */
void cbo_load_f32(const void* x, int dtype, int64_t n, float* out);
void cbo_store_from_f32(const float* v, int64_t n, void* y, int dtype);
void cbo_cast_e4m3(const float* v, int64_t n, uint8_t* q);
void cbo_decode_e4m3(const uint8_t* q, int64_t n, float* out);
void cbo_cast_int8(const float* v, int64_t n, int8_t* q);

/* reductions and scales */
float cbo_amax(const void* x, int dtype, int64_t n);
float cbo_inv_scale(float amax, float eps, float qmax);
float cbo_scale_from_inv(float inv);

/* quantization entry points (return 0 on success, nonzero on bad args) */
int cbo_quant_fp8_tensor(const void* x, int dtype, int64_t n, float eps,
                         uint8_t* q, float* scale);
int cbo_quant_int8_tensor(const void* x, int dtype, int64_t n, float eps,
                          int8_t* q, float* scale);
int cbo_quant_int8_channel(const void* x, int dtype, int64_t rows, int64_t cols,
                           int axis, float eps, int8_t* q, float* scale);
int cbo_quant_int8_group(const void* x, int dtype, int64_t num_groups,
                         int64_t group_size, float eps, int8_t* q, float* scale);

/* dequantization entry points */
int cbo_dequant_fp8_tensor(const uint8_t* q, const float* scale, int64_t n,
                           void* y, int out_dtype);
int cbo_dequant_int8_tensor(const int8_t* q, const float* scale, int64_t n,
                            void* y, int out_dtype);
int cbo_dequant_int8_channel(const int8_t* q, const float* scale, int64_t rows,
                             int64_t cols, int axis, void* y, int out_dtype);
int cbo_dequant_int8_group(const int8_t* q, const float* scale,
                           int64_t num_groups, int64_t group_size, void* y,
                           int out_dtype);

/* W8A16 linear in exact-accumulation form (double accumulators, fp32 out).
 * Restates cublade/quantization/linear.py:97-135 without the intermediate
 * fp16 roundings:
 *   y[m,n] = s[n] * sum_i x[m, normal_cols[i]] * wq[n, i]
 *          + sum_j x[m, outlier_cols[j]] * w_out[n, j]     (n_out > 0)
 *          + bias[n]                                       (bias != NULL)
 * wq is int8 [N, Kn] row-major. normal_cols may be NULL, meaning Kn == K and
 * normal column i is column i. x, scales, bias and w_out are in act_dtype.
 * rows_idx (optional, length n_rows) restricts the computation to those rows
 * of x; y then has n_rows rows of N floats.
 */
int cbo_w8a16_linear(const void* x, int act_dtype, const int8_t* wq,
                     int64_t Kn, const int64_t* normal_cols,
                     const void* scales, const void* bias,
                     const int64_t* outlier_cols, int64_t n_out,
                     const void* w_out, int64_t M, int64_t N, int64_t K,
                     const int64_t* rows_idx, int64_t n_rows, float* y);

/* Dense GEMM restatements (wmma.cu): C = A[M,K] . B, B [K,N] or stored [N,K]
 * (b_nk). 8-bit integers with wrapping int32 accumulation; fp16 / bf16 with
 * double accumulation. */
int cbo_mm_int8(const void* A, const void* B, int is_unsigned, int b_nk, int64_t M,
                int64_t N, int64_t K, int32_t* C);
int cbo_mm_float(const void* A, const void* B, int dtype, int b_nk, int64_t M, int64_t N,
                 int64_t K, double* C);

#ifdef __cplusplus
}
#endif

#endif /* CBQ_ORACLE_H */
