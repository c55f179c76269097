/*
 * cbq_oracle.c - CPU restatement of cuBlade's quantization numerics.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP kernels in
 * cublade_amd/csrc, loaded only by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py. Never part of the product path.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the cuBlade source tree, package `cublade`). Build flags must keep IEEE fp32
 * semantics: no -ffast-math, -ffp-contract=off (see oracle/Makefile).
 *
 * Pinning (how each function is checked independently of this file):
 *   conversions  - exhaustive over all 16-bit / 8-bit codes against torch CPU
 *                  and numpy library conversions (tests/test_oracle_numerics.py)
 *   amax         - numpy max over |x| on random and adversarial inputs
 *   scales       - closed-form known answers (toy cases) and torch fp32 division
 *   quant/dequant- committed golden vectors built with torch CPU ops
 *                  (tests/golden/make_golden.py), plus invariants
 *   w8a16        - numpy float64 matmul on the same operands
 */
#include "cbq_oracle.h"

#include <math.h>
#include <stddef.h>
#include <string.h>

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* Scalar conversions.                                                      */
/* fp8_pack.cuh:30-35, 54-58 (to_float2/from_float2: exact widening, RNE    */
/* narrowing), fp8_pack.cuh:38-41, 64-68 (E4M3 -> half exact).              */
/* ------------------------------------------------------------------------ */

float cbo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

float cbo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));      /* inf/nan */
    if (e == 0) {                                                   /* subnormal */
        float v = (float)m * 0x1p-24f;                               /* exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* OCP E4M3 ("e4m3fn"): bias 7, no infinities, S.1111.111 is NaN. */
float cbo_e4m3_to_f32(uint8_t b) {
    uint32_t sign = (uint32_t)(b & 0x80u) << 24;
    uint32_t e = (b >> 3) & 0xfu;
    uint32_t m = b & 0x7u;
    if (e == 0xf && m == 0x7) return u2f(sign | 0x7fc00000u);
    if (e == 0) {
        float v = (float)m * 0x1p-9f;                                /* exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

/* Round-to-nearest-even narrowing to bf16 (__float22bfloat162_rn). */
uint16_t cbo_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* Round-to-nearest-even narrowing to IEEE binary16 (__float22half2_rn). */
uint16_t cbo_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);        /* >= 65520 */
    if (a >= 0x38800000u) {                                          /* >= 2^-14 */
        a += 0xfffu + ((a >> 13) & 1u);
        return (uint16_t)(sign | ((a - 0x38000000u) >> 13));
    }
    /* subnormal range: units of 2^-24; scaling by 2^24 is exact in double */
    double units = nearbyint((double)u2f(a) * 16777216.0);
    return (uint16_t)(sign | (uint16_t)units);
}

/* FP32 -> E4M3 with saturation to +-448 and NaN preserved: the semantics of
 * __nv_cvt_float2_to_fp8x2(..., __NV_SATFINITE, __NV_E4M3) used at
 * quantize_per_tensor_fp8.cu:117,129. RNE including subnormals. */
uint8_t cbo_f32_to_e4m3_satfinite(float f) {
    uint32_t u = f2u(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);            /* NaN */
    if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu);           /* >= 448 */
    if (a >= 0x3c800000u) {                                          /* >= 2^-6 */
        a += 0x7ffffu + ((a >> 20) & 1u);
        uint32_t code = (a - (120u << 23)) >> 20;
        if (code > 0x7eu) code = 0x7eu;   /* (448, 464) rounds to 448 */
        return (uint8_t)(sign | code);
    }
    double units = nearbyint((double)u2f(a) * 512.0);                /* 2^-9 */
    return (uint8_t)(sign | (uint8_t)units);
}

/* int8_pack.cuh:51-56: __float2int_rn (RNE, NaN -> 0) then clamp to +-127. */
int8_t cbo_round_clamp_int8(float v) {
    if (v != v) return 0;
    float r = nearbyintf(v);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    return (int8_t)r;
}

/* ------------------------------------------------------------------------ */
/* Array helpers                                                            */
/* ------------------------------------------------------------------------ */

static inline float load_one(const void* x, int dtype, int64_t i) {
    switch (dtype) {
        case DT_F16: return cbo_f16_to_f32(((const uint16_t*)x)[i]);
        case DT_BF16: return cbo_bf16_to_f32(((const uint16_t*)x)[i]);
        default: return ((const float*)x)[i];
    }
}

static inline void store_one(void* y, int dtype, int64_t i, float v) {
    switch (dtype) {
        case DT_F16: ((uint16_t*)y)[i] = cbo_f32_to_f16(v); break;
        case DT_BF16: ((uint16_t*)y)[i] = cbo_f32_to_bf16(v); break;
        default: ((float*)y)[i] = v; break;
    }
}

void cbo_load_f32(const void* x, int dtype, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = load_one(x, dtype, i);
}
void cbo_store_from_f32(const float* v, int64_t n, void* y, int dtype) {
    for (int64_t i = 0; i < n; ++i) store_one(y, dtype, i, v[i]);
}
void cbo_cast_e4m3(const float* v, int64_t n, uint8_t* q) {
    for (int64_t i = 0; i < n; ++i) q[i] = cbo_f32_to_e4m3_satfinite(v[i]);
}
void cbo_decode_e4m3(const uint8_t* q, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = cbo_e4m3_to_f32(q[i]);
}
void cbo_cast_int8(const float* v, int64_t n, int8_t* q) {
    for (int64_t i = 0; i < n; ++i) q[i] = cbo_round_clamp_int8(v[i]);
}

/* ------------------------------------------------------------------------ */
/* amax and scales                                                          */
/* ------------------------------------------------------------------------ */

/* quantize_per_tensor_fp8.cu:38-86 and quantize_int8.cu:47-101: fmaxf fold of
 * |x| from 0.0 (fmaxf drops NaN). Max is order independent. */
float cbo_amax(const void* x, int dtype, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) m = fmaxf(m, fabsf(load_one(x, dtype, i)));
    return m;
}

/* quantize_per_tensor_fp8.cu:99 (448.0f / fmaxf(amax, eps)) and
 * quantize_int8.cu:120-122 (fp32(127.0 / (double)fmaxf(amax, eps))). Both are
 * the correctly rounded fp32 quotient: a double quotient of two floats narrowed
 * to float is correctly rounded because 53 >= 2*24 + 2. */
float cbo_inv_scale(float amax, float eps, float qmax) {
    return qmax / fmaxf(amax, eps);
}

/* quantize_per_tensor_fp8.cu:101-102 (1.0f / scale) and
 * quantize_int8.cu:124-126 (fp32(1.0 / (double)scale)). */
float cbo_scale_from_inv(float inv) { return 1.0f / inv; }

/* ------------------------------------------------------------------------ */
/* Quantization                                                             */
/* ------------------------------------------------------------------------ */

/* quantize_per_tensor_fp8.cu:140-182. An empty tensor launches no kernel in
 * the reference, so the zero-initialised scale (:171) is returned as 0. */
int cbo_quant_fp8_tensor(const void* x, int dtype, int64_t n, float eps,
                         uint8_t* q, float* scale) {
    if (dtype != DT_F16 && dtype != DT_BF16) return 1;
    if (n == 0) { *scale = 0.0f; return 0; }
    float inv = cbo_inv_scale(cbo_amax(x, dtype, n), eps, 448.0f);
    *scale = cbo_scale_from_inv(inv);
    for (int64_t i = 0; i < n; ++i)
        q[i] = cbo_f32_to_e4m3_satfinite(load_one(x, dtype, i) * inv);
    return 0;
}

/* quantize_int8.cu:103-166, 395-410, 470-484. */
int cbo_quant_int8_tensor(const void* x, int dtype, int64_t n, float eps,
                          int8_t* q, float* scale) {
    if (dtype < DT_F32 || dtype > DT_BF16) return 1;
    if (n == 0) { *scale = 0.0f; return 0; }
    float inv = cbo_inv_scale(cbo_amax(x, dtype, n), eps, 127.0f);
    *scale = cbo_scale_from_inv(inv);
    for (int64_t i = 0; i < n; ++i)
        q[i] = cbo_round_clamp_int8(load_one(x, dtype, i) * inv);
    return 0;
}

/* axis 0: quantize_int8.cu:173-297, 412-431, 487-509 (one scale per row of
 * the (rows, cols) view). axis 1 has no reference kernel (quantizers.py:117-
 * 120 rejects ch_axis != 0); it is the same math with the max taken over
 * rows, i.e. the axis-0 restatement applied to the transpose. A row (or
 * column) with no elements keeps the zero-initialised scale, as the
 * reference's empty launch does. */
int cbo_quant_int8_channel(const void* x, int dtype, int64_t rows, int64_t cols,
                           int axis, float eps, int8_t* q, float* scale) {
    if (dtype < DT_F32 || dtype > DT_BF16) return 1;
    if (axis == 0) {
        for (int64_t r = 0; r < rows; ++r) {
            if (cols == 0) { scale[r] = 0.0f; continue; }
            float m = 0.0f;
            for (int64_t c = 0; c < cols; ++c)
                m = fmaxf(m, fabsf(load_one(x, dtype, r * cols + c)));
            float inv = cbo_inv_scale(m, eps, 127.0f);
            scale[r] = cbo_scale_from_inv(inv);
            for (int64_t c = 0; c < cols; ++c)
                q[r * cols + c] = cbo_round_clamp_int8(load_one(x, dtype, r * cols + c) * inv);
        }
        return 0;
    }
    if (axis == 1) {
        for (int64_t c = 0; c < cols; ++c) {
            if (rows == 0) { scale[c] = 0.0f; continue; }
            float m = 0.0f;
            for (int64_t r = 0; r < rows; ++r)
                m = fmaxf(m, fabsf(load_one(x, dtype, r * cols + c)));
            float inv = cbo_inv_scale(m, eps, 127.0f);
            scale[c] = cbo_scale_from_inv(inv);
            for (int64_t r = 0; r < rows; ++r)
                q[r * cols + c] = cbo_round_clamp_int8(load_one(x, dtype, r * cols + c) * inv);
        }
        return 0;
    }
    return 1;
}

/* quantize_int8.cu:307-371, 433-447, 514-536: one scale per contiguous group
 * of group_size elements, 0 < group_size <= 4096. */
int cbo_quant_int8_group(const void* x, int dtype, int64_t num_groups,
                         int64_t group_size, float eps, int8_t* q, float* scale) {
    if (dtype < DT_F32 || dtype > DT_BF16) return 1;
    if (group_size <= 0 || group_size > 4096) return 1;
    for (int64_t g = 0; g < num_groups; ++g) {
        const int64_t base = g * group_size;
        float m = 0.0f;
        for (int64_t i = 0; i < group_size; ++i)
            m = fmaxf(m, fabsf(load_one(x, dtype, base + i)));
        float inv = cbo_inv_scale(m, eps, 127.0f);
        scale[g] = cbo_scale_from_inv(inv);
        for (int64_t i = 0; i < group_size; ++i)
            q[base + i] = cbo_round_clamp_int8(load_one(x, dtype, base + i) * inv);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Dequantization: y = T(float(q) * s), RNE narrowing                       */
/* ------------------------------------------------------------------------ */

/* dequantize_per_tensor_fp8.cu:23-66. */
int cbo_dequant_fp8_tensor(const uint8_t* q, const float* scale, int64_t n,
                           void* y, int out_dtype) {
    if (out_dtype != DT_F16 && out_dtype != DT_BF16) return 1;
    const float s = *scale;
    for (int64_t i = 0; i < n; ++i) store_one(y, out_dtype, i, cbo_e4m3_to_f32(q[i]) * s);
    return 0;
}

/* dequantize_int8.cu:29-64. */
int cbo_dequant_int8_tensor(const int8_t* q, const float* scale, int64_t n,
                            void* y, int out_dtype) {
    if (out_dtype != DT_F16 && out_dtype != DT_BF16) return 1;
    const float s = *scale;
    for (int64_t i = 0; i < n; ++i) store_one(y, out_dtype, i, (float)q[i] * s);
    return 0;
}

/* dequantize_int8.cu:70-109 (axis 0); axis 1 is the transpose of it. */
int cbo_dequant_int8_channel(const int8_t* q, const float* scale, int64_t rows,
                             int64_t cols, int axis, void* y, int out_dtype) {
    if (out_dtype != DT_F16 && out_dtype != DT_BF16) return 1;
    if (axis != 0 && axis != 1) return 1;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) {
            const float s = scale[axis == 0 ? r : c];
            store_one(y, out_dtype, r * cols + c, (float)q[r * cols + c] * s);
        }
    return 0;
}

/* dequantize_int8.cu:118-134. */
int cbo_dequant_int8_group(const int8_t* q, const float* scale,
                           int64_t num_groups, int64_t group_size, void* y,
                           int out_dtype) {
    if (out_dtype != DT_F16 && out_dtype != DT_BF16) return 1;
    if (group_size <= 0 || group_size > 4096) return 1;
    for (int64_t g = 0; g < num_groups; ++g)
        for (int64_t i = 0; i < group_size; ++i) {
            const int64_t k = g * group_size + i;
            store_one(y, out_dtype, k, (float)q[k] * scale[g]);
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* W8A16 linear (linear.py:83-137), exact accumulation                       */
/* ------------------------------------------------------------------------ */

int cbo_w8a16_linear(const void* x, int act_dtype, const int8_t* wq,
                     int64_t Kn, const int64_t* normal_cols,
                     const void* scales, const void* bias,
                     const int64_t* outlier_cols, int64_t n_out,
                     const void* w_out, int64_t M, int64_t N, int64_t K,
                     const int64_t* rows_idx, int64_t n_rows, float* y) {
    if (act_dtype < DT_F32 || act_dtype > DT_BF16) return 1;
    if (normal_cols == NULL && Kn != K) return 1;
    const int64_t R = rows_idx ? n_rows : M;
    for (int64_t ri = 0; ri < R; ++ri) {
        const int64_t m = rows_idx ? rows_idx[ri] : ri;
        if (m < 0 || m >= M) return 1;
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            const int8_t* wrow = wq + n * Kn;
            for (int64_t i = 0; i < Kn; ++i) {
                const int64_t k = normal_cols ? normal_cols[i] : i;
                acc += (double)load_one(x, act_dtype, m * K + k) * (double)wrow[i];
            }
            double out = acc * (double)load_one(scales, act_dtype, n);
            for (int64_t j = 0; j < n_out; ++j) {
                const int64_t k = outlier_cols[j];
                out += (double)load_one(x, act_dtype, m * K + k) *
                       (double)load_one(w_out, act_dtype, n * n_out + j);
            }
            if (bias) out += (double)load_one(bias, act_dtype, n);
            y[ri * N + n] = (float)out;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Dense GEMM (kernels/cuda/wmma.cu:29-169, host :186-261)                  */
/* ------------------------------------------------------------------------ */

/* C[m][n] = sum_k A[m][k] * B[k][n] with 8-bit integer operands (is_unsigned:
 * uint8, else int8) and int32 accumulation; the sum wraps modulo 2^32 as the
 * reference's int32 accumulator fragments do (wmma.cu:229-250). A is [M, K]
 * row-major; B is [K, N] row-major (b_nk == 0) or stored [N, K] (b_nk != 0). */
int cbo_mm_int8(const void* A, const void* B, int is_unsigned, int b_nk, int64_t M,
                int64_t N, int64_t K, int32_t* C) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            uint32_t acc = 0;
            for (int64_t k = 0; k < K; ++k) {
                const int64_t ib = b_nk ? n * K + k : k * N + n;
                int32_t a, b;
                if (is_unsigned) {
                    a = ((const uint8_t*)A)[m * K + k];
                    b = ((const uint8_t*)B)[ib];
                } else {
                    a = ((const int8_t*)A)[m * K + k];
                    b = ((const int8_t*)B)[ib];
                }
                acc += (uint32_t)(a * b);
            }
            C[m * N + n] = (int32_t)acc;
        }
    return 0;
}

/* The same for fp16 / bf16 operands (dtype codes as above), accumulated in
 * double: the exact product sum rounded once to double; callers compare
 * against it with a tolerance (the reference accumulates in fp32 or fp16
 * fragments, wmma.cu:173-176). */
int cbo_mm_float(const void* A, const void* B, int dtype, int b_nk, int64_t M, int64_t N,
                 int64_t K, double* C) {
    if (dtype != DT_F16 && dtype != DT_BF16) return 1;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const int64_t ib = b_nk ? n * K + k : k * N + n;
                acc += (double)load_one(A, dtype, m * K + k) * (double)load_one(B, dtype, ib);
            }
            C[m * N + n] = acc;
        }
    return 0;
}
