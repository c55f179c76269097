/*
 * cublade_quant.h - C ABI of the MI355X (gfx950) quantization library
 * libcublade_quant.so.
 *
 * Every entry point takes raw device pointers, element counts, dtype codes and
 * a HIP stream, launches asynchronously on that stream, and returns a status
 * code (CBQ_OK on success). No entry point allocates, frees or synchronises:
 * the caller owns every buffer, including the workspace. On failure
 * cbq_last_error() returns a thread-local message.
 *
 * Each function names the reference interface it replaces (paths relative to
 * the cuBlade source tree, package `cublade`). The reference's pybind entry
 * points allocate their outputs and launch on the legacy default stream; here
 * the caller allocates and chooses the stream.
 *
 * Numerics (all bit-exact restatements of the reference kernels):
 *   amax  = max |x| (NaN inputs ignored), per tensor / row / column / group
 *   inv   = fp32(Q / max(amax, eps))     Q = 448 (FP8 E4M3) or 127 (INT8),
 *                                        IEEE correctly rounded division
 *   q     = FP8:  e4m3fn(x * inv), round-to-nearest-even, saturated to +-448
 *           INT8: clamp(round_half_even(x * inv), -127, 127), NaN -> 0
 *   scale = fp32(1 / inv)
 *   dequant y = T(float(q) * scale), round-to-nearest-even to fp16 / bf16
 */
#ifndef CUBLADE_QUANT_H
#define CUBLADE_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t passed as an opaque pointer (NULL = the null stream). */
typedef void* cbq_stream_t;

/* Floating-point dtype codes for activations, inputs and outputs. */
enum { CBQ_F32 = 0, CBQ_F16 = 1, CBQ_BF16 = 2 };
/* Integer dtype codes (GEMM operands and accumulators). */
enum { CBQ_I8 = 3, CBQ_U8 = 4, CBQ_I32 = 5 };

/* Status codes. */
enum { CBQ_OK = 0, CBQ_EINVAL = 1, CBQ_ELAUNCH = 2 };

/* Workspace contract.  Entry points that take (ws, ws_bytes) need a
 * 16-byte aligned device buffer of at least the size their *_ws_bytes query
 * returns. The first CBQ_WS_CTRL_BYTES bytes are a control block: zero-fill
 * it once before the first call on that workspace and do not write to it
 * afterwards (zero-filling all of it again between calls is allowed: it
 * resets it). The per-tensor quant entry points keep their cross-workgroup
 * state there (a generation tag at byte 0, the tag of the last call that
 * timed out at byte 520, tagged per-workgroup slots from byte 1024) and a
 * sticky int32 status word at byte 512 (cbq_tensor_quant_status): 1 once the
 * workgroups of a call gave up waiting for each other (only possible when
 * other work keeps part of the grid off the GPU for about a second). Such a
 * call writes a NaN scale whenever any of its codes is not exact (FP8 codes
 * NaN, INT8 codes 0 there); a scale that is not NaN comes with every code
 * exact. The next call on the workspace is exact again, with no reset; the
 * status word stays 1 until cbq_tensor_quant_status_clear. The other entry
 * points leave the control block alone. The rest is per-call scratch. One
 * workspace serves one stream at a time: calls that overlap in time must not
 * share it. */
#define CBQ_WS_CTRL_BYTES 16384

/* Message of the last failed call on this thread ("" if none). */
const char* cbq_last_error(void);

/* ABI version (major * 100 + minor). A caller built against another major
 * version must not call the library: signatures differ between majors. */
int cbq_abi_version(void);

/* Workspace bytes needed by cbq_quant_fp8_tensor / cbq_quant_int8_tensor
 * (one partial maximum per workgroup of the persistent grid). */
size_t cbq_quant_tensor_ws_bytes(void);

/* Workspace bytes needed by cbq_quant_int8_channel (axis 1 needs per-column
 * partial maxima; axis 0 needs only the control block, except for few long
 * rows, cut into slices over the CUs with one partial maximum per slice: with
 * a smaller workspace those take the one-workgroup-per-row path). */
size_t cbq_quant_int8_channel_ws_bytes(int64_t rows, int64_t cols, int axis);

/* ---- FP8 E4M3 per tensor ------------------------------------------------ */

/* Replaces quantize_per_tensor_fp8_cuda (kernels/cuda/quantization/
 * quantize_per_tensor_fp8.cu:162-182; kernels :38-132), bound as
 * cublade.bindings.cuda.quantize_fp8.quantize_per_tensor_fp8
 * (bindings/cuda/quantize_fp8.py:15-34).
 * x: n elements of dtype CBQ_F16 or CBQ_BF16. q: n FP8 E4M3 codes.
 * scale: one fp32, written when n > 0. ws: cbq_quant_tensor_ws_bytes(). */
int cbq_quant_fp8_tensor(const void* x, int dtype, int64_t n, float eps,
                         void* ws, size_t ws_bytes, uint8_t* q, float* scale,
                         cbq_stream_t stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): cbq_quant_fp8_tensor without the workspace argument, same
 * kernels and results. Its workspace is a 24 KiB static device array inside
 * the library, one per GPU, held until the process ends and shared by every
 * call on that GPU: calls that overlap in time on one GPU (other streams,
 * other threads) race and must be serialised by the caller. Allocates nothing;
 * the first call on a device looks the array's address up
 * (hipGetSymbolAddress), so make that call outside graph capture. A timed-out
 * exchange behaves as described under the workspace contract: read and clear
 * its status with cbq_tensor_quant_status / _clear and ws = NULL. */
int cbq_quant_fp8_tensor_noalloc(const void* x, int dtype, int64_t n, float eps,
                                 uint8_t* q, float* scale, cbq_stream_t stream);

/* No counterpart in the reference (its per-tensor kernels never wait on each
 * other). Status of the one-launch per-tensor quant's control block:
 * *status = the sticky word described under the workspace contract (0: no
 * call on this workspace timed out since the word was last cleared). ws: a
 * workspace given to cbq_quant_{fp8,int8}_tensor, or NULL for the static
 * array of cbq_quant_fp8_tensor_noalloc on the current device. Reads the word
 * in stream order and synchronises the stream (not under graph capture). */
int cbq_tensor_quant_status(const void* ws, cbq_stream_t stream, int* status);

/* Clears that status word, in stream order (a one-thread kernel: allowed
 * under graph capture). ws as for cbq_tensor_quant_status. */
int cbq_tensor_quant_status_clear(void* ws, cbq_stream_t stream);

/* Sets how many polls a per-tensor quant's workgroups make while waiting for
 * each other before they give up (default 1048576, about a second; the
 * environment variable CBQ_TENSOR_SPIN_LIMIT read at the first call
 * overrides the default). Takes effect for later launches; returns the
 * previous value. 0 makes every workgroup that does not find all the others
 * at its first poll give up: tests use it to force the timeout path while
 * every kernel still ends normally. */
uint32_t cbq_set_tensor_spin_limit(uint32_t polls);

/* Replaces dequantize_per_tensor_fp8_cuda (dequantize_per_tensor_fp8.cu:84-109;
 * kernel :23-66), bound as dequantize_fp8.dequantize_per_tensor_fp8
 * (bindings/cuda/dequantize_fp8.py:15-35). out_dtype: CBQ_F16 or CBQ_BF16. */
int cbq_dequant_fp8_tensor(const uint8_t* q, const float* scale, int64_t n,
                           void* y, int out_dtype, cbq_stream_t stream);

/* ---- INT8 --------------------------------------------------------------- */

/* Replaces quantize_per_tensor_int8_cuda (quantize_int8.cu:470-484; kernels
 * :47-166), bound as quantize_int8.quantize_per_tensor_int8
 * (bindings/cuda/quantize_int8.py:18-38). dtype: CBQ_F32/F16/BF16. */
int cbq_quant_int8_tensor(const void* x, int dtype, int64_t n, float eps,
                          void* ws, size_t ws_bytes, int8_t* q, float* scale,
                          cbq_stream_t stream);

/* Replaces quantize_per_channel_int8_cuda (quantize_int8.cu:487-509; kernels
 * :173-297), bound as quantize_int8.quantize_per_channel_int8
 * (bindings/cuda/quantize_int8.py:41-62). x is viewed as rows x cols.
 * axis 0: one scale per row (the reference's only axis); axis 1: one scale per
 * column (an extension: same math with the maximum taken over rows).
 * Unlike the reference, cols need not be a multiple of 16 / element size. */
int cbq_quant_int8_channel(const void* x, int dtype, int64_t rows, int64_t cols,
                           int axis, float eps, void* ws, size_t ws_bytes,
                           int8_t* q, float* scale, cbq_stream_t stream);

/* Replaces quantize_per_group_int8_cuda (quantize_int8.cu:514-536; kernels
 * :307-371), bound as quantize_int8.quantize_per_group_int8
 * (bindings/cuda/quantize_int8.py:65-87). x: num_groups x group_size,
 * 0 < group_size <= 4096. scale: num_groups fp32. */
int cbq_quant_int8_group(const void* x, int dtype, int64_t num_groups,
                         int64_t group_size, float eps, int8_t* q, float* scale,
                         cbq_stream_t stream);

/* ---- N-D axes without transposing copies --------------------------------- */

/* Channel quant over any axis of an N-D tensor, viewed as outer x channels x
 * inner (channels = the axis length, outer/inner the products of the dims
 * before/after it); one fp32 scale per channel. The reference only supports
 * the leading axis (quantizers.py:116-121, quantize_int8.cu:487-509); this is
 * the same math with the channel maximum taken over outer and inner, and no
 * copies. outer == 1 runs the row kernels (the control block only, or the
 * slices' partial maxima for few long rows, as cbq_quant_int8_channel axis 0).
 * Otherwise the
 * workspace below holds, for inner >= 512, [outer, channels] segment maxima
 * plus [channels] multipliers; for shorter inner, the column path's partial
 * maxima over outer x (channels * inner). */
size_t cbq_quant_int8_channel_nd_ws_bytes(int64_t outer, int64_t channels,
                                          int64_t inner);
int cbq_quant_int8_channel_nd(const void* x, int dtype, int64_t outer,
                              int64_t channels, int64_t inner, float eps,
                              void* ws, size_t ws_bytes, int8_t* q,
                              float* scale, cbq_stream_t stream);

/* Group quant along any axis, viewed as outer x len x inner with groups of
 * group_size consecutive positions along len. Replaces the reference's
 * movedim(ch_axis, -1).contiguous() / view(-1, G) / kernel / movedim-back
 * sequence (quantizers.py:122-132, two full copies) with no copies. scale:
 * outer * inner * (len / group_size) fp32 in the reference's order,
 * index (o * inner + i) * (len / group_size) + g. The workspace (optional:
 * null or smaller gives the same results, slower) holds the scales in
 * group-major order before one transposing pass writes that order:
 * cbq_quant_int8_group_nd_ws_bytes() = the control block + 4 bytes per scale
 * when inner % 8 == 0 and more than one group lies along len, else the
 * control block. */
size_t cbq_quant_int8_group_nd_ws_bytes(int64_t outer, int64_t len,
                                        int64_t inner, int64_t group_size);
int cbq_quant_int8_group_nd(const void* x, int dtype, int64_t outer,
                            int64_t len, int64_t inner, int64_t group_size,
                            float eps, void* ws, size_t ws_bytes, int8_t* q,
                            float* scale, cbq_stream_t stream);

/* Replaces dequantize_per_tensor_int8_cuda (dequantize_int8.cu:210-225; kernel
 * :29-64), bound as dequantize_int8.dequantize_per_tensor_int8
 * (bindings/cuda/dequantize_int8.py:18-38). */
int cbq_dequant_int8_tensor(const int8_t* q, const float* scale, int64_t n,
                            void* y, int out_dtype, cbq_stream_t stream);

/* Replaces dequantize_per_channel_int8_cuda (dequantize_int8.cu:227-247;
 * kernel :70-109), bound as dequantize_int8.dequantize_per_channel_int8
 * (bindings/cuda/dequantize_int8.py:41-58). axis 0: scale[rows];
 * axis 1 (extension): scale[cols]. */
int cbq_dequant_int8_channel(const int8_t* q, const float* scale, int64_t rows,
                             int64_t cols, int axis, void* y, int out_dtype,
                             cbq_stream_t stream);

/* Replaces dequantize_per_group_int8_cuda (dequantize_int8.cu:249-273; kernel
 * :118-134), bound as dequantize_int8.dequantize_per_group_int8
 * (bindings/cuda/dequantize_int8.py:61-79). */
int cbq_dequant_int8_group(const int8_t* q, const float* scale,
                           int64_t num_groups, int64_t group_size, void* y,
                           int out_dtype, cbq_stream_t stream);

/* Channel dequant over any axis (outer x channels x inner, scale[channels]);
 * the reference only dequantizes axis 0 (dequantizers.py:51-57). */
int cbq_dequant_int8_channel_nd(const int8_t* q, const float* scale,
                                int64_t outer, int64_t channels, int64_t inner,
                                void* y, int out_dtype, cbq_stream_t stream);

/* Group dequant along any axis (outer x len x inner, scale order as in
 * cbq_quant_int8_group_nd). Replaces the movedim / view / kernel / movedim
 * sequence of dequantizers.py:58-72 (two full copies). The workspace
 * (optional: null or smaller gives the same results, slower) receives the
 * scales transposed to group-major order, read contiguously by the kernel;
 * cbq_dequant_int8_group_nd_ws_bytes() sizes it as for the group quant. */
size_t cbq_dequant_int8_group_nd_ws_bytes(int64_t outer, int64_t len,
                                          int64_t inner, int64_t group_size);
int cbq_dequant_int8_group_nd(const int8_t* q, const float* scale,
                              int64_t outer, int64_t len, int64_t inner,
                              int64_t group_size, void* ws, size_t ws_bytes,
                              void* y, int out_dtype, cbq_stream_t stream);

/* ---- W8A16 linear ------------------------------------------------------- */

/* Workspace bytes for cbq_w8a16_linear at this shape and activation dtype:
 * the control block, plus the split-K scratch of the kernel that dtype
 * selects. CBQ_F16 / CBQ_BF16 with K % 16 == 0 (MFMA): for M > 64 when the
 * last wave of output tiles is short, the fp32 partial tiles of that wave
 * (ranges x tail tiles x 256 / 192 / 128 KiB for tiles of 256 / 192 / 128 x
 * 256; at most 16 ranges and at most one partial tile per CU, i.e. <= 64 MiB
 * on MI355X; the same with outlier columns), else nothing. CBQ_F32 on the matrix-core path (see
 * cbq_w8a16_linear): two bf16 planes of x (4 M K bytes) and the fp32
 * partial tiles of both planes (8 bytes per output of the padded tiles; for
 * M <= 64 times the k-ranges per plane, at most 8: 32 MB at M = 16, N = 4096,
 * K = 11008), capped at 256 MiB: a larger M runs in chunks of rows
 * (multiples of 256, one after another, reusing the workspace), so the size
 * is that of the largest chunk (M = 4096, N = 11008, K = 4096: chunks of 2560
 * and 1536 rows, 241 MB instead of 428 MB; chunks of 256 rows that alone
 * exceed the cap are used as they are). Other CBQ_F32
 * shapes and K % 16 != 0 (general kernel): fp32 partial sums, up to 16 x M x
 * N x 4 bytes when its tiles give fewer than two workgroups per CU. The
 * reference allocates its temporaries inside the forward (linear.py:105-131). */
size_t cbq_w8a16_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t n_out, int act_dtype);

/* Replaces the forward chain of cuBladeW8A16LinearLayer
 * (quantization/linear.py:83-137): int8 -> activation copy of the weight
 * (:105, :123), the Triton GEMM bindings/triton/matmul.py:17-132 (kernel
 * kernels/triton/matmul_kernel.py:9-99), the per-channel scale multiply
 * (:113, :131), the outlier side-GEMM (:116-120) and the bias add (:134-135),
 * in one launch:
 *   y[m,n] = T( s[n] * sum_k x[m,k] * wq[n,k]
 *               + sum_j x[m, outlier_cols[j]] * w_out[n,j] + bias[n] )
 * with fp32 accumulation and one final round-to-nearest-even to T.
 * x: [M,K] and y: [M,N] in act_dtype, row-major. CBQ_F16 / CBQ_BF16 run
 * on MFMA. CBQ_F32 (the reference's fp32 Triton path, TF32 precision on its
 * hardware) with K % 64 == 0, no outlier columns, M > 64 or a weight of at
 * least 8 MB, and a workspace of cbq_w8a16_ws_bytes also runs on MFMA (for
 * M <= 64 with K split into up to 8 ranges): x is split into two bf16 planes
 * (hi = x truncated, lo = bf16(x - hi): 16 significant bits of x, exact
 * products with the int8 weights, fp32 accumulation); other CBQ_F32 calls,
 * K % 16 != 0 and unaligned operands run a tiled fp32-FMA kernel. K == 0
 * gives y = bias (or 0); x and wq may then be null.
 * wq: int8 [N,K] row-major; its outlier columns hold 0.
 * scales, bias (nullable): [N] act_dtype. outlier_cols: n_out int64 indices in
 * [0, K) (nullable when n_out == 0); w_out: [N, n_out] act_dtype.
 * ws: cbq_w8a16_ws_bytes(...) bytes, 256-byte aligned, control block zeroed;
 * a smaller or missing workspace selects a kernel without split-K (same
 * results within fp32 accumulation order, slower at those shapes). */
int cbq_w8a16_linear(const void* x, int act_dtype, const int8_t* wq,
                     const void* scales, const void* bias,
                     const int64_t* outlier_cols, int64_t n_out,
                     const void* w_out, int64_t M, int64_t N, int64_t K,
                     void* ws, size_t ws_bytes, void* y, cbq_stream_t stream);

/* ---- Dense GEMM on the matrix cores -------------------------------------- */

/* Storage of B for cbq_mm: [K, N] row-major (the reference's layout), or
 * [N, K] row-major, i.e. B = W^T for a weight W [N, K] (read in place). */
enum { CBQ_MM_B_KN = 0, CBQ_MM_B_NK = 1 };

/* Workspace bytes for cbq_mm at this shape: the control block, plus staging
 * buffers when B is [K, N] (transposed copy), the inputs are uint8 (offset
 * copies and row sums) or K * element bytes is not a multiple of 64 (padded
 * copies), plus, when the 256 x 256 output tiles are fewer than the CUs,
 * the 4-byte partial sums of a split over K (up to 16 x M x N x 4 bytes). */
size_t cbq_mm_ws_bytes(int64_t M, int64_t N, int64_t K, int in_dtype,
                       int b_layout);

/* Replaces wmma_gemm (kernels/cuda/wmma.cu:186-261, kernel :29-169), bound as
 * bindings/cuda/wmma.py:15-43: C[M,N] = A[M,K] . B[K,N], row-major A and C.
 * in_dtype -> out_dtype, as the reference's precision table:
 *   CBQ_I8 -> CBQ_I32, CBQ_U8 -> CBQ_I32 (exact modulo 2^32),
 *   CBQ_F16 -> CBQ_F32 or CBQ_F16, CBQ_BF16 -> CBQ_F32
 * (fp32 accumulation; fp16 output rounded once at the end).
 * M, N, K multiples of 16 (the reference's WMMA constraint); A, B and C
 * 16-byte aligned; ws: cbq_mm_ws_bytes(...) bytes, 256-byte aligned.
 * K == 0 gives C = 0; A and B may then be null. */
int cbq_mm(const void* A, const void* B, int in_dtype, int b_layout,
           int64_t M, int64_t N, int64_t K, void* C, int out_dtype, void* ws,
           size_t ws_bytes, cbq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CUBLADE_QUANT_H */
