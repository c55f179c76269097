// cbq_w8a16.hip - W8A16 linear for gfx950: y = x . dequant(Wq)^T (+ outlier
// side-GEMM) (+ bias), one kernel.
//
// Replaces the reference forward chain (quantization/linear.py:83-137): the
// int8 -> activation-dtype copy of the weight (:105, :123), the transposed
// copy and Triton GEMM (bindings/triton/matmul.py:17-132,
// kernels/triton/matmul_kernel.py:9-99), the per-channel scale multiply
// (:113, :131), the outlier side-GEMM (:116-120) and the bias add (:134-135).
//
//   y[m, n] = T( s[n] * sum_k x[m, k] * wq[n, k]
//                + sum_j x[m, oc[j]] * w_out[n, j]          (n_out > 0)
//                + bias[n] )                                 (bias != null)
//
// fp32 accumulation, one rounding to T at the end (the reference rounds to T
// after the GEMM, after the scale multiply and after each add).
//
// k_w8a16_gemm: WG tile 128 (m) x 128 (n) x 64 (k), 4 waves in a 2 x 2 grid,
// each wave 64 x 64 as 4 x 4 v_mfma_f32_16x16x32_{f16,bf16} tiles. The MFMA
// A operand is the weight tile (rows n), B the activation tile (rows m), so
// each lane owns 4 consecutive n of one m and stores 8 contiguous bytes.
// INT8 weights are dequantized exactly (|q| <= 127) to the activation dtype
// on their way from registers into LDS; global loads of the next k-tile are
// in flight while the current one is multiplied (double-buffered LDS).
#include "cbq_device.h"
#include "cbq_host.h"

namespace cbq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

template <int ACT>
__device__ __forceinline__ f4 mfma16x16x32(const uint4& a, const uint4& b, f4 c) {
  if constexpr (ACT == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a),
                                                  __builtin_bit_cast(h8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a),
                                                   __builtin_bit_cast(b8, b), c, 0, 0, 0);
}

// 4 int8 codes -> 4 exact values of the activation dtype (2 words).
template <int ACT>
__device__ __forceinline__ void i8x4_to_act(uint32_t w, uint32_t& lo, uint32_t& hi) {
  if constexpr (ACT == kF16) {
    // fp16 0x6400 | b is 1024 + b for a byte b; b = q + 128, minus 1152 -> q.
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t l = (u & 0xffu) | ((u & 0xff00u) << 8) | 0x64006400u;
    const uint32_t h = ((u >> 16) & 0xffu) | ((u >> 8) & 0x00ff0000u) | 0x64006400u;
    const h2 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, l) - bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, h) - bias);
  } else {
    float f[4];
    int8x4_to_f32(w, f);
    lo = pack2_out<kBF16>(f[0], f[1]);
    hi = pack2_out<kBF16>(f[2], f[3]);
  }
}

template <int ACT>
__device__ __forceinline__ float act_to_f32(uint16_t v) {
  if constexpr (ACT == kBF16) return __uint_as_float(static_cast<uint32_t>(v) << 16);
  else return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;   // LDS row stride in 16-bit elements (144 bytes)

template <int ACT>
__global__ __launch_bounds__(kBlock, 2) void k_w8a16_gemm(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ bias,
    const int64_t* __restrict__ oc, int n_out, const uint16_t* __restrict__ w_out,
    uint16_t* __restrict__ y, int M, int N, int K, int tiles_m) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1;
  const int tm = static_cast<int>(blockIdx.x) % tiles_m;
  const int tn = static_cast<int>(blockIdx.x) / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  uint4 rx[4], rw[2];
  const uint4 zero = make_uint4(0, 0, 0, 0);

  // x tile: 128 rows x 64 values = 1024 16-byte chunks (4 per thread);
  // w tile: 128 rows x 64 codes = 512 16-byte chunks (2 per thread).
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + kBlock * u;
      const int m = m0 + (c >> 3), k = k0 + (c & 7) * 8;
      rx[u] = (m < M && k < K)
                  ? *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(m) * K + k)
                  : zero;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + kBlock * u;
      const int n = n0 + (c >> 2), k = k0 + (c & 3) * 16;
      rw[u] = (n < N && k < K)
                  ? *reinterpret_cast<const uint4*>(wq + static_cast<int64_t>(n) * K + k)
                  : zero;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + kBlock * u;
      *reinterpret_cast<uint4*>(&sX[buf][(c >> 3) * LDK + (c & 7) * 8]) = rx[u];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + kBlock * u;
      uint4 lo, hi;
      i8x4_to_act<ACT>(rw[u].x, lo.x, lo.y);
      i8x4_to_act<ACT>(rw[u].y, lo.z, lo.w);
      i8x4_to_act<ACT>(rw[u].z, hi.x, hi.y);
      i8x4_to_act<ACT>(rw[u].w, hi.z, hi.w);
      uint16_t* dst = &sW[buf][(c >> 2) * LDK + (c & 3) * 16];
      *reinterpret_cast<uint4*>(dst) = lo;
      *reinterpret_cast<uint4*>(dst + 8) = hi;
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nk = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;
  for (int t = 0; t < nk; ++t) {
    const int cur = t & 1;
    if (t + 1 < nk) gload((t + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      uint4 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const uint4*>(
            &sW[cur][(wn * 64 + i * 16 + frag_row) * LDK + kk + frag_k]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const uint4*>(
            &sX[cur][(wm * 64 + j * 16 + frag_row) * LDK + kk + frag_k]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32<ACT>(a[i], b[j], acc[i][j]);
    }
    if (t + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns y[m, nb .. nb+3] of each 16 x 16 tile.
  const bool vec_store = (N % 4) == 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wm * 64 + j * 16 + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nb = n0 + wn * 64 + i * 16 + (lane >> 4) * 4;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nb + r;
        float val = 0.0f;
        if (n < N) {
          val = acc[i][j][r] * act_to_f32<ACT>(scales[n]);
          for (int jj = 0; jj < n_out; ++jj) {
            const int64_t k = oc[jj];
            if (k >= 0 && k < K)
              val += act_to_f32<ACT>(x[static_cast<int64_t>(m) * K + k]) *
                     act_to_f32<ACT>(w_out[static_cast<int64_t>(n) * n_out + jj]);
          }
          if (bias) val += act_to_f32<ACT>(bias[n]);
        }
        v[r] = val;
      }
      uint16_t* dst = y + static_cast<int64_t>(m) * N + nb;
      if (vec_store && nb + 3 < N) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack2_out<ACT>(v[0], v[1]),
                                                    pack2_out<ACT>(v[2], v[3]));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) dst[r] = out1<ACT>(v[r]);
      }
    }
  }
}

// Any shape or activation dtype (fp32 activations, K not a multiple of 16,
// unaligned pointers): one output per thread, fp32 accumulation in k order.
template <int ACT>
__global__ __launch_bounds__(kBlock) void k_w8a16_simple(
    const void* __restrict__ x, const int8_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ bias, const int64_t* __restrict__ oc, int64_t n_out,
    const void* __restrict__ w_out, void* __restrict__ y, int64_t M, int64_t N, int64_t K) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx % N;
  float acc = 0.0f;
  for (int64_t k = 0; k < K; ++k) acc += ld1<ACT>(x, m * K + k) * static_cast<float>(wq[n * K + k]);
  float val = acc * ld1<ACT>(scales, n);
  for (int64_t jj = 0; jj < n_out; ++jj) {
    const int64_t k = oc[jj];
    if (k >= 0 && k < K) val += ld1<ACT>(x, m * K + k) * ld1<ACT>(w_out, n * n_out + jj);
  }
  if (bias) val += ld1<ACT>(bias, n);
  if constexpr (ACT == kF32) static_cast<float*>(y)[idx] = val;
  else static_cast<uint16_t*>(y)[idx] = out1<ACT>(val);
}

template <int ACT>
int w8a16_simple(const void* x, const int8_t* wq, const void* scales, const void* bias,
                 const int64_t* oc, int64_t n_out, const void* w_out, int64_t M, int64_t N,
                 int64_t K, void* y, hipStream_t s) {
  const int64_t blocks = cdiv(M * N, kBlock);
  if (blocks > 0x7fffffffLL / kBlock) {
    set_error("cbq_w8a16_linear: output too large for the general path");
    return CBQ_EINVAL;
  }
  k_w8a16_simple<ACT><<<dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s>>>(
      x, wq, scales, bias, oc, n_out, w_out, y, M, N, K);
  return launch_status("cbq_w8a16_linear");
}

template <int ACT>
int w8a16_t(const void* x, const int8_t* wq, const void* scales, const void* bias,
            const int64_t* oc, int64_t n_out, const void* w_out, int64_t M, int64_t N, int64_t K,
            void* y, hipStream_t s) {
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ss = static_cast<const uint16_t*>(scales);
  const auto* bs = static_cast<const uint16_t*>(bias);
  const auto* wo = static_cast<const uint16_t*>(w_out);
  auto* ys = static_cast<uint16_t*>(y);
  const bool fast = (K % 16 == 0) && aligned(x, 16) && aligned(wq, 16) && aligned(y, 8) &&
                    M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= 0x7fffffffLL;
  if (fast) {
    const int64_t tiles_m = cdiv(M, BM), tiles_n = cdiv(N, BN);
    const int64_t tiles = tiles_m * tiles_n;
    if (tiles > 0x7fffffffLL / kBlock) {
      set_error("cbq_w8a16_linear: too many output tiles (%lld)", (long long)tiles);
      return CBQ_EINVAL;
    }
    k_w8a16_gemm<ACT><<<dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0, s>>>(
        xs, wq, ss, bs, oc, static_cast<int>(n_out), wo, ys, static_cast<int>(M),
        static_cast<int>(N), static_cast<int>(K), static_cast<int>(tiles_m));
  } else {
    return w8a16_simple<ACT>(x, wq, scales, bias, oc, n_out, w_out, M, N, K, y, s);
  }
  return launch_status("cbq_w8a16_linear");
}

}  // namespace
}  // namespace cbq

using namespace cbq;

extern "C" size_t cbq_w8a16_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t n_out) {
  (void)M; (void)N; (void)K; (void)n_out;
  return CBQ_WS_CTRL_BYTES;
}

extern "C" int cbq_w8a16_linear(const void* x, int act_dtype, const int8_t* wq,
                                const void* scales, const void* bias,
                                const int64_t* outlier_cols, int64_t n_out, const void* w_out,
                                int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes,
                                void* y, cbq_stream_t stream) {
  clear_error();
  (void)ws; (void)ws_bytes;
  const char* what = "cbq_w8a16_linear";
  CBQ_REQUIRE(act_dtype == kF16 || act_dtype == kBF16 || act_dtype == kF32,
              "%s: activation dtype must be fp16, bf16 or fp32 (code %d)", what, act_dtype);
  CBQ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && n_out >= 0, "%s: negative size", what);
  CBQ_REQUIRE(n_out <= 0x7fffffffLL, "%s: too many outlier columns", what);
  if (M == 0 || N == 0) return CBQ_OK;
  CBQ_REQUIRE(x && wq && scales && y, "%s: null pointer", what);
  CBQ_REQUIRE(n_out == 0 || (outlier_cols && w_out), "%s: outlier columns need indices and weights",
              what);
  if (act_dtype == kF32)
    return w8a16_simple<kF32>(x, wq, scales, bias, outlier_cols, n_out, w_out, M, N, K, y,
                              as_stream(stream));
  return act_dtype == kF16
             ? w8a16_t<kF16>(x, wq, scales, bias, outlier_cols, n_out, w_out, M, N, K, y,
                             as_stream(stream))
             : w8a16_t<kBF16>(x, wq, scales, bias, outlier_cols, n_out, w_out, M, N, K, y,
                              as_stream(stream));
}
