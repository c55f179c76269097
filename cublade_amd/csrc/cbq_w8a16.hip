// cbq_w8a16.hip - W8A16 linear for gfx950: y = x . dequant(Wq)^T (+ outlier
// side-GEMM) (+ bias), one kernel per call.
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
// k_gemm<ACT, BM, BN, BK, WGM, WGN>: output tile BM (m) x BN (n), k-step BK,
// WGM x WGN waves, each wave (BM/WGM) x (BN/WGN) as 16 x 16 tiles of
// v_mfma_f32_16x16x32_{f16,bf16}. The MFMA A operand is the weight tile (rows
// n), B the activation tile (rows m), so a lane owns 4 consecutive n of one m
// and stores 8 contiguous bytes. INT8 weights are dequantized exactly
// (|q| <= 127) to the activation dtype on their way from registers into LDS;
// the next k-tile's global loads are in flight while the current one is
// multiplied: two LDS buffers and two register staging buffers (prefetch
// distance two), one barrier per k-step.
//
// Tile order: workgroups are dispatched round-robin over the 8 XCDs, each
// with its own L2. Workgroup b is renumbered so that XCD b % 8 receives a
// contiguous run of tiles, and tiles run in groups of 8 m-tiles, so the
// workgroups resident on one XCD share activation and weight k-slices in L2.
//
// k_skinny<ACT, TM, TN, U> (M <= 64): weight streaming with the K split across
// the waves of a workgroup and reduced through LDS (see below). A split of K
// across workgroups was measured slower on MI355X: publishing partial tiles
// needs agent-scope release fences, which write back the whole L2.
#include <type_traits>

#include "cbq_device.h"
#include "cbq_host.h"

namespace cbq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Operands and staging registers use native vector types: HIP's uint4 is a
// struct around a union, and arrays of it are kept on the stack (scratch or
// LDS) instead of in VGPRs.
template <int ACT>
__device__ __forceinline__ f4 mfma16x16x32(const u32x4& a, const u32x4& b, f4 c) {
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

struct GemmArgs {
  const uint16_t* x;        // [M, K]
  const int8_t* wq;         // [N, K]
  const uint16_t* scales;   // [N]
  const uint16_t* bias;     // [N] or null
  const int64_t* oc;        // [n_out]
  const uint16_t* w_out;    // [N, n_out]
  uint16_t* y;              // [M, N]
  int M, N, K, n_out;
  int tiles_m, tiles_n;
};

// Workgroup -> (tile m, tile n); see the file comment.
__device__ __forceinline__ void decode_tile(int b, const GemmArgs& a, int& tm, int& tn) {
  const int total = a.tiles_m * a.tiles_n;
  const int per = total >> 3;
  if (b < per * 8) b = (b & 7) * per + (b >> 3);
  const int t = b;
  constexpr int G = 8;
  const int group = t / (G * a.tiles_n);
  const int first_m = group * G;
  const int gsize = min(a.tiles_m - first_m, G);
  const int r = t % (G * a.tiles_n);
  tm = first_m + r % gsize;
  tn = r / gsize;
}

template <int ACT, int BM, int BN, int BK, int WGM, int WGN, int PD>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm(GemmArgs a) {
  static_assert(PD == 1 || PD == 2, "prefetch distance");
  constexpr int T = 64 * WGM * WGN;
  constexpr int TM = BM / WGM / 16, TN = BN / WGN / 16;
  constexpr int LDK = BK + 8;                 // LDS row stride, 16-bit elements
  constexpr int XC = BM * BK / 8;             // 16-byte chunks (8 values) of x
  constexpr int WC = BN * BK / 16;            // 16-byte chunks (16 codes) of w
  constexpr int XCH = (XC + T - 1) / T, WCH = (WC + T - 1) / T;
  static_assert(TM >= 1 && TN >= 1 && BK % 32 == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  int tm, tn;
  decode_tile(blockIdx.x, a, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int k_begin = 0;
  const int k_end = a.K;
  const int nk = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;

  // PD register staging buffers. With PD == 2, tile t+2 is loaded while tile
  // t is multiplied and tile t+1 waits in the other buffer (global latency
  // hidden behind two k-steps); PD == 1 uses one buffer (fewer VGPRs). Buffer
  // indices are compile-time (the k loop is unrolled by two) so the buffers
  // stay in VGPRs.
  u32x4 rx[PD][XCH], rw[PD][WCH];
  const u32x4 zero = {0u, 0u, 0u, 0u};
  auto gload = [&](u32x4 (&gx)[XCH], u32x4 (&gw)[WCH], int k0) {
#pragma unroll
    for (int u = 0; u < XCH; ++u) {
      const int c = tid + T * u;
      const int m = m0 + c / (BK / 8), k = k0 + (c % (BK / 8)) * 8;
      gx[u] = (c < XC && m < a.M && k < k_end)
                  ? *reinterpret_cast<const u32x4*>(a.x + static_cast<int64_t>(m) * a.K + k)
                  : zero;
    }
#pragma unroll
    for (int u = 0; u < WCH; ++u) {
      const int c = tid + T * u;
      const int n = n0 + c / (BK / 16), k = k0 + (c % (BK / 16)) * 16;
      gw[u] = (c < WC && n < a.N && k < k_end)
                  ? *reinterpret_cast<const u32x4*>(a.wq + static_cast<int64_t>(n) * a.K + k)
                  : zero;
    }
  };
  auto sstore = [&](const u32x4 (&gx)[XCH], const u32x4 (&gw)[WCH], uint16_t* lx, uint16_t* lw) {
#pragma unroll
    for (int u = 0; u < XCH; ++u) {
      const int c = tid + T * u;
      if (c < XC)
        *reinterpret_cast<u32x4*>(&lx[(c / (BK / 8)) * LDK + (c % (BK / 8)) * 8]) = gx[u];
    }
#pragma unroll
    for (int u = 0; u < WCH; ++u) {
      const int c = tid + T * u;
      if (c < WC) {
        uint32_t o[8];
        i8x4_to_act<ACT>(gw[u].x, o[0], o[1]);
        i8x4_to_act<ACT>(gw[u].y, o[2], o[3]);
        i8x4_to_act<ACT>(gw[u].z, o[4], o[5]);
        i8x4_to_act<ACT>(gw[u].w, o[6], o[7]);
        uint16_t* dst = &lw[(c / (BK / 16)) * LDK + (c % (BK / 16)) * 16];
        *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<u32x4*>(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
      }
    }
  };

  f4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;
  auto compute = [&](const uint16_t* lx, const uint16_t* lw) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      u32x4 fa[TN], fb[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i)
        fa[i] = *reinterpret_cast<const u32x4*>(
            &lw[(wn * (BN / WGN) + i * 16 + frag_row) * LDK + kk + frag_k]);
#pragma unroll
      for (int j = 0; j < TM; ++j)
        fb[j] = *reinterpret_cast<const u32x4*>(
            &lx[(wm * (BM / WGM) + j * 16 + frag_row) * LDK + kk + frag_k]);
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = mfma16x16x32<ACT>(fa[i], fb[j], acc[i][j]);
    }
  };
  // One k-step: tile t sits in LDS buffer P, tile t+1 in registers 1-P.
  auto step = [&](int t, auto parity) {
    constexpr int P = decltype(parity)::value;
    if (t + 2 < nk) gload(rx[P % PD], rw[P % PD], k_begin + (t + 2) * BK);
    compute(sX[P], sW[P]);
    if (t + 1 < nk) sstore(rx[(1 - P) % PD], rw[(1 - P) % PD], sX[1 - P], sW[1 - P]);
    __syncthreads();
  };

  if constexpr (PD == 2) {
    if (nk > 0) {
      gload(rx[0], rw[0], k_begin);
      if (nk > 1) gload(rx[1], rw[1], k_begin + BK);
      sstore(rx[0], rw[0], sX[0], sW[0]);
      __syncthreads();
    }
    for (int t = 0; t < nk; t += 2) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < nk) step(t + 1, std::integral_constant<int, 1>{});
    }
  } else {
    // Prefetch distance one: a single staging buffer (fewer VGPRs).
    auto step1 = [&](int t, auto parity) {
      constexpr int P = decltype(parity)::value;
      if (t + 1 < nk) gload(rx[0], rw[0], k_begin + (t + 1) * BK);
      compute(sX[P], sW[P]);
      if (t + 1 < nk) sstore(rx[0], rw[0], sX[1 - P], sW[1 - P]);
      __syncthreads();
    };
    if (nk > 0) {
      gload(rx[0], rw[0], k_begin);
      sstore(rx[0], rw[0], sX[0], sW[0]);
      __syncthreads();
    }
    for (int t = 0; t < nk; t += 2) {
      step1(t, std::integral_constant<int, 0>{});
      if (t + 1 < nk) step1(t + 1, std::integral_constant<int, 1>{});
    }
  }

  // Epilogue: lane owns y[m, nb .. nb+3] of each 16 x 16 tile.
  const bool vec_store = (a.N % 4) == 0;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int m = m0 + wm * (BM / WGM) + j * 16 + (lane & 15);
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int nb = n0 + wn * (BN / WGN) + i * 16 + (lane >> 4) * 4;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nb + r;
        float val = 0.0f;
        if (n < a.N) {
          val = acc[i][j][r] * act_to_f32<ACT>(a.scales[n]);
          for (int jj = 0; jj < a.n_out; ++jj) {
            const int64_t k = a.oc[jj];
            if (k >= 0 && k < a.K)
              val += act_to_f32<ACT>(a.x[static_cast<int64_t>(m) * a.K + k]) *
                     act_to_f32<ACT>(a.w_out[static_cast<int64_t>(n) * a.n_out + jj]);
          }
          if (a.bias) val += act_to_f32<ACT>(a.bias[n]);
        }
        v[r] = val;
      }
      uint16_t* dst = a.y + static_cast<int64_t>(m) * a.N + nb;
      if (vec_store && nb + 3 < a.N) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack2_out<ACT>(v[0], v[1]),
                                                    pack2_out<ACT>(v[2], v[3]));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < a.N) dst[r] = out1<ACT>(v[r]);
      }
    }
  }
}

// Small M (M <= 16 * TM): weight streaming. A workgroup owns 16 * TN weight
// rows; its 4 waves take a quarter of K each and stream those rows straight
// from HBM into registers (16 bytes per lane per row tile and 64-k block, U
// blocks in flight), with the activation fragments read from L2 (x is small
// and shared by every workgroup) and reused for the TN row tiles. Per 64-k
// block a lane holds W[n][k0 + 16 g .. +16] and x[m][k0 + 16 g .. +16]
// (g = lane / 16) and issues two MFMAs on the low and high 8 values: A and B
// lanes of the same group see the same k, which is all the MFMA contraction
// needs. The 4 partial tiles are summed through LDS in wave order
// (deterministic) and wave 0 runs the epilogue.
template <int ACT, int TM, int TN, int U>
__global__ __launch_bounds__(256) void k_skinny(GemmArgs a) {
  __shared__ f4 red[3][TN][TM][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16 * TN;
  const int row = lane & 15, g = lane >> 4;
  const int kq = ((a.K / 4 + 15) / 16) * 16;
  const int kb = min(a.K, wave * kq), ke = min(a.K, kb + kq);
  const u32x4 zero = {0u, 0u, 0u, 0u};

  f4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int k0 = kb; k0 < ke; k0 += 64 * U) {
    u32x4 w[U][TN], xl[U][TM], xh[U][TM];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + u * 64 + g * 16;
      const bool kv = k < ke;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int n = n0 + i * 16 + row;
        w[u][i] = (kv && n < a.N)
                      ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                            a.wq + static_cast<int64_t>(n) * a.K + k))
                      : zero;
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int m = j * 16 + row;
        const u32x4* xp = reinterpret_cast<const u32x4*>(a.x + static_cast<int64_t>(m) * a.K + k);
        const bool v = kv && m < a.M;
        xl[u][j] = v ? xp[0] : zero;
        xh[u][j] = v ? xp[1] : zero;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        uint32_t o[8];
        i8x4_to_act<ACT>(w[u][i].x, o[0], o[1]);
        i8x4_to_act<ACT>(w[u][i].y, o[2], o[3]);
        i8x4_to_act<ACT>(w[u][i].z, o[4], o[5]);
        i8x4_to_act<ACT>(w[u][i].w, o[6], o[7]);
        const u32x4 lo = {o[0], o[1], o[2], o[3]}, hi = {o[4], o[5], o[6], o[7]};
#pragma unroll
        for (int j = 0; j < TM; ++j) {
          acc[i][j] = mfma16x16x32<ACT>(lo, xl[u][j], acc[i][j]);
          acc[i][j] = mfma16x16x32<ACT>(hi, xh[u][j], acc[i][j]);
        }
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) red[wave - 1][i][j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) acc[i][j] += red[w][i][j][lane];

  const bool vec_store = (a.N % 4) == 0;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int m = j * 16 + row;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int nb = n0 + i * 16 + g * 4;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nb + r;
        float val = 0.0f;
        if (n < a.N) {
          val = acc[i][j][r] * act_to_f32<ACT>(a.scales[n]);
          for (int jj = 0; jj < a.n_out; ++jj) {
            const int64_t k = a.oc[jj];
            if (k >= 0 && k < a.K)
              val += act_to_f32<ACT>(a.x[static_cast<int64_t>(m) * a.K + k]) *
                     act_to_f32<ACT>(a.w_out[static_cast<int64_t>(n) * a.n_out + jj]);
          }
          if (a.bias) val += act_to_f32<ACT>(a.bias[n]);
        }
        v[r] = val;
      }
      uint16_t* dst = a.y + static_cast<int64_t>(m) * a.N + nb;
      if (vec_store && nb + 3 < a.N) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack2_out<ACT>(v[0], v[1]),
                                                    pack2_out<ACT>(v[2], v[3]));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < a.N) dst[r] = out1<ACT>(v[r]);
      }
    }
  }
}

template <int ACT, int TM, int TN, int U>
void launch_skinny(GemmArgs a, hipStream_t s) {
  k_skinny<ACT, TM, TN, U><<<dim3(static_cast<unsigned>(cdiv(a.N, 16 * TN))), dim3(256), 0, s>>>(a);
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

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Kernel choice by M (measured on MI355X at N = 11008, K = 4096):
//   M <= 64       k_skinny (weight streaming), TM = ceil(M / 16)
//   64 < M < 1024 k_gemm 128 x 64 x 64, 2 x 2 waves
//   M >= 1024     k_gemm 256 x 256 x 64, 4 x 2 waves
enum Kind { kSkinny1, kSkinny2, kSkinny4, kTileMid, kTileLarge };

Kind choose(int64_t M) {
  if (M <= 16) return kSkinny1;
  if (M <= 32) return kSkinny2;
  if (M <= 64) return kSkinny4;
  return M >= 1024 ? kTileLarge : kTileMid;
}

template <int ACT, int BM, int BN, int BK, int WGM, int WGN, int PD>
void launch_gemm(GemmArgs a, hipStream_t s) {
  a.tiles_m = static_cast<int>(cdiv(a.M, BM));
  a.tiles_n = static_cast<int>(cdiv(a.N, BN));
  const unsigned grid = static_cast<unsigned>(a.tiles_m) * a.tiles_n;
  k_gemm<ACT, BM, BN, BK, WGM, WGN, PD><<<dim3(grid), dim3(64 * WGM * WGN), 0, s>>>(a);
}

template <int ACT>
void launch_kind(Kind k, const GemmArgs& a, hipStream_t s) {
  switch (k) {
    case kSkinny1: launch_skinny<ACT, 1, 1, 4>(a, s); break;
    case kSkinny2: launch_skinny<ACT, 2, 1, 4>(a, s); break;
    case kSkinny4: launch_skinny<ACT, 4, 1, 2>(a, s); break;
    case kTileMid: launch_gemm<ACT, 128, 64, 64, 2, 2, 1>(a, s); break;
    default: launch_gemm<ACT, 256, 256, 64, 4, 2, 1>(a, s); break;
  }
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

// The MFMA kernels need 16-byte rows (K % 16 == 0), aligned operands and
// 32-bit index arithmetic (tile counts and row offsets fit in int).
bool mfma_path(int64_t M, int64_t N, int64_t K, const void* x, const int8_t* wq, const void* y) {
  return (K % 16 == 0) && aligned(x, 16) && aligned(wq, 16) && aligned(y, 8) && M < (1LL << 30) &&
         N < (1LL << 30) && K < (1LL << 30) && cdiv(M, 64) * cdiv(N, 64) < (1LL << 31);
}

template <int ACT>
int w8a16_t(const void* x, const int8_t* wq, const void* scales, const void* bias,
            const int64_t* oc, int64_t n_out, const void* w_out, int64_t M, int64_t N, int64_t K,
            void* y, hipStream_t s) {
  if (!mfma_path(M, N, K, x, wq, y))
    return w8a16_simple<ACT>(x, wq, scales, bias, oc, n_out, w_out, M, N, K, y, s);
  GemmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.wq = wq;
  a.scales = static_cast<const uint16_t*>(scales);
  a.bias = static_cast<const uint16_t*>(bias);
  a.oc = oc;
  a.w_out = static_cast<const uint16_t*>(w_out);
  a.y = static_cast<uint16_t*>(y);
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.n_out = static_cast<int>(n_out);
  launch_kind<ACT>(choose(M), a, s);
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
  (void)ws;
  (void)ws_bytes;
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
