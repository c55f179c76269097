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
// k_gemm_dma<ACT, SPLIT, TM> (M > 64, K % 64 == 0): 64 TM x 256 tiles (TM =
// 4, 3, 2) of v_mfma_f32_32x32x16 fed by LDS DMA, 8 waves (two per SIMD),
// int8 weights widened after the fragment read, explicitly scheduled k-steps
// (see the kernel's comment). With SPLIT, the tiles of a short last wave run
// over several k-ranges into fp32 partial tiles in the caller's workspace and
// k_splitk_reduce sums them in a fixed order (no cross-workgroup fences);
// dma_plan picks the tile height and the split with a fitted time model.
// Where the time model prefers them (mostly 64 < M < 384 with up to one
// round of tiles), the same kernel runs 128 x 128 tiles instead (two waves
// along M, four along N, one 32-row weight tile each): no partials at all.
// Outlier columns run on the matrix cores too: per 16 columns the tile's
// gathered x columns and w_out rows are staged in LDS in one round of loads,
// then one rank-16 MFMA update per 32 x 32 block onto the scaled
// accumulators. Split tiles leave them to k_splitk_reduce, which stages the
// same operands per workgroup and adds them per output.
//
// k_stream1<ACT> (M <= 16) and k_stream<ACT, TM> (M <= 64): persistent
// weight streaming for large weights (see the kernels' comments).
//
// k_skinny<ACT, TM, TN, U> (M <= 64): weight streaming with the K split across
// the waves of a workgroup and reduced through LDS (see below). A split of K
// across workgroups that publishes partial tiles for a last-arriving
// workgroup was measured slower on MI355X: it needs agent-scope release
// fences, which write back the whole L2.
#include <algorithm>
#include <type_traits>

#include "cbq_device.h"
#include "cbq_host.h"
#include "cbq_lds_dma.h"

namespace cbq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));

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
    // One v_cvt_f16_i16 per code: the SDWA source select takes byte b of w
    // sign-extended, the destination select writes one half of lo / hi and
    // keeps the other (exact: every int8 is an fp16). The compiler does not
    // form these selects from shifts and casts itself (it shifts each byte
    // first and packs the halves: 5 instructions per word instead of 4).
    // Wait states the hardware needs and the compiler cannot insert inside
    // the statement (it does not look into asm text):
    // - a sub-dword (dst_sel WORD_n) write needs one before the next VALU
    //   instruction that touches the register, and the preserving write of
    //   the high half reads it: lo's and hi's writes alternate so that each
    //   pair has one instruction between them;
    // - an MFMA that reads a VGPR needs two after a VALU write of it. The
    //   compiler counts the statement as a sub-dword write, not as a VALU: it
    //   keeps one wait state (an s_nop 0 of its own, or any instruction)
    //   between the statement and the next reader of lo / hi, whatever that
    //   reader is. The closing s_nop 0 is the second one for an MFMA.
    //   (Bit-identical outputs; 0.5% at M = 4096 against no wait.)
    asm("v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3\n\t"
        "s_nop 0"
        : "=&v"(lo), "=&v"(hi)
        : "v"(w));
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
  float* part;              // split-K partial tiles (k_gemm_dma<ACT, true, TM>)
  int M, N, K, n_out;
  int tiles_m, tiles_n;
  int splits, split_steps;  // split-K: number of k-ranges, 64-k steps per range
  int full_tiles;           // split-K: tiles [0, full_tiles) run whole, the rest split
  const uint16_t* x2;       // k_gemm_dma<.., PLANES>: the second x plane (splits >= splits / 2)
};

// Workgroup b of n goes to XCD b % 8; renumbered so that each XCD takes a
// contiguous run of [0, n) (neighbouring tiles share operand rows in its L2).
__device__ __forceinline__ int xcd_renumber(int b, int n) {
  const int per = n >> 3;
  return b < per * 8 ? (b & 7) * per + (b >> 3) : b;
}

// Linear tile t -> (tile m, tile n): groups of 8 tile rows, column-major
// inside a group.
__device__ __forceinline__ void group_tile(int t, const GemmArgs& a, int& tm, int& tn) {
  constexpr int G = 8;
  const int group = t / (G * a.tiles_n);
  const int first_m = group * G;
  const int gsize = min(a.tiles_m - first_m, G);
  const int r = t % (G * a.tiles_n);
  tm = first_m + r % gsize;
  tn = r / gsize;
}

// Workgroup -> (tile m, tile n); see the file comment.
__device__ __forceinline__ void decode_tile(int b, const GemmArgs& a, int& tm, int& tn) {
  group_tile(xcd_renumber(b, a.tiles_m * a.tiles_n), a, tm, tn);
}

// Outlier side-GEMM for 4 consecutive outputs y[m, nb .. nb+3]:
// v[r] += sum_j x[m, oc[j]] * w_out[nb + r, j], in j order. Columns go in
// groups of 4 whose loads (indices, x values, weights) are all issued before
// any is used: addresses are clamped to valid elements and the terms of
// missing columns / rows or of an index outside [0, K) are zeroed by selects,
// so no branch makes the compiler wait for each load in turn (a dependent
// chain of 3 loads per column and quad cost 2x the whole GEMM at M = 4096,
// N = 11008 with 6 columns). The group loop is kept rolled so that the
// unrolled tile epilogues stay small enough to keep their accumulators in
// registers.
template <int ACT>
__device__ __forceinline__ f4 outlier_quad(const GemmArgs& a, int m, int nb, f4 v) {
  constexpr int G = 4;
  const int64_t xrow = static_cast<int64_t>(m) * a.K;
#pragma nounroll
  for (int j0 = 0; j0 < a.n_out; j0 += G) {
    float xv[G], wv[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int j = min(j0 + g, a.n_out - 1);
      const int64_t k = a.oc[j];
      const bool ok = j0 + g < a.n_out && k >= 0 && k < a.K;
      const int64_t kc = k < 0 ? 0 : (k >= a.K ? a.K - 1 : k);
      const float x = act_to_f32<ACT>(a.x[xrow + kc]);
      xv[g] = ok ? x : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = min(nb + r, a.N - 1);
        wv[g][r] = act_to_f32<ACT>(a.w_out[static_cast<int64_t>(n) * a.n_out + j]);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += xv[g] * wv[g][r];
  }
  return v;
}

// Tile epilogue for one MFMA accumulator quad: y[m, nb + r] =
// T(acc[r] * s[n] (+ outlier sum) (+ bias[n])), fp32 until the one rounding.
template <int ACT>
__device__ __forceinline__ void store_quad(const GemmArgs& a, const f4& acc, int m, int nb,
                                           bool vec_store) {
  f4 v;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    v[r] = nb + r < a.N ? acc[r] * act_to_f32<ACT>(a.scales[nb + r]) : 0.0f;
  if (a.n_out > 0) v = outlier_quad<ACT>(a, m, nb, v);
  if (a.bias) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (nb + r < a.N) v[r] += act_to_f32<ACT>(a.bias[nb + r]);
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
    if (m < a.M) {
#pragma unroll
      for (int i = 0; i < TN; ++i)
        store_quad<ACT>(a, acc[i][j], m, n0 + wn * (BN / WGN) + i * 16 + (lane >> 4) * 4, vec_store);
    }
  }
}

// ---------------------------------------------------------------------------
// k_gemm_dma<ACT>: large-M tile kernel fed by LDS DMA.
//
// Tile 256 (m) x 256 (n) x 64 (k), 8 waves (two per SIMD) in 2 (m) x 4 (n),
// each wave 128 x 64 as 4 x 2 tiles of v_mfma_f32_32x32x16_{f16,bf16} (128
// accumulator registers). On MI355X this MFMA runs at the full dense rate
// (2.47 PFLOP/s measured), the 16x16x32 form at about half of it. With two
// waves per SIMD one wave's MFMAs run while the other waits at the barrier or
// for fragments: rocprof's MfmaUtil rose from 38% (4 waves of 128 x 128) to
// 51% at M = 4096, N = 11008, K = 4096. Operand tiles go from global memory
// straight into LDS with global_load_lds_dwordx4 (no VGPR staging, no LDS
// store instructions): x as 256 rows of 128 bytes, the weight tile as 256
// rows of 64 int8 codes. The codes are widened to the activation dtype after
// the fragment read, so LDS holds half the bytes of a widened tile. Three
// LDS stages (3 x 48 KiB): while the MFMAs of tile t run, tiles t + 1 and
// t + 2 are in flight; each k-half's fragments are read while the previous
// half is multiplied; one barrier per k-step, between its two halves.
//
// LDS rows are XOR-swizzled at 16-byte granularity so that the 16 lanes of a
// fragment read phase (16 rows, one 16-byte chunk each) hit 16 distinct
// 4-bank groups: x chunk c of row r sits at position c ^ ((r >> 1) & 7),
// weight chunk c at c ^ ((r >> 2) & 3). The DMA writes 64 consecutive
// 16-byte slots per wave instruction, so each lane loads the source chunk its
// slot holds.
//
// k order: in a 64-k step, lane half h = lane / 32 owns k in [32 h, 32 h + 32)
// of its weight row (two 16-byte reads) and of its x row (four reads). MFMA s
// (0..3) takes k [32 h + 8 s, 32 h + 8 s + 8) from both operands, so A and B
// see the same k permutation and the products are unchanged.
//
// Requirements (checked on the host): K % 64 == 0, x and wq 16-byte aligned,
// M * K * 2 and N * K below 2^32 (32-bit per-lane offsets from a scalar base).
// Rows past M or N are clamped to the last row; their products land in
// outputs that are never stored.

template <int ACT>
__device__ __forceinline__ f16x mfma32x32x16(const u32x4& a, const u32x4& b, f16x c) {
  if constexpr (ACT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, a),
                                                  __builtin_bit_cast(h8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8, a),
                                                   __builtin_bit_cast(b8, b), c, 0, 0, 0);
}

// Outlier side-GEMM of a tile on the matrix cores, 16 outlier columns at a
// time (a rank-16 update with v_mfma_f32_32x32x16, the layout of the main
// accumulators). stage_outliers writes the tile's operands for columns
// c0 .. c0 + 15 to LDS in one round of independent loads by the whole
// workgroup: xo[r][0, 16) = x[m0 + r, oc[c0 ..]] (BM rows, 32 B each),
// then wo[r][0, 16) = w_out[n0 + r, c0 ..] (256 rows). Columns past n_out
// and indices outside [0, K) give zeros; rows past M / N are clamped for
// the loads (their outputs are never stored). Thread t fills 16 bytes: row
// t / 2, columns 8 (t % 2) .. + 8. A lane then reads its MFMA fragment (row
// l % 32, columns 8 (l / 32) .. + 8) with one ds_read_b128.
constexpr int kOutStageBytes = (256 + 256) * 32;

template <int ACT, int BM>
__device__ __forceinline__ void stage_outliers(const GemmArgs& a, int m0, int n0, int c0,
                                               uint8_t* so) {
  const int t = threadIdx.x, row = t >> 1, cb = c0 + 8 * (t & 1);
  uint32_t v[8];
  if (row < BM) {
    const int64_t xrow = static_cast<int64_t>(min(m0 + row, a.M - 1)) * a.K;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = cb + e;
      const int64_t k = a.oc[min(j, a.n_out - 1)];
      const int64_t kc = k < 0 ? 0 : (k >= a.K ? a.K - 1 : k);
      const uint32_t x = a.x[xrow + kc];
      v[e] = (j < a.n_out && k >= 0 && k < a.K) ? x : 0u;
    }
    *reinterpret_cast<u32x4*>(so + t * 16) =
        u32x4{v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16)};
  }
  const uint16_t* wr = a.w_out + static_cast<int64_t>(min(n0 + row, a.N - 1)) * a.n_out;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int j = cb + e;
    v[e] = j < a.n_out ? wr[min(j, a.n_out - 1)] : 0u;
  }
  *reinterpret_cast<u32x4*>(so + BM * 32 + t * 16) =
      u32x4{v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16)};
}

constexpr int kDmaThreads = 512;   // 8 waves, two per SIMD
constexpr int kDmaTN = 2;          // 32-row weight tiles per wave

// acc[i][j] += the side-GEMM block of the staged chunk (see stage_outliers)
// for the wave's weight rows 32 i .. of its 32 TN and x rows 32 j .. of its
// 32 TM (the accumulator layout of k_gemm_dma; WM waves along M).
template <int ACT, int TM, int TN, int WM>
__device__ __forceinline__ void outlier_mfma(const uint8_t* so, int wm, int wn, int lane,
                                             f16x (&acc)[TN][TM]) {
  constexpr int BM = WM * 32 * TM;
  const int r32 = lane & 31, h = lane >> 5;
  u32x4 wf[TN];
#pragma unroll
  for (int i = 0; i < TN; ++i)
    wf[i] = *reinterpret_cast<const u32x4*>(so + BM * 32 + (wn * 32 * TN + i * 32 + r32) * 32 + h * 16);
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const u32x4 xf = *reinterpret_cast<const u32x4*>(so + (wm * TM * 32 + j * 32 + r32) * 32 + h * 16);
#pragma unroll
    for (int i = 0; i < TN; ++i) acc[i][j] = mfma32x32x16<ACT>(wf[i], xf, acc[i][j]);
  }
}

// TM: 32-row x tiles per wave; TNW: 32-row weight tiles per wave; WM waves
// along M and 8 / WM along N. The workgroup tile is 32 WM TM x 256 TNW /
// WM: with the default TNW = WM = 2, 64 TM x 256 (TM = 4: 256 x 256; TM = 3
// or 2: 192 or 128 x 256 for small M and for tile counts that leave the
// last wave of workgroups short); TNW = 1 with TM = WM = 2 gives 128 x 128
// (k_gemm_dma128).
// SPLIT: workgroups [0, full_tiles) take whole tiles 0 .. full_tiles - 1;
// the others split the remaining tiles over `splits` k-ranges, workgroup
// full_tiles + b covering tail tile b % rest of k-range b / rest (after the
// XCD renumbering, so the workgroups of one XCD share a k-range of x).
template <int ACT, bool SPLIT, int TM, bool PLANES = false, int TNW = kDmaTN, int WM = 2>
__global__ __launch_bounds__(kDmaThreads) void k_gemm_dma(GemmArgs a) {
  constexpr int WN = 8 / WM;   // waves along N
  constexpr int BM = WM * 32 * TM, BN = WN * 32 * TNW, BK = 64, NS = 3;
  constexpr int XB = BM * BK * 2;          // x stage bytes (32 / 24 / 16 KiB)
  constexpr int WB = BN * BK;              // weight stage bytes (16 KiB)
  constexpr int SB = XB + WB;
  constexpr int XL = XB / (kDmaThreads * 16);   // DMA instructions per thread: TM
  constexpr int WL = WB / (kDmaThreads * 16);   // 2 (1 for 128 columns)
  static_assert(!SPLIT || (TNW == kDmaTN && WM == 2), "k_splitk_reduce reads the default layout");
  constexpr int TN = TNW;
  static_assert(TM >= 2 && TM <= 4, "x tile of 128, 192 or 256 rows");
  // operand stages; after the main loop the outlier staging area (at the
  // start) and the epilogue's output tiles
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * SB];
  static_assert(kOutStageBytes <= NS * SB, "outlier stage fits in LDS");
  uint8_t* const so = smem;
  // The tile's 256 scales and biases in fp32 (0 past N), loaded while the
  // first stages' DMA is in flight, so that the epilogue reads them from LDS
  // instead of waiting on global loads at the end of the tile (which cost
  // 3-8 us per call at N = 11008, K = 4096: M = 512 / 768 / 1024 / 2048 /
  // 3072 / 4096 took 56.3 / 73.9 / 92.2 / 173.0 / 247.5 / 323.4 us and take
  // 53.3 / 71.0 / 89.1 / 167.1 / 242.0 / 315.3 us, bit-identical). Split
  // tail tiles load them too and do not use them.
  __shared__ float s_scale[256], s_bias[256];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;   // 32 TM x rows, 32 TN weight rows
  int tm, tn, split = 0, ptile = 0;
  bool partial = false;
  if constexpr (SPLIT) {
    const int b = blockIdx.x;
    if (b < a.full_tiles) {
      group_tile(xcd_renumber(b, a.full_tiles), a, tm, tn);
    } else {
      partial = true;
      const int rest = a.tiles_m * a.tiles_n - a.full_tiles;
      const int r = xcd_renumber(b - a.full_tiles, rest * a.splits);
      split = r / rest;
      ptile = r % rest;
      group_tile(a.full_tiles + ptile, a, tm, tn);
    }
  } else {
    decode_tile(blockIdx.x, a, tm, tn);
  }
  const int m0 = tm * BM, n0 = tn * BN;
  // PLANES: splits = 2 KS, split s runs k-range s % KS of x plane s / KS
  const int ks = PLANES ? a.splits / 2 : 1;
  const int krange = PLANES ? split % ks : split;
  const int kb = partial ? krange * a.split_steps : 0;   // first 64-k step
  const int nk = partial ? min(a.split_steps, a.K / BK - kb) : a.K / BK;
  const uint16_t* const xsrc = (PLANES && split >= ks) ? a.x2 : a.x;
  const uint32_t sbase = __builtin_amdgcn_readfirstlane(lds_addr(smem));

  // Per-lane DMA source offsets (bytes from the k0 column of the tile). x
  // instruction u fills rows (u * 8 + wave) * 8 + lane / 8 (128-byte rows,
  // 8 chunks); weight instruction u fills rows (u * 8 + wave) * 16 + lane / 4
  // (64-byte rows, 4 chunks). Each lane loads the source chunk its LDS slot
  // holds under the swizzle.
  uint32_t xo[XL], wo[WL];
#pragma unroll
  for (int u = 0; u < XL; ++u) {
    const int row = (u * 8 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    const int m = min(m0 + row, a.M - 1);
    xo[u] = static_cast<uint32_t>(m) * static_cast<uint32_t>(a.K) * 2u + c * 16u;
  }
#pragma unroll
  for (int u = 0; u < WL; ++u) {
    const int row = (u * 8 + wave) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 2) & 3);
    const int n = min(n0 + row, a.N - 1);
    wo[u] = static_cast<uint32_t>(n) * static_cast<uint32_t>(a.K) + c * 16u;
  }
  // DMA instruction u (0..XL+WL-1) of tile t into `stage`.
  auto issue_one = [&](int t, int stage, int u) {
    if (u < XL)
      lds_dma16(xo[u], uniform_ptr(xsrc + (kb + t) * BK), sbase + stage * SB + wave * 1024 + u * 8192);
    else
      lds_dma16(wo[u - XL], uniform_ptr(a.wq + (kb + t) * BK),
                sbase + stage * SB + XB + wave * 1024 + (u - XL) * 8192);
  };
  auto issue = [&](int t, int stage) {
#pragma unroll
    for (int u = 0; u < XL + WL; ++u) issue_one(t, stage, u);
  };

  // Fragment read offsets within a stage: row r32 of each 32-row tile, lane
  // half h; x chunk 4 h + 2 e + s (half e, slice s), weight chunk 2 h + e.
  const int r32 = lane & 31, h = lane >> 5;
  uint32_t xr[2][2], wr[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      xr[e][q] = (wm * TM * 32 + r32) * 128 + (((4 * h + 2 * e + q) ^ ((r32 >> 1) & 7)) << 4);
    wr[e] = XB + (wn * 32 * TN + r32) * 64 + (((2 * h + e) ^ ((r32 >> 2) & 3)) << 4);
  }

  f16x acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f16x{};

  // Half e of a k-step: weight chunk e of each lane's rows (k [32 h + 16 e,
  // +16)) and x chunks 4 h + 2 e, 4 h + 2 e + 1: MFMA k-slices s = 0, 1 of the
  // half. One fragment set per half: TN weight reads, then 2 TM x reads.
  struct Frags {
    u32x4 x[TM][2];
    u32x4 w[TN];
  };
  Frags fr[2];
  auto read_one = [&](int stage, int e, Frags& f, int r) {
    const uint8_t* st = smem + stage * SB;
    if (r < TN) {
      f.w[r] = *reinterpret_cast<const u32x4*>(st + wr[e] + r * 2048);
    } else {
      const int rx = r - TN;
      f.x[rx >> 1][rx & 1] = *reinterpret_cast<const u32x4*>(st + xr[e][rx & 1] + (rx >> 1) * 4096);
    }
  };
  auto read_half = [&](int stage, int e, Frags& f) {
#pragma unroll
    for (int r = 0; r < 2 * TM + TN; ++r) read_one(stage, e, f, r);
  };
  // Widen word c (0..3: 4 codes) of weight tile i into w (slice c / 2).
  auto cvt_word = [&](const Frags& f, int i, int c, u32x4 (&w)[2]) {
    const uint32_t src = c == 0 ? f.w[i].x : c == 1 ? f.w[i].y : c == 2 ? f.w[i].z : f.w[i].w;
    uint32_t lo, hi;
    i8x4_to_act<ACT>(src, lo, hi);
    const int q = c >> 1, k = (c & 1) * 2;
    w[q][k] = lo;
    w[q][k + 1] = hi;
  };
  // MFMA p (0 .. 2 TM - 1) of weight tile i: slice p / TM, x tile p % TM
  // (an accumulator is reused TM MFMAs later).
  auto mma_one = [&](const Frags& f, int i, const u32x4 (&w)[2], int p) {
    const int q = p / TM, j = p % TM;
    acc[i][j] = mfma32x32x16<ACT>(w[q], f.x[j][q], acc[i][j]);
  };
  // A half: weight tile i's 4 MFMAs, each followed by one word of the next
  // tile's widening (tile 0 of the next half after the last tile) and by
  // `extra` (DMA issue / fragment reads); sched_barrier pins the order.
  u32x4 wa[2], wb[2];   // widened weights: current and next tile
  // With one weight tile per wave (TN = 1) the next set's tile is only read
  // at the half's first slot: its words widen at slots 1, 2, ... (two at the
  // last slot of a 4-MFMA half), and the buffers alternate per half (par).
  auto half = [&](Frags& f, Frags* fnext, int par, auto&& extra) {
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      u32x4 (&cur)[2] = ((i + par) & 1) ? wb : wa;
      u32x4 (&nxt)[2] = ((i + par) & 1) ? wa : wb;
#pragma unroll
      for (int p = 0; p < 2 * TM; ++p) {
        mma_one(f, i, cur, p);
        if constexpr (TN == 1) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (fnext && (c + 1 < 2 * TM ? c + 1 : 2 * TM - 1) == p) cvt_word(*fnext, 0, c, nxt);
        } else if (p < 4) {
          if (i + 1 < TN) cvt_word(f, i + 1, p, nxt);
          else if (fnext) cvt_word(*fnext, 0, p, nxt);
        }
        extra(i, p);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // Step t: set 0 holds half 0 of tile t, wa weight tile 0 of set 0
  // widened; tiles t + 1 and t + 2 are in flight. Half 0, with the reads of
  // tile t's half 1 into set 1 spread over its first MFMAs (tile t landed
  // before the previous step's barrier; the last tile of half 0 widens tile
  // 0 of set 1); the wait for tile t + 1 and the barrier, after which every
  // wave is done with tile t's stage, so the DMA of tile t + 3 goes there;
  // half 1 with one DMA instruction and one read of tile t + 1's half 0 into
  // set 0 after each of its first MFMAs. Spreading the DMA and the reads
  // (rather than issuing them in bursts) took 4-5% off the step at M = 4096,
  // N = 11008 / 4096 on MI355X. The other wave of the SIMD keeps the MFMA
  // pipe busy while a wave waits.
  // SC: t % NS when known at compile time (the main loop is unrolled by NS,
  // so the stage offsets fold into the LDS instructions' immediate offsets
  // instead of costing an address add per fragment read: 3-4% at M = 4096),
  // else -1.
  auto step = [&](int t, auto dma, int nwait, auto sc) {
    constexpr int SC = decltype(sc)::value;
    const int stage_cur = SC >= 0 ? SC : t % NS;
    const int stage_next = SC >= 0 ? (SC + 1) % NS : (t + 1) % NS;
    half(fr[0], &fr[1], 0, [&](int i, int p) {
      const int r = i * 2 * TM + p;
      if (r < 2 * TM + TN) read_one(stage_cur, 1, fr[1], r);
      if (r == 2 * TM * TN - 1)   // reads past the MFMA slots (TN = 1)
        for (int rr = r + 1; rr < 2 * TM + TN; ++rr) read_one(stage_cur, 1, fr[1], rr);
    });
    __builtin_amdgcn_sched_barrier(0);
    if (nwait >= 1) dma_wait_barrier<XL + WL>();
    else dma_wait_barrier<0>();
    __builtin_amdgcn_sched_barrier(0);
    half(fr[1], &fr[0], TN & 1, [&](int i, int p) {
      const int r = i * 2 * TM + p;
      if constexpr (decltype(dma)::value) {
        if (r < XL + WL) issue_one(t + NS, stage_cur, r);
      }
      if (r < 2 * TM + TN) read_one(stage_next, 0, fr[0], r);
      if (r == 2 * TM * TN - 1)
        for (int rr = r + 1; rr < 2 * TM + TN; ++rr) read_one(stage_next, 0, fr[0], rr);
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  using yes = std::true_type;
  using no = std::false_type;

#pragma unroll
  for (int t = 0; t < NS; ++t)
    if (t < nk) issue(t, t);
  if (!PLANES && tid < 256) {   // the two-plane launches carry no scales
    const int n = n0 + tid;
    const int nc = min(n, a.N - 1);
    const float sv = act_to_f32<ACT>(a.scales[nc]);
    const float bv = a.bias ? act_to_f32<ACT>(a.bias[nc]) : 0.0f;
    s_scale[tid] = n < a.N ? sv : 0.0f;
    s_bias[tid] = n < a.N ? bv : 0.0f;
  }
  if (nk > 0) {
    if (nk > 2) dma_wait_barrier<2 * (XL + WL)>();
    else if (nk > 1) dma_wait_barrier<XL + WL>();
    else dma_wait_barrier<0>();
    read_half(0, 0, fr[0]);
#pragma unroll
    for (int c = 0; c < 4; ++c) cvt_word(fr[0], 0, c, wa);
    int t = 0;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using SR = std::integral_constant<int, -1>;
    static_assert(NS == 3, "the main loop is unrolled by the stage count");
    // Tile t + 2 in flight, DMA of t + 3.
    for (; t + NS + 2 < nk; t += NS) {
      step(t, yes{}, 1, S0{});
      step(t + 1, yes{}, 1, S1{});
      step(t + 2, yes{}, 1, S2{});
    }
    for (; t + NS < nk; ++t) step(t, yes{}, 1, SR{});
    for (; t + 1 < nk; ++t) step(t, no{}, nk - 2 - t, SR{});
    half(fr[0], &fr[1], 0, [&](int i, int p) {
      const int r = i * 2 * TM + p;
      if (r < 2 * TM + TN) read_one((nk - 1) % NS, 1, fr[1], r);
      if (r == 2 * TM * TN - 1)
        for (int rr = r + 1; rr < 2 * TM + TN; ++rr) read_one((nk - 1) % NS, 1, fr[1], rr);
    });
    half(fr[1], nullptr, TN & 1, [&](int, int) {});
  }

  const int mw = m0 + wm * TM * 32, nw = n0 + wn * 32 * TN;
  if (SPLIT && partial) {
    // Partial tile in lane order: f4 (split, tail tile, wave, i, j, q, lane),
    // one contiguous 1 KiB store per (i, j, q); k_splitk_reduce finishes it
    // (scale, outlier columns, bias).
    const int rest = a.tiles_m * a.tiles_n - a.full_tiles;
    f4* dst = reinterpret_cast<f4*>(a.part) +
              ((static_cast<int64_t>(split) * rest + ptile) * 8 + wave) * (TN * TM * 4 * 64) + lane;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dst[((i * TM + j) * 4 + q) * 64] =
              f4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    return;
  }
  // Epilogue. Accumulator values 4q .. 4q+3 of tile (i, j) are the wave's
  // outputs (m, n .. n+3) with m = 32 j + r32, n = 32 i + 8 q + 4 h. Each is
  // finished in fp32 (scale, outlier sum, bias, in that order), rounded once,
  // and written to an LDS copy of the wave's 32 TM x 64 output tile; the
  // tile is then stored with 16-byte row-contiguous stores. Scales and
  // biases come from s_scale / s_bias.
  constexpr int EPS = 32 * TN + 8;   // LDS row stride of the output tile (halfs)
  static_assert(8 * TM * 32 * EPS * 2 <= NS * SB, "epilogue tile fits in LDS");
  dma_wait_barrier<0>();     // every wave is done with the operand stages
  uint16_t* ep = reinterpret_cast<uint16_t*>(smem) + wave * (TM * 32 * EPS);
  const bool outl = a.n_out > 0;
  if (outl) {
    // y = s * acc + sum_j x[m, oc[j]] w_out[n, j] + bias: the scale first, in
    // place, then the side-GEMM accumulates onto the scaled tiles (fp32, one
    // rank-16 MFMA update per 16 outlier columns and block)
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sc = s_scale[wn * 32 * TN + i * 32 + 8 * q + 4 * h + r];
#pragma unroll
          for (int j = 0; j < TM; ++j) acc[i][j][4 * q + r] *= sc;
        }
    for (int c0 = 0; c0 < a.n_out; c0 += 16) {
      if (c0 > 0) __syncthreads();   // every wave has read the previous chunk
      stage_outliers<ACT, BM>(a, m0, n0, c0, so);
      __syncthreads();
      outlier_mfma<ACT, TM, TN, WM>(so, wm, wn, lane, acc);
    }
    __syncthreads();   // the output tiles below overwrite the stage
  }
#pragma unroll
  for (int i = 0; i < TN; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = i * 32 + 8 * q + 4 * h;
      float sc[4], bs[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = outl ? 1.0f : s_scale[wn * 32 * TN + nl + r];   // x 1: exact
        bs[r] = s_bias[wn * 32 * TN + nl + r];
      }
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        f4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = acc[i][j][4 * q + r] * sc[r];
        if (a.bias) {
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] += bs[r];
        }
        *reinterpret_cast<uint2*>(&ep[(j * 32 + r32) * EPS + nl]) =
            make_uint2(pack2_out<ACT>(v[0], v[1]), pack2_out<ACT>(v[2], v[3]));
      }
    }
  }
  // Row-contiguous stores: 4 TN lanes cover one 32 TN-wide row (8 outputs
  // each).
  const bool vec16 = (a.N % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
  constexpr int LR = 4 * TN;
#pragma unroll 4
  for (int u = 0; u < 2 * TM * TN; ++u) {
    const int row = u * (64 / LR) + lane / LR, c8 = (lane % LR) * 8;
    const int m = mw + row, n = nw + c8;
    if (m >= a.M || n >= a.N) continue;
    const u32x4 val = *reinterpret_cast<const u32x4*>(&ep[row * EPS + c8]);
    uint16_t* dst = a.y + static_cast<int64_t>(m) * a.N + n;
    if (vec16 && n + 8 <= a.N) {
      *reinterpret_cast<u32x4*>(dst) = val;
    } else {
      const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (n + r < a.N) dst[r] = static_cast<uint16_t>(w[r >> 1] >> (16 * (r & 1)));
    }
  }
}

template <int ACT, int TM>
void launch_gemm_dma(GemmArgs a, hipStream_t s) {
  a.tiles_m = static_cast<int>(cdiv(a.M, 64 * TM));
  a.tiles_n = static_cast<int>(cdiv(a.N, 256));
  const unsigned grid = static_cast<unsigned>(a.tiles_m) * a.tiles_n;
  k_gemm_dma<ACT, false, TM><<<dim3(grid), dim3(kDmaThreads), 0, s>>>(a);
}

// 128 x 128 tiles, whole (k_gemm_dma128): 98 VGPRs and 74 KiB of LDS, so two
// workgroups fit a CU.
template <int ACT>
void launch_gemm_dma128(GemmArgs a, hipStream_t s) {
  a.tiles_m = static_cast<int>(cdiv(a.M, 128));
  a.tiles_n = static_cast<int>(cdiv(a.N, 128));
  const unsigned grid = static_cast<unsigned>(a.tiles_m) * a.tiles_n;
  k_gemm_dma<ACT, false, 2, false, 1, 2><<<dim3(grid), dim3(kDmaThreads), 0, s>>>(a);
}

// Split-K finish: each thread takes two partial f4 of a tail tile, kBlock
// apart (4 outputs y[m, n .. n+3] each); sums the splits in order
// (deterministic), then scale, outlier columns, bias and one rounding, as in
// the tile kernels' epilogue. Partial index, fastest first: lane (64), q (4),
// j (TM), i (2), wave (8), tail tile.
//
// Outlier columns (the OUTL instance): a workgroup's partial f4 all lie in
// one wave's part of one tail tile (rows 32 TM, columns 64), so per 6
// outlier columns it stages that part's x[m, oc[j]] and w_out[n, j] in LDS
// (one independent load per thread and column, the indices oc[j] read as
// scalars), issued before the partial planes' loads so that both latencies
// overlap. The sum is then added per output in j order, onto the scaled
// value (as outlier_quad does). Chunks of 6 columns keep the kernel within 64
// VGPRs (8 waves per SIMD, every workgroup of M = 256, N = 11008 resident at
// once; chunks of 16 needed 86 VGPRs and took two rounds: 14 against 8 us).
// Measured at N = 11008, K = 4096, 6 columns: M = 256 45.4 against 50.4 us,
// M = 128 33.0 against 37.8 us, where the first k-range used to store the
// tail tile's side-GEMM block as one more partial plane for the reduce to
// read (11 MB at M = 256), and per-quad global loads (outlier_quad) in the
// reduce took 56.8 us.
constexpr int kReduceF4 = 2;   // partial f4 per thread

template <int ACT, int TM, bool OUTL>   // OUTL: n_out > 0
__global__ __launch_bounds__(kBlock) void k_splitk_reduce(GemmArgs a) {
  constexpr int kWaveF4 = kDmaTN * TM * 4 * 64;
  constexpr int kTileF4 = 8 * kWaveF4;
  constexpr int R = 32 * TM;           // rows of a wave's part
  constexpr int OC = 6;                // outlier columns per staged chunk (see above)
  static_assert(kWaveF4 % (kBlock * kReduceF4) == 0, "a workgroup's f4 share a wave's part");
  static_assert(R + 64 <= kBlock, "one staging load per thread and column");
  __shared__ float xs[OUTL ? OC : 1][R];     // x[mw + row, oc[c0 + c]]
  __shared__ float wsh[OUTL ? OC : 1][64];   // w_out[nw + col, c0 + c]
  const int rest = a.tiles_m * a.tiles_n - a.full_tiles;
  const int64_t per_split = static_cast<int64_t>(rest) * kTileF4;
  const int64_t idx0 = static_cast<int64_t>(blockIdx.x) * (kBlock * kReduceF4) + threadIdx.x;
  // per_split is a multiple of the workgroup's span: uniform per workgroup
  if (static_cast<int64_t>(blockIdx.x) * (kBlock * kReduceF4) >= per_split) return;
  const int tid = threadIdx.x;
  int tm, tn;
  group_tile(a.full_tiles + static_cast<int>(idx0 / kTileF4), a, tm, tn);
  const int wave = static_cast<int>((idx0 / kWaveF4) & 7);
  const int mw = tm * 64 * TM + (wave & 1) * R;      // first row of the wave's part
  const int nw = tn * 256 + (wave >> 1) * 64;        // first column

  // Staging loads of outlier chunk c0 into registers: thread t < R loads
  // x[mw + t, oc[c0 + c]], thread R <= t < R + 64 loads w_out[nw + t - R,
  // c0 + c] (rows and columns clamped; an index outside [0, K) gives 0).
  float sv[OC];
  auto stage_load = [&](int c0) {
    const int C = min(OC, a.n_out - c0);
#pragma unroll
    for (int c = 0; c < OC; ++c) {
      sv[c] = 0.0f;
      if (c < C) {
        if (tid < R) {
          const int64_t k = a.oc[c0 + c];
          const bool ok = k >= 0 && k < a.K;
          const int m = min(mw + tid, a.M - 1);
          const float xv = act_to_f32<ACT>(a.x[static_cast<int64_t>(m) * a.K + (ok ? k : 0)]);
          sv[c] = ok ? xv : 0.0f;
        } else if (tid < R + 64) {
          const int n = min(nw + tid - R, a.N - 1);
          sv[c] = act_to_f32<ACT>(a.w_out[static_cast<int64_t>(n) * a.n_out + c0 + c]);
        }
      }
    }
  };
  auto stage_store = [&]() {
#pragma unroll
    for (int c = 0; c < OC; ++c) {
      if (tid < R) xs[c][tid] = sv[c];
      else if (tid < R + 64) wsh[c][tid - R] = sv[c];
    }
  };
  int mr[kReduceF4], nr[kReduceF4];   // row / column offsets in the wave's part
#pragma unroll
  for (int u = 0; u < kReduceF4; ++u) {
    const int w = static_cast<int>((idx0 + u * kBlock) % kWaveF4);
    const int lane = w & 63, q = (w >> 6) & 3, j = (w >> 8) % TM, i = (w >> 8) / TM;
    mr[u] = j * 32 + (lane & 31);
    nr[u] = i * 32 + 8 * q + 4 * (lane >> 5);
  }
  // The part's 64 scales and biases (fp32, 0 past N): loaded by the first
  // 64 threads before the partial planes and read from LDS by the finish, so
  // that it does not wait on global loads after the sums.
  __shared__ float ssc[64], sbs[64];
  float sc_t = 0.0f, bs_t = 0.0f;
  if (tid < 64) {
    const int n = min(nw + tid, a.N - 1);
    sc_t = act_to_f32<ACT>(a.scales[n]);
    bs_t = a.bias ? act_to_f32<ACT>(a.bias[n]) : 0.0f;
  }
  if constexpr (OUTL) stage_load(0);

  const f4* src = reinterpret_cast<const f4*>(a.part) + idx0;
  // planes summed in order 0, 1, ..., splits - 1 (deterministic); the loads
  // of up to 8 planes are issued before their adds (a plane at a time was
  // latency-bound: 6.2 us for 2 tail tiles over 16 ranges)
  f4 sum[kReduceF4];
#pragma unroll
  for (int u = 0; u < kReduceF4; ++u) sum[u] = src[u * kBlock];
  int sp = 1;
  for (; sp + 4 <= a.splits; sp += 4) {
    f4 v[4][kReduceF4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int u = 0; u < kReduceF4; ++u) v[p][u] = src[(sp + p) * per_split + u * kBlock];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int u = 0; u < kReduceF4; ++u) sum[u] += v[p][u];
  }
  for (; sp < a.splits; ++sp) {
    f4 v[kReduceF4];
#pragma unroll
    for (int u = 0; u < kReduceF4; ++u) v[u] = src[sp * per_split + u * kBlock];
#pragma unroll
    for (int u = 0; u < kReduceF4; ++u) sum[u] += v[u];
  }
  if (tid < 64) {
    ssc[tid] = sc_t;
    sbs[tid] = bs_t;
  }
  __syncthreads();
  f4 v[kReduceF4];
#pragma unroll
  for (int u = 0; u < kReduceF4; ++u) {
    const int nb = nw + nr[u];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[u][r] = nb + r < a.N ? sum[u][r] * ssc[nr[u] + r] : 0.0f;
  }
  if constexpr (OUTL) {
    for (int c0 = 0; c0 < a.n_out; c0 += OC) {
      if (c0 > 0) {
        __syncthreads();   // every thread has read the previous chunk
        stage_load(c0);
      }
      stage_store();
      __syncthreads();
      const int C = min(OC, a.n_out - c0);
      for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int u = 0; u < kReduceF4; ++u) {
          const float xv = xs[c][mr[u]];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[u][r] += xv * wsh[c][nr[u] + r];
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kReduceF4; ++u) {
    const int m = mw + mr[u], nb = nw + nr[u];
    if (m >= a.M || nb >= a.N) continue;
    if (a.bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[u][r] += sbs[nr[u] + r];
    }
    uint16_t* dst = a.y + static_cast<int64_t>(m) * a.N + nb;
    if ((a.N % 4) == 0 && nb + 3 < a.N) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack2_out<ACT>(v[u][0], v[u][1]),
                                                  pack2_out<ACT>(v[u][2], v[u][3]));
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < a.N) dst[r] = out1<ACT>(v[u][r]);
    }
  }
}

// fp32 activations on the matrix cores. The weights are int8, exact in
// bf16, so x . w = hi . w + lo . w + r . w with hi = x truncated to bf16
// (never rounds up to inf), lo = bf16(x - hi) (x - hi is exact: the low 16
// bits of x's significand) and |r| <= 2^-16 |x|: each bf16 x int8 product is
// exact in the fp32 accumulators, and x keeps 16 significant bits (the
// reference's fp32 Triton dot runs at TF32 precision, 11 bits). Non-finite x:
// hi carries it (NaN canonical), lo = 0. k_f32_planes writes the two planes;
// k_gemm_dma<BF16, true, TM, true> then runs every tile once per plane and
// k-range (KS ranges per plane: 1, or up to 8 for M <= 64) into fp32 partial
// tiles, and k_planes_reduce adds them in order and applies the fp32 scale
// and bias.
__global__ __launch_bounds__(kBlock) void k_f32_planes(const float* __restrict__ x, int64_t n4,
                                                     uint16_t* __restrict__ xh,
                                                     uint16_t* __restrict__ xl) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n4) return;
  const f4 v = reinterpret_cast<const f4*>(x)[i];
  uint32_t hb[4];
  float lo[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t b = __float_as_uint(v[r]);
    const bool fin = (b & 0x7f800000u) != 0x7f800000u;
    const bool nan = !fin && (b & 0x007fffffu) != 0;
    hb[r] = nan ? 0x7fc0u : (b >> 16);
    lo[r] = fin ? v[r] - __uint_as_float(hb[r] << 16) : 0.0f;
  }
  reinterpret_cast<uint2*>(xh)[i] = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
  reinterpret_cast<uint2*>(xl)[i] =
      make_uint2(pack2_out<kBF16>(lo[0], lo[1]), pack2_out<kBF16>(lo[2], lo[3]));
}

// The 2 KS partial planes of every tile (layout as in k_splitk_reduce, all
// tiles split: the k-ranges of x plane hi, then those of plane lo), summed in
// that order -> y = fp32(sum * s[n] + bias[n]). Each thread takes two
// partial f4, kBlock apart.
template <int TM>
__global__ __launch_bounds__(kBlock) void k_planes_reduce(GemmArgs a, const float* __restrict__ sc,
                                                          const float* __restrict__ bias,
                                                          float* __restrict__ y) {
  constexpr int kWaveF4 = kDmaTN * TM * 4 * 64;
  constexpr int kTileF4 = 8 * kWaveF4;
  static_assert(kTileF4 % (kBlock * 2) == 0, "a thread's f4 share a tile");
  const int tiles = a.tiles_m * a.tiles_n;
  const int64_t per_plane = static_cast<int64_t>(tiles) * kTileF4;
  const int64_t idx0 = static_cast<int64_t>(blockIdx.x) * (kBlock * 2) + threadIdx.x;
  if (idx0 >= per_plane) return;
  const f4* src = reinterpret_cast<const f4*>(a.part) + idx0;
  f4 sum[2] = {src[0], src[kBlock]};
#pragma unroll 4
  for (int p = 1; p < a.splits; ++p) {
    const f4* q = src + p * per_plane;
    sum[0] += q[0];
    sum[1] += q[kBlock];
  }
  int tm, tn;
  group_tile(static_cast<int>(idx0 / kTileF4), a, tm, tn);
  const bool vec = (a.N % 4) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int w = static_cast<int>((idx0 + u * kBlock) % kWaveF4);
    const int lane = w & 63, q = (w >> 6) & 3, j = (w >> 8) % TM, i = (w >> 8) / TM;
    const int wave = static_cast<int>(((idx0 + u * kBlock) / kWaveF4) & 7);
    const int m = tm * 64 * TM + (wave & 1) * 32 * TM + j * 32 + (lane & 31);
    const int nb = tn * 256 + (wave >> 1) * 64 + i * 32 + 8 * q + 4 * (lane >> 5);
    if (m >= a.M || nb >= a.N) continue;
    f4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = nb + r < a.N ? sum[u][r] * sc[nb + r] : 0.0f;
    if (bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < a.N) v[r] += bias[nb + r];
    }
    float* dst = y + static_cast<int64_t>(m) * a.N + nb;
    if (vec && nb + 3 < a.N) {
      *reinterpret_cast<f4*>(dst) = v;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (nb + r < a.N) dst[r] = v[r];
    }
  }
}

// Launch plan of the k_gemm_dma path: x tile of 64 tm rows; tiles
// [0, full) whole, the rest split over `splits` k-ranges (splits == 1:
// every tile whole, no partials).
struct DmaPlan {
  int tm, full, splits;
};

// Bytes of split-K partials of a plan: one fp32 tile per tail tile and range.
int64_t splitk_bytes(int64_t M, int64_t N, const DmaPlan& p) {
  if (p.splits <= 1) return 0;
  const int64_t tiles = cdiv(M, 64 * p.tm) * cdiv(N, 256);
  return (tiles - p.full) * p.splits * (p.tm * 64) * 256 * 4;
}

template <int ACT, int TM>
void launch_gemm_dma_splitk(GemmArgs a, const DmaPlan& p, hipStream_t s) {
  a.tiles_m = static_cast<int>(cdiv(a.M, 64 * TM));
  a.tiles_n = static_cast<int>(cdiv(a.N, 256));
  a.full_tiles = p.full;
  const int nk = a.K / 64;
  a.split_steps = static_cast<int>(cdiv(nk, p.splits));
  a.splits = static_cast<int>(cdiv(nk, a.split_steps));   // no empty ranges
  const int rest = a.tiles_m * a.tiles_n - a.full_tiles;
  const unsigned grid = static_cast<unsigned>(a.full_tiles + rest * a.splits);
  k_gemm_dma<ACT, true, TM><<<dim3(grid), dim3(kDmaThreads), 0, s>>>(a);
  const int64_t n4 = static_cast<int64_t>(rest) * 8 * kDmaTN * TM * 4 * 64;
  const dim3 rgrid(static_cast<unsigned>(cdiv(n4, kBlock * kReduceF4)));
  if (a.n_out > 0) k_splitk_reduce<ACT, TM, true><<<rgrid, dim3(kBlock), 0, s>>>(a);
  else k_splitk_reduce<ACT, TM, false><<<rgrid, dim3(kBlock), 0, s>>>(a);
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
    if (m < a.M) {
#pragma unroll
      for (int i = 0; i < TN; ++i) store_quad<ACT>(a, acc[i][j], m, n0 + i * 16 + g * 4, vec_store);
    }
  }
}

template <int ACT, int TM, int TN, int U>
void launch_skinny(GemmArgs a, hipStream_t s) {
  k_skinny<ACT, TM, TN, U><<<dim3(static_cast<unsigned>(cdiv(a.N, 16 * TN))), dim3(256), 0, s>>>(a);
}

// ---------------------------------------------------------------------------
// k_stream<ACT, TM> (M <= 16 * TM, TM <= 4): persistent weight streaming.
//
// One 16-wave workgroup per CU owns up to kStreamMaxTiles (3) row tiles of
// 16 weight rows (tile b, b + G, b + 2G for grid size G). The activations
// are staged in LDS by DMA once per K-chunk (the M rows, kc columns; at most
// 128 KiB) and shared by every tile of the workgroup, so x crosses L2 once
// per CU and chunk instead of once per row tile. Within a chunk the 16 waves
// split the 64-k blocks. Each wave issues the x DMA, then the weight loads of
// all its (tile, block) pairs straight from HBM into registers
// (non-temporal, 16 bytes per lane, a fixed count so that the wait for the
// DMA, vmcnt(#weight loads), leaves them in flight), then multiplies: per
// block two x fragment reads from LDS serve every tile. Per block a lane
// holds W[n][k0 + 16 g .. +16] and x[m][k0 + 16 g .. +16] (g = lane / 16):
// the low and high 8 values feed two v_mfma_f32_16x16x32 with the same k
// permutation on both operands. After the last chunk all partial tiles go
// through LDS at once; wave (tile r, m-tile j) sums its 16 partials in wave
// order (deterministic) and runs the epilogue with scales loaded at start.
//
// x LDS rows are padded by 16 bytes so that the 16 rows of a fragment read
// fall in distinct bank groups; rows past M are not staged (their outputs
// are never stored). Requirements (host): K % 1024 == 0, 16-byte aligned x
// and wq, M <= 16 * TM, M * K * 2 < 2^32.
constexpr int kStreamWaves = 16;
constexpr int kStreamMaxTiles = 3;
constexpr int kStreamLdsBytes = 132096;   // x chunk, then the partial tiles

template <int TM>
constexpr int stream_kc() { return TM == 1 ? 4096 : TM == 2 ? 2048 : 1024; }

template <int ACT, int TM>
__global__ __launch_bounds__(64 * kStreamWaves) void k_stream(GemmArgs a) {
  constexpr int MP = 16 * TM;                 // padded rows
  constexpr int KC = stream_kc<TM>();         // chunk columns
  constexpr int RS = KC * 2 + 16;             // LDS row stride, bytes
  constexpr int NB = KC / 64 / kStreamWaves;  // 64-k blocks per wave per chunk
  constexpr int RT = kStreamMaxTiles;
  constexpr int NLOAD = NB * RT;              // weight loads per wave per chunk
  static_assert(MP * RS <= kStreamLdsBytes, "x chunk fits in LDS");
  static_assert(RT * TM <= kStreamWaves, "one reduction pair per wave");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStreamLdsBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = lane & 15, g = lane >> 4;
  const int tiles = (a.N + 15) / 16;
  const int G = gridDim.x;
  const uint32_t sbase = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  int ntile = 0;
#pragma unroll
  for (int r = 0; r < RT; ++r) ntile += (static_cast<int>(blockIdx.x) + r * G < tiles) ? 1 : 0;

  // Reduction pair of this wave: tile rr, m-tile jr. Its scales and bias are
  // loaded now, long before they are needed.
  const int rr = wave / TM, jr = wave % TM;
  const bool has_pair = rr < ntile && jr * 16 < a.M;
  const int nq = (static_cast<int>(blockIdx.x) + rr * G) * 16 + g * 4;
  // Raw values, loaded unconditionally (clamped index) so that they do not
  // serialize the kernel's start; converted in the epilogue.
  uint16_t sraw[4], braw[4];
  const uint16_t* bsrc = a.bias ? a.bias : a.scales;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = min(nq + q, a.N - 1);
    sraw[q] = a.scales[n];
    braw[q] = bsrc[n];
  }

  f4 acc[RT][TM];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[r][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  // Weight row of this lane in each tile (clamped: loads of missing tiles
  // and blocks read valid memory and their products are skipped).
  const int8_t* wrow[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int tile = min(static_cast<int>(blockIdx.x) + r * G, tiles - 1);
    wrow[r] = a.wq + static_cast<int64_t>(min(tile * 16 + row, a.N - 1)) * a.K + 16 * g;
  }

  for (int c0 = 0; c0 < a.K; c0 += KC) {
    const int clen = min(KC, a.K - c0);       // a multiple of 1024
    const int nb = clen / 64;
    __syncthreads();                          // previous chunk's x reads done
    // Stage x[0 .. M, c0 .. c0 + clen) in LDS: one wave instruction moves
    // 1 KiB (512 values) of one row.
    const int segs = clen / 512;
    for (int q = wave; q < a.M * segs && q < MP * segs; q += kStreamWaves) {
      const int m = q / segs, sg = q % segs;
      lds_dma16(static_cast<uint32_t>((m * a.K + c0 + sg * 512) * 2) + lane * 16u,
                uniform_ptr(a.x), sbase + m * RS + sg * 1024);
    }
    // Weight loads of all (block, tile) pairs of this wave, always NLOAD.
    // Wave blocks are contiguous (b = wave * nbw + i) so that one wave reads
    // both 64-byte halves of each 128-byte line of its rows.
    const int nbw = nb / kStreamWaves;        // nb is a multiple of 16
    u32x4 w[NB][RT];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = min(wave * nbw + i, nb - 1);
#pragma unroll
      for (int r = 0; r < RT; ++r)
        w[i][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[r] + c0 + b * 64));
    }
    // The DMA was issued before the NLOAD weight loads; loads complete in
    // order, so at most NLOAD outstanding means the DMA has landed.
    dma_wait_barrier<NLOAD>();
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = wave * nbw + i;
      if (i >= nbw) continue;
      u32x4 xl[TM], xh[TM];
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const uint8_t* p = smem + (j * 16 + row) * RS + (b * 64 + 16 * g) * 2;
        xl[j] = *reinterpret_cast<const u32x4*>(p);
        xh[j] = *reinterpret_cast<const u32x4*>(p + 16);
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (r >= ntile) continue;
        uint32_t o[8];
        i8x4_to_act<ACT>(w[i][r].x, o[0], o[1]);
        i8x4_to_act<ACT>(w[i][r].y, o[2], o[3]);
        i8x4_to_act<ACT>(w[i][r].z, o[4], o[5]);
        i8x4_to_act<ACT>(w[i][r].w, o[6], o[7]);
        const u32x4 lo = {o[0], o[1], o[2], o[3]}, hi = {o[4], o[5], o[6], o[7]};
#pragma unroll
        for (int j = 0; j < TM; ++j) {
          acc[r][j] = mfma16x16x32<ACT>(lo, xl[j], acc[r][j]);
          acc[r][j] = mfma16x16x32<ACT>(hi, xh[j], acc[r][j]);
        }
      }
    }
  }

  // All partial tiles through LDS (rounds of RPR tiles if they do not fit);
  // wave (rr, jr) sums its 16 partials in wave order and stores.
  constexpr int RPR = kStreamLdsBytes / (kStreamWaves * TM * 1024) < RT
                          ? kStreamLdsBytes / (kStreamWaves * TM * 1024) : RT;
  f4* red = reinterpret_cast<f4*>(smem);
  const bool vec_store = (a.N % 4) == 0;
#pragma unroll
  for (int r0 = 0; r0 < RT; r0 += RPR) {
    __syncthreads();
#pragma unroll
    for (int r = r0; r < r0 + RPR && r < RT; ++r)
#pragma unroll
      for (int j = 0; j < TM; ++j)
        red[(((r - r0) * TM + j) * kStreamWaves + wave) * 64 + lane] = acc[r][j];
    __syncthreads();
    if (has_pair && rr >= r0 && rr < r0 + RPR) {
      const f4* src = red + ((rr - r0) * TM + jr) * kStreamWaves * 64 + lane;
      f4 sum = src[0];
      for (int w2 = 1; w2 < kStreamWaves; ++w2) sum += src[w2 * 64];
      const int m = jr * 16 + row;
      if (m < a.M) {
        f4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = sum[q] * act_to_f32<ACT>(sraw[q]);
        if (a.n_out > 0) v = outlier_quad<ACT>(a, m, nq, v);
        if (a.bias) {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] += act_to_f32<ACT>(braw[q]);
        }
        uint16_t* dst = a.y + static_cast<int64_t>(m) * a.N + nq;
        if (vec_store && nq + 3 < a.N) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack2_out<ACT>(v[0], v[1]),
                                                      pack2_out<ACT>(v[2], v[3]));
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nq + q < a.N) dst[q] = out1<ACT>(v[q]);
        }
      }
    }
  }
}

// k_stream1<ACT, RT> (M <= 16): weight streaming with row-contiguous loads.
//
// One 16-wave workgroup owns RT consecutive row tiles (16 RT weight rows;
// RT = 3, or 4 when 48-row workgroups would outnumber the CUs). Every wave
// issues all of its weight loads at once, as 1 KiB row-contiguous requests
// (wave w: rows RT w .. RT w + RT - 1, step by step; 64 lanes x 16 bytes per
// request), which stream from HBM far faster than MFMA-shaped requests
// (16 rows x 64 bytes). Per 1024-k step the rows are written to a
// padded LDS stage (row stride 1040 bytes: the 16 rows of a fragment read
// fall in distinct bank groups), one barrier, and read back in the MFMA
// layout: wave w takes 64-k block w of the step for all RT tiles, with its
// x fragments loaded from L2 up front. k order within a block as in
// k_stream. The 16 partial tiles are summed in wave order (deterministic).
// Requirements (host): K % 1024 == 0, K <= 4096, 16-byte aligned x and wq,
// M <= 16.
constexpr int kStream1Stride = 1040;
constexpr int kStream1MaxSteps = 4;
constexpr int kStream1MaxRT = 4;   // two stages of 64 rows: 130 KiB of LDS

template <int ACT, int RT>
__global__ __launch_bounds__(1024) void k_stream1(GemmArgs a) {
  constexpr int ROWS = 16 * RT, SB = ROWS * kStream1Stride, NST = kStream1MaxSteps;
  static_assert(RT >= 3 && RT <= kStream1MaxRT, "3 or 4 row tiles");
  static_assert(2 * SB <= 160 * 1024, "two LDS stages");
  static_assert(16 * RT * 64 * 16 <= 2 * SB, "reduction fits in the stages");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * SB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * ROWS;
  const int nsteps = a.K / 1024;

  // Scale and bias of this lane's outputs (wave r < 3 finishes tile r).
  const int nq = n0 + wave * 16 + g * 4;
  const uint16_t* bsrc = a.bias ? a.bias : a.scales;
  uint16_t sraw[4], braw[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = min(nq + q, a.N - 1);
    sraw[q] = a.scales[n];
    braw[q] = bsrc[n];
  }
  __builtin_amdgcn_sched_barrier(0);
  // Loads in step order: the x fragments of block `wave` of step s (row
  // `row`; rows past M repeat row M - 1, their outputs are never stored),
  // then step s of this wave's weight rows n0 + 3 wave + i (clamped), each
  // a 1 KiB row-contiguous request. Loads complete in issue order, so step
  // s can start once its own loads have landed. Pinned with scheduling
  // barriers; measured at M = 16, N = 11008, K = 4096: 15.3 us event-timed,
  // against 16.3 us with each row's four steps issued together and x last,
  // and 16.8 us with all of x first.
  const int mr = min(row, a.M - 1);
  u32x4 xl[NST], xh[NST], wr[NST][RT];
#pragma unroll
  for (int s = 0; s < NST; ++s) {
    const int sc = min(s, nsteps - 1);
    const u32x4* xp = reinterpret_cast<const u32x4*>(
        a.x + static_cast<int64_t>(mr) * a.K + sc * 1024 + wave * 64 + 16 * g);
    xl[s] = xp[0];
    xh[s] = xp[1];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int n = min(n0 + RT * wave + i, a.N - 1);
      wr[s][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          a.wq + static_cast<int64_t>(n) * a.K + sc * 1024 + lane * 16));
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  f4 acc[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) acc[r] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < NST; ++s) {
    if (s >= nsteps) break;
    uint8_t* st = smem + (s & 1) * SB;
    // Stage s: rows 3 wave + i. The previous use of this stage (step
    // s - 2) ended before the barrier of step s - 1.
#pragma unroll
    for (int i = 0; i < RT; ++i)
      *reinterpret_cast<u32x4*>(st + (RT * wave + i) * kStream1Stride + lane * 16) = wr[s][i];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const u32x4 wf =
          *reinterpret_cast<const u32x4*>(st + (r * 16 + row) * kStream1Stride + wave * 64 + 16 * g);
      uint32_t o[8];
      i8x4_to_act<ACT>(wf.x, o[0], o[1]);
      i8x4_to_act<ACT>(wf.y, o[2], o[3]);
      i8x4_to_act<ACT>(wf.z, o[4], o[5]);
      i8x4_to_act<ACT>(wf.w, o[6], o[7]);
      const u32x4 lo = {o[0], o[1], o[2], o[3]}, hi = {o[4], o[5], o[6], o[7]};
      acc[r] = mfma16x16x32<ACT>(lo, xl[s], acc[r]);
      acc[r] = mfma16x16x32<ACT>(hi, xh[s], acc[r]);
    }
  }

  // Partial tiles through LDS; wave r (< 3) sums tile r in wave order.
  __syncthreads();
  f4* red = reinterpret_cast<f4*>(smem);
#pragma unroll
  for (int r = 0; r < RT; ++r) red[(r * 16 + wave) * 64 + lane] = acc[r];
  __syncthreads();
  if (wave < RT && n0 + wave * 16 < a.N && row < a.M) {
    const f4* src = red + wave * 16 * 64 + lane;
    f4 sum = src[0];
    for (int w2 = 1; w2 < 16; ++w2) sum += src[w2 * 64];
    f4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = sum[q] * act_to_f32<ACT>(sraw[q]);
    if (a.n_out > 0) v = outlier_quad<ACT>(a, row, nq, v);
    if (a.bias) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += act_to_f32<ACT>(braw[q]);
    }
    uint16_t* dst = a.y + static_cast<int64_t>(row) * a.N + nq;
    if ((a.N % 4) == 0 && nq + 3 < a.N) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack2_out<ACT>(v[0], v[1]),
                                                  pack2_out<ACT>(v[2], v[3]));
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (nq + q < a.N) dst[q] = out1<ACT>(v[q]);
    }
  }
}

// Row tiles per k_stream1 workgroup: 3 while 48-row workgroups fit on the
// CUs at once, else 4 (0: neither fits; the host picks another kernel).
// Measured on MI355X, M = 16, K = 4096, N = 14336: 299 workgroups of 48 rows
// do not fit, and the kernel it then fell back to (k_skinny) took 30.0 us;
// 224 workgroups of 64 rows took 23.8 us.
int stream1_tiles(int64_t N) {
  const int64_t cus = device_cus();
  if (cdiv(N, 48) <= cus) return 3;
  if (cdiv(N, 16 * kStream1MaxRT) <= cus) return kStream1MaxRT;
  return 0;
}

template <int ACT>
void launch_stream1(GemmArgs a, hipStream_t s) {
  const int rt = stream1_tiles(a.N);
  const unsigned grid = static_cast<unsigned>(cdiv(a.N, 16 * rt));
  if (rt == 3) k_stream1<ACT, 3><<<dim3(grid), dim3(1024), 0, s>>>(a);
  else k_stream1<ACT, kStream1MaxRT><<<dim3(grid), dim3(1024), 0, s>>>(a);
}

template <int ACT, int TM>
void launch_stream(GemmArgs a, hipStream_t s) {
  const int tiles = static_cast<int>(cdiv(a.N, 16));
  int grid = std::min(tiles, device_cus());
  grid = std::max(grid, static_cast<int>(cdiv(tiles, kStreamMaxTiles)));
  k_stream<ACT, TM><<<dim3(static_cast<unsigned>(grid)), dim3(64 * kStreamWaves), 0, s>>>(a);
}

// Any shape or activation dtype (fp32 activations, K not a multiple of 16,
// unaligned pointers): k_w8a16_general<ACT, BM, BN, SPLIT>. Output tile
// BM (m) x BN (n) per 256-thread workgroup, 64 x 64 or, for M <= 16,
// 16 x 256; each thread owns 4 rows x 4 consecutive n. Per 32-k step the
// workgroup loads the activation tile (BM x 32, element loads along k,
// coalesced) and the int8 weight tile (BN x 32) into registers, converts
// both to fp32 and stores them k-major in LDS; the next step's loads are in
// flight while the current one is multiplied (two LDS buffers, one barrier
// per step). fp32 FMA accumulation on the VALU (no MFMA: fp32 operands are
// the point of this path), then the same epilogue as the MFMA kernels:
// scale, outlier side-GEMM, bias, one rounding. When the tiles alone leave
// the GPU under-occupied (small M) the host splits K into `splits` ranges:
// workgroup (split, tile) writes its fp32 sums to the workspace and
// k_general_reduce adds the ranges in order (deterministic) before the
// epilogue.
constexpr int kGenBK = 32;
constexpr int kGenThreads = 256;

struct GenArgs {
  const void* x;           // [M, K] act
  const int8_t* wq;        // [N, K]
  const void* scales;      // [N] act
  const void* bias;        // [N] act or null
  const int64_t* oc;       // [n_out]
  const void* w_out;       // [N, n_out] act
  void* y;                 // [M, N] act
  float* part;             // [splits, M, N] fp32 (split mode)
  int64_t n_out, M, N, K;
  int64_t tiles_n, tiles;  // output tiles along n, in total
  int64_t kper;            // k per split (a multiple of kGenBK, hence of every k step)
  int splits;
};

// Epilogue of one output: scale, outlier side-GEMM, bias, one rounding.
template <int ACT>
__device__ __forceinline__ void general_out(const GenArgs& a, int64_t m, int64_t n, float acc) {
  float val = acc * ld1<ACT>(a.scales, n);
  for (int64_t jj = 0; jj < a.n_out; ++jj) {
    const int64_t k = a.oc[jj];
    if (k >= 0 && k < a.K)
      val += ld1<ACT>(a.x, m * a.K + k) * ld1<ACT>(a.w_out, n * a.n_out + jj);
  }
  if (a.bias) val += ld1<ACT>(a.bias, n);
  if constexpr (ACT == kF32) static_cast<float*>(a.y)[m * a.N + n] = val;
  else static_cast<uint16_t*>(a.y)[m * a.N + n] = out1<ACT>(val);
}

template <int ACT, int BM, int BN, bool SPLIT>
__global__ __launch_bounds__(kGenThreads) void k_w8a16_general(GenArgs a) {
  constexpr int TM = 4, TN = 4;
  // 32-k steps; 16 for the 256-wide tile (32 weight codes per thread per
  // step would cost more address registers than the loads are worth)
  constexpr int BK = BN > 64 ? 16 : kGenBK;
  static_assert((BM / TM) * (BN / TN) == kGenThreads, "one 4 x 4 output block per thread");
  constexpr int XL = BM * BK / kGenThreads;        // activation elements per thread per step
  constexpr int WL = BN * BK / kGenThreads;        // weight codes per thread per step
  // k-major tiles; rows padded by 4 floats (keeps the float4 reads aligned)
  __shared__ __align__(16) float xs[2][BK][BM + 4];
  __shared__ __align__(16) float ws[2][BK][BN + 4];
  const int tid = threadIdx.x;
  const int tn = tid % (BN / TN), tm = tid / (BN / TN);
  const int64_t bid = blockIdx.x;
  const int64_t split = SPLIT ? bid / a.tiles : 0;
  const int64_t tile = SPLIT ? bid % a.tiles : bid;
  const int64_t m0 = (tile / a.tiles_n) * BM, n0 = (tile % a.tiles_n) * BN;
  const int64_t kb = SPLIT ? split * a.kper : 0;
  const int64_t ke = SPLIT ? min(a.K, kb + a.kper) : a.K;
  const int64_t M = a.M, N = a.N, K = a.K;

  float xr[XL], wr[WL];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kGenThreads, r = e / BK, kk = e % BK;
      const int64_t m = m0 + r, k = k0 + kk;
      xr[i] = (m < M && k < ke) ? ld1<ACT>(a.x, m * K + k) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const int e = tid + i * kGenThreads, r = e / BK, kk = e % BK;
      const int64_t n = n0 + r, k = k0 + kk;
      wr[i] = (n < N && k < ke) ? static_cast<float>(a.wq[n * K + k]) : 0.0f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int e = tid + i * kGenThreads;
      xs[buf][e % BK][e / BK] = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const int e = tid + i * kGenThreads;
      ws[buf][e % BK][e / BK] = wr[i];
    }
  };

  float acc[TM][TN] = {};
  const int64_t nt = ke > kb ? (ke - kb + BK - 1) / BK : 0;
  if (nt > 0) {
    load(kb);
    store(0);
    __syncthreads();
  }
  for (int64_t t = 0; t < nt; ++t) {
    const int buf = static_cast<int>(t & 1);
    if (t + 1 < nt) load(kb + (t + 1) * BK);
#pragma unroll 8
    for (int kk = 0; kk < BK; ++kk) {
      float xv[TM], wv[TN];
      const float4 v = *reinterpret_cast<const float4*>(&xs[buf][kk][tm * 4]);
      xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
      const float4 w4 = *reinterpret_cast<const float4*>(&ws[buf][kk][tn * 4]);
      wv[0] = w4.x; wv[1] = w4.y; wv[2] = w4.z; wv[3] = w4.w;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_fmaf(xv[i], wv[j], acc[i][j]);
    }
    if (t + 1 < nt) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + tn * 4 + j;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = m0 + tm * TM + i;
      if (m >= M) continue;
      if constexpr (SPLIT) a.part[(split * M + m) * N + n] = acc[i][j];
      else general_out<ACT>(a, m, n, acc[i][j]);
    }
  }
}

// Split-K finish of the general path: one thread per output, the ranges
// summed in order, then the epilogue.
template <int ACT>
__global__ __launch_bounds__(kBlock) void k_general_reduce(GenArgs a) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t mn = a.M * a.N;
  if (idx >= mn) return;
  float sum = a.part[idx];
  int sp = 1;
  for (; sp + 8 <= a.splits; sp += 8) {   // in order; 8 loads issued before their adds
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = a.part[(sp + u) * mn + idx];
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += v[u];
  }
  for (; sp < a.splits; ++sp) sum += a.part[sp * mn + idx];
  general_out<ACT>(a, idx / a.N, idx % a.N, sum);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Kernel choice by M (measured on MI355X at N = 11008, K = 4096):
//   M <= 16       k_stream1 when the weight is at least 8 MB, K % 1024 == 0,
//                 K <= 4096 and the 48-row (else 64-row) groups fit one
//                 wave of workgroups; else k_skinny (TM = 1)
//   M <= 64       k_stream<2 or 4> under the same size rules (3 row tiles
//                 per workgroup); else k_skinny, TM = ceil(M / 16); for
//                 M > 24 and K > 8192 the split k_gemm_dma plan below first
//   M > 64        k_gemm_dma (K % 64 == 0 and 32-bit operand offsets) with
//                 the x tile (256 or 128 rows) and split-K plan of dma_plan:
//                 the last, short wave of tiles split over K (2-16 k-ranges,
//                 partial tiles in the workspace, k_splitk_reduce) when the
//                 time model prefers it and the caller's workspace holds the
//                 partials, unless one round of 128 x 128 tiles
//                 (k_gemm_dma128, no partials) is modelled faster;
//   M > 64        else k_gemm_dma without a split (x tile of dma_plan), or
//                 k_gemm_dma128 where modelled faster; without k_gemm_dma
//                 (K % 64 != 0 or offsets past 32 bits) k_gemm 128 x 64 x 64,
//                 2 x 2 waves (M >= 1024: 256 x 256 x 64, 4 x 2 waves)
enum Kind { kSkinny1, kSkinny2, kSkinny4, kTileMid, kTileLarge, kTileDma, kStream1, kStream2,
            kStream4, kTileDmaSplit, kTileDma128 };

// The streaming kernels pay a fixed cost for their large workgroups; below
// 8 MB of weight the k_skinny kernels are faster.
bool stream_ok(int64_t M, int64_t N, int64_t K) {
  return K % 1024 == 0 && N * K >= (8LL << 20) && M * K * 2 < (1LL << 31);
}

// k_gemm_dma addresses x and wq with 32-bit byte offsets from a scalar base
// and needs whole 64-k steps.
bool dma_ok(int64_t M, int64_t N, int64_t K) {
  constexpr int64_t kLim = (1LL << 32) - 4096;
  return K % 64 == 0 && M * K * 2 < kLim && N * K < kLim;
}

// Plan of the k_gemm_dma path with the lowest modelled time (0.01 us): the
// 64-k steps of the longest chain of workgroups on one CU times the cost of
// a step, which grows with the share of CUs busy (clock and bandwidth under
// load): 1.30 + 0.55 occ us for 256 x 256 tiles, 0.96 + 0.50 occ us for
// 192 x 256, 0.84 + 0.28 occ us for 128 x 256; plus, when split, 5 us for the reduce pass and 0.12 us per
// 256 KiB of partial tiles written and re-read. With `rest` tiles in the
// last, short wave, a split runs the full waves whole and the rest over sp
// k-ranges (rest x sp workgroups fit one wave of CUs, each range keeps at
// least four 64-k steps). Fitted on MI355X over M = 96..4096 at N = 11008,
// K = 4096 and N = 4096, K = 11008 (fp16; over those 20 shapes the plan
// picked is 0.6% slower than the best one measured on average, 3.4% at
// worst). E.g. M = 1536, N = 11008: whole 256 x 256 tiles 208 us, the 2
// tail tiles over 16 ranges 133 us; M = 768: 172 tiles of 192 x 256 in one
// wave 74.9 us, 258 of 128 x 256 with the tail split 79.6 us; M = 128:
// 256 x 256 over 5 ranges 46.8 us, 128 x 256 over 4 ranges 29.8 us.
int64_t dma_step_cost(int tm, int64_t wgs, int64_t cus) {
  const int64_t busy = std::min(wgs, cus);
  if (tm == 4) return 130 + 55 * busy / cus;
  if (tm == 3) return 96 + 50 * busy / cus;
  return 84 + 28 * busy / cus;
}

DmaPlan dma_plan(int64_t M, int64_t N, int64_t K, bool allow_split, int64_t* cost = nullptr) {
  const int64_t cus = device_cus(), nk = K / 64;
  DmaPlan best{4, 0, 1};
  int64_t best_cost = INT64_MAX;
  for (const int tm : {4, 2, 3}) {
    const int64_t tiles = cdiv(M, 64 * tm) * cdiv(N, 256);
    const int64_t rounds = tiles / cus, rest = tiles % cus;
    const int64_t whole = nk * cdiv(tiles, cus) * dma_step_cost(tm, tiles, cus);
    if (whole < best_cost) {
      best = {tm, static_cast<int>(tiles), 1};
      best_cost = whole;
    }
    if (!allow_split || rest == 0) continue;
    const int64_t max_sp = std::min<int64_t>({16, cus / rest, nk / 4});
    for (int64_t sp = 2; sp <= max_sp; ++sp) {
      const int64_t wgs = rounds * cus + rest * sp;
      const int64_t cost = (rounds * nk + cdiv(nk, sp)) * dma_step_cost(tm, wgs, cus) + 500 +
                           3 * tm * rest * sp;
      if (cost < best_cost) {
        best = {tm, static_cast<int>(rounds * cus), static_cast<int>(sp)};
        best_cost = cost;
      }
    }
  }
  if (cost) *cost = best_cost;
  return best;
}

// Modelled time of the 128 x 128 tiles (k_gemm_dma128) on dma_plan's scale,
// for M > 64 (else no estimate). When the tiles fit one workgroup per CU:
// 6.9 us plus (0.41 + 0.17 x share of CUs busy) us per 64-k step, as timed
// on MI355X (op level, fp16) over M = 128..256, N = 8192..28672,
// K = 2048..8192, times the 1.13 by which dma_plan's model exceeds the
// measured time of its split plans at those shapes. Measured against the
// plans it displaces (op level): M = 256, N = 11008, K = 4096 39.7 against
// 41.6 us (split 128 x 256 tiles); N = 14336 41.8 against 46.9; N = 16384
// 44.4 against 54.2; M = 128, N = 28672 48.2 against 55.6; K = 2048 23.3
// against 47.2 (no split: k_gemm). It loses where a split keeps more CUs busy
// for fewer steps (K = 8192: 67.7 against 64.4; M = 160: 39.4 against 37.0;
// N = 4096, K = 11008: 95 against 40), which the model leaves to the split.
// With more tiles than CUs two workgroups share each CU: 1.2 model units
// (1.06 us) per 64-k step and round of 2 x CUs tiles, which leaves those
// shapes to the whole 128-256 row tiles where they are faster (M = 320,
// N = 22016: 69.0 against 89.1 us; M = 256, N = 65536: 116.4 against
// 138.0; M = 200, N = 50000, K = 2048: 53.4 against 64.5).
int64_t dma128_cost(int64_t M, int64_t N, int64_t K) {
  const int64_t cus = device_cus();
  const int64_t tiles = cdiv(M, 128) * cdiv(N, 128), nk = K / 64;
  if (M <= 64) return INT64_MAX;
  if (tiles <= cus) return 780 + nk * (46 + 19 * tiles / cus);
  return 780 + nk * 120 * cdiv(tiles, 2 * cus);
}

// Whether k_gemm_dma is a candidate: M > 64, or 24 < M <= 64 with K above
// 8 x-chunks of k_stream<4> (from 8 chunks on its per-chunk staging and
// barriers cost more than the empty rows of a 128-row MFMA tile: N = 4096,
// K = 11008, M = 64: k_stream 52.2 us, 128 x 256 tiles over 11 k-ranges
// about 31 us; M = 32: k_stream<2> 32.4 us; at M = 24 the two are level, and
// at K = 4096 k_stream is ahead, 29.8 us at M = 64).
bool dma_candidate(int64_t M, int64_t N, int64_t K) {
  return (M > 64 || (M > 24 && K > 8 * stream_kc<4>())) && dma_ok(M, N, K);
}

// The split plan when it applies (and the 128 x 128 tiles are not modelled
// faster), else none.
DmaPlan split_plan(int64_t M, int64_t N, int64_t K) {
  if (!dma_candidate(M, N, K)) return DmaPlan{4, 0, 1};
  int64_t cost = 0;
  const DmaPlan p = dma_plan(M, N, K, true, &cost);
  if (p.splits > 1 && dma128_cost(M, N, K) < cost) return DmaPlan{4, 0, 1};
  return p;
}

Kind choose(int64_t M, int64_t N, int64_t K, int64_t n_out, size_t ws_bytes, DmaPlan& plan) {
  const int64_t cus = device_cus();
  const bool stream = stream_ok(M, N, K);
  if (M <= 16)
    return (stream && K <= 4096 && stream1_tiles(N) > 0) ? kStream1 : kSkinny1;
  const bool tiles_fit = cdiv(N, 16) <= kStreamMaxTiles * cus;
  const Kind narrow = M <= 32 ? ((stream && tiles_fit) ? kStream2 : kSkinny2)
                              : ((stream && tiles_fit) ? kStream4 : kSkinny4);
  if (M <= 64 && !dma_candidate(M, N, K)) return narrow;
  if (!dma_ok(M, N, K)) return M < 1024 ? kTileMid : kTileLarge;
  int64_t cost = 0;
  plan = dma_plan(M, N, K, true, &cost);
  const int64_t cost128 = dma128_cost(M, N, K);
  if (plan.splits > 1 &&
      ws_bytes >= static_cast<size_t>(CBQ_WS_CTRL_BYTES + splitk_bytes(M, N, plan)))
    return cost128 < cost ? kTileDma128 : kTileDmaSplit;
  if (M <= 64) return narrow;
  // no split: whole tiles of 128-256 rows or the 128 x 128 tiles, by the
  // model (below 384 rows both are about 2x faster than k_gemm's 128 x 64
  // tiles: 40.0 against 78.5 us at M = 256, N = 11008, K = 4096 without a
  // workspace; 38.4 against 74.2 us at M = 128, N = K = 4096)
  plan = dma_plan(M, N, K, false, &cost);
  return cost128 < cost ? kTileDma128 : kTileDma;
}

template <int ACT, int BM, int BN, int BK, int WGM, int WGN, int PD>
void launch_gemm(GemmArgs a, hipStream_t s) {
  a.tiles_m = static_cast<int>(cdiv(a.M, BM));
  a.tiles_n = static_cast<int>(cdiv(a.N, BN));
  const unsigned grid = static_cast<unsigned>(a.tiles_m) * a.tiles_n;
  k_gemm<ACT, BM, BN, BK, WGM, WGN, PD><<<dim3(grid), dim3(64 * WGM * WGN), 0, s>>>(a);
}

template <int ACT>
void launch_kind(Kind k, const GemmArgs& a, const DmaPlan& p, hipStream_t s) {
  switch (k) {
    case kSkinny1: launch_skinny<ACT, 1, 1, 4>(a, s); break;
    case kSkinny2: launch_skinny<ACT, 2, 1, 4>(a, s); break;
    case kSkinny4: launch_skinny<ACT, 4, 1, 2>(a, s); break;
    case kStream1: launch_stream1<ACT>(a, s); break;
    case kStream2: launch_stream<ACT, 2>(a, s); break;
    case kStream4: launch_stream<ACT, 4>(a, s); break;
    case kTileMid: launch_gemm<ACT, 128, 64, 64, 2, 2, 1>(a, s); break;
    case kTileDma:
      if (p.tm == 2) launch_gemm_dma<ACT, 2>(a, s);
      else if (p.tm == 3) launch_gemm_dma<ACT, 3>(a, s);
      else launch_gemm_dma<ACT, 4>(a, s);
      break;
    case kTileDma128: launch_gemm_dma128<ACT>(a, s); break;
    case kTileDmaSplit:
      if (p.tm == 2) launch_gemm_dma_splitk<ACT, 2>(a, p, s);
      else if (p.tm == 3) launch_gemm_dma_splitk<ACT, 3>(a, p, s);
      else launch_gemm_dma_splitk<ACT, 4>(a, p, s);
      break;
    default: launch_gemm<ACT, 256, 256, 64, 4, 2, 1>(a, s); break;
  }
}

// Tile of the general path: 16 x 256 for M <= 16, else 64 x 64.
int general_bm(int64_t M) { return M <= 16 ? 16 : 64; }
int general_bn(int64_t M) { return M <= 16 ? 256 : 64; }

// k-ranges of the general path (1: no split): enough workgroups for about
// four per CU when the tiles alone are fewer than two per CU, each range at
// least four 32-k steps, at most 16 ranges (measured on MI355X, M = 16,
// N = 11008, K = 4096, fp32: 289 us in one range).
int general_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = cdiv(M, general_bm(M)) * cdiv(N, general_bn(M));
  const int64_t cus = device_cus();
  if (tiles >= 2 * cus) return 1;
  const int64_t sp = std::min<int64_t>({16, cdiv(4 * cus, tiles), K / (4 * kGenBK)});
  return sp >= 2 ? static_cast<int>(sp) : 1;
}

int64_t general_split_bytes(int64_t M, int64_t N, int64_t K) {
  const int sp = general_splits(M, N, K);
  return sp > 1 ? static_cast<int64_t>(sp) * M * N * 4 : 0;
}

// Two-plane fp32 path (see k_f32_planes): no outlier columns, the DMA
// kernel's shape limits, and for M <= 64 a weight of at least 8 MB (below
// that the general kernel's single launch is as fast). The x-tile height
// with the fewest modelled step units over both planes' workgroups: rounds
// of workgroups on the CUs times the full-occupancy cost of a 64-k step
// (dma_plan's model: 1.12 / 1.46 / 1.85 us for 128 / 192 / 256-row tiles).
// For M <= 64 (one row of 128-row tiles) K is also split into KS ranges, so
// that the 2 KS planes' workgroups fill the CUs (at most 8 ranges of at
// least four 64-k steps): fp32 x at M = 16, N = 11008, K = 4096 takes two
// ranges, 172 workgroups.
bool planes_ok(int64_t M, int64_t N, int64_t K, int64_t n_out) {
  return n_out == 0 && dma_ok(M, N, K) && 2 * cdiv(M, 128) * cdiv(N, 256) < (1LL << 30) &&
         (M > 64 || N * K >= (8LL << 20));
}

int planes_tm(int64_t M, int64_t N) {
  const int64_t cus = device_cus();
  const double cost[5] = {0.0, 0.0, 1.12, 1.46, 1.85};
  int best_tm = 4;
  double best = 1e300;
  for (int tm = 2; tm <= 4; ++tm) {
    const int64_t wgs = 2 * cdiv(M, static_cast<int64_t>(64 * tm)) * cdiv(N, static_cast<int64_t>(256));
    const double t = static_cast<double>(cdiv(wgs, cus)) * cost[tm];
    if (t < best - 1e-9) {
      best = t;
      best_tm = tm;
    }
  }
  return best_tm;
}

struct PlanesPlan {
  int tm, ks, steps;   // x-tile height / 64, k-ranges per plane, 64-k steps per range
};

PlanesPlan planes_plan(int64_t M, int64_t N, int64_t K) {
  const int tm = planes_tm(M, N);
  const int64_t tiles = cdiv(M, static_cast<int64_t>(64 * tm)) * cdiv(N, static_cast<int64_t>(256));
  const int64_t nk = K / 64;
  int64_t ks = 1;
  if (M <= 64) ks = std::max<int64_t>(1, std::min<int64_t>({device_cus() / (2 * tiles), 8, nk / 4}));
  const int64_t steps = cdiv(nk, ks);
  return {tm, static_cast<int>(cdiv(nk, steps)), static_cast<int>(steps)};   // no empty ranges
}

// Bytes after the control block: the two bf16 planes (each 256-byte
// aligned), then the fp32 partial tiles of every plane and k-range.
int64_t planes_x_bytes(int64_t M, int64_t K) { return cdiv(M * K * 2, static_cast<int64_t>(256)) * 256; }

int64_t planes_bytes(int64_t M, int64_t N, int64_t K) {
  const PlanesPlan p = planes_plan(M, N, K);
  const int64_t tiles = cdiv(M, static_cast<int64_t>(64 * p.tm)) * cdiv(N, static_cast<int64_t>(256));
  return 2 * planes_x_bytes(M, K) + tiles * 2 * p.ks * (64 * p.tm) * 256 * 4;
}

// Workspace cap of the two-plane path: M is processed in chunks of rows
// (multiples of 256, one after the other on the stream, reusing the
// workspace) whose planes and partial tiles fit kPlanesMaxBytes (at M = 4096,
// N = 11008, K = 4096 one launch would need 428 MB: two chunks of 2560 and
// 1536 rows). A remainder of at most 64 rows joins the chunk before it, so
// that every chunk keeps the plan of M > 64; chunks of 256 rows that alone
// exceed the cap (very wide weights) are taken as they are.
constexpr int64_t kPlanesMaxBytes = int64_t(256) << 20;

int64_t planes_chunk_rows(int64_t M, int64_t N, int64_t K) {
  if (planes_bytes(M, N, K) <= kPlanesMaxBytes) return M;
  int64_t mc = 256;
  while (mc + 256 < M && planes_bytes(mc + 256, N, K) <= kPlanesMaxBytes) mc += 256;
  return mc;
}

// Rows of the chunk starting at m0.
int64_t planes_chunk_at(int64_t m0, int64_t M, int64_t mc) {
  const int64_t left = M - m0;
  return left <= mc + 64 ? left : mc;
}

// Workspace of the two-plane path: the most any of its chunks needs (the
// chunks of w8a16_f32_planes, walked the same way).
int64_t planes_ws_bytes(int64_t M, int64_t N, int64_t K) {
  const int64_t mc = planes_chunk_rows(M, N, K);
  int64_t most = 0;
  for (int64_t m0 = 0; m0 < M;) {
    const int64_t mr = planes_chunk_at(m0, M, mc);
    most = std::max(most, planes_bytes(mr, N, K));
    m0 += mr;
  }
  return most;
}

template <int TM>
void launch_planes(GemmArgs a, const PlanesPlan& p, const float* sc, const float* bias, float* y,
                   hipStream_t s) {
  a.tiles_m = static_cast<int>(cdiv(a.M, 64 * TM));
  a.tiles_n = static_cast<int>(cdiv(a.N, 256));
  a.full_tiles = 0;
  a.splits = 2 * p.ks;
  a.split_steps = p.steps;
  const int tiles = a.tiles_m * a.tiles_n;
  k_gemm_dma<kBF16, true, TM, true><<<dim3(static_cast<unsigned>(a.splits * tiles)),
                                      dim3(kDmaThreads), 0, s>>>(a);
  const int64_t n4 = static_cast<int64_t>(tiles) * 8 * kDmaTN * TM * 4 * 64;
  k_planes_reduce<TM><<<dim3(static_cast<unsigned>(cdiv(n4, kBlock * 2))), dim3(kBlock), 0, s>>>(
      a, sc, bias, y);
}

// The two-plane path when it applies (returns its status), else -1.
int w8a16_f32_planes(const void* x, const int8_t* wq, const void* scales, const void* bias,
                     int64_t n_out, int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes,
                     void* y, hipStream_t s) {
  if (!planes_ok(M, N, K, n_out) || !ws || !aligned(x, 16) || !aligned(wq, 16) ||
      ws_bytes < static_cast<size_t>(CBQ_WS_CTRL_BYTES + planes_ws_bytes(M, N, K)))
    return -1;
  const int64_t mc = planes_chunk_rows(M, N, K);
  for (int64_t m0 = 0; m0 < M;) {
    const int64_t mr = planes_chunk_at(m0, M, mc);
    uint8_t* base = static_cast<uint8_t*>(ws) + CBQ_WS_CTRL_BYTES;
    uint16_t* xh = reinterpret_cast<uint16_t*>(base);
    uint16_t* xl = reinterpret_cast<uint16_t*>(base + planes_x_bytes(mr, K));
    const int64_t n4 = mr * K / 4;   // K % 64 == 0
    k_f32_planes<<<dim3(static_cast<unsigned>(cdiv(n4, static_cast<int64_t>(kBlock)))),
                   dim3(kBlock), 0, s>>>(static_cast<const float*>(x) + m0 * K, n4, xh, xl);
    GemmArgs a{};
    a.x = xh;
    a.x2 = xl;
    a.wq = wq;
    a.part = reinterpret_cast<float*>(base + 2 * planes_x_bytes(mr, K));
    a.M = static_cast<int>(mr);
    a.N = static_cast<int>(N);
    a.K = static_cast<int>(K);
    const float* sc = static_cast<const float*>(scales);
    const float* bs = static_cast<const float*>(bias);
    float* yo = static_cast<float*>(y) + m0 * N;
    const PlanesPlan p = planes_plan(mr, N, K);
    switch (p.tm) {
      case 2: launch_planes<2>(a, p, sc, bs, yo, s); break;
      case 3: launch_planes<3>(a, p, sc, bs, yo, s); break;
      default: launch_planes<4>(a, p, sc, bs, yo, s); break;
    }
    m0 += mr;
  }
  return launch_status("cbq_w8a16_linear");
}

template <int ACT>
int w8a16_general(const void* x, const int8_t* wq, const void* scales, const void* bias,
                  const int64_t* oc, int64_t n_out, const void* w_out, int64_t M, int64_t N,
                  int64_t K, void* ws, size_t ws_bytes, void* y, hipStream_t s) {
  const int bm = general_bm(M), bn = general_bn(M);
  GenArgs a{};
  a.x = x; a.wq = wq; a.scales = scales; a.bias = bias; a.oc = oc; a.w_out = w_out; a.y = y;
  a.n_out = n_out; a.M = M; a.N = N; a.K = K;
  a.tiles_n = cdiv(N, static_cast<int64_t>(bn));
  a.tiles = cdiv(M, static_cast<int64_t>(bm)) * a.tiles_n;
  int sp = general_splits(M, N, K);
  if (sp > 1 && (!ws || ws_bytes < static_cast<size_t>(CBQ_WS_CTRL_BYTES + general_split_bytes(M, N, K))))
    sp = 1;   // no room for the partial sums: one range
  if (sp > 1) {
    a.kper = cdiv(cdiv(K, static_cast<int64_t>(kGenBK)), sp) * kGenBK;
    a.splits = static_cast<int>(cdiv(K, a.kper));   // no empty ranges
    a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + CBQ_WS_CTRL_BYTES);
  } else {
    a.kper = K;
    a.splits = 1;
  }
  const int64_t blocks = a.tiles * a.splits;
  if (blocks > 0x7fffffffLL || cdiv(M * N, static_cast<int64_t>(kBlock)) > 0x7fffffffLL) {
    set_error("cbq_w8a16_linear: output too large for the general path");
    return CBQ_EINVAL;
  }
  const dim3 g(static_cast<unsigned>(blocks)), b(kGenThreads);
  if (a.splits > 1) {
    if (bm == 16) k_w8a16_general<ACT, 16, 256, true><<<g, b, 0, s>>>(a);
    else k_w8a16_general<ACT, 64, 64, true><<<g, b, 0, s>>>(a);
    k_general_reduce<ACT><<<dim3(static_cast<unsigned>(cdiv(M * N, static_cast<int64_t>(kBlock)))),
                            dim3(kBlock), 0, s>>>(a);
  } else if (bm == 16) {
    k_w8a16_general<ACT, 16, 256, false><<<g, b, 0, s>>>(a);
  } else {
    k_w8a16_general<ACT, 64, 64, false><<<g, b, 0, s>>>(a);
  }
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
            void* ws, size_t ws_bytes, void* y, hipStream_t s) {
  if (!mfma_path(M, N, K, x, wq, y))
    return w8a16_general<ACT>(x, wq, scales, bias, oc, n_out, w_out, M, N, K, ws, ws_bytes, y, s);
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
  DmaPlan plan{4, 0, 1};
  const Kind kind = choose(M, N, K, n_out, ws ? ws_bytes : 0, plan);
  if (kind == kTileDmaSplit)
    a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + CBQ_WS_CTRL_BYTES);
  launch_kind<ACT>(kind, a, plan, s);
  return launch_status("cbq_w8a16_linear");
}

}  // namespace
}  // namespace cbq

using namespace cbq;

extern "C" size_t cbq_w8a16_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t n_out,
                                     int act_dtype) {
  if (M <= 0 || N <= 0 || K <= 0) return CBQ_WS_CTRL_BYTES;
  // fp16 / bf16 with K % 16 == 0 run the MFMA kernels (split-K partials of
  // the last wave of tiles); fp32 and K % 16 != 0 run the general kernel
  // (its partial sums). Unaligned fp16 / bf16 operands also take the general
  // kernel; with this size it then runs without a split (same results).
  const bool mfma = (act_dtype == kF16 || act_dtype == kBF16) && K % 16 == 0;
  const int64_t bytes =
      mfma ? splitk_bytes(M, N, split_plan(M, N, K))
      : (act_dtype == kF32 && planes_ok(M, N, K, n_out))
          ? std::max(planes_ws_bytes(M, N, K), general_split_bytes(M, N, K))
          : general_split_bytes(M, N, K);
  return CBQ_WS_CTRL_BYTES + static_cast<size_t>(bytes);
}

extern "C" int cbq_w8a16_linear(const void* x, int act_dtype, const int8_t* wq,
                                const void* scales, const void* bias,
                                const int64_t* outlier_cols, int64_t n_out, const void* w_out,
                                int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes,
                                void* y, cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_w8a16_linear";
  CBQ_REQUIRE(act_dtype == kF16 || act_dtype == kBF16 || act_dtype == kF32,
              "%s: activation dtype must be fp16, bf16 or fp32 (code %d)", what, act_dtype);
  CBQ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && n_out >= 0, "%s: negative size", what);
  CBQ_REQUIRE(n_out <= 0x7fffffffLL, "%s: too many outlier columns", what);
  if (M == 0 || N == 0) return CBQ_OK;
  // K == 0: the empty contraction, y = bias (or 0); x and wq hold no bytes.
  CBQ_REQUIRE(scales && y && (K == 0 || (x && wq)), "%s: null pointer", what);
  CBQ_REQUIRE(n_out == 0 || (outlier_cols && w_out), "%s: outlier columns need indices and weights",
              what);
  // The split-K partials go after the control block; a workspace that is
  // missing, unaligned or too small selects a path without partials.
  if (ws && !aligned(ws, 256)) ws = nullptr;
  if (K == 0) {
    hipStream_t s = as_stream(stream);
    return act_dtype == kF32 ? w8a16_general<kF32>(x, wq, scales, bias, nullptr, 0, nullptr, M, N,
                                                  K, nullptr, 0, y, s)
           : act_dtype == kF16 ? w8a16_general<kF16>(x, wq, scales, bias, nullptr, 0, nullptr, M,
                                                    N, K, nullptr, 0, y, s)
                               : w8a16_general<kBF16>(x, wq, scales, bias, nullptr, 0, nullptr, M,
                                                     N, K, nullptr, 0, y, s);
  }
  if (act_dtype == kF32) {
    const int rc = w8a16_f32_planes(x, wq, scales, bias, n_out, M, N, K, ws, ws_bytes, y,
                                    as_stream(stream));
    if (rc >= 0) return rc;
    return w8a16_general<kF32>(x, wq, scales, bias, outlier_cols, n_out, w_out, M, N, K, ws,
                              ws_bytes, y, as_stream(stream));
  }
  return act_dtype == kF16
             ? w8a16_t<kF16>(x, wq, scales, bias, outlier_cols, n_out, w_out, M, N, K, ws,
                             ws_bytes, y, as_stream(stream))
             : w8a16_t<kBF16>(x, wq, scales, bias, outlier_cols, n_out, w_out, M, N, K, ws,
                              ws_bytes, y, as_stream(stream));
}
