// cbq_gemm.hip - dense GEMM on gfx950 matrix cores: C[M, N] = A[M, K] . B[K, N].
//
// Replaces the reference's WMMA GEMM (kernels/cuda/wmma.cu:29-169, host
// wmma_gemm :186-261, bound as bindings/cuda/wmma.py:15-43) and keeps its
// precision table:
//   int8  x int8  -> int32   v_mfma_i32_32x32x32_i8
//   uint8 x uint8 -> int32   the same on u ^ 0x80 (= u - 128), corrected exactly
//                            in the epilogue (or the split-K reduce):
//        sum_k ua ub = sum_k sa sb + 128 (sum_k sa + sum_k sb) + 16384 K
//   fp16  x fp16  -> fp32    v_mfma_f32_32x32x16_f16
//   fp16  x fp16  -> fp16    fp32 accumulation, one rounding at the end (the
//                            reference accumulates in fp16 fragments)
//   bf16  x bf16  -> fp32    v_mfma_f32_32x32x16_bf16
// Integer results are exact modulo 2^32 (int32 wrap-around, as the int32
// accumulators of the reference).
//
// k_mm_dma<IN, OUT, SPLIT, T>: T x T output tiles; T = 256: 8 waves (two per SIMD) of
// 128 (m) x 64 (n) (4 x 2 tiles of 32 x 32), k-steps of 64 bytes per row (64
// int8 or 32 fp16 k), four LDS stages of 32 KiB filled by LDS DMA
// (global_load_lds_dwordx4), three k-steps in flight, one barrier per k-step
// placed between its two MFMA substeps so that the next k-step's fragment
// reads overlap the second substep's MFMAs. Measured on MI355X at 8192^3
// (random data): two waves per SIMD raise rocprof's MfmaUtil from ~47% to
// 58% (int8) / 65% (fp16); the int8 kernel then runs level with hipBLASLt.
// T = 128 (4 waves of 64 x 64, two workgroups per CU) serves shapes whose
// 256 x 256 tiles would leave CUs idle, and the host may also split K into
// ranges (mm_choose picks both from a time model): k_mm_dma<IN, OUT, true, T>
// writes each range's raw int32 / fp32 sums to the workspace and k_mm_reduce
// adds the ranges in order (int32 wrap-around: bit-exact; fp32:
// deterministic).
// A is read as K-contiguous rows [M, K]. A B that is stored [N, K] (B = W^T,
// the usual weight layout) is read in place as B^T rows; a contiguous
// [K, N] B whose K fills whole 64-byte k-steps is read in place too, as
// k-rows, its fragments assembled by gfx950's transposing LDS reads
// (k_mm_dma<.., BKN>). Otherwise a [K, N] B is transposed into the workspace
// first (k_stage_bt); uint8 operands and row lengths that are not a multiple
// of 64 bytes are staged too (k_stage_rows: offset to int8, zero padding).
//
// LDS layout of a stage: A rows (64 B each) then B^T rows; 16-byte chunk c of
// row r sits at chunk c ^ ((r >> 2) & 3), so that the fragment reads of 16
// consecutive rows hit distinct banks. In a k-step, MFMA s (0, 1) of lane
// half h (lane / 32) takes chunk 2 h + s of its A row and of its B^T row: A
// and B see the same k order, which is all the contraction needs.
//
// The MFMA A operand is the A fragment (D rows = m) and B the B^T fragment
// (D columns = n): lane l holds C[m][n] for n = l % 32 and m = 8 (v / 4) +
// 4 (l / 32) + v % 4, so each store instruction writes two 128-byte runs of a
// row (int32 / fp32).
#include <algorithm>
#include <type_traits>

#include "cbq_device.h"
#include "cbq_host.h"
#include "cbq_lds_dma.h"

namespace cbq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16x __attribute__((ext_vector_type(16)));
typedef int v2i32_t __attribute__((ext_vector_type(2)));
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef short v8i16_t __attribute__((ext_vector_type(8)));

// Input kinds of the kernels (the C ABI's dtype codes map onto these).
enum : int { kInI8 = 0, kInF16 = 1, kInBF16 = 2 };
// Output kinds.
enum : int { kOutI32 = 0, kOutF32 = 1, kOutF16 = 2 };

template <int IN> struct AccOf { typedef f16x type; };
template <> struct AccOf<kInI8> { typedef i16x type; };

template <int IN>
__device__ __forceinline__ typename AccOf<IN>::type mfma32(const u32x4& a, const u32x4& b,
                                                           typename AccOf<IN>::type c) {
  if constexpr (IN == kInI8)
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i4v, a),
                                                 __builtin_bit_cast(i4v, b), c, 0, 0, 0);
  else if constexpr (IN == kInF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, a),
                                                  __builtin_bit_cast(h8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8, a),
                                                   __builtin_bit_cast(b8, b), c, 0, 0, 0);
}

struct MmArgs {
  const uint8_t* a;      // [M, ldk] bytes, K-contiguous rows
  const uint8_t* bt;     // [N, ldk] bytes (B^T); k_mm_dma<.., BKN>: B itself, [K, ldb] bytes
  int ldb;               // k_mm_dma<.., BKN>: B's row pitch in bytes (N x element bytes)
  void* c;               // [M, N] row-major, OUT elements
  const int* row_sum;    // uint8 correction: sum_k of each signed A row [M]
  const int* col_sum;    // and of each signed B^T row [N] (null: none)
  int M, N;
  int ldk;               // row pitch of a and bt in bytes (multiple of 64)
  int nk;                // 64-byte k-steps
  int K;                 // true K (the uint8 correction's 16384 K term)
  int tiles_m, tiles_n;
  // split-K: `splits` k-ranges of `split_steps` 64-byte steps; range s writes
  // its raw sums (int32 or fp32) to part[s][M][N] and k_mm_reduce adds them
  void* part;
  int splits, split_steps;
};

// Workgroup -> (tile m, tile n) of the tiles_m x tiles_n grid: XCD b % 8
// gets a contiguous run of logical tiles, which run in groups of 8 m-tiles so
// that the workgroups resident on one XCD share A and B^T k-slices in its L2.
__device__ __forceinline__ void mm_tile(int b, const MmArgs& a, int& tm, int& tn) {
  const int total = a.tiles_m * a.tiles_n;
  const int per = total >> 3;
  if (b < per * 8) b = (b & 7) * per + (b >> 3);
  constexpr int G = 8;
  const int group = b / (G * a.tiles_n);
  const int first_m = group * G;
  const int gsize = min(a.tiles_m - first_m, G);
  const int r = b % (G * a.tiles_n);
  tm = first_m + r % gsize;
  tn = r / gsize;
}

constexpr int kMmNS = 4;                 // LDS stages

// Geometry of a T x T output tile (T = 256: 8 waves of 128 x 64, two per
// SIMD, one workgroup per CU; T = 128: 4 waves of 64 x 64, two workgroups
// per CU). Each wave computes J x 2 tiles of 32 x 32.
template <int T> struct MmGeom {
  static constexpr int kThreads = T == 256 ? 512 : 256;
  static constexpr int kWaves = kThreads / 64;
  static constexpr int kHalf = T * 64;                     // bytes of one operand per stage
  static constexpr int kSB = 2 * kHalf;                    // stage bytes
  static constexpr int kL = kHalf / (kThreads * 16);       // DMA instructions per operand per thread
  static constexpr int kWM = T / 2;                        // rows of a wave tile
  static constexpr int kJ = kWM / 32;                      // 32-row tiles per wave
  static_assert(kL == 2 && T / (kWaves / 2) == 64, "two DMA rows per thread, 64-column wave tiles");
};

// XOR swizzle (in 16-byte chunks) of k-row r of a [K, N]-layout B tile in
// LDS: the 16 (row, chunk) pairs that a transposing fragment read touches
// per 32 lanes (8 rows x 2 chunks for int8, 4 rows x 4 chunks for 16-bit
// elements) fall in distinct 16-byte bank groups.
template <int IN, int T>
__device__ __forceinline__ int kn_swizzle(int r) {
  if constexpr (IN != kInI8) return 4 * (r & 3);
  else if constexpr (T == 256) return 2 * (r & 7);
  else return 2 * ((r >> 1) & 3);
}

// BKN: B is read in place as [K, N] (row pitch a.ldb), without the
// transposing staging pass: its k-step tile is held in LDS as k-rows of T
// columns (swizzled, see kn_swizzle), and each B^T fragment (16 consecutive
// bytes of k for one column) is assembled by two transposing reads,
// ds_read_b64_tr_b8 / ds_read_b64_tr_b16. Measured on MI355X: lane i of a
// 16-lane group receives element i % EV of the 8-byte vectors that lanes
// i / EV + (16 / EV) j address (EV = 8 / element bytes, j = 0 .. EV - 1), so
// lanes that address k-rows k0 + sl / (16 / EV) at columns c + EV (sl %
// (16 / EV)) give lane i column c + i, k-rows k0 .. k0 + EV - 1 in order.
// Needs K to fill whole 64-byte k-steps (no padding).
template <int IN, int OUT, bool SPLIT, int T, bool BKN = false>
__global__ __launch_bounds__(MmGeom<T>::kThreads) void k_mm_dma(MmArgs a) {
  typedef typename AccOf<IN>::type Acc;
  typedef MmGeom<T> G;
  constexpr int kMmHalf = G::kHalf, kMmSB = G::kSB, kMmL = G::kL, J = G::kJ;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kMmNS * kMmSB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;   // T/2-row half of m, 64-column slice of n
  int tm, tn, split = 0;
  if constexpr (SPLIT) {
    const int tiles = a.tiles_m * a.tiles_n;
    split = blockIdx.x / tiles;
    mm_tile(blockIdx.x % tiles, a, tm, tn);
  } else {
    mm_tile(blockIdx.x, a, tm, tn);
  }
  const int m0 = tm * T, n0 = tn * T;
  const int kb = SPLIT ? split * a.split_steps : 0;   // first 64-byte k-step of this range
  const int nk = SPLIT ? min(a.split_steps, a.nk - kb) : a.nk;
  const uint32_t sbase = __builtin_amdgcn_readfirstlane(lds_addr(smem));

  // DMA sources: instruction u of an operand fills rows (u * waves + wave) *
  // 16 + lane / 4, chunk slot lane % 4, which holds source chunk slot ^ swizzle.
  // Rows past M or N are clamped to the last row; their products land in
  // outputs that are never stored.
  constexpr int ES = IN == kInI8 ? 1 : 2;     // element bytes
  constexpr int KCPR = T * ES / 16;            // BKN: 16-byte chunks per k-row of the B tile
  constexpr int KRPI = 64 / KCPR;              // BKN: k-rows per wave DMA instruction
  uint32_t ao[kMmL], bo[kMmL];
#pragma unroll
  for (int u = 0; u < kMmL; ++u) {
    const int row = (u * G::kWaves + wave) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 2) & 3);
    ao[u] = static_cast<uint32_t>(min(m0 + row, a.M - 1)) * static_cast<uint32_t>(a.ldk) + c * 16u;
    if constexpr (BKN) {
      // k-row kr of the tile, slot lane % KCPR holding chunk slot ^ swizzle;
      // columns past N are clamped to the row's last chunk
      const int kr = (u * G::kWaves + wave) * KRPI + lane / KCPR;
      const int kc = (lane % KCPR) ^ kn_swizzle<IN, T>(kr);
      const int col = min(n0 * ES + kc * 16, a.N * ES - 16);
      bo[u] = static_cast<uint32_t>(kr) * static_cast<uint32_t>(a.ldb) + static_cast<uint32_t>(col);
    } else {
      bo[u] = static_cast<uint32_t>(min(n0 + row, a.N - 1)) * static_cast<uint32_t>(a.ldk) + c * 16u;
    }
  }
  // DMA instruction u (0 .. 2 kMmL - 1: A rows, then B^T rows) of tile t.
  auto issue_one = [&](int t, int stage, int u) {
    const uint32_t dst = sbase + stage * kMmSB + wave * 1024;
    if (u < kMmL)
      lds_dma16(ao[u], uniform_ptr(a.a + (kb + t) * 64), dst + u * G::kWaves * 1024);
    else
      lds_dma16(bo[u - kMmL],
                uniform_ptr(BKN ? a.bt + static_cast<int64_t>(kb + t) * (64 / ES) * a.ldb
                                : a.bt + (kb + t) * 64),
                dst + kMmHalf + (u - kMmL) * G::kWaves * 1024);
  };
  auto issue = [&](int t, int stage) {
#pragma unroll
    for (int u = 0; u < 2 * kMmL; ++u) issue_one(t, stage, u);
  };

  // Fragment read offsets: row r32 of 32-row tile j (A) / i (B^T), chunk
  // 2 h + s.
  const int r32 = lane & 31, h = lane >> 5;
  uint32_t ar[2], br[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const uint32_t slot = static_cast<uint32_t>((2 * h + s) ^ ((r32 >> 2) & 3)) << 4;
    ar[s] = (wm * G::kWM + r32) * 64 + slot;
    br[s] = kMmHalf + (wn * 64 + r32) * 64 + slot;
  }
  // BKN: LDS offsets of the two transposing reads (p) of B tile i, substep
  // s. Substep s of lane half h takes k-chunk 2 h + s (16 bytes of k). A read
  // gives each lane EV = 8 / ES consecutive k of its column: source lane sl
  // (of 16) addresses k-row k0 + sl / LPR, bytes 8 (sl % LPR) past the
  // group's first column (LPR = 16 / EV lanes per k-row); lanes 16 g .. 16 g
  // + 15 of the half take columns 16 g .. 16 g + 15 of the 32-column tile.
  uint32_t bkr[2][2][2];   // [i][s][p]
  if constexpr (BKN) {
    constexpr int EV = 8 / ES, LPR = 16 / EV;
    const int sl = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int kr = ((2 * h + s) * 16) / ES + p * EV + sl / LPR;
          const int cb = (wn * 64 + i * 32 + 16 * g) * ES + 8 * (sl % LPR);
          const int chunk = (cb >> 4) ^ kn_swizzle<IN, T>(kr);
          bkr[i][s][p] = kMmHalf + kr * (T * ES) + chunk * 16 + (cb & 15);
        }
  }

  const int mw = m0 + wm * G::kWM, nw = n0 + wn * 64;
  Acc acc[J][2];   // [j: m-tile][i: n-tile]
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int i = 0; i < 2; ++i) acc[j][i] = Acc{};

  // Fragments of one k-substep: J A tiles, 2 B^T tiles (J + 2 reads, 2 J
  // MFMAs).
  struct Frags {
    u32x4 x[J];
    u32x4 w[2];
  };
  auto read_one = [&](int stage, int s, Frags& f, int r) {
    const uint8_t* st = smem + stage * kMmSB;
    if (r < J) {
      f.x[r] = *reinterpret_cast<const u32x4*>(st + ar[s] + r * 2048);
    } else if constexpr (BKN) {
      const int i = r - J;
      typedef __attribute__((address_space(3))) v2i32_t* lp2;
      if constexpr (ES == 1) {
        const v2i32_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lp2)(st + bkr[i][s][0]));
        const v2i32_t hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lp2)(st + bkr[i][s][1]));
        f.w[i] = u32x4{static_cast<uint32_t>(lo.x), static_cast<uint32_t>(lo.y),
                       static_cast<uint32_t>(hi.x), static_cast<uint32_t>(hi.y)};
      } else {
        typedef __attribute__((address_space(3))) v4i16_t* lp4;
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp4)(st + bkr[i][s][0]));
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp4)(st + bkr[i][s][1]));
        f.w[i] = __builtin_bit_cast(u32x4, v8i16_t{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
      }
    } else {
      f.w[r - J] = *reinterpret_cast<const u32x4*>(st + br[s] + (r - J) * 2048);
    }
  };
  auto read = [&](int stage, int s, Frags& f) {
#pragma unroll
    for (int r = 0; r < J + 2; ++r) read_one(stage, s, f, r);
  };
  // MFMA q (0 .. 2 J - 1) of a substep: tile (j, i) = (q / 2, q % 2); an
  // accumulator is reused every (2 J)th MFMA.
  auto mma_one = [&](const Frags& f, int q) {
    acc[q >> 1][q & 1] = mfma32<IN>(f.x[q >> 1], f.w[q & 1], acc[q >> 1][q & 1]);
  };

  // Step t: F0 holds the fragments of tile t's substep 0. The substep-0
  // MFMAs run with tile t's substep-1 reads into F1 between them (tile t
  // landed before the previous step's barrier); then the wait for tile t + 1
  // and the barrier (which also means every wave is past its reads of tile
  // t - 1, whose stage tile t + 3 takes); then the substep-1 MFMAs, each
  // followed by one DMA instruction of tile t + 3 and one substep-0 read of
  // tile t + 1 into F0. Spreading the DMA and the reads over the MFMAs
  // (rather than issuing them in bursts) took 1-4% off 8192^3 on MI355X.
  // The other wave of the SIMD fills the MFMA pipe while a wave waits.
  Frags f0, f1;
  // One step (see above). DMA: issue tile t + 3; ALL: tile t + 1 is the last
  // tile in flight (wait for everything).
  auto step = [&](int t, auto dma, auto all) {
#pragma unroll
    for (int q = 0; q < 2 * J; ++q) {
      mma_one(f0, q);
      if (q < J + 2) read_one(t % kMmNS, 1, f1, q);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (decltype(all)::value) dma_wait_barrier<0>();
    else dma_wait_barrier<2 * kMmL>();
    __builtin_amdgcn_sched_barrier(0);
    const int next = (t + 1) % kMmNS;
#pragma unroll
    for (int q = 0; q < 2 * J; ++q) {
      mma_one(f1, q);
      if constexpr (decltype(dma)::value) {
        if (q < 2 * kMmL) issue_one(t + kMmNS - 1, (t + kMmNS - 1) % kMmNS, q);
      }
      if (q < J + 2) read_one(next, 0, f0, q);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using yes = std::true_type;
  using no = std::false_type;
#pragma unroll
  for (int t = 0; t < kMmNS - 1; ++t)
    if (t < nk) issue(t, t);
  if (nk > 0) {
    if (nk > 2) dma_wait_barrier<2 * 2 * kMmL>();
    else if (nk > 1) dma_wait_barrier<2 * kMmL>();
    else dma_wait_barrier<0>();
    read(0, 0, f0);
    int t = 0;
    for (; t + kMmNS - 1 < nk; ++t) step(t, yes{}, no{});    // tiles t + 1, t + 2 in flight
    if (t + 2 < nk) step(t++, no{}, no{});                  // tile t + 2 still in flight
    if (t + 1 < nk) step(t++, no{}, yes{});
#pragma unroll
    for (int q = 0; q < 2 * J; ++q) {
      mma_one(f0, q);
      if (q < J + 2) read_one((nk - 1) % kMmNS, 1, f1, q);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = 0; q < 2 * J; ++q) mma_one(f1, q);
  }

  // Epilogue: C[m][n], n = 32 i + r32, m = 32 j + 8 (v / 4) + 4 h + v % 4;
  // 32-bit offsets from the wave's corner (T/2 rows of N elements). A split
  // range stores its raw 4-byte sums to its plane of the partial buffer.
  typedef typename std::conditional<IN == kInI8, int, float>::type PartT;
  constexpr int ES_OUT = (OUT == kOutF16 && !SPLIT) ? 2 : 4;
  // uint8 inputs (col_sum set): the correction 128 (row_sum[m] + col_sum[n])
  // + 16384 K of the offset operands' product, added before the store (int32
  // wrap-around). M and N are multiples of 16, so each lane's four row sums
  // of a group (rows m .. m + 3, m % 4 == 0) are one 16-byte load.
  constexpr bool kFix = (OUT == kOutI32) && !SPLIT;
  const bool u8fix = kFix && a.col_sum != nullptr;
  uint32_t ccol[2] = {0u, 0u};
  if (u8fix) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      ccol[i] = 128u * static_cast<uint32_t>(a.col_sum[min(nw + 32 * i + r32, a.N - 1)]) +
                16384u * static_cast<uint32_t>(a.K);
  }
  uint8_t* cw = SPLIT ? static_cast<uint8_t*>(a.part) +
                            ((static_cast<int64_t>(split) * a.M + mw) * a.N + nw) * ES_OUT
                      : static_cast<uint8_t*>(a.c) + (static_cast<int64_t>(mw) * a.N + nw) * ES_OUT;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    uint32_t crow[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) crow[v] = 0u;
    if (u8fix) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int mb = mw + 32 * j + 8 * g + 4 * h;
        if (mb < a.M) {
          const int4 r = *reinterpret_cast<const int4*>(a.row_sum + mb);
          crow[4 * g] = 128u * static_cast<uint32_t>(r.x);
          crow[4 * g + 1] = 128u * static_cast<uint32_t>(r.y);
          crow[4 * g + 2] = 128u * static_cast<uint32_t>(r.z);
          crow[4 * g + 3] = 128u * static_cast<uint32_t>(r.w);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int nl = 32 * i + r32;
      if (nw + nl < a.N) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ml = 32 * j + 8 * (v >> 2) + 4 * h + (v & 3);
          if (mw + ml < a.M) {
            const uint32_t off = (static_cast<uint32_t>(ml) * static_cast<uint32_t>(a.N) + nl) * ES_OUT;
            if constexpr (SPLIT)
              *reinterpret_cast<PartT*>(cw + off) = acc[j][i][v];
            else if constexpr (OUT == kOutI32)
              *reinterpret_cast<uint32_t*>(cw + off) =
                  static_cast<uint32_t>(acc[j][i][v]) + (u8fix ? crow[v] + ccol[i] : 0u);
            else if constexpr (OUT == kOutF32)
              *reinterpret_cast<float*>(cw + off) = acc[j][i][v];
            else
              *reinterpret_cast<_Float16*>(cw + off) = static_cast<_Float16>(acc[j][i][v]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Split-K finish: C = the sum of the ranges' partial planes, in range order
// (int32 wrap-around for integer inputs, plus the uint8 correction when
// col_sum is set; fp32 for float inputs, then one rounding for fp16 outputs).
// One thread per output.
template <int IN, int OUT>
__global__ __launch_bounds__(kBlock) void k_mm_reduce(MmArgs a) {
  const int64_t mn = static_cast<int64_t>(a.M) * a.N;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= mn) return;
  if constexpr (IN == kInI8) {
    const uint32_t* p = static_cast<const uint32_t*>(a.part) + idx;
    uint32_t sum = p[0];
    for (int s = 1; s < a.splits; ++s) sum += p[s * mn];
    if (a.col_sum) {
      const int64_t m = idx / a.N, n = idx - m * a.N;
      sum += 128u * (static_cast<uint32_t>(a.row_sum[m]) + static_cast<uint32_t>(a.col_sum[n])) +
             16384u * static_cast<uint32_t>(a.K);
    }
    static_cast<uint32_t*>(a.c)[idx] = sum;
  } else {
    const float* p = static_cast<const float*>(a.part) + idx;
    float sum = p[0];
    for (int s = 1; s < a.splits; ++s) sum += p[s * mn];
    if constexpr (OUT == kOutF16) static_cast<_Float16*>(a.c)[idx] = static_cast<_Float16>(sum);
    else static_cast<float*>(a.c)[idx] = sum;
  }
}

// ---------------------------------------------------------------------------
// Staging into the workspace
// ---------------------------------------------------------------------------

// Rows of kb bytes (multiple of 16) -> rows of ldk bytes (multiple of 64),
// zero-padded; XOR flips the sign bit of every byte (uint8 -> int8 offset).
// Grid-stride over 16-byte chunks of the destination.
template <bool XOR>
__global__ __launch_bounds__(kBlock) void k_stage_rows(const uint8_t* __restrict__ src,
                                                       int64_t rows, int64_t kb, int64_t ldk,
                                                       uint8_t* __restrict__ dst) {
  const int64_t cpr = ldk >> 4;
  const int64_t total = rows * cpr;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; c < total;
       c += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = c / cpr, k = (c % cpr) * 16;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (k < kb) {
      v = *reinterpret_cast<const u32x4*>(src + r * kb + k);
      if constexpr (XOR) v ^= 0x80808080u;
    }
    *reinterpret_cast<u32x4*>(dst + r * ldk + k) = v;
  }
}

// B [K, N] (ES-byte elements, row-major) -> B^T [N, ldk bytes], zero-padded
// past K; XOR as above (ES == 1 only). A workgroup transposes a 64 (k) x 64 (n)
// element tile through LDS: 16-byte loads along n, element reads down k,
// 16-byte stores along k.
template <int ES, bool XOR>
__global__ __launch_bounds__(kBlock) void k_stage_bt(const uint8_t* __restrict__ b, int64_t K,
                                                     int64_t N, int64_t ldk,
                                                     uint8_t* __restrict__ dst) {
  constexpr int T = 64;                        // elements per tile side
  constexpr int RB = T * ES;                   // bytes per tile row
  constexpr int PITCH = RB + 4;                // LDS row pitch
  constexpr int CPR = RB / 16;                 // 16-byte chunks per tile row
  __shared__ uint8_t tile[T * PITCH];
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * T;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * T;
  // Load: T rows (k) x CPR chunks.
  for (int c = threadIdx.x; c < T * CPR; c += kBlock) {
    const int kr = c / CPR, ch = c % CPR;
    const int64_t k = k0 + kr, n = n0 + (ch * 16) / ES;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (k < K && n < N) v = *reinterpret_cast<const u32x4*>(b + (k * N + n) * ES);
    uint32_t* d = reinterpret_cast<uint32_t*>(tile + kr * PITCH + ch * 16);
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
  }
  __syncthreads();
  // Store: T rows (n) x CPR chunks of k.
  for (int c = threadIdx.x; c < T * CPR; c += kBlock) {
    const int nr = c / CPR, ch = c % CPR;
    const int64_t n = n0 + nr;
    const int kc = (ch * 16) / ES;             // first k of the chunk in the tile
    if (n >= N) continue;
    const int64_t kbyte = (k0 + kc) * ES;
    if (kbyte >= ldk) continue;
    uint8_t bytes[16];
#pragma unroll
    for (int e = 0; e < 16 / ES; ++e) {
#pragma unroll
      for (int x = 0; x < ES; ++x) {
        const bool in = k0 + kc + e < K;
        bytes[e * ES + x] = in ? tile[(kc + e) * PITCH + nr * ES + x] : 0;
      }
    }
    u32x4 v;
    v.x = bytes[0] | (bytes[1] << 8) | (bytes[2] << 16) | (static_cast<uint32_t>(bytes[3]) << 24);
    v.y = bytes[4] | (bytes[5] << 8) | (bytes[6] << 16) | (static_cast<uint32_t>(bytes[7]) << 24);
    v.z = bytes[8] | (bytes[9] << 8) | (bytes[10] << 16) | (static_cast<uint32_t>(bytes[11]) << 24);
    v.w = bytes[12] | (bytes[13] << 8) | (bytes[14] << 16) | (static_cast<uint32_t>(bytes[15]) << 24);
    if constexpr (XOR) {
      // Flip the sign bit of the bytes that hold data (k < K); padding stays 0.
      uint32_t m[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k0 + kc + e < K) m[e >> 2] |= 0x80u << (8 * (e & 3));
      v.x ^= m[0]; v.y ^= m[1]; v.z ^= m[2]; v.w ^= m[3];
    }
    *reinterpret_cast<u32x4*>(dst + n * ldk + kbyte) = v;
  }
}

// Sum of the signed bytes of each row of a staged [rows, ldk] int8 buffer
// (padding is 0): one workgroup per row (grid-stride), dot4 with 1s.
__global__ __launch_bounds__(kBlock) void k_row_sums(const uint8_t* __restrict__ src,
                                                     int64_t rows, int64_t ldk,
                                                     int* __restrict__ sums) {
  __shared__ int red[kBlock / kWave];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    int s = 0;
    for (int64_t k = threadIdx.x * 16; k < ldk; k += kBlock * 16) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(src + r * ldk + k);
      s = __builtin_amdgcn_sdot4(static_cast<int>(v.x), 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(v.y), 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(v.z), 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(v.w), 0x01010101, s, false);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) sums[r] = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Host
// ---------------------------------------------------------------------------
struct MmPlan {
  int in, es;          // kernel input kind, element bytes
  bool u8;
  int64_t kb, ldk;     // row bytes, padded row bytes
  bool stage_a, stage_b;
  bool kn_direct;      // [K, N] B read in place by k_mm_dma<.., BKN>
  int tile;            // output tile edge (256 or 128)
  int splits;          // k-ranges (1: no split-K)
  size_t a_off, b_off, rs_off, cs_off, part_off, bytes;
};

// Tile and k-ranges for C = A . B: the pair with the lowest modelled time
// (0.01 us units, fitted on MI355X at 512^3 .. 8192^3 and M = 16 .. 2048 x
// N = 4096 / 11008, int8 and fp16). Per 64-byte k-step of the longest range
// and per round of workgroups over the CUs: 1.0 us for a 256 x 256 tile,
// 0.4 us for a 128 x 128 tile (its workgroups are a quarter of the work but
// less efficient: 1024^3 int8 12.4 us against 21.2, 2048^3 fp16 32.5 against
// 59.4; 8192^3 stays on 256 tiles). A split of K into 2-16 ranges adds
// 0.09 us per 256 KiB of 4-byte partial sums written and re-read and 5 us
// for the reduce pass; ranges keep at least four k-steps, and the split
// workgroups must fit one round (256 tiles) or two (128 tiles, two per CU).
void mm_choose(int64_t M, int64_t N, int64_t nk, int& tile, int& splits) {
  const int64_t cus = device_cus();
  tile = 256;
  splits = 1;
  int64_t best = -1;
  for (int t : {256, 128}) {
    const int64_t tiles = cdiv(M, t) * cdiv(N, t);
    const int64_t step = t == 256 ? 100 : 40;
    const int64_t max_wg = t == 256 ? cus : 2 * cus;
    for (int64_t sp = 1; sp <= 16; ++sp) {
      if (sp > 1 && (tiles * sp > max_wg || nk / sp < 4)) break;
      int64_t cost = step * cdiv(nk, sp) * cdiv(tiles * sp, cus);
      if (sp > 1) cost += 9 * cdiv(sp * M * N * 4, 262144) + 500;
      if (best < 0 || cost < best) {
        best = cost;
        tile = t;
        splits = static_cast<int>(sp);
      }
    }
  }
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

bool mm_plan(int64_t M, int64_t N, int64_t K, int in_dtype, int b_layout, MmPlan& p) {
  switch (in_dtype) {
    case CBQ_I8: p.in = kInI8; p.es = 1; p.u8 = false; break;
    case CBQ_U8: p.in = kInI8; p.es = 1; p.u8 = true; break;
    case CBQ_F16: p.in = kInF16; p.es = 2; p.u8 = false; break;
    case CBQ_BF16: p.in = kInBF16; p.es = 2; p.u8 = false; break;
    default: return false;
  }
  p.kb = K * p.es;
  p.ldk = cdiv(p.kb, 64) * 64;
  const bool padded = p.ldk != p.kb;
  p.stage_a = p.u8 || padded;
  p.kn_direct = b_layout == CBQ_MM_B_KN && !p.u8 && !padded;
  p.stage_b = p.u8 || padded || (b_layout == CBQ_MM_B_KN && !p.kn_direct);
  size_t off = CBQ_WS_CTRL_BYTES;
  p.a_off = off;
  if (p.stage_a) off = align256(off + static_cast<size_t>(M) * p.ldk);
  p.b_off = off;
  if (p.stage_b) off = align256(off + static_cast<size_t>(N) * p.ldk);
  p.rs_off = off;
  if (p.u8) off = align256(off + static_cast<size_t>(M) * 4);
  p.cs_off = off;
  if (p.u8) off = align256(off + static_cast<size_t>(N) * 4);
  p.tile = 256;
  p.splits = 1;
  if (M > 0 && N > 0 && K > 0) mm_choose(M, N, p.ldk / 64, p.tile, p.splits);
  p.part_off = off;
  if (p.splits > 1) off = align256(off + static_cast<size_t>(p.splits) * M * N * 4);
  p.bytes = off;
  return true;
}

template <int IN, int OUT, int T, bool BKN>
void launch_mm_t(const MmArgs& a, hipStream_t s) {
  const unsigned tiles = static_cast<unsigned>(a.tiles_m * a.tiles_n);
  const dim3 b(MmGeom<T>::kThreads);
  if (a.splits > 1) {
    k_mm_dma<IN, OUT, true, T, BKN><<<dim3(tiles * a.splits), b, 0, s>>>(a);
    const int64_t mn = static_cast<int64_t>(a.M) * a.N;
    k_mm_reduce<IN, OUT><<<dim3(static_cast<unsigned>(cdiv(mn, kBlock))), dim3(kBlock), 0, s>>>(a);
  } else {
    k_mm_dma<IN, OUT, false, T, BKN><<<dim3(tiles), b, 0, s>>>(a);
  }
}

// a.tiles_m / a.tiles_n must be counted in tiles of `tile`; kn: a.bt is B
// as [K, N] (row pitch a.ldb), else B^T as [N, ldk].
template <int IN, int OUT>
void launch_mm(const MmArgs& a, int tile, bool kn, hipStream_t s) {
  if (kn) {
    if (tile == 128) launch_mm_t<IN, OUT, 128, true>(a, s);
    else launch_mm_t<IN, OUT, 256, true>(a, s);
  } else {
    if (tile == 128) launch_mm_t<IN, OUT, 128, false>(a, s);
    else launch_mm_t<IN, OUT, 256, false>(a, s);
  }
}

unsigned grid_for(int64_t work, int64_t per_block) {
  int64_t g = cdiv(work, per_block);
  const int64_t cap = static_cast<int64_t>(device_cus()) * 16;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace cbq

using namespace cbq;

extern "C" size_t cbq_mm_ws_bytes(int64_t M, int64_t N, int64_t K, int in_dtype, int b_layout) {
  MmPlan p;
  if (M <= 0 || N <= 0 || K < 0 || !mm_plan(M, N, K, in_dtype, b_layout, p))
    return CBQ_WS_CTRL_BYTES;
  return p.bytes;
}

extern "C" int cbq_mm(const void* A, const void* B, int in_dtype, int b_layout, int64_t M,
                      int64_t N, int64_t K, void* C, int out_dtype, void* ws, size_t ws_bytes,
                      cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_mm";
  MmPlan p;
  CBQ_REQUIRE(mm_plan(1, 1, 1, in_dtype, b_layout, p),
              "%s: unsupported dtype code %d; expected int8, uint8, float16 or bfloat16", what,
              in_dtype);
  const bool int_in = in_dtype == CBQ_I8 || in_dtype == CBQ_U8;
  if (int_in) {
    CBQ_REQUIRE(out_dtype == CBQ_I32, "%s: int8 / uint8 inputs only support an int32 accumulator",
                what);
  } else if (in_dtype == CBQ_BF16) {
    CBQ_REQUIRE(out_dtype == CBQ_F32, "%s: bfloat16 inputs only support a float32 accumulator",
                what);
  } else {
    CBQ_REQUIRE(out_dtype == CBQ_F32 || out_dtype == CBQ_F16,
                "%s: float16 inputs support a float32 or float16 accumulator", what);
  }
  CBQ_REQUIRE(b_layout == CBQ_MM_B_KN || b_layout == CBQ_MM_B_NK, "%s: bad b_layout %d", what,
              b_layout);
  CBQ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", what);
  CBQ_REQUIRE(M % 16 == 0 && N % 16 == 0 && K % 16 == 0,
              "%s: dimensions must be multiples of 16 (M=%lld N=%lld K=%lld)", what, (long long)M,
              (long long)N, (long long)K);
  if (M == 0 || N == 0) return CBQ_OK;
  // K == 0 is the empty contraction (C = 0): A and B hold no bytes and may be null.
  CBQ_REQUIRE(C && (K == 0 || (A && B)), "%s: null pointer", what);
  CBQ_REQUIRE(aligned(A, 16) && aligned(B, 16) && aligned(C, 16),
              "%s: A, B and C must be 16-byte aligned", what);
  mm_plan(M, N, K, in_dtype, b_layout, p);
  CBQ_REQUIRE(static_cast<uint64_t>(M) * p.ldk < (1ULL << 32) &&
                  static_cast<uint64_t>(N) * p.ldk < (1ULL << 32),
              "%s: M * K and N * K must stay below 4 GiB of operand bytes", what);
  CBQ_REQUIRE(cdiv(M, 256) * cdiv(N, 256) < (1LL << 31), "%s: too many tiles", what);
  CBQ_REQUIRE(b_layout == CBQ_MM_B_NK || cdiv(p.ldk / p.es, 64) <= 65535,
              "%s: K too large for a [K, N] B (store B as [N, K])", what);
  CBQ_REQUIRE(ws && aligned(ws, 256) && ws_bytes >= p.bytes,
              "%s: workspace must be >= %zu bytes, 256-byte aligned", what, p.bytes);
  hipStream_t s = as_stream(stream);
  uint8_t* w = static_cast<uint8_t*>(ws);
  MmArgs a;
  a.a = static_cast<const uint8_t*>(A);
  a.bt = static_cast<const uint8_t*>(B);
  a.c = C;
  a.row_sum = nullptr;
  a.col_sum = nullptr;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.ldk = static_cast<int>(p.ldk);
  a.ldb = static_cast<int>(N * p.es);
  a.nk = static_cast<int>(p.ldk / 64);
  a.K = static_cast<int>(K);
  a.tiles_m = static_cast<int>(cdiv(M, p.tile));
  a.tiles_n = static_cast<int>(cdiv(N, p.tile));
  a.part = nullptr;
  a.splits = 1;
  a.split_steps = a.nk;
  if (p.splits > 1) {
    a.split_steps = static_cast<int>(cdiv(a.nk, p.splits));
    a.splits = static_cast<int>(cdiv(a.nk, a.split_steps));   // no empty ranges
    a.part = w + p.part_off;
  }
  if (p.stage_a && K > 0) {
    uint8_t* da = w + p.a_off;
    const unsigned g = grid_for(M * (p.ldk / 16), kBlock);
    if (p.u8) k_stage_rows<true><<<g, kBlock, 0, s>>>(a.a, M, p.kb, p.ldk, da);
    else k_stage_rows<false><<<g, kBlock, 0, s>>>(a.a, M, p.kb, p.ldk, da);
    a.a = da;
  }
  if (p.stage_b && K > 0) {
    uint8_t* db = w + p.b_off;
    if (b_layout == CBQ_MM_B_KN) {
      const dim3 g(static_cast<unsigned>(cdiv(N, 64)), static_cast<unsigned>(cdiv(p.ldk / p.es, 64)));
      if (p.es == 2) k_stage_bt<2, false><<<g, kBlock, 0, s>>>(a.bt, K, N, p.ldk, db);
      else if (p.u8) k_stage_bt<1, true><<<g, kBlock, 0, s>>>(a.bt, K, N, p.ldk, db);
      else k_stage_bt<1, false><<<g, kBlock, 0, s>>>(a.bt, K, N, p.ldk, db);
    } else {
      const unsigned g = grid_for(N * (p.ldk / 16), kBlock);
      if (p.u8) k_stage_rows<true><<<g, kBlock, 0, s>>>(a.bt, N, p.kb, p.ldk, db);
      else k_stage_rows<false><<<g, kBlock, 0, s>>>(a.bt, N, p.kb, p.ldk, db);
    }
    a.bt = db;
  }
  if (p.u8 && K > 0) {   // K == 0: the empty contraction, C = 0, needs no correction
    int* rs = reinterpret_cast<int*>(w + p.rs_off);
    int* cs = reinterpret_cast<int*>(w + p.cs_off);
    k_row_sums<<<grid_for(M, 1), kBlock, 0, s>>>(a.a, M, p.ldk, rs);
    k_row_sums<<<grid_for(N, 1), kBlock, 0, s>>>(a.bt, N, p.ldk, cs);
    a.row_sum = rs;
    a.col_sum = cs;
  }
  const bool kn = p.kn_direct && K > 0;
  if (p.in == kInI8) launch_mm<kInI8, kOutI32>(a, p.tile, kn, s);
  else if (p.in == kInF16 && out_dtype == CBQ_F16) launch_mm<kInF16, kOutF16>(a, p.tile, kn, s);
  else if (p.in == kInF16) launch_mm<kInF16, kOutF32>(a, p.tile, kn, s);
  else launch_mm<kInBF16, kOutF32>(a, p.tile, kn, s);
  return launch_status(what);
}
