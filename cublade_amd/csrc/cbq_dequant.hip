// cbq_dequant.hip - FP8 E4M3 / INT8 dequantization kernels for gfx950 and
// their C-ABI entry points: y = T(float(q) * scale), rounded to nearest even.
//
// Kernels (reference kernels they replace, kernels/cuda/quantization/...):
//   k_deq_tensor     one scale: a full grid, 2 or 4 x 8 codes per thread,
//                    8-byte loads and 16-byte stores
//                    (dequantize_per_tensor_fp8.cu:23-66, dequantize_int8.cu:29-64)
//   k_deq_rows_sub   rows of 8..2048 codes (per-group, short per-channel rows)
//                    owned by power-of-two lane groups; 8-byte loads, 16-byte
//                    stores (dequantize_int8.cu:118-134, :70-109)
//   k_deq_rows_sub_any rows of any multiple of 8 below 4096 codes without a
//                    fixed-shape kernel: k_deq_rows_sub's layout, masked slots
//   k_deq_rows_wg    one workgroup per row of any longer length that is a
//                    multiple of 8 (long per-channel rows)
//   k_deq_rows_sub_any1 rows of up to 2048 codes that 8-byte loads cannot
//                    take: k_deq_rows_sub's layout with code loads
//   k_deq_rows_scalar any longer such row, element at a time
//   k_deq_cols       per-column scales (axis 1), and per-channel scales of an
//                    N-D tensor seen as [outer, channels * inner]: each thread
//                    keeps the scales of its eight columns in registers while
//                    walking rows
//   k_deq_cols_narrow the same for rows of at most 1024 codes: several rows
//                    per workgroup pass, so every thread has a chunk
//   k_deq_cols_narrow1 the same with one code per thread, for rows of at most
//                    128 codes that 8-byte loads cannot take
//   k_deq_group_tile groups along a non-last axis (the reference moves the
//                    axis last with two copies, dequantizers.py:58-72): 1-2
//                    waves per group and 512 inner positions, in place
//   k_deq_group_strided the same for inner % 8 != 0 or unaligned buffers
#include <algorithm>

#include "cbq_device.h"
#include "cbq_host.h"

namespace cbq {
namespace {


template <bool FP8>
__device__ __forceinline__ void dec4(uint32_t w, float* f) {
  if constexpr (FP8) fp8x4_to_f32(w, f);
  else int8x4_to_f32(w, f);
}

template <bool FP8>
__device__ __forceinline__ float dec1(uint8_t b) {
  float f[4];
  dec4<FP8>(static_cast<uint32_t>(b), f);
  return f[0];
}

template <int OUT>
__device__ __forceinline__ void st8(void* y, int64_t elem, const float (&f)[8]) {
  stg16(static_cast<uint16_t*>(y) + elem, pack8_out<OUT>(f));
}

template <int OUT>
__device__ __forceinline__ void st1(void* y, int64_t i, float v) {
  static_cast<uint16_t*>(y)[i] = out1<OUT>(v);
}

// ---------------------------------------------------------------------------
// Per tensor
// ---------------------------------------------------------------------------
// Workgroup b covers codes [b * span, (b + 1) * span), span = kBlock * U * 8:
// each thread loads U chunks of 8 codes (8-byte non-temporal loads, all in
// flight) and writes each as one 16-byte store. A full (non-persistent) grid.
// Measured on MI355X in steady state (launches over distinct 2 GB of
// buffers, so no input or output stays in the Infinity Cache), 64M codes:
// U = 2 runs at 33.3 us, as fast as a plain 16-byte copy of the same bytes
// (33.2 us); U = 4 at 35.4 us, U = 1 or 3 at 34.3-34.7 us, a persistent
// grid at 33.5-35.4 us. Below 32M codes U = 4 is faster (fewer workgroups
// to launch).
template <bool FP8, int OUT, int U>
__global__ __launch_bounds__(kBlock) void k_deq_tensor(
    const uint8_t* __restrict__ q, const float* __restrict__ scale, int64_t n, int vec,
    void* __restrict__ y) {
  const float s = scale[0];
  if (vec) {
    const int64_t n8 = n >> 3;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * (kBlock * U) + threadIdx.x;
    uint2 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
      if (c < n8) r[u] = ldg8(q + c * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
      if (c < n8) {
        float f[8];
        dec4<FP8>(r[u].x, f);
        dec4<FP8>(r[u].y, f + 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] *= s;
        st8<OUT>(y, c * 8, f);
      }
    }
    if (blockIdx.x == 0) {
      const int64_t i = n8 * 8 + threadIdx.x;   // the < 8 trailing codes
      if (i < n) st1<OUT>(y, i, dec1<FP8>(q[i]) * s);
    }
  } else {
    const int64_t step = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += step)
      st1<OUT>(y, i, dec1<FP8>(q[i]) * s);
  }
}

// ---------------------------------------------------------------------------
// Rows: scale[row] for rows of L codes
// ---------------------------------------------------------------------------
template <int OUT, int LPR, int VPL, int RI>
__global__ __launch_bounds__(kBlock) void k_deq_rows_sub(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows,
    void* __restrict__ y) {
  constexpr int RPW = kWave / LPR;
  constexpr int64_t L = static_cast<int64_t>(LPR) * VPL * 8;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int sub = lane / LPR;
  const int lr = lane % LPR;
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * (RI * RPW) + sub;
  uint2 r[RI][VPL];
  float s[RI];
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
      s[it] = scale[row];
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        r[it][v] = ldg8(q + row * L + (v * LPR + lr) * 8);
    }
  }
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        float f[8];
        int8x4_to_f32(r[it][v].x, f);
        int8x4_to_f32(r[it][v].y, f + 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] *= s[it];
        st8<OUT>(y, row * L + (v * LPR + lr) * 8, f);
      }
    }
  }
}

// Rows of cg chunks of 8 codes for any cg < 512 without a fixed-shape
// kernel (group sizes such as 56 or 112): the layout of k_deq_rows_sub with
// LPR * VPL >= cg chunk slots per row, slots past cg idle.
template <int OUT, int LPR, int VPL, int RI>
__global__ __launch_bounds__(kBlock) void k_deq_rows_sub_any(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int cg,
    void* __restrict__ y) {
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int sub = lane / LPR;
  const int lr = lane % LPR;
  const int64_t L = static_cast<int64_t>(cg) * 8;
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * (RI * RPW) + sub;
  uint2 r[RI][VPL];
  float s[RI];
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
      s[it] = scale[row];
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int j = v * LPR + lr;
        r[it][v] = ldg8(q + row * L + (j < cg ? j : 0) * 8);
      }
    }
  }
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int j = v * LPR + lr;
        if (j >= cg) continue;
        float f[8];
        int8x4_to_f32(r[it][v].x, f);
        int8x4_to_f32(r[it][v].y, f + 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] *= s[it];
        st8<OUT>(y, row * L + j * 8, f);
      }
    }
  }
}

// One workgroup per row (striding over rows); L % 8 == 0, aligned pointers.
template <int OUT>
__global__ __launch_bounds__(kBlock) void k_deq_rows_wg(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int64_t L,
    void* __restrict__ y, int64_t sc) {
  // slice blockIdx.y of each row: chunks [c0, nc) of sc (all of them when
  // gridDim.y == 1; few long rows are cut into slices to fill the CUs)
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * sc;
  const int64_t nc = c0 + sc < (L >> 3) ? c0 + sc : (L >> 3);
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float s = scale[row];
    const int64_t base = row * L;
    int64_t c = c0 + threadIdx.x;
    for (; c + 3 * kBlock < nc; c += 4 * kBlock) {
      uint2 r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        r[u] = ldg8(q + base + (c + u * kBlock) * 8);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float f[8];
        int8x4_to_f32(r[u].x, f);
        int8x4_to_f32(r[u].y, f + 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] *= s;
        st8<OUT>(y, base + (c + u * kBlock) * 8, f);
      }
    }
    for (; c < nc; c += kBlock) {
      const uint2 r = ldg8(q + base + c * 8);
      float f[8];
      int8x4_to_f32(r.x, f);
      int8x4_to_f32(r.y, f + 4);
#pragma unroll
      for (int k = 0; k < 8; ++k) f[k] *= s;
      st8<OUT>(y, base + c * 8, f);
    }
  }
}

template <int OUT>
__global__ __launch_bounds__(kBlock) void k_deq_rows_scalar(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int64_t L,
    void* __restrict__ y) {
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float s = scale[row];
    const int64_t base = row * L;
    for (int64_t i = threadIdx.x; i < L; i += kBlock)
      st1<OUT>(y, base + i, static_cast<float>(q[base + i]) * s);
  }
}

// Rows of any length L <= 2048 that 8-byte code loads cannot take (L % 8 !=
// 0, e.g. groups of 100, or unaligned buffers): LPR lanes per row, VPL codes
// per lane, code j = v * LPR + lr, loads and stores contiguous across the
// lanes of a row.
template <int OUT, int LPR, int VPL, int RI, int E>
__global__ __launch_bounds__(kBlock) void k_deq_rows_sub_any1(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int L,
    void* __restrict__ y) {
  // E = 2: code pairs (L even, q and y aligned to a pair): one 2-byte load
  // and one 4-byte store per pair
  static_assert(E == 1 || E == 2, "codes per load");
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int sub = lane / LPR;
  const int lr = lane % LPR;
  const int U = L / E;
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * (RI * RPW) + sub;
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row >= rows) continue;
    const float s = scale[row];
    uint32_t c[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int j = v * LPR + lr;
      const int64_t e = row * L + static_cast<int64_t>(j < U ? j : 0) * E;
      if constexpr (E == 1) c[v] = static_cast<uint8_t>(q[e]);
      else c[v] = *reinterpret_cast<const uint16_t*>(q + e);
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int j = v * LPR + lr;
      if (j >= U) continue;
      const int64_t e = row * L + static_cast<int64_t>(j) * E;
      const float a = static_cast<float>(static_cast<int8_t>(c[v] & 0xffu)) * s;
      if constexpr (E == 1) {
        st1<OUT>(y, e, a);
      } else {
        float b = static_cast<float>(static_cast<int8_t>((c[v] >> 8) & 0xffu)) * s;
        float a2 = a;
        asm volatile("" : "+v"(a2), "+v"(b));   // finished fp32 products, as in out1
        *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(y) + e) = pack2_out<OUT>(a2, b);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Columns: scale[col] (axis 1). Row block blockIdx.y of RB rows.
// ---------------------------------------------------------------------------
// inner: adjacent columns sharing one scale (1 for per-column scales; the
// N-D channel path views [outer, channels, inner] as [outer, channels * inner]).
template <int OUT>
__global__ __launch_bounds__(kBlock) void k_deq_cols(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int64_t cols,
    int64_t RB, int vec, int64_t inner, void* __restrict__ y) {
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  if (vec) {
    const int64_t c = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 8;
    if (c >= cols) return;
    float s[8];
    channel_vals8(scale, c, inner, s);
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      uint2 raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[u] = ldg8(q + (r + u) * cols + c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float f[8];
        int8x4_to_f32(raw[u].x, f);
        int8x4_to_f32(raw[u].y, f + 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] *= s[k];
        st8<OUT>(y, (r + u) * cols + c, f);
      }
    }
    for (; r < r1; ++r) {
      const uint2 raw = ldg8(q + r * cols + c);
      float f[8];
      int8x4_to_f32(raw.x, f);
      int8x4_to_f32(raw.y, f + 4);
#pragma unroll
      for (int k = 0; k < 8; ++k) f[k] *= s[k];
      st8<OUT>(y, r * cols + c, f);
    }
  } else {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= cols) return;
    const float s = scale[c / inner];
    for (int64_t r = r0; r < r1; ++r)
      st1<OUT>(y, r * cols + c, static_cast<float>(q[r * cols + c]) * s);
  }
}

// Narrow columns (cols % 8 == 0, u = cols / 8 <= kBlock / 2 chunks per row,
// e.g. [262144, 64]): k_deq_cols would leave all but u threads of a
// workgroup idle; here thread t takes chunk t % u of rows r0 + t / u,
// stepping by rpi = kBlock / u rows.
template <int OUT>
__global__ __launch_bounds__(kBlock) void k_deq_cols_narrow(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int64_t cols,
    int64_t RB, int u, int rpi, int64_t inner, void* __restrict__ y) {
  const int sub = static_cast<int>(threadIdx.x) / u, cu = static_cast<int>(threadIdx.x) - sub * u;
  if (sub >= rpi) return;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  const int64_t c = static_cast<int64_t>(cu) * 8;
  float s[8];
  channel_vals8(scale, c, inner, s);
  int64_t r = r0 + sub;
  for (; r + 3 * rpi < r1; r += 4 * rpi) {
    uint2 raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k] = ldg8(q + (r + k * rpi) * cols + c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float f[8];
      int8x4_to_f32(raw[k].x, f);
      int8x4_to_f32(raw[k].y, f + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] *= s[e];
      st8<OUT>(y, (r + k * rpi) * cols + c, f);
    }
  }
  for (; r < r1; r += rpi) {
    const uint2 raw = ldg8(q + r * cols + c);
    float f[8];
    int8x4_to_f32(raw.x, f);
    int8x4_to_f32(raw.y, f + 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] *= s[e];
    st8<OUT>(y, r * cols + c, f);
  }
}

// The same for narrow rows that 8-byte code loads cannot take (cols <=
// kBlock / 2 with cols % 8 != 0, or unaligned buffers): one code per thread.
template <int OUT>
__global__ __launch_bounds__(kBlock) void k_deq_cols_narrow1(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t rows, int64_t cols,
    int64_t RB, int rpi, int64_t inner, void* __restrict__ y) {
  const int u = static_cast<int>(cols);
  const int sub = static_cast<int>(threadIdx.x) / u, c = static_cast<int>(threadIdx.x) - sub * u;
  if (sub >= rpi) return;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  const float s = scale[c / inner];
  int64_t r = r0 + sub;
  for (; r + 3 * rpi < r1; r += 4 * rpi) {
    int8_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = q[(r + k * rpi) * cols + c];
#pragma unroll
    for (int k = 0; k < 4; ++k) st1<OUT>(y, (r + k * rpi) * cols + c, static_cast<float>(v[k]) * s);
  }
  for (; r < r1; r += rpi) st1<OUT>(y, r * cols + c, static_cast<float>(q[r * cols + c]) * s);
}

// Groups along a non-last axis ([outer, len, inner], groups of G along len):
// one thread per group (o, g, i), i fastest; scale index in the reference's
// movedim layout, (o * inner + i) * (len / G) + g (dequantizers.py:61-72).
template <int OUT>
__global__ __launch_bounds__(kBlock) void k_deq_group_strided(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t outer, int64_t len,
    int64_t inner, int64_t G, void* __restrict__ y) {
  const int64_t ng = len / G;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (t >= outer * ng * inner) return;
  const int64_t i = t % inner, g = (t / inner) % ng, o = t / (inner * ng);
  const int64_t base = (o * len + g * G) * inner + i;
  const float s = scale[(o * inner + i) * ng + g];
  for (int64_t k = 0; k < G; ++k)
    st1<OUT>(y, base + k * inner, static_cast<float>(q[base + k * inner]) * s);
}

// Groups along a non-last axis, tiled (inner % 8 == 0, 8-byte aligned q,
// 16-byte aligned y). A workgroup of NW (1 or 2) waves covers 64 x 8
// adjacent inner positions of one group of G = NW * rpt positions; each
// thread keeps its eight columns' scales in registers and walks its rpt
// positions (8-byte loads, 16-byte stores). Workgroup index: inner tile
// fastest, then g, then o. Measured on MI355X ([16384, 14336] bf16, G = 128
// along axis 0): 157 us against 202 us with 8 waves per group; shorter walks
// per thread lose more to the scale gathers (the eight scales of a thread are
// len / G floats apart) than they gain.
constexpr int kDgCols = kWave * 8;

// TS: scale is group-major scratch [outer, ng, inner] (the movedim order
// transposed by k_transpose_f32 beforehand), so a thread's eight scales are
// two contiguous 16-byte loads and short walks pay: RPTC > 0 is the walk
// rounded up to a power of two at compile time (unguarded loads, clamped
// past rpt; stores guarded).
template <int OUT, int NW, bool TS = false, int RPTC = 0>
__global__ __launch_bounds__(NW * kWave) void k_deq_group_tile(
    const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t len, int64_t inner,
    int64_t G, int rpt, int64_t ng, int64_t tiles, void* __restrict__ y) {
  const int64_t b = blockIdx.x;
  const int64_t ti = b % tiles, g = (b / tiles) % ng, o = b / (ng * tiles);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int64_t i = ti * kDgCols + lane * 8;
  if (i >= inner) return;
  float s[8];
  if constexpr (TS) {
    const float4* sp = reinterpret_cast<const float4*>(scale + (o * ng + g) * inner + i);
    const float4 a = sp[0], c = sp[1];
    s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w; s[4] = c.x; s[5] = c.y; s[6] = c.z; s[7] = c.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = scale[(o * inner + i + j) * ng + g];
  }
  const int64_t base = (o * len + g * G + w) * inner + i;
  const int64_t rs = static_cast<int64_t>(NW) * inner;
  if constexpr (RPTC > 0) {
    uint2 raw[RPTC];
#pragma unroll
    for (int k = 0; k < RPTC; ++k) raw[k] = ldg8(q + base + min(k, rpt - 1) * rs);
#pragma unroll
    for (int k = 0; k < RPTC; ++k)
      if (k < rpt) {
        float f[8];
        int8x4_to_f32(raw[k].x, f);
        int8x4_to_f32(raw[k].y, f + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= s[j];
        st8<OUT>(y, base + k * rs, f);
      }
    return;
  }
  for (int k0 = 0; k0 < rpt; k0 += 8) {
    uint2 raw[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < rpt) raw[k] = ldg8(q + base + (k0 + k) * rs);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < rpt) {
        float f[8];
        int8x4_to_f32(raw[k].x, f);
        int8x4_to_f32(raw[k].y, f + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= s[j];
        st8<OUT>(y, base + (k0 + k) * rs, f);
      }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
bool valid_out(int dt) { return dt == kF16 || dt == kBF16; }

unsigned rows_grid(int64_t rows) {
  const int64_t cap = 1 << 20;
  return static_cast<unsigned>(rows < cap ? rows : cap);
}

constexpr int64_t kDeqU2Min = 1LL << 25;   // codes from which k_deq_tensor takes U = 2

template <bool FP8, int OUT>
int deq_tensor_t(const uint8_t* q, const float* scale, int64_t n, void* y, hipStream_t s,
                 const char* what) {
  const bool vec = aligned(q, 8) && aligned(y, 16);
  const int u = n >= kDeqU2Min ? 2 : 4;
  int64_t grid;
  if (vec) {
    grid = cdiv(n, static_cast<int64_t>(kBlock) * u * 8);
    if (grid > 0x7fffffffLL / kBlock) {
      set_error("%s: tensor too large (%lld elements)", what, (long long)n);
      return CBQ_EINVAL;
    }
  } else {
    const int64_t cap = static_cast<int64_t>(device_cus()) * 8;
    grid = cdiv(n, kBlock) < cap ? cdiv(n, kBlock) : cap;
  }
  if (grid < 1) grid = 1;
  const dim3 g(static_cast<unsigned>(grid)), b(kBlock);
  if (u == 2) k_deq_tensor<FP8, OUT, 2><<<g, b, 0, s>>>(q, scale, n, vec ? 1 : 0, y);
  else k_deq_tensor<FP8, OUT, 4><<<g, b, 0, s>>>(q, scale, n, vec ? 1 : 0, y);
  return launch_status(what);
}

template <bool FP8>
int deq_tensor(const uint8_t* q, const float* scale, int64_t n, void* y, int out, hipStream_t s,
               const char* what) {
  CBQ_REQUIRE(valid_out(out), "%s: out_dtype must be fp16 or bf16 (code %d)", what, out);
  CBQ_REQUIRE(n >= 0, "%s: negative element count", what);
  if (n == 0) return CBQ_OK;
  CBQ_REQUIRE(q && scale && y, "%s: null pointer", what);
  return out == kF16 ? deq_tensor_t<FP8, kF16>(q, scale, n, y, s, what)
                     : deq_tensor_t<FP8, kBF16>(q, scale, n, y, s, what);
}

template <int OUT, int LPR, int VPL>
void launch_deq_rows_sub(const int8_t* q, const float* scale, int64_t rows, void* y,
                         hipStream_t s) {
  constexpr int RI = (LPR * VPL >= 64) ? 2 : 4;
  constexpr int64_t rows_per_wg = static_cast<int64_t>(kBlock / kWave) * RI * (kWave / LPR);
  k_deq_rows_sub<OUT, LPR, VPL, RI><<<dim3(static_cast<unsigned>(cdiv(rows, rows_per_wg))),
                                       dim3(kBlock), 0, s>>>(q, scale, rows, y);
}

template <int OUT, int LPR, int VPL>
void launch_deq_rows_sub_any(const int8_t* q, const float* scale, int64_t rows, int cg, void* y,
                             hipStream_t s) {
  constexpr int RI = (LPR * VPL >= 64) ? 2 : 4;
  constexpr int64_t rows_per_wg = static_cast<int64_t>(kBlock / kWave) * RI * (kWave / LPR);
  k_deq_rows_sub_any<OUT, LPR, VPL, RI><<<dim3(static_cast<unsigned>(cdiv(rows, rows_per_wg))),
                                           dim3(kBlock), 0, s>>>(q, scale, rows, cg, y);
}

// Rows of cg < 512 chunks without a fixed-shape kernel (k_deq_rows_wg would
// give each short row a workgroup of its own): LPR lanes x VPL chunks.
template <int OUT>
void deq_rows_any(const int8_t* q, const float* scale, int64_t rows, int cg, void* y,
                  hipStream_t s) {
  if (cg <= 1) launch_deq_rows_sub_any<OUT, 1, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 2) launch_deq_rows_sub_any<OUT, 2, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 4) launch_deq_rows_sub_any<OUT, 4, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 8) launch_deq_rows_sub_any<OUT, 8, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 16) launch_deq_rows_sub_any<OUT, 16, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 32) launch_deq_rows_sub_any<OUT, 32, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 64) launch_deq_rows_sub_any<OUT, 64, 1>(q, scale, rows, cg, y, s);
  else if (cg <= 128) launch_deq_rows_sub_any<OUT, 64, 2>(q, scale, rows, cg, y, s);
  else if (cg <= 256) launch_deq_rows_sub_any<OUT, 64, 4>(q, scale, rows, cg, y, s);
  else launch_deq_rows_sub_any<OUT, 64, 8>(q, scale, rows, cg, y, s);
}

template <int OUT, int LPR, int VPL, int E>
void launch_deq_rows_sub_any1(const int8_t* q, const float* scale, int64_t rows, int L, void* y,
                              hipStream_t s) {
  constexpr int RI = VPL >= 16 ? 1 : 2;
  constexpr int64_t rows_per_wg = static_cast<int64_t>(kBlock / kWave) * RI * (kWave / LPR);
  k_deq_rows_sub_any1<OUT, LPR, VPL, RI, E>
      <<<dim3(static_cast<unsigned>(cdiv(rows, rows_per_wg))), dim3(kBlock), 0, s>>>(q, scale,
                                                                                     rows, L, y);
}

template <int OUT, int E>
void deq_rows_any1_e(const int8_t* q, const float* scale, int64_t rows, int L, void* y,
                     hipStream_t s) {
  const int U = L / E;
  if (U <= 1) launch_deq_rows_sub_any1<OUT, 1, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 2) launch_deq_rows_sub_any1<OUT, 2, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 4) launch_deq_rows_sub_any1<OUT, 4, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 8) launch_deq_rows_sub_any1<OUT, 8, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 16) launch_deq_rows_sub_any1<OUT, 16, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 32) launch_deq_rows_sub_any1<OUT, 32, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 64) launch_deq_rows_sub_any1<OUT, 64, 1, E>(q, scale, rows, L, y, s);
  else if (U <= 128) launch_deq_rows_sub_any1<OUT, 64, 2, E>(q, scale, rows, L, y, s);
  else if (U <= 256) launch_deq_rows_sub_any1<OUT, 64, 4, E>(q, scale, rows, L, y, s);
  else if (U <= 512) launch_deq_rows_sub_any1<OUT, 64, 8, E>(q, scale, rows, L, y, s);
  else launch_deq_rows_sub_any1<OUT, 64, 16, E>(q, scale, rows, L, y, s);
}

template <int OUT>
void deq_rows_any1(const int8_t* q, const float* scale, int64_t rows, int L, void* y,
                   hipStream_t s) {
  if (L % 2 == 0 && aligned(q, 2) && aligned(y, 4))
    deq_rows_any1_e<OUT, 2>(q, scale, rows, L, y, s);
  else if (L <= 1024)
    deq_rows_any1_e<OUT, 1>(q, scale, rows, L, y, s);
  else
    launch_deq_rows_sub_any1<OUT, 64, 32, 1>(q, scale, rows, L, y, s);
}

template <int OUT>
int deq_rows_t(const int8_t* q, const float* scale, int64_t rows, int64_t L, void* y,
               hipStream_t s, const char* what) {
  CBQ_REQUIRE(rows <= 0x7fffffffLL, "%s: too many rows (%lld)", what, (long long)rows);
  const bool vec = (L % 8 == 0) && aligned(q, 8) && aligned(y, 16);
  if (vec) {
    switch (L) {
      case 8: launch_deq_rows_sub<OUT, 1, 1>(q, scale, rows, y, s); return launch_status(what);
      case 16: launch_deq_rows_sub<OUT, 2, 1>(q, scale, rows, y, s); return launch_status(what);
      case 32: launch_deq_rows_sub<OUT, 4, 1>(q, scale, rows, y, s); return launch_status(what);
      case 64: launch_deq_rows_sub<OUT, 8, 1>(q, scale, rows, y, s); return launch_status(what);
      case 128: launch_deq_rows_sub<OUT, 16, 1>(q, scale, rows, y, s); return launch_status(what);
      case 256: launch_deq_rows_sub<OUT, 32, 1>(q, scale, rows, y, s); return launch_status(what);
      case 512: launch_deq_rows_sub<OUT, 64, 1>(q, scale, rows, y, s); return launch_status(what);
      case 1024: launch_deq_rows_sub<OUT, 64, 2>(q, scale, rows, y, s); return launch_status(what);
      case 2048: launch_deq_rows_sub<OUT, 64, 4>(q, scale, rows, y, s); return launch_status(what);
      default:
        if ((L >> 3) < 512) {
          deq_rows_any<OUT>(q, scale, rows, static_cast<int>(L >> 3), y, s);
          return launch_status(what);
        }
        {
          // fewer than two rows per CU: each row cut into slices of at least
          // 8192 codes, about four workgroups per CU in all. Measured on
          // MI355X, [64, 2^20] codes to bf16: 108.3 us with one workgroup
          // per row
          const int64_t nc = L >> 3, cus = device_cus();
          int64_t sp = 1;
          if (rows < 2 * cus)
            sp = std::max<int64_t>(1, std::min<int64_t>({cdiv(4 * cus, rows), nc / 1024, 256}));
          k_deq_rows_wg<OUT><<<dim3(rows_grid(rows), static_cast<unsigned>(sp)), dim3(kBlock), 0,
                               s>>>(q, scale, rows, L, y, cdiv(nc, sp));
        }
        return launch_status(what);
    }
  }
  if (L <= 2048) {
    deq_rows_any1<OUT>(q, scale, rows, static_cast<int>(L), y, s);
    return launch_status(what);
  }
  k_deq_rows_scalar<OUT><<<dim3(rows_grid(rows)), dim3(kBlock), 0, s>>>(q, scale, rows, L, y);
  return launch_status(what);
}

int deq_rows(const int8_t* q, const float* scale, int64_t rows, int64_t L, void* y, int out,
             hipStream_t s, const char* what) {
  return out == kF16 ? deq_rows_t<kF16>(q, scale, rows, L, y, s, what)
                     : deq_rows_t<kBF16>(q, scale, rows, L, y, s, what);
}

constexpr int64_t kDeqNarrowRows = 8;

template <int OUT>
int deq_cols_t(const int8_t* q, const float* scale, int64_t rows, int64_t cols, int64_t inner,
               void* y, hipStream_t s, const char* what) {
  const bool vec = (cols % 8 == 0) && aligned(q, 8) && aligned(y, 16);
  const int64_t u = cols >> 3;
  if (!vec && cols <= kBlock / 2) {
    // narrow rows, one code per thread: 16 rows per thread
    const int rpi = kBlock / static_cast<int>(cols);
    int64_t RB = rpi * 2 * kDeqNarrowRows;
    if (cdiv(rows, RB) > 65535) RB = cdiv(cdiv(rows, 65535), rpi) * rpi;
    k_deq_cols_narrow1<OUT><<<dim3(1, static_cast<unsigned>(cdiv(rows, RB))), dim3(kBlock), 0, s>>>(
        q, scale, rows, cols, RB, rpi, inner, y);
    return launch_status(what);
  }
  if (vec && u <= kBlock / 2) {
    // narrow rows: kDeqNarrowRows rows per thread, rpi threads per chunk
    const int rpi = kBlock / static_cast<int>(u);
    int64_t RB = rpi * kDeqNarrowRows;
    if (cdiv(rows, RB) > 65535) RB = cdiv(cdiv(rows, 65535), rpi) * rpi;
    k_deq_cols_narrow<OUT><<<dim3(1, static_cast<unsigned>(cdiv(rows, RB))), dim3(kBlock), 0, s>>>(
        q, scale, rows, cols, RB, static_cast<int>(u), rpi, inner, y);
    return launch_status(what);
  }
  const int64_t col_blocks = vec ? cdiv(cdiv(cols, 8), kBlock) : cdiv(cols, kBlock);
  // Short row blocks (16 rows per thread): many workgroups in flight;
  // measured on MI355X, walks of ~60 rows per thread lose ~5-20%, and
  // 4-row blocks lose 3% on [7, 4096 x 8192] (channel axis 1 of 3-D).
  int64_t RB = 16;
  if (cdiv(rows, RB) > 65535) RB = cdiv(rows, 65535);
  const int64_t nrb = cdiv(rows, RB);
  k_deq_cols<OUT><<<dim3(static_cast<unsigned>(col_blocks), static_cast<unsigned>(nrb)),
                    dim3(kBlock), 0, s>>>(q, scale, rows, cols, RB, vec ? 1 : 0, inner, y);
  return launch_status(what);
}

template <int OUT, int NW>
void launch_deq_group_tile(const int8_t* q, const float* scale, int64_t outer, int64_t len,
                           int64_t inner, int64_t G, void* y, hipStream_t s) {
  const int64_t ng = len / G, tiles = cdiv(inner, kDgCols);
  const int64_t nblocks = outer * tiles * ng;
  k_deq_group_tile<OUT, NW><<<dim3(static_cast<unsigned>(nblocks)), dim3(NW * kWave), 0, s>>>(
      q, scale, len, inner, G, static_cast<int>(G / NW), ng, tiles, y);
}

// Scale scratch for the tiled group dequant: ng > 1 and a 32-bit transpose
// grid (as in the group quant).
bool deq_group_scratch_applies(int64_t outer, int64_t ng, int64_t inner) {
  return ng > 1 && outer * cdiv(ng, static_cast<int64_t>(kTrTile)) *
                           cdiv(inner, static_cast<int64_t>(kTrTile)) < (1LL << 31);
}

// The scratch path: the scales transposed to group-major [outer, ng, inner]
// in tmp, then 8 waves per group (G % 8 == 0, G <= 128: walks of at most 16
// positions, compile-time) or the 1-2 wave tiles reading the scratch.
template <int OUT>
void launch_deq_group_scratch(const int8_t* q, const float* scale, int64_t outer, int64_t len,
                              int64_t inner, int64_t G, float* tmp, void* y, hipStream_t s) {
  const int64_t ng = len / G, tiles = cdiv(inner, kDgCols);
  const int64_t rt = cdiv(inner, static_cast<int64_t>(kTrTile));
  const int64_t ct = cdiv(ng, static_cast<int64_t>(kTrTile));
  k_transpose_f32<<<dim3(static_cast<unsigned>(outer * rt * ct)), dim3(kBlock), 0, s>>>(
      scale, inner, ng, rt, ct, (ng % 4 == 0 && aligned(scale, 16)) ? 1 : 0, 1, tmp);
  const int64_t nblocks = outer * tiles * ng;
  const dim3 grid(static_cast<unsigned>(nblocks));
  if (G % 8 == 0 && G / 8 <= 16) {
    const int rpt = static_cast<int>(G / 8);
    const dim3 block(8 * kWave);
    const int rc = rpt <= 1 ? 1 : rpt <= 2 ? 2 : rpt <= 4 ? 4 : rpt <= 8 ? 8 : 16;
    switch (rc) {
      case 1: k_deq_group_tile<OUT, 8, true, 1><<<grid, block, 0, s>>>(q, tmp, len, inner, G, rpt, ng, tiles, y); break;
      case 2: k_deq_group_tile<OUT, 8, true, 2><<<grid, block, 0, s>>>(q, tmp, len, inner, G, rpt, ng, tiles, y); break;
      case 4: k_deq_group_tile<OUT, 8, true, 4><<<grid, block, 0, s>>>(q, tmp, len, inner, G, rpt, ng, tiles, y); break;
      case 8: k_deq_group_tile<OUT, 8, true, 8><<<grid, block, 0, s>>>(q, tmp, len, inner, G, rpt, ng, tiles, y); break;
      default: k_deq_group_tile<OUT, 8, true, 16><<<grid, block, 0, s>>>(q, tmp, len, inner, G, rpt, ng, tiles, y); break;
    }
  } else if (G % 2 == 0) {
    k_deq_group_tile<OUT, 2, true><<<grid, dim3(2 * kWave), 0, s>>>(
        q, tmp, len, inner, G, static_cast<int>(G / 2), ng, tiles, y);
  } else {
    k_deq_group_tile<OUT, 1, true><<<grid, dim3(kWave), 0, s>>>(
        q, tmp, len, inner, G, static_cast<int>(G), ng, tiles, y);
  }
}

}  // namespace
}  // namespace cbq

using namespace cbq;

extern "C" int cbq_dequant_fp8_tensor(const uint8_t* q, const float* scale, int64_t n, void* y,
                                      int out_dtype, cbq_stream_t stream) {
  clear_error();
  return deq_tensor<true>(q, scale, n, y, out_dtype, as_stream(stream), "cbq_dequant_fp8_tensor");
}

extern "C" int cbq_dequant_int8_tensor(const int8_t* q, const float* scale, int64_t n, void* y,
                                       int out_dtype, cbq_stream_t stream) {
  clear_error();
  return deq_tensor<false>(reinterpret_cast<const uint8_t*>(q), scale, n, y, out_dtype,
                           as_stream(stream), "cbq_dequant_int8_tensor");
}

extern "C" int cbq_dequant_int8_channel(const int8_t* q, const float* scale, int64_t rows,
                                        int64_t cols, int axis, void* y, int out_dtype,
                                        cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_dequant_int8_channel";
  CBQ_REQUIRE(valid_out(out_dtype), "%s: out_dtype must be fp16 or bf16 (code %d)", what,
              out_dtype);
  CBQ_REQUIRE(axis == 0 || axis == 1, "%s: axis must be 0 or 1, got %d", what, axis);
  CBQ_REQUIRE(rows >= 0 && cols >= 0, "%s: negative shape", what);
  if (rows == 0 || cols == 0) return CBQ_OK;
  CBQ_REQUIRE(q && scale && y, "%s: null pointer", what);
  if (axis == 0) return deq_rows(q, scale, rows, cols, y, out_dtype, as_stream(stream), what);
  return out_dtype == kF16 ? deq_cols_t<kF16>(q, scale, rows, cols, 1, y, as_stream(stream), what)
                           : deq_cols_t<kBF16>(q, scale, rows, cols, 1, y, as_stream(stream), what);
}

extern "C" int cbq_dequant_int8_channel_nd(const int8_t* q, const float* scale, int64_t outer,
                                           int64_t channels, int64_t inner, void* y,
                                           int out_dtype, cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_dequant_int8_channel_nd";
  CBQ_REQUIRE(valid_out(out_dtype), "%s: out_dtype must be fp16 or bf16 (code %d)", what,
              out_dtype);
  CBQ_REQUIRE(outer >= 0 && channels >= 0 && inner >= 0, "%s: negative shape", what);
  if (outer == 0 || channels == 0 || inner == 0) return CBQ_OK;
  CBQ_REQUIRE(q && scale && y, "%s: null pointer", what);
  if (outer == 1) return deq_rows(q, scale, channels, inner, y, out_dtype, as_stream(stream), what);
  const int64_t cols = channels * inner;
  return out_dtype == kF16
             ? deq_cols_t<kF16>(q, scale, outer, cols, inner, y, as_stream(stream), what)
             : deq_cols_t<kBF16>(q, scale, outer, cols, inner, y, as_stream(stream), what);
}

extern "C" int cbq_dequant_int8_group(const int8_t* q, const float* scale, int64_t num_groups,
                                      int64_t group_size, void* y, int out_dtype,
                                      cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_dequant_int8_group";
  CBQ_REQUIRE(valid_out(out_dtype), "%s: out_dtype must be fp16 or bf16 (code %d)", what,
              out_dtype);
  CBQ_REQUIRE(group_size > 0 && group_size <= 4096, "%s: group_size must be in (0, 4096], got %lld",
              what, (long long)group_size);
  CBQ_REQUIRE(num_groups >= 0, "%s: negative group count", what);
  if (num_groups == 0) return CBQ_OK;
  CBQ_REQUIRE(q && scale && y, "%s: null pointer", what);
  return deq_rows(q, scale, num_groups, group_size, y, out_dtype, as_stream(stream), what);
}

extern "C" size_t cbq_dequant_int8_group_nd_ws_bytes(int64_t outer, int64_t len, int64_t inner,
                                                     int64_t group_size) {
  if (outer <= 0 || len <= 0 || inner <= 1 || group_size <= 0 || len % group_size != 0 ||
      inner % 8 != 0)
    return CBQ_WS_CTRL_BYTES;
  const int64_t ng = len / group_size;
  if (!deq_group_scratch_applies(outer, ng, inner)) return CBQ_WS_CTRL_BYTES;
  return CBQ_WS_CTRL_BYTES + static_cast<size_t>(outer * ng * inner) * 4;
}

extern "C" int cbq_dequant_int8_group_nd(const int8_t* q, const float* scale, int64_t outer,
                                         int64_t len, int64_t inner, int64_t group_size,
                                         void* ws, size_t ws_bytes, void* y, int out_dtype,
                                         cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_dequant_int8_group_nd";
  CBQ_REQUIRE(valid_out(out_dtype), "%s: out_dtype must be fp16 or bf16 (code %d)", what,
              out_dtype);
  CBQ_REQUIRE(group_size > 0 && group_size <= 4096, "%s: group_size must be in (0, 4096], got %lld",
              what, (long long)group_size);
  CBQ_REQUIRE(outer >= 0 && len >= 0 && inner >= 0, "%s: negative shape", what);
  CBQ_REQUIRE(len % group_size == 0, "%s: group_size %lld must divide the axis length %lld", what,
              (long long)group_size, (long long)len);
  if (outer == 0 || len == 0 || inner == 0) return CBQ_OK;
  CBQ_REQUIRE(q && scale && y, "%s: null pointer", what);
  const int64_t ng = len / group_size;
  CBQ_REQUIRE(cdiv(outer * ng * inner, kBlock) < (1LL << 31), "%s: too many groups", what);
  if (inner == 1)
    return deq_rows(q, scale, outer * ng, group_size, y, out_dtype, as_stream(stream), what);
  const int64_t tiles = cdiv(inner, kDgCols);
  if (inner % 8 == 0 && aligned(q, 8) && aligned(y, 16) && outer * tiles * ng < (1LL << 31)) {
    if (ws && aligned(ws, 16) && deq_group_scratch_applies(outer, ng, inner) &&
        ws_bytes >= CBQ_WS_CTRL_BYTES + static_cast<size_t>(outer * ng * inner) * 4) {
      float* tmp = reinterpret_cast<float*>(static_cast<char*>(ws) + CBQ_WS_CTRL_BYTES);
      if (out_dtype == kF16)
        launch_deq_group_scratch<kF16>(q, scale, outer, len, inner, group_size, tmp, y, as_stream(stream));
      else
        launch_deq_group_scratch<kBF16>(q, scale, outer, len, inner, group_size, tmp, y, as_stream(stream));
      return launch_status(what);
    }
    const bool two = group_size % 2 == 0;
    if (out_dtype == kF16) {
      if (two) launch_deq_group_tile<kF16, 2>(q, scale, outer, len, inner, group_size, y, as_stream(stream));
      else launch_deq_group_tile<kF16, 1>(q, scale, outer, len, inner, group_size, y, as_stream(stream));
    } else {
      if (two) launch_deq_group_tile<kBF16, 2>(q, scale, outer, len, inner, group_size, y, as_stream(stream));
      else launch_deq_group_tile<kBF16, 1>(q, scale, outer, len, inner, group_size, y, as_stream(stream));
    }
    return launch_status(what);
  }
  const unsigned grid = static_cast<unsigned>(cdiv(outer * ng * inner, kBlock));
  if (out_dtype == kF16)
    k_deq_group_strided<kF16><<<dim3(grid), dim3(kBlock), 0, as_stream(stream)>>>(
        q, scale, outer, len, inner, group_size, y);
  else
    k_deq_group_strided<kBF16><<<dim3(grid), dim3(kBlock), 0, as_stream(stream)>>>(
        q, scale, outer, len, inner, group_size, y);
  return launch_status(what);
}
