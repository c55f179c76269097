// cbq_quant.hip - symmetric FP8 E4M3 / INT8 quantization kernels for gfx950
// and their C-ABI entry points.
//
// Kernels (reference kernels they replace, kernels/cuda/quantization/...):
//   k_quant_tensor_1pass
//                   per-tensor quant in one launch (x of 2^20 elements and
//                   more): one resident workgroup per CU reads x once,
//                   holds up to 96 MiB of it in registers, exchanges
//                   workgroup maxima through tagged slots in the workspace,
//                   then casts from registers (quantize_per_tensor_fp8.cu:38-132,
//                   quantize_int8.cu:47-166: both passes in one)
//   k_amax_tensor   per-tensor |x| max over a persistent grid: 16-byte loads,
//                   wave64 DPP reduce, one partial maximum per workgroup
//                   written to the workspace (no atomics: measured on MI355X,
//                   ~4k same-address device atomics cost ~100 us)
//                   (quantize_per_tensor_fp8.cu:38-86, quantize_int8.cu:47-101)
//   k_cast_tensor   per-tensor cast on the same persistent grid (the two-pass
//                   path for smaller or unaligned x): each workgroup
//                   issues its first 16-byte loads, reduces the partial maxima
//                   (L2-resident) to inv meanwhile, then 8-byte packed stores;
//                   workgroup 0 writes the scale
//                   (quantize_per_tensor_fp8.cu:88-132, quantize_int8.cu:103-166)
//   k_rows_sub      fused single-pass quant of rows of 8..2048 elements: each
//                   row is owned by a power-of-two group of lanes, reduced
//                   with DPP and cast from registers (per-group
//                   quantize_int8.cu:307-371, short per-channel rows :173-297)
//   k_rows_wg       fused single-pass quant of rows of 4096..16384 elements,
//                   one workgroup per row held in registers (per-channel)
//   k_rows_sub_any  rows / groups of any multiple of 8 below 4096 elements
//                   without a fixed-shape kernel (k_rows_sub's layout with
//                   masked chunk slots)
//   k_rows_sub_any1 the same layout with element loads, for rows / groups of
//                   up to 2048 elements that 16-byte loads cannot take
//   k_rows_generic  row lengths no kernel above takes (two passes over the
//                   row; the second read hits L2); aligned rows of 512 to
//                   8192 chunks of 8 elements take k_chan_wg (below) instead
//   k_rows_split_max / k_rows_split_cast
//                   few long rows (fewer than about two per CU): each row cut
//                   into slices over the CUs, one partial maximum per slice
//                   in the workspace, then the cast of each slice
//   k_quant_cols_1pass
//                   per-column (axis 1) quant in one launch for rows of 8192,
//                   16384 or 32768 elements and x of 2^22 elements up to
//                   480 MiB: k_quant_tensor_1pass's step layout with running
//                   column maxima per thread, then two grid-wide exchanges
//                   (partial column maxima; each workgroup's slice of
//                   multipliers) and the cast from registers / LDS
//   k_colmax / k_col_finalize / k_cast_cols
//                   per-column (axis 1) quant otherwise: partial column
//                   maxima per row block, one finalize pass, then the cast
//                   with each thread's eight column multipliers held in
//                   registers
//   k_colmax_narrow / k_cast_cols_narrow
//                   the same for rows of at most 1024 columns: several rows
//                   per workgroup pass, so every thread has a chunk
//   k_colmax_narrow1 / k_cast_cols_narrow1
//                   the same with one element per thread, for rows of at
//                   most 128 columns that 16-byte loads cannot take
//   k_chan_wg       per-channel quant of an N-D tensor seen as
//                   [outer, channels, inner] in one pass: one workgroup per
//                   channel holding its outer segments (512 .. 65536
//                   elements, inner % 8 == 0) in registers
//   k_segmax / k_chan_finalize
//                   the same channels when they do not fit k_chan_wg:
//                   per-channel maxima with inner >= 512, one wave per
//                   contiguous run, then the maximum over outer (the cast is
//                   k_cast_cols with inner columns per channel; shorter runs
//                   take k_colmax). The reference supports ch_axis = 0 only.
//   k_group_tile    groups along a non-last axis in place (the reference moves
//                   the axis last with two copies, quantizers.py:122-132):
//                   a workgroup holds one group x 512 inner positions in
//                   registers, one pass over x
//   k_group_strided the same for inner % 8 != 0 or unaligned buffers
//
// Numerics: see cbq_device.h. Every kernel guards its indices against the
// sizes it is given; the entry points check shapes, dtypes and alignment.
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "cbq_device.h"
#include "cbq_host.h"

namespace cbq {
namespace {

#ifndef CBQ_TENSOR_WG_PER_CU
#define CBQ_TENSOR_WG_PER_CU 8
#endif
constexpr int kU = 4;                 // 8-element chunks in flight per thread
constexpr int kTensorWgPerCu = CBQ_TENSOR_WG_PER_CU;   // persistent grid per CU
constexpr int kMaxTensorWg = 2048;    // cap on that grid (= partial maxima)

// ---------------------------------------------------------------------------
// Per tensor
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kBlock) void k_amax_tensor(
    const void* __restrict__ x, int64_t n, int vec, float* __restrict__ partial) {
  __shared__ float red[kBlock / kWave];
  float m = 0.0f;
  if (vec) {
    const int64_t n8 = n >> 3;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kU * kBlock;
    for (int64_t c0 = static_cast<int64_t>(blockIdx.x) * kU * kBlock + threadIdx.x; c0 < n8;
         c0 += step) {
      Raw8<DT> r[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
        if (c < n8) r[u] = ld8<DT, (CBQ_NT_LOADS_AMAX != 0)>(x, c * 8);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
        if (c < n8) {
          float f[8];
          cvt8<DT>(r[u], f);
          m = absmax8(f, m);
        }
      }
    }
    if (blockIdx.x == 0) {
      const int64_t i = n8 * 8 + threadIdx.x;   // the < 8 trailing elements
      if (i < n) m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, i)));
    }
  } else {
    const int64_t step = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += step)
      m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, i)));
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Maximum of the nparts partial maxima -> inv; every thread gets it.
__device__ __forceinline__ float reduce_partials(const float* __restrict__ partial, int nparts,
                                                 float* red) {
  float m = 0.0f;
  for (int i = threadIdx.x; i < nparts; i += kBlock) m = fmaxf(m, partial[i]);
  return block_max(m, red);
}

// Persistent grid (the amax pass's): each workgroup issues its first chunk
// loads, reduces the partial maxima (<= kMaxTensorWg floats, L2-resident) to
// inv while they are in flight, then strides over the tensor. Measured on
// MI355X, a full grid is slower here: every one of its workgroups pays the
// partial reduction.
template <int DT, bool FP8>
__global__ __launch_bounds__(kBlock) void k_cast_tensor(
    const void* __restrict__ x, int64_t n, int vec, const float* __restrict__ partial,
    int nparts, float eps, uint8_t* __restrict__ q, float* __restrict__ scale_out) {
  __shared__ float red[kBlock / kWave];
  constexpr float kQ = FP8 ? kQmaxFp8 : kQmaxInt8;
  if (vec) {
    const int64_t n8 = n >> 3;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kU * kBlock;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * kU * kBlock + threadIdx.x;
    Raw8<DT> r[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t c = first + static_cast<int64_t>(u) * kBlock;
      if (c < n8) r[u] = ld8<DT>(x, c * 8);
    }
    const float inv = inv_scale(reduce_partials(partial, nparts, red), eps, kQ);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = 1.0f / inv;
    for (int64_t c0 = first; c0 < n8; c0 += step) {
      if (c0 != first) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
          if (c < n8) r[u] = ld8<DT>(x, c * 8);
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
        if (c < n8) {
          float f[8];
          cvt8<DT>(r[u], f);
          stg8(q + c * 8, FP8 ? pack8_fp8(f, inv) : pack8_int8(f, inv));
        }
      }
    }
    if (blockIdx.x == 0) {
      const int64_t i = n8 * 8 + threadIdx.x;   // the < 8 trailing elements
      if (i < n) {
        const float v = ld1<DT>(x, i) * inv;
        q[i] = FP8 ? q_fp8_1(v) : static_cast<uint8_t>(q_int8(v));
      }
    }
  } else {
    const float inv = inv_scale(reduce_partials(partial, nparts, red), eps, kQ);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = 1.0f / inv;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += step) {
      const float v = ld1<DT>(x, i) * inv;
      q[i] = FP8 ? q_fp8_1(v) : static_cast<uint8_t>(q_int8(v));
    }
  }
}

// ---------------------------------------------------------------------------
// Per tensor in one launch. A resident grid of one 1024-thread workgroup per
// CU reads x once in grid-stride steps (4 chunks of 16 bytes per thread and
// step: measured on MI355X, deeper load pipelines read 15-25% slower),
// keeping the last HOLD_STEPS steps of each thread in registers; the
// workgroups exchange their maxima through the workspace's control block;
// then each casts its held chunks from registers and re-reads only the steps
// that did not fit (x beyond 96 MiB of 2-byte elements, 48 MiB of fp32).
// HBM traffic: 2N + N bytes up to that size, against 2N + 2N + N for the
// amax + cast passes above.
//
// Step i of workgroup b covers the 4096 consecutive chunks starting at chunk
// (i * gridDim.x + b) * 4096, lane t of the workgroup taking chunks + t,
// + 1024 + t, + 2048 + t, + 3072 + t (one 64-byte-per-lane stretch of 16 KiB
// per workgroup and step, the whole grid covering 16 MiB of x per step).
//
// Exchange (no atomics: same-address device atomics serialize at ~25 ns each
// on MI355X, 6 us for one per workgroup). Control block layout, bytes:
//   0      gen      tag of the last call whose exchange completed (low 32
//                   bits of a 64-bit word; 0 in a zero-filled block)
//   512    status   sticky int32 for the caller: 1 once a workgroup of any
//                   call gave up waiting (cleared only by the caller)
//   520    suspect  tag of the last call in which a workgroup gave up
//   1024   slot[b]  64-bit per workgroup: tag << 32 | its |x| maximum (bits)
// A call's tag is gen + 1 (skipping 0, the tag of a zero-filled slot). Each
// workgroup reads gen when it starts, publishes its slot (and refreshes the
// slots b + G, b + 2G, ... beyond the grid, so that no slot ever holds a tag
// older than the previous call's), and polls slots [0, G) until every tag is
// the call's. Only a workgroup whose wait completed advances gen (workgroup
// 0 normally): a completed wait proves that every workgroup has read gen, so
// every workgroup of a call uses the same tag, and the next call (stream
// order: it starts after this one has ended) uses a tag no slot carries.
//
// A wait gives up after spin_limit polls (only possible when the grid is not
// resident at once, e.g. other work holding CUs for about a second). Then the
// workgroup stores suspect = tag and status = 1, waits for both stores, and
// polls once more:
//  * if every slot now carries the tag, it goes on as a completed wait;
//  * otherwise it gives up: its codes are NaN (INT8: 0) and it writes a NaN
//    scale. Some slot j was missing at that final poll, so workgroup j
//    published after the suspect store, and every completed wait of the call
//    (each must see slot j) reads suspect == tag afterwards. Those
//    workgroups advance gen (the last workgroup to publish always completes,
//    so gen always advances), and workgroup 0 returns NaN, so the scale is
//    NaN whenever any workgroup gave up.
// A scale that is not NaN therefore comes with every code exact. Later calls
// are exact again without any reset; status tells the caller that a call
// since it last cleared the word was touched by a timeout.
// ---------------------------------------------------------------------------
constexpr int kFusedBlock = 1024;                // 16 waves: four per SIMD
constexpr int kFusedU = 4;                       // chunks per thread and step
constexpr int64_t kFusedMinElems = int64_t(1) << 20;
constexpr uint32_t kFusedSpinLimit = 1u << 20;   // polls (each >= one memory round trip)
constexpr int kCtlGen = 0, kCtlStatus = 512, kCtlSuspect = 520, kCtlSlots = 1024;
constexpr int kMaxFusedGrid = (CBQ_WS_CTRL_BYTES - kCtlSlots) / 8;

// Steps held in registers: 24 chunks (96 VGPRs) of 2-byte input, 12 of fp32.
template <int DT> constexpr int fused_hold_steps() { return DT == kF32 ? 3 : 6; }
// The first streamed steps are parked in LDS (128 KiB of a workgroup's
// 160 KiB): two steps of 2-byte input, one of fp32. With the registers, a
// 2-byte x of up to 128 MiB (fp32: 80 MiB) is read from HBM exactly once.
constexpr int kFusedLdsBytes = 128 * 1024;
template <int DT>
constexpr int fused_lds_steps() {
  return kFusedLdsBytes / (kFusedBlock * kFusedU * 8 * elem_bytes<DT>());
}

// Chunk loads and code stores addressed as a wave-uniform base plus a 32-bit
// per-thread offset (keeps one offset register per thread instead of one
// address pair per held chunk).
template <int DT>
__device__ __forceinline__ Raw8<DT> ld8_at(const char* base, uint32_t off) {
  Raw8<DT> r;
  r.a = ldg16(base + off);
  if constexpr (DT == kF32) r.b = ldg16(base + off + 16);
  return r;
}

template <int DT, bool FP8>
__device__ __forceinline__ void cast_store8(const Raw8<DT>& r, float inv, uint8_t* base,
                                            uint32_t off) {
  float f[8];
  cvt8<DT>(r, f);
  stg8(base + off, FP8 ? pack8_fp8(f, inv) : pack8_int8(f, inv));
}

// Buffer resources for the held steps: num_records bounds each access, so a
// chunk past the end of x reads as zeros and its code store is dropped by the
// hardware, without branches (a guarded load would make the compiler wait
// for every outstanding load where the branch rejoins).

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  const int nr = bytes <= 0 ? 0 : static_cast<int>(bytes);   // callers pass <= 128 KiB
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nr, kBufDword3);
}

template <int DT>
__device__ __forceinline__ Raw8<DT> ld8_buf(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  Raw8<DT> r;
  const u32x4 a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rs, off, 0, CBQ_NT_LOADS ? kAuxNT : 0));
  r.a = make_uint4(a.x, a.y, a.z, a.w);
  if constexpr (DT == kF32) {
    const u32x4 b = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rs, off + 16, 0, CBQ_NT_LOADS ? kAuxNT : 0));
    r.b = make_uint4(b.x, b.y, b.z, b.w);
  }
  return r;
}

template <int DT, bool FP8>
__device__ __forceinline__ void cast_store8_buf(const Raw8<DT>& r, float inv,
                                                __amdgpu_buffer_rsrc_t rs, uint32_t off) {
  float f[8];
  cvt8<DT>(r, f);
  const uint2 c = FP8 ? pack8_fp8(f, inv) : pack8_int8(f, inv);
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, u32x2{c.x, c.y}), rs, off, 0,
                                        CBQ_NT_STORES_NARROW ? kAuxNT : 0);
}

// Grid-wide maximum of the workgroups' m (see the exchange above); NaN in a
// workgroup that gave up waiting, and in workgroup 0 of a call in which any
// workgroup did. Every thread of the workgroup gets the result.
__device__ float grid_max_exchange(float m, char* ctl, uint32_t spin_limit, float* red) {
  __shared__ uint32_t s_tag;
  __shared__ int s_nan;
  auto* gen_w = reinterpret_cast<unsigned long long*>(ctl + kCtlGen);
  auto* status = reinterpret_cast<unsigned int*>(ctl + kCtlStatus);
  auto* suspect = reinterpret_cast<unsigned int*>(ctl + kCtlSuspect);
  auto* slots = reinterpret_cast<unsigned long long*>(ctl + kCtlSlots);
  const int G = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  if (threadIdx.x == 0) {
    const uint32_t g = static_cast<uint32_t>(
        __hip_atomic_load(gen_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const uint32_t tag = g + 1 == 0 ? 1u : g + 1;
    s_tag = tag;
    __hip_atomic_store(slots + b,
                       (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(m),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);   // the slot store has been performed before any poll
  }
  __syncthreads();
  const uint32_t tag = s_tag;
  const unsigned long long mine = (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(m);
  for (int k = static_cast<int>(threadIdx.x) + 1; b + static_cast<int64_t>(k) * G < kMaxFusedGrid;
       k += static_cast<int>(blockDim.x))   // slots beyond the grid: refreshed, never read
    __hip_atomic_store(slots + b + k * G, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  auto poll = [&](float& mx) {
    int ok = 1;
    mx = 0.0f;
    for (int i = threadIdx.x; i < G; i += blockDim.x) {
      const unsigned long long v = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok &= static_cast<uint32_t>(v >> 32) == tag;
      mx = fmaxf(mx, __uint_as_float(static_cast<uint32_t>(v)));
    }
    return __syncthreads_and(ok);
  };
  uint32_t spins = 0;
  float mx;
  int ok;
  for (;;) {
    ok = poll(mx);
    if (ok || spins >= spin_limit) break;
    ++spins;
    __builtin_amdgcn_s_sleep(2);
  }
  if (!ok) {
    if (threadIdx.x == 0) {
      __hip_atomic_store(suspect, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);   // both performed before the final poll
    }
    __syncthreads();
    ok = poll(mx);
  }
  if (threadIdx.x == 0) {
    int nan = !ok;
    if (ok) {
      const uint32_t sp = __hip_atomic_load(suspect, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (sp == tag) {
        // a workgroup of this call gave up: make sure gen advances, and let
        // workgroup 0 write a NaN scale
        __hip_atomic_store(gen_w, static_cast<unsigned long long>(tag), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        nan = b == 0;
      } else if (b == 0) {
        __hip_atomic_store(gen_w, static_cast<unsigned long long>(tag), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (sp != 0) {   // an earlier call's record: clear it unless a workgroup of this call
                         // has just replaced it
          uint32_t expect = sp;
          __hip_atomic_compare_exchange_strong(suspect, &expect, 0u, __ATOMIC_RELAXED,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    s_nan = nan;
  }
  mx = block_max(mx, red);   // contains a barrier: s_nan is visible after it
  return s_nan ? __builtin_nanf("") : mx;
}

template <int DT, bool FP8>
__global__ __launch_bounds__(kFusedBlock) void k_quant_tensor_1pass(
    const void* __restrict__ x, int64_t n, float eps, uint8_t* __restrict__ q,
    float* __restrict__ scale_out, char* __restrict__ ctl, uint32_t spin_limit) {
  constexpr int U = kFusedU;
  constexpr int HS = fused_hold_steps<DT>();
  constexpr int LS = fused_lds_steps<DT>();
  constexpr int EB = 8 * elem_bytes<DT>();            // bytes of x per chunk
  constexpr int QW = EB / 16;                         // 16-byte words per chunk
  constexpr float kQ = FP8 ? kQmaxFp8 : kQmaxInt8;
  __shared__ float red[kFusedBlock / kWave];
  // parked steps: word w of chunk (i, u) of lane t at ((i * U + u) * QW + w) * B + t
  __shared__ u32x4 park[LS * U * QW * kFusedBlock];

  const int64_t SB = static_cast<int64_t>(kFusedBlock) * U;   // chunks per workgroup and step
  const int64_t GS = static_cast<int64_t>(gridDim.x) * SB;    // chunks per grid step
  const int64_t n8 = n >> 3;
  const int64_t I = (n8 + GS - 1) / GS;               // steps
  const int64_t held0 = I > HS ? I - HS : 0;          // first held step; earlier steps are full
  // chunk (i, u) = i * GS + b * SB + u * kFusedBlock + t: a wave-uniform part
  // (the bases below plus i * GS + u * kFusedBlock) and the lane's t.
  const char* xw = static_cast<const char*>(x) + static_cast<int64_t>(blockIdx.x) * SB * EB;
  uint8_t* qw = q + static_cast<int64_t>(blockIdx.x) * SB * 8;
  const uint32_t xo = threadIdx.x * EB, qo = threadIdx.x * 8;

  // Pass 1: |x| max; streamed steps first (the first LS of them parked in
  // LDS), then the held steps into r[].
  float m = 0.0f;
  for (int64_t i = 0; i < held0; ++i) {
    Raw8<DT> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld8_at<DT>(xw + (i * GS + u * kFusedBlock) * EB, xo);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float f[8];
      cvt8<DT>(v[u], f);
      m = absmax8(f, m);
    }
    if (i < LS) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        u32x4* pk = park + (static_cast<int>(i) * U + u) * QW * kFusedBlock + threadIdx.x;
        pk[0] = u32x4{v[u].a.x, v[u].a.y, v[u].a.z, v[u].a.w};
        if constexpr (DT == kF32) pk[kFusedBlock] = u32x4{v[u].b.x, v[u].b.y, v[u].b.z, v[u].b.w};
      }
    }
  }
  // Held steps through buffer resources bounded at the end of x (the
  // workgroup's part of a step: SB chunks from chunk c0 + b * SB).
  // Steps wholly past the end (the workgroup's part starts at or after chunk
  // n8) are skipped with a workgroup-uniform branch.
  const int64_t cb = static_cast<int64_t>(blockIdx.x) * SB;
  Raw8<DT> r[HS * U];
#pragma unroll
  for (int k = 0; k < HS; ++k) {
    const int64_t c0 = (held0 + k) * GS + cb;
    const int64_t left = n8 - c0;                     // chunks of x from the step's base
    // one step's loads in flight at a time (the scheduler would otherwise
    // hoist the loads of every held step)
    __builtin_amdgcn_sched_barrier(0);
    if (left > 0) {
      const auto rs = rsrc(static_cast<const char*>(x) + c0 * EB, (left < SB ? left : SB) * EB);
#pragma unroll
      for (int u = 0; u < U; ++u) r[k * U + u] = ld8_buf<DT>(rs, u * kFusedBlock * EB + xo);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float f[8];
        cvt8<DT>(r[k * U + u], f);
        m = absmax8(f, m);
      }
    }
  }
  float tail = 0.0f;                                  // the < 8 trailing elements
  if (blockIdx.x == 0 && threadIdx.x < 8 && n8 * 8 + threadIdx.x < n) {
    tail = ld1<DT>(x, n8 * 8 + threadIdx.x);
    m = fmaxf(m, __builtin_fabsf(tail));
  }
  // Pass 2 converts the held chunks again from their raw words (keeping the
  // first conversion live would take 8 registers per chunk instead of 4).
#pragma unroll
  for (int j = 0; j < HS * U; ++j) reload_barrier<DT>(r[j]);
  const float amax = grid_max_exchange(block_max(m, red), ctl, spin_limit, red);
  const float inv = amax == amax ? inv_scale(amax, eps, kQ) : amax;
  if (threadIdx.x == 0 && (blockIdx.x == 0 || inv != inv)) *scale_out = 1.0f / inv;

  // Pass 2: cast the held steps from registers, then the parked ones from
  // LDS, then re-read the others.
#pragma unroll
  for (int k = 0; k < HS; ++k) {
    const int64_t c0 = (held0 + k) * GS + cb;
    const int64_t left = n8 - c0;
    if (left > 0) {
      const auto rs = rsrc(q + c0 * 8, (left < SB ? left : SB) * 8);
#pragma unroll
      for (int u = 0; u < U; ++u)
        cast_store8_buf<DT, FP8>(r[k * U + u], inv, rs, u * kFusedBlock * 8 + qo);
    }
  }
  const int64_t parked = held0 < LS ? held0 : LS;
  for (int64_t i = 0; i < parked; ++i) {            // each lane reads back its own words
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const u32x4* pk = park + (static_cast<int>(i) * U + u) * QW * kFusedBlock + threadIdx.x;
      Raw8<DT> v;
      const u32x4 a = pk[0];
      v.a = make_uint4(a.x, a.y, a.z, a.w);
      if constexpr (DT == kF32) {
        const u32x4 b = pk[kFusedBlock];
        v.b = make_uint4(b.x, b.y, b.z, b.w);
      }
      cast_store8<DT, FP8>(v, inv, qw + (i * GS + u * kFusedBlock) * 8, qo);
    }
  }
  for (int64_t i = parked; i < held0; ++i) {
    Raw8<DT> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld8_at<DT>(xw + (i * GS + u * kFusedBlock) * EB, xo);
#pragma unroll
    for (int u = 0; u < U; ++u)
      cast_store8<DT, FP8>(v[u], inv, qw + (i * GS + u * kFusedBlock) * 8, qo);
  }
  if (blockIdx.x == 0 && threadIdx.x < 8 && n8 * 8 + threadIdx.x < n) {
    const float v = tail * inv;
    q[n8 * 8 + threadIdx.x] = FP8 ? q_fp8_1(v) : static_cast<uint8_t>(q_int8(v));
  }
}

// ---------------------------------------------------------------------------
// Per column (axis 1) in one launch, for rows of 8192, 16384 or 32768
// elements (c8 = cols / 8 = 1024 CPT chunks, CPT = 1, 2 or 4) and x of up to
// CBQ_COLS_1PASS_MAX_BYTES (the host checks both). The step
// layout of k_quant_tensor_1pass: a resident grid of G workgroups (a power
// of two) reads x once in grid-wide steps of G x 4096 chunks, holding the
// last HS steps of each thread in registers and parking the first LS streamed
// steps in LDS (128 MiB of 2-byte x in all on 256 CUs); since a step starts
// at a multiple of c8 chunks, chunk u of thread t is always of chunk-column
// t + 1024 (u % CPT), so each thread keeps the running |x| maxima of its CPT
// chunk-columns (8 columns each). Then two grid-wide exchanges through the
// workspace:
//  1. every workgroup stores its [cols] partial maxima (part[b], in planes
//     of 64-bit words: a wave's stores cover 512 contiguous bytes; with
//     8-byte stores 32 bytes apart the exchange ran at under 1 TB/s; 16-bit
//     values of the input dtype for 2-byte input, see st8_max) and
//     publishes its slot with tag T1; once every slot carries T1 (or T2),
//     workgroup b reduces the partials of its slice of c8 / G chunk-columns
//     (<= 16) over all G workgroups, stores the slice's multipliers inv[c] =
//     fp32(127 / max(amax_c, eps)) and publishes T2;
//  2. once every slot carries T2, every thread loads the multipliers of its
//     chunk-columns and casts its held steps from registers, the parked ones
//     from LDS, and re-reads the rest; workgroup b writes its slice's scales.
// HBM traffic 2N (+ the re-read beyond 128 MiB) + N + the partial maxima
// (2 G cols bytes for 2-byte input, 4 G cols for fp32, each written and read
// once), against 2N + 2N + N for k_colmax + k_cast_cols.
//
// Tags and timeouts follow the per-tensor exchange (the same control block:
// gen, status, suspect, slots). T1 = gen + 1 and T2 = T1 + 1 (skipping 0);
// only a workgroup whose second wait completed advances gen (workgroup 0, or
// any of them once suspect holds T1 or T2). A workgroup that gives up on the
// first wait publishes NaN multipliers for its slice (so those columns get a
// NaN scale and 0 codes everywhere); one that gives up on the second writes 0
// codes, and then every workgroup that completes the second wait finds
// suspect == T2 and writes NaN scales. A scale that is not NaN therefore
// comes with every code of its column exact.
// ---------------------------------------------------------------------------
constexpr int kColsMaxSlice = 16;   // chunk-columns per workgroup in the slice reduction
constexpr int64_t kColsMinElems = int64_t(1) << 22;
// Largest x (bytes) the one-launch column path takes; larger ones take
// k_colmax + k_cast_cols. Measured on MI355X (bf16, cols 8192, op time after
// a cache sweep, one-launch against two-pass, same process): 64 MiB 32.6 /
// 37.8 us, 128 MiB 48.4 / 62.4, 256 MiB 101.6 / 112.2, 384 MiB 154.2 /
// 159.3, 448 MiB 182.2 / 184.0, 576 MiB 235.7 / 232.9 us: past what
// registers and LDS hold (128 MiB) the re-read of the rest and the exchange
// cost about what the single read saves. A compile-time tuning knob.
#ifndef CBQ_COLS_1PASS_MAX_BYTES
#define CBQ_COLS_1PASS_MAX_BYTES (int64_t(480) << 20)
#endif

// Steps held in registers: those of k_quant_tensor_1pass, less what the CPT
// chunk-columns' 8 maxima (then multipliers) per thread take.
template <int DT, int CPT>
constexpr int cols_hold_steps() {
  return DT == kF32 ? (CPT == 1 ? 3 : CPT == 2 ? 2 : 1) : (CPT == 1 ? 6 : CPT == 2 ? 5 : 3);
}

__device__ __forceinline__ uint32_t next_tag(uint32_t g) { return g + 1 == 0 ? 1u : g + 1; }

// Agent-scope 64-bit accesses (coherent across the XCDs' L2s, like the
// slots) to the exchange arrays, which hold 8 floats per chunk-column as 4
// planes of pairs: element (i, c) = floats 2i, 2i + 1 of chunk-column c, so
// that the 64 lanes of a wave (consecutive c) access 512 contiguous bytes.
__device__ __forceinline__ void ld8_pairs(const unsigned long long* p, int64_t plane,
                                          int64_t c, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned long long d =
        __hip_atomic_load(p + i * plane + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v[2 * i] = __uint_as_float(static_cast<uint32_t>(d));
    v[2 * i + 1] = __uint_as_float(static_cast<uint32_t>(d >> 32));
  }
}

__device__ __forceinline__ void st8_pairs(unsigned long long* p, int64_t plane, int64_t c,
                                          const float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    __hip_atomic_store(p + i * plane + c,
                       static_cast<unsigned long long>(__float_as_uint(v[2 * i])) |
                           (static_cast<unsigned long long>(__float_as_uint(v[2 * i + 1])) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The column maxima of one chunk-column (8 columns) as they cross the
// exchange: for 2-byte input as the input dtype's 16-bit values, 4 per
// 64-bit word in 2 planes (each maximum is the absolute value of an input
// element, so it is exact in that dtype; half the bytes of fp32), for fp32
// input as fp32 pairs in 4 planes.
template <int DT> constexpr int max_planes() { return DT == kF32 ? 4 : 2; }

template <int DT>
__device__ __forceinline__ uint32_t max_to16(float f) {
  if constexpr (DT == kBF16) return __float_as_uint(f) >> 16;
  else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT>
__device__ __forceinline__ float max_from16(uint32_t h) {
  if constexpr (DT == kBF16) return __uint_as_float(h << 16);
  else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

template <int DT>
__device__ __forceinline__ void st8_max(unsigned long long* p, int64_t plane, int64_t c,
                                        const float (&v)[8]) {
  if constexpr (DT == kF32) {
    st8_pairs(p, plane, c, v);
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      unsigned long long w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w |= static_cast<unsigned long long>(max_to16<DT>(v[4 * i + j])) << (16 * j);
      __hip_atomic_store(p + i * plane + c, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int DT>
__device__ __forceinline__ void ld8_max(const unsigned long long* p, int64_t plane, int64_t c,
                                        float (&v)[8]) {
  if constexpr (DT == kF32) {
    ld8_pairs(p, plane, c, v);
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const unsigned long long w =
          __hip_atomic_load(p + i * plane + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[4 * i + j] = max_from16<DT>(static_cast<uint32_t>(w >> (16 * j)) & 0xffffu);
    }
  }
}

// Waits until every slot [0, G) carries tag or alt; after spin_limit polls
// records suspect = tag and status = 1 (both performed before it) and polls
// once more. Returns whether the wait completed (every thread gets it).
__device__ int slot_wait(char* ctl, uint32_t tag, uint32_t alt, uint32_t spin_limit) {
  auto* slots = reinterpret_cast<unsigned long long*>(ctl + kCtlSlots);
  const int G = static_cast<int>(gridDim.x);
  auto poll = [&]() {
    int ok = 1;
    for (int i = threadIdx.x; i < G; i += blockDim.x) {
      const uint32_t t = static_cast<uint32_t>(
          __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32);
      ok &= (t == tag) | (t == alt);
    }
    return __syncthreads_and(ok);
  };
  uint32_t spins = 0;
  int ok;
  for (;;) {
    ok = poll();
    if (ok || spins >= spin_limit) break;
    ++spins;
    __builtin_amdgcn_s_sleep(2);
  }
  if (!ok) {
    if (threadIdx.x == 0) {
      __hip_atomic_store(reinterpret_cast<unsigned int*>(ctl + kCtlSuspect), tag, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(reinterpret_cast<unsigned int*>(ctl + kCtlStatus), 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    ok = poll();
  }
  return ok;
}

// Thread 0 publishes the workgroup's slot with tag (after the workgroup's
// data stores, which every thread has waited for before the barrier that
// precedes this call); with refresh, the slots b + G, b + 2G, ... beyond the
// grid too (by the whole workgroup).
__device__ __forceinline__ void slot_publish(char* ctl, uint32_t tag, bool refresh) {
  auto* slots = reinterpret_cast<unsigned long long*>(ctl + kCtlSlots);
  const int G = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
  const unsigned long long v = static_cast<unsigned long long>(tag) << 32;
  if (threadIdx.x == 0) {
    __hip_atomic_store(slots + b, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
  }
  if (refresh)
    for (int k = static_cast<int>(threadIdx.x) + 1; b + static_cast<int64_t>(k) * G < kMaxFusedGrid;
         k += static_cast<int>(blockDim.x))
      __hip_atomic_store(slots + b + k * G, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
}

template <int DT, int CPT>
__device__ __forceinline__ void colmax8(const Raw8<DT>& r, float (&m)[8]) {
  float f[8];
  cvt8<DT>(r, f);
#pragma unroll
  for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], __builtin_fabsf(f[e]));
}

template <int DT>
__device__ __forceinline__ uint2 cast8_cols(const Raw8<DT>& r, const float (&inv)[8]) {
  float f[8];
  cvt8<DT>(r, f);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] *= inv[e];
  return pack8_int8(f, 1.0f);   // x 1: exact
}

template <int DT, int CPT>
__global__ __launch_bounds__(kFusedBlock) void k_quant_cols_1pass(
    const void* __restrict__ x, int64_t n8, float eps, int8_t* __restrict__ q,
    float* __restrict__ scale_out, char* __restrict__ ctl, float* __restrict__ part,
    float* __restrict__ invs, uint32_t spin_limit) {
  constexpr int U = kFusedU;
  constexpr int HS = cols_hold_steps<DT, CPT>();
  constexpr int LS = fused_lds_steps<DT>();
  constexpr int EB = 8 * elem_bytes<DT>();            // bytes of x per chunk
  constexpr int QW = EB / 16;                         // 16-byte words per chunk
  constexpr int C8 = 1024 * CPT;                      // chunk-columns
  static_assert(U % CPT == 0, "chunk u of a thread is of chunk-column t + 1024 (u % CPT)");
  __shared__ u32x4 park[LS * U * QW * kFusedBlock];
  __shared__ float red[(kFusedBlock / kWave) * kColsMaxSlice * 8];
  __shared__ uint32_t s_t1;
  __shared__ int s_nan;

  const int G = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
  const int t = static_cast<int>(threadIdx.x), lane = t % kWave, wave = t / kWave;
  auto* gen_w = reinterpret_cast<unsigned long long*>(ctl + kCtlGen);
  auto* suspect = reinterpret_cast<unsigned int*>(ctl + kCtlSuspect);
  if (t == 0)
    s_t1 = next_tag(static_cast<uint32_t>(
        __hip_atomic_load(gen_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));

  const int64_t SB = static_cast<int64_t>(kFusedBlock) * U;   // chunks per workgroup and step
  const int64_t GS = static_cast<int64_t>(G) * SB;            // chunks per grid step
  const int64_t I = (n8 + GS - 1) / GS;
  const int64_t held0 = I > HS ? I - HS : 0;
  const char* xw = static_cast<const char*>(x) + static_cast<int64_t>(b) * SB * EB;
  int8_t* qw = q + static_cast<int64_t>(b) * SB * 8;
  const uint32_t xo = t * EB, qo = t * 8;

  // Pass 1: column maxima; streamed steps (the first LS parked), then the
  // held steps into r[].
  float m[CPT][8];
#pragma unroll
  for (int s = 0; s < CPT; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) m[s][e] = 0.0f;
  for (int64_t i = 0; i < held0; ++i) {
    Raw8<DT> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld8_at<DT>(xw + (i * GS + u * kFusedBlock) * EB, xo);
#pragma unroll
    for (int u = 0; u < U; ++u) colmax8<DT, CPT>(v[u], m[u % CPT]);
    if (i < LS) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        u32x4* pk = park + (static_cast<int>(i) * U + u) * QW * kFusedBlock + t;
        pk[0] = u32x4{v[u].a.x, v[u].a.y, v[u].a.z, v[u].a.w};
        if constexpr (DT == kF32) pk[kFusedBlock] = u32x4{v[u].b.x, v[u].b.y, v[u].b.z, v[u].b.w};
      }
    }
  }
  const int64_t cb = static_cast<int64_t>(b) * SB;
  Raw8<DT> r[HS * U];
#pragma unroll
  for (int k = 0; k < HS; ++k) {
    const int64_t c0 = (held0 + k) * GS + cb;
    const int64_t left = n8 - c0;
    __builtin_amdgcn_sched_barrier(0);
    if (left > 0) {
      const auto rs = rsrc(static_cast<const char*>(x) + c0 * EB, (left < SB ? left : SB) * EB);
#pragma unroll
      for (int u = 0; u < U; ++u) r[k * U + u] = ld8_buf<DT>(rs, u * kFusedBlock * EB + xo);
#pragma unroll
      for (int u = 0; u < U; ++u) colmax8<DT, CPT>(r[k * U + u], m[u % CPT]);
    }
  }
#pragma unroll
  for (int j = 0; j < HS * U; ++j) reload_barrier<DT>(r[j]);

  // Exchange 1: this workgroup's partial maxima (part: [G][NP planes][C8]
  // words), then tag T1.
  constexpr int NP = max_planes<DT>();
  auto* part64 = reinterpret_cast<unsigned long long*>(part);
  auto* inv64 = reinterpret_cast<unsigned long long*>(invs);   // [4 planes][C8] pairs
#pragma unroll
  for (int s = 0; s < CPT; ++s)
    st8_max<DT>(part64 + static_cast<int64_t>(b) * NP * C8, C8, t + 1024 * s, m[s]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const uint32_t T1 = s_t1, T2 = next_tag(T1);
  slot_publish(ctl, T1, false);
  const int ok1 = slot_wait(ctl, T1, T2, spin_limit);

  // Slice reduction: chunk-columns [b SCC, b SCC + SCC) over the G partials.
  // Thread t takes chunk-column cc = t % SCC of partials (t + 1024 j) / SCC,
  // then the lanes of a wave with the same cc combine (xor shuffles), then
  // the waves through LDS.
  const int SCC = C8 / G;                             // power of two, <= kColsMaxSlice
  const int cc = t & (SCC - 1);
  float sm[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sm[e] = 0.0f;
  if (ok1) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int p = (t + 1024 * j) / SCC;             // < G: G * SCC = C8 = 1024 CPT
      float v[8];
      ld8_max<DT>(part64 + static_cast<int64_t>(p) * NP * C8, C8, b * SCC + cc, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) sm[e] = fmaxf(sm[e], v[e]);
    }
  }
  for (int o = SCC; o < kWave; o <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) sm[e] = fmaxf(sm[e], __shfl_xor(sm[e], o));
  if (lane < SCC) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[(wave * SCC + lane) * 8 + e] = sm[e];
  }
  __syncthreads();
  float inv_mine = 0.0f;                              // thread t < 8 SCC: column 8 (b SCC) + t
  if (t < 8 * SCC) {
    float mx = 0.0f;
    for (int w = 0; w < kFusedBlock / kWave; ++w) mx = fmaxf(mx, red[(w * SCC + (t >> 3)) * 8 + (t & 7)]);
    inv_mine = ok1 ? inv_scale(mx, eps, kQmaxInt8) : __builtin_nanf("");
    // column 8 (b SCC + t / 8) + t % 8: plane (t % 8) / 2, half t % 2 of the pair
    __hip_atomic_store(reinterpret_cast<unsigned int*>(inv64 + ((t & 7) >> 1) * C8 + b * SCC + (t >> 3)) +
                           (t & 1),
                       __float_as_uint(inv_mine), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  slot_publish(ctl, T2, true);
  const int ok2 = slot_wait(ctl, T2, T2, spin_limit);
  if (t == 0) {
    int nan = !ok2;
    if (ok2) {
      const uint32_t sp = __hip_atomic_load(suspect, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (b == 0 || sp == T1 || sp == T2)
        __hip_atomic_store(gen_w, static_cast<unsigned long long>(T2), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      nan = sp == T2;
      if (b == 0 && sp != 0 && sp != T1 && sp != T2) {   // an earlier call's record
        uint32_t expect = sp;
        __hip_atomic_compare_exchange_strong(suspect, &expect, 0u, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    s_nan = nan;
  }
  __syncthreads();
  if (t < 8 * SCC) scale_out[b * SCC * 8 + t] = s_nan ? __builtin_nanf("") : 1.0f / inv_mine;

  // Pass 2: multipliers of the thread's chunk-columns, then the cast.
  float iv[CPT][8];
#pragma unroll
  for (int s = 0; s < CPT; ++s) {
    if (ok2) {
      ld8_pairs(inv64, C8, t + 1024 * s, iv[s]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) iv[s][e] = __builtin_nanf("");
    }
  }
#pragma unroll
  for (int k = 0; k < HS; ++k) {
    const int64_t c0 = (held0 + k) * GS + cb;
    const int64_t left = n8 - c0;
    if (left > 0) {
      const auto rs = rsrc(q + c0 * 8, (left < SB ? left : SB) * 8);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint2 c = cast8_cols<DT>(r[k * U + u], iv[u % CPT]);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, u32x2{c.x, c.y}), rs,
                                              u * kFusedBlock * 8 + qo, 0,
                                              CBQ_NT_STORES_NARROW ? kAuxNT : 0);
      }
    }
  }
  const int64_t parked = held0 < LS ? held0 : LS;
  for (int64_t i = 0; i < parked; ++i) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const u32x4* pk = park + (static_cast<int>(i) * U + u) * QW * kFusedBlock + t;
      Raw8<DT> v;
      const u32x4 a = pk[0];
      v.a = make_uint4(a.x, a.y, a.z, a.w);
      if constexpr (DT == kF32) {
        const u32x4 bb = pk[kFusedBlock];
        v.b = make_uint4(bb.x, bb.y, bb.z, bb.w);
      }
      stg8(qw + (i * GS + u * kFusedBlock) * 8 + qo, cast8_cols<DT>(v, iv[u % CPT]));
    }
  }
  for (int64_t i = parked; i < held0; ++i) {
    Raw8<DT> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld8_at<DT>(xw + (i * GS + u * kFusedBlock) * EB, xo);
#pragma unroll
    for (int u = 0; u < U; ++u)
      stg8(qw + (i * GS + u * kFusedBlock) * 8 + qo, cast8_cols<DT>(v[u], iv[u % CPT]));
  }
}

// ---------------------------------------------------------------------------
// Rows (per-channel axis 0 and per-group): fused single pass
// ---------------------------------------------------------------------------

// Rows of L = LPR * VPL * 8 elements; LPR lanes own a row, each lane holding
// VPL chunks. A wave covers 64 / LPR rows per iteration and RI iterations,
// all loads issued before the first reduction.
template <int DT, int LPR, int VPL, int RI>
__global__ __launch_bounds__(kBlock) void k_rows_sub(
    const void* __restrict__ x, int64_t rows, float eps, int8_t* __restrict__ q,
    float* __restrict__ scale) {
  constexpr int RPW = kWave / LPR;
  constexpr int64_t L = static_cast<int64_t>(LPR) * VPL * 8;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int sub = lane / LPR;
  const int lr = lane % LPR;
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * (RI * RPW) + sub;

  Raw8<DT> r[RI][VPL];
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) r[it][v] = ld8<DT>(x, row * L + (v * LPR + lr) * 8);
    }
  }
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    const bool ok = row < rows;
    float f[VPL][8];
    float m = 0.0f;
    if (ok) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        cvt8<DT>(r[it][v], f[v]);
        m = absmax8(f[v], m);
      }
    }
    m = group_max<LPR>(m);   // every lane participates
    const float inv = inv_scale(m, eps, kQmaxInt8);
    if (ok) {
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        stg8(q + row * L + (v * LPR + lr) * 8, pack8_int8(f[v], inv));
      if (lr == 0) scale[row] = 1.0f / inv;
    }
  }
}

// Rows (groups) of cg chunks of 8 elements for any cg < 512 without a
// fixed-shape kernel (e.g. groups of 56, 112, 224 elements): the layout of
// k_rows_sub with LPR * VPL >= cg chunk slots per row, chunk j = v * LPR + lr
// in slot (v, lr); slots past cg load the row's first chunk (in bounds), stay
// out of the maximum and store nothing.
template <int DT, int LPR, int VPL, int RI>
__global__ __launch_bounds__(kBlock) void k_rows_sub_any(
    const void* __restrict__ x, int64_t rows, int cg, float eps, int8_t* __restrict__ q,
    float* __restrict__ scale) {
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int sub = lane / LPR;
  const int lr = lane % LPR;
  const int64_t L = static_cast<int64_t>(cg) * 8;
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * (RI * RPW) + sub;

  Raw8<DT> r[RI][VPL];
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int j = v * LPR + lr;
        r[it][v] = ld8<DT>(x, row * L + (j < cg ? j : 0) * 8);
      }
    }
  }
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    const bool ok = row < rows;
    float f[VPL][8];
    float m = 0.0f;
    if (ok) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        cvt8<DT>(r[it][v], f[v]);
        const float mv = absmax8(f[v], 0.0f);
        m = v * LPR + lr < cg ? fmaxf(m, mv) : m;
      }
    }
    m = group_max<LPR>(m);   // every lane participates
    const float inv = inv_scale(m, eps, kQmaxInt8);
    if (ok) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int j = v * LPR + lr;
        if (j < cg) stg8(q + row * L + j * 8, pack8_int8(f[v], inv));
      }
      if (lr == 0) scale[row] = 1.0f / inv;
    }
  }
}

// Rows (groups) of any length L <= 2048 that 16-byte loads cannot take (L %
// 8 != 0, e.g. groups of 100, or unaligned buffers): LPR lanes per row, VPL
// elements per lane, element j = v * LPR + lr, 2- or 4-byte loads that are
// contiguous across the lanes of a row. Slots past L load the row's first
// element, stay out of the maximum and store nothing.
template <int DT, int LPR, int VPL, int RI, int E>
__global__ __launch_bounds__(kBlock) void k_rows_sub_any1(
    const void* __restrict__ x, int64_t rows, int L, float eps, int8_t* __restrict__ q,
    float* __restrict__ scale) {
  // E = 2: element pairs (L even, x and q aligned to a pair) in one load and
  // one 2-byte code store
  static_assert(E == 1 || E == 2, "elements per load");
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int sub = lane / LPR;
  const int lr = lane % LPR;
  const int U = L / E;   // load units per row
  const int64_t row0 =
      (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * (RI * RPW) + sub;

  float f[RI][VPL][E];
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    if (row < rows) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int j = v * LPR + lr;
        const int64_t e = row * L + static_cast<int64_t>(j < U ? j : 0) * E;
        if constexpr (E == 1) {
          f[it][v][0] = ld1<DT>(x, e);
        } else if constexpr (DT == kF32) {
          const float2 w = *reinterpret_cast<const float2*>(static_cast<const float*>(x) + e);
          f[it][v][0] = w.x;
          f[it][v][1] = w.y;
        } else {
          const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(x) + e);
          if constexpr (DT == kBF16) {
            f[it][v][0] = __uint_as_float(w << 16);
            f[it][v][1] = __uint_as_float(w & 0xffff0000u);
          } else {
            f[it][v][0] = static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu)));
            f[it][v][1] = static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)));
          }
        }
      }
    }
  }
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int64_t row = row0 + static_cast<int64_t>(it) * RPW;
    const bool ok = row < rows;
    float m = 0.0f;
    if (ok) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        float mv = __builtin_fabsf(f[it][v][0]);
        if constexpr (E == 2) mv = fmaxf(mv, __builtin_fabsf(f[it][v][1]));
        m = v * LPR + lr < U ? fmaxf(m, mv) : m;
      }
    }
    m = group_max<LPR>(m);   // every lane participates
    const float inv = inv_scale(m, eps, kQmaxInt8);
    if (ok) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int j = v * LPR + lr;
        if (j < U) {
          if constexpr (E == 1) {
            q[row * L + j] = static_cast<int8_t>(q_int8(f[it][v][0] * inv));
          } else {
            const uint32_t c0 = static_cast<uint8_t>(q_int8(f[it][v][0] * inv));
            const uint32_t c1 = static_cast<uint8_t>(q_int8(f[it][v][1] * inv));
            *reinterpret_cast<uint16_t*>(q + row * L + static_cast<int64_t>(j) * 2) =
                static_cast<uint16_t>(c0 | (c1 << 8));
          }
        }
      }
      if (lr == 0) scale[row] = 1.0f / inv;
    }
  }
}

// Few long rows (e.g. per-channel axis 0 of [64, 1024, 1024]): each row is
// cut into `splits` slices of sc chunks and workgroup (row, slice) = blockIdx
// (y, x) works on one slice, so the grid fills the CUs however few the rows.
// k_rows_split_max writes one partial maximum per slice; k_rows_split_cast
// reduces its row's partials (L2) while its first loads are in flight, then
// casts its slice. L % 8 == 0, 16-byte aligned x, 8-byte aligned q.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_rows_split_max(
    const void* __restrict__ x, int64_t L, int64_t sc, float* __restrict__ partial) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.y, n8 = L >> 3;
  const int64_t c_end = min((static_cast<int64_t>(blockIdx.x) + 1) * sc, n8);
  const int64_t base = row * L;
  float m = 0.0f;
  for (int64_t c0 = static_cast<int64_t>(blockIdx.x) * sc + threadIdx.x; c0 < c_end;
       c0 += kU * kBlock) {
    Raw8<DT> r[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
      if (c < c_end) r[u] = ld8<DT>(x, base + c * 8);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
      if (c < c_end) {
        float f[8];
        cvt8<DT>(r[u], f);
        m = absmax8(f, m);
      }
    }
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) partial[row * gridDim.x + blockIdx.x] = m;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_rows_split_cast(
    const void* __restrict__ x, int64_t L, int64_t sc, const float* __restrict__ partial,
    float eps, int8_t* __restrict__ q, float* __restrict__ scale) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.y, n8 = L >> 3;
  const int64_t c_end = min((static_cast<int64_t>(blockIdx.x) + 1) * sc, n8);
  const int64_t base = row * L;
  int64_t c0 = static_cast<int64_t>(blockIdx.x) * sc + threadIdx.x;
  Raw8<DT> r[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
    if (c < c_end) r[u] = ld8<DT>(x, base + c * 8);
  }
  const float m = reduce_partials(partial + row * gridDim.x, static_cast<int>(gridDim.x), red);
  const float inv = inv_scale(m, eps, kQmaxInt8);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[row] = 1.0f / inv;
  for (;;) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
      if (c < c_end) {
        float f[8];
        cvt8<DT>(r[u], f);
        stg8(q + base + c * 8, pack8_int8(f, inv));
      }
    }
    c0 += kU * kBlock;
    if (c0 >= c_end) break;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t c = c0 + static_cast<int64_t>(u) * kBlock;
      if (c < c_end) r[u] = ld8<DT>(x, base + c * 8);
    }
  }
}

// One workgroup of B threads per row of L = B * VPL * 8 elements, held in
// registers. Workgroups stride over rows (the row loop is uniform per
// workgroup). Measured on MI355X, rows of 8192 bf16 (C3 axis 0): 512 threads
// x 2 chunks 110.0 us, 256 x 4 111.4-113.7 us, 1024 x 1 148 us.
template <int DT, int VPL, int B = kBlock>
__global__ __launch_bounds__(B) void k_rows_wg(
    const void* __restrict__ x, int64_t rows, float eps, int8_t* __restrict__ q,
    float* __restrict__ scale) {
  __shared__ float red[B / kWave];
  constexpr int64_t L = static_cast<int64_t>(B) * VPL * 8;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    Raw8<DT> r[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) r[v] = ld8<DT>(x, row * L + (v * B + threadIdx.x) * 8);
    float f[VPL][8];
    float m = 0.0f;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      cvt8<DT>(r[v], f[v]);
      m = absmax8(f[v], m);
    }
    m = block_max(m, red);
    const float inv = inv_scale(m, eps, kQmaxInt8);
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      stg8(q + row * L + (v * B + threadIdx.x) * 8, pack8_int8(f[v], inv));
    if (threadIdx.x == 0) scale[row] = 1.0f / inv;
  }
}

// Any row length: one workgroup per row (striding over rows), a reduce pass
// then a cast pass. vec != 0 requires L % 8 == 0 and 16-byte / 8-byte
// aligned x / q.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_rows_generic(
    const void* __restrict__ x, int64_t rows, int64_t L, int vec, float eps,
    int8_t* __restrict__ q, float* __restrict__ scale) {
  __shared__ float red[kBlock / kWave];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * L;
    float m = 0.0f;
    if (vec) {
      const int64_t nc = L >> 3;
      for (int64_t c = threadIdx.x; c < nc; c += kBlock) {
        float f[8];
        cvt8<DT>(ld8<DT>(x, base + c * 8), f);
        m = absmax8(f, m);
      }
    } else {
      for (int64_t i = threadIdx.x; i < L; i += kBlock)
        m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, base + i)));
    }
    m = block_max(m, red);
    const float inv = inv_scale(m, eps, kQmaxInt8);
    if (vec) {
      const int64_t nc = L >> 3;
      for (int64_t c = threadIdx.x; c < nc; c += kBlock) {
        float f[8];
        cvt8<DT>(ld8<DT>(x, base + c * 8), f);
        stg8(q + base + c * 8, pack8_int8(f, inv));
      }
    } else {
      for (int64_t i = threadIdx.x; i < L; i += kBlock)
        q[base + i] = static_cast<int8_t>(q_int8(ld1<DT>(x, base + i) * inv));
    }
    if (threadIdx.x == 0) scale[row] = 1.0f / inv;
  }
}

// ---------------------------------------------------------------------------
// Columns (per-channel axis 1)
// ---------------------------------------------------------------------------

// Partial column maxima of row block blockIdx.y (rows [y*RB, y*RB+RB)).
// vec: each thread owns 8 adjacent columns (cols % 8 == 0, aligned x);
// otherwise one column. partial is [gridDim.y, cols] fp32.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_colmax(
    const void* __restrict__ x, int64_t rows, int64_t cols, int64_t RB, int vec,
    float* __restrict__ partial) {
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  float* out = partial + static_cast<int64_t>(blockIdx.y) * cols;
  if (vec) {
    const int64_t c = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 8;
    if (c >= cols) return;
    float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      Raw8<DT> raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[u] = ld8<DT>(x, (r + u) * cols + c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float f[8];
        cvt8<DT>(raw[u], f);
#pragma unroll
        for (int k = 0; k < 8; ++k) m[k] = fmaxf(m[k], __builtin_fabsf(f[k]));
      }
    }
    for (; r < r1; ++r) {
      float f[8];
      cvt8<DT>(ld8<DT>(x, r * cols + c), f);
#pragma unroll
      for (int k = 0; k < 8; ++k) m[k] = fmaxf(m[k], __builtin_fabsf(f[k]));
    }
    float4* o = reinterpret_cast<float4*>(out + c);
    o[0] = make_float4(m[0], m[1], m[2], m[3]);
    o[1] = make_float4(m[4], m[5], m[6], m[7]);
  } else {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= cols) return;
    float m = 0.0f;
    for (int64_t r = r0; r < r1; ++r) m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, r * cols + c)));
    out[c] = m;
  }
}

// Column maxima from the partials: a workgroup covers kFinCols columns; its
// kBlock / kFinCols thread slices stride over the row blocks, then combine
// through LDS.
// FC columns per workgroup: kFinCols, or 4 for narrow rows, whose few
// columns would otherwise leave a handful of workgroups walking all the row
// blocks.
constexpr int kFinCols = 32;
template <int FC>
__global__ __launch_bounds__(kBlock) void k_col_finalize(
    const float* __restrict__ partial, int64_t nrb, int64_t cols, float eps,
    float* __restrict__ inv_out, float* __restrict__ scale) {
  constexpr int kSlices = kBlock / FC;
  __shared__ float red[kSlices][FC];
  const int cl = threadIdx.x % FC, sl = threadIdx.x / FC;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * FC + cl;
  float m = 0.0f;
  if (c < cols)
    for (int64_t b = sl; b < nrb; b += kSlices) m = fmaxf(m, partial[b * cols + c]);
  red[sl][cl] = m;
  __syncthreads();
  if (sl == 0 && c < cols) {
#pragma unroll
    for (int k = 1; k < kSlices; ++k) m = fmaxf(m, red[k][cl]);
    const float inv = inv_scale(m, eps, kQmaxInt8);
    inv_out[c] = inv;
    scale[c] = 1.0f / inv;
  }
}

// The same with 4 columns per lane (cols % 4 == 0): 16 lanes x 4 columns per
// slice, 16 slices striding over the row blocks, so each thread keeps
// 16-byte loads in flight instead of one 4-byte load per row block.
// Measured on MI355X (C3 axis 1: 256 row blocks x 8192 columns): 9.6 us for
// the scalar kernel above.
constexpr int kFin4Cols = 64;
__global__ __launch_bounds__(kBlock) void k_col_finalize4(
    const float* __restrict__ partial, int64_t nrb, int64_t cols, float eps,
    float* __restrict__ inv_out, float* __restrict__ scale) {
  constexpr int kLanes = kFin4Cols / 4, kSlices = kBlock / kLanes;
  __shared__ float4 red[kSlices][kLanes];
  const int cl = threadIdx.x % kLanes, sl = threadIdx.x / kLanes;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kFin4Cols + cl * 4;
  float4 m = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (c < cols) {
    int64_t b = sl;
    for (; b + 3 * kSlices < nrb; b += 4 * kSlices) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = *reinterpret_cast<const float4*>(partial + (b + u * kSlices) * cols + c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        m.x = fmaxf(m.x, v[u].x); m.y = fmaxf(m.y, v[u].y);
        m.z = fmaxf(m.z, v[u].z); m.w = fmaxf(m.w, v[u].w);
      }
    }
    for (; b < nrb; b += kSlices) {
      const float4 v = *reinterpret_cast<const float4*>(partial + b * cols + c);
      m.x = fmaxf(m.x, v.x); m.y = fmaxf(m.y, v.y); m.z = fmaxf(m.z, v.z); m.w = fmaxf(m.w, v.w);
    }
  }
  red[sl][cl] = m;
  __syncthreads();
  if (sl == 0 && c < cols) {
#pragma unroll
    for (int k = 1; k < kSlices; ++k) {
      const float4 v = red[k][cl];
      m.x = fmaxf(m.x, v.x); m.y = fmaxf(m.y, v.y); m.z = fmaxf(m.z, v.z); m.w = fmaxf(m.w, v.w);
    }
    const float mm[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float inv = inv_scale(mm[k], eps, kQmaxInt8);
      inv_out[c + k] = inv;
      scale[c + k] = 1.0f / inv;
    }
  }
}

// inner: adjacent columns sharing one scale (1 for per-column scales; the
// N-D channel path views [outer, channels, inner] as [outer, channels * inner]).
template <int DT>
__global__ __launch_bounds__(kBlock) void k_cast_cols(
    const void* __restrict__ x, int64_t rows, int64_t cols, int64_t RB, int vec,
    const float* __restrict__ inv_c, int64_t inner, int8_t* __restrict__ q) {
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  if (vec) {
    const int64_t c = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 8;
    if (c >= cols) return;
    float inv[8];
    channel_vals8(inv_c, c, inner, inv);
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      Raw8<DT> raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[u] = ld8<DT>(x, (r + u) * cols + c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float f[8];
        cvt8<DT>(raw[u], f);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] *= inv[k];
        stg8(q + (r + u) * cols + c, pack8_int8(f, 1.0f));
      }
    }
    for (; r < r1; ++r) {
      float f[8];
      cvt8<DT>(ld8<DT>(x, r * cols + c), f);
#pragma unroll
      for (int k = 0; k < 8; ++k) f[k] *= inv[k];
      stg8(q + r * cols + c, pack8_int8(f, 1.0f));
    }
  } else {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= cols) return;
    const float inv = inv_c[c / inner];
    for (int64_t r = r0; r < r1; ++r)
      q[r * cols + c] = static_cast<int8_t>(q_int8(ld1<DT>(x, r * cols + c) * inv));
  }
}

// Narrow columns (cols % 8 == 0, u = cols / 8 <= kBlock / 2 chunks per row,
// e.g. [262144, 64] or the [outer, 512] view of a channel on the last axis):
// the wide kernels above leave all but u threads of a workgroup idle, so
// here thread t takes chunk t % u of rows r0 + t / u, stepping by rpi =
// kBlock / u rows. k_colmax_narrow folds its rpi sub-rows through LDS and
// writes the same [gridDim.y, cols] partials as k_colmax.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_colmax_narrow(
    const void* __restrict__ x, int64_t rows, int64_t cols, int64_t RB, int u, int rpi,
    float* __restrict__ partial) {
  __shared__ float4 red[kBlock][2];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  const int sub = static_cast<int>(threadIdx.x) / u, cu = static_cast<int>(threadIdx.x) - sub * u;
  const int64_t c = static_cast<int64_t>(cu) * 8;
  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (sub < rpi) {
    int64_t r = r0 + sub;
    for (; r + 3 * rpi < r1; r += 4 * rpi) {
      Raw8<DT> raw[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) raw[k] = ld8<DT>(x, (r + k * rpi) * cols + c);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float f[8];
        cvt8<DT>(raw[k], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], __builtin_fabsf(f[e]));
      }
    }
    for (; r < r1; r += rpi) {
      float f[8];
      cvt8<DT>(ld8<DT>(x, r * cols + c), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], __builtin_fabsf(f[e]));
    }
  }
  red[threadIdx.x][0] = make_float4(m[0], m[1], m[2], m[3]);
  red[threadIdx.x][1] = make_float4(m[4], m[5], m[6], m[7]);
  __syncthreads();
  if (sub == 0) {
    for (int k = 1; k < rpi; ++k) {
      const float4 a = red[k * u + cu][0], b = red[k * u + cu][1];
      m[0] = fmaxf(m[0], a.x); m[1] = fmaxf(m[1], a.y); m[2] = fmaxf(m[2], a.z); m[3] = fmaxf(m[3], a.w);
      m[4] = fmaxf(m[4], b.x); m[5] = fmaxf(m[5], b.y); m[6] = fmaxf(m[6], b.z); m[7] = fmaxf(m[7], b.w);
    }
    float4* o = reinterpret_cast<float4*>(partial + static_cast<int64_t>(blockIdx.y) * cols + c);
    o[0] = make_float4(m[0], m[1], m[2], m[3]);
    o[1] = make_float4(m[4], m[5], m[6], m[7]);
  }
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_cast_cols_narrow(
    const void* __restrict__ x, int64_t rows, int64_t cols, int64_t RB, int u, int rpi,
    const float* __restrict__ inv_c, int64_t inner, int8_t* __restrict__ q) {
  const int sub = static_cast<int>(threadIdx.x) / u, cu = static_cast<int>(threadIdx.x) - sub * u;
  if (sub >= rpi) return;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  const int64_t c = static_cast<int64_t>(cu) * 8;
  float inv[8];
  channel_vals8(inv_c, c, inner, inv);
  int64_t r = r0 + sub;
  for (; r + 3 * rpi < r1; r += 4 * rpi) {
    Raw8<DT> raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k] = ld8<DT>(x, (r + k * rpi) * cols + c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float f[8];
      cvt8<DT>(raw[k], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] *= inv[e];
      stg8(q + (r + k * rpi) * cols + c, pack8_int8(f, 1.0f));
    }
  }
  for (; r < r1; r += rpi) {
    float f[8];
    cvt8<DT>(ld8<DT>(x, r * cols + c), f);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] *= inv[e];
    stg8(q + r * cols + c, pack8_int8(f, 1.0f));
  }
}

// The same for narrow rows that 16-byte loads cannot take (cols <= kBlock /
// 2 with cols % 8 != 0, or unaligned buffers): one element per thread, thread
// t on column t % cols of rows r0 + t / cols, stepping by rpi = kBlock / cols.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_colmax_narrow1(
    const void* __restrict__ x, int64_t rows, int64_t cols, int64_t RB, int rpi,
    float* __restrict__ partial) {
  __shared__ float red[kBlock];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  const int u = static_cast<int>(cols);
  const int sub = static_cast<int>(threadIdx.x) / u, c = static_cast<int>(threadIdx.x) - sub * u;
  float m = 0.0f;
  if (sub < rpi) {
    int64_t r = r0 + sub;
    for (; r + 3 * rpi < r1; r += 4 * rpi) {
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = ld1<DT>(x, (r + k * rpi) * cols + c);
#pragma unroll
      for (int k = 0; k < 4; ++k) m = fmaxf(m, __builtin_fabsf(v[k]));
    }
    for (; r < r1; r += rpi) m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, r * cols + c)));
  }
  red[threadIdx.x] = m;
  __syncthreads();
  if (sub == 0) {
    for (int k = 1; k < rpi; ++k) m = fmaxf(m, red[k * u + c]);
    partial[static_cast<int64_t>(blockIdx.y) * cols + c] = m;
  }
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_cast_cols_narrow1(
    const void* __restrict__ x, int64_t rows, int64_t cols, int64_t RB, int rpi,
    const float* __restrict__ inv_c, int64_t inner, int8_t* __restrict__ q) {
  const int u = static_cast<int>(cols);
  const int sub = static_cast<int>(threadIdx.x) / u, c = static_cast<int>(threadIdx.x) - sub * u;
  if (sub >= rpi) return;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * RB;
  const int64_t r1 = r0 + RB < rows ? r0 + RB : rows;
  const float inv = inv_c[c / inner];
  int64_t r = r0 + sub;
  for (; r + 3 * rpi < r1; r += 4 * rpi) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = ld1<DT>(x, (r + k * rpi) * cols + c);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      q[(r + k * rpi) * cols + c] = static_cast<int8_t>(q_int8(v[k] * inv));
  }
  for (; r < r1; r += rpi) q[r * cols + c] = static_cast<int8_t>(q_int8(ld1<DT>(x, r * cols + c) * inv));
}

// N-D channel quant in one pass: one workgroup of B threads per channel
// (a middle axis of [outer, channels, inner], inner % 8 == 0), the channel's
// outer segments of inner elements held in registers. Chunk j (8 elements)
// of the channel is chunk j % (inner / 8) of segment j / (inner / 8); thread
// t holds chunks t, t + B, ..., up to V of them. Chunks past the channel's
// end are loaded from its first chunk (in bounds) and left out of the
// maximum, so the loads need no branch. Reads x once: 2N + N + 4C bytes.
template <int DT, int V, int B>
__global__ __launch_bounds__(B) void k_chan_wg(
    const void* __restrict__ x, int64_t channels, int64_t inner, int nchunks, float eps,
    int8_t* __restrict__ q, float* __restrict__ scale) {
  __shared__ float red[B / kWave];
  const int64_t c = blockIdx.x;
  const int cps = static_cast<int>(inner >> 3);          // chunks per segment
  // element offset of this thread's chunk v (chunk 0 of the channel when v
  // is past its end); recomputed where needed rather than held
  auto elem = [&](int v) {
    const int j = v * B + static_cast<int>(threadIdx.x);
    const int jj = j < nchunks ? j : 0;
    const int o = jj / cps, k = jj - o * cps;
    return (static_cast<int64_t>(o) * channels + c) * inner + static_cast<int64_t>(k) * 8;
  };
  Raw8<DT> r[V];
#pragma unroll
  for (int v = 0; v < V; ++v) r[v] = ld8<DT>(x, elem(v));
  float m = 0.0f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    float f[8];
    cvt8<DT>(r[v], f);
    const float mv = absmax8(f, 0.0f);
    m = v * B + static_cast<int>(threadIdx.x) < nchunks ? fmaxf(m, mv) : m;
  }
  // the cast converts from the raw words again instead of keeping the
  // first conversion's fp32 values live
#pragma unroll
  for (int v = 0; v < V; ++v) reload_barrier<DT>(r[v]);
  m = block_max(m, red);
  const float inv = inv_scale(m, eps, kQmaxInt8);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (v * B + static_cast<int>(threadIdx.x) >= nchunks) continue;
    float f[8];
    cvt8<DT>(r[v], f);
    stg8(q + elem(v), pack8_int8(f, inv));
  }
  if (threadIdx.x == 0) scale[c] = 1.0f / inv;
}

// Channel maxima of the N-D channel path: channel ch owns columns
// [ch * inner, ch * inner + inner) of the partial maxima; one workgroup per
// channel reduces its nrb * inner partials (block reduce), then writes inv
// and scale.
__global__ __launch_bounds__(kBlock) void k_chan_finalize(
    const float* __restrict__ partial, int64_t nrb, int64_t cols, int64_t inner, float eps,
    float* __restrict__ inv_out, float* __restrict__ scale) {
  __shared__ float red[kBlock / kWave];
  const int64_t ch = blockIdx.x;
  float m = 0.0f;
  const int64_t n = nrb * inner;
  for (int64_t e = threadIdx.x; e < n; e += kBlock) {
    const int64_t b = e / inner, j = e % inner;
    m = fmaxf(m, partial[b * cols + ch * inner + j]);
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) {
    const float inv = inv_scale(m, eps, kQmaxInt8);
    inv_out[ch] = inv;
    scale[ch] = 1.0f / inv;
  }
}

// ---------------------------------------------------------------------------
// Groups along a non-last axis: x viewed as [outer, len, inner], groups of G
// consecutive positions along len. One thread per group (o, g, i) with i
// fastest, so that a wave's loads of one position are contiguous in x. The
// scale index follows the reference's movedim layout,
// (o * inner + i) * (len / G) + g (quantizers.py:123-130).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kBlock) void k_group_strided(
    const void* __restrict__ x, int64_t outer, int64_t len, int64_t inner, int64_t G, float eps,
    int8_t* __restrict__ q, float* __restrict__ scale) {
  const int64_t ng = len / G;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (t >= outer * ng * inner) return;
  const int64_t i = t % inner, g = (t / inner) % ng, o = t / (inner * ng);
  const int64_t base = (o * len + g * G) * inner + i;
  float m = 0.0f;
  for (int64_t k = 0; k < G; ++k) m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, base + k * inner)));
  const float inv = inv_scale(m, eps, kQmaxInt8);
  scale[(o * inner + i) * ng + g] = 1.0f / inv;
  for (int64_t k = 0; k < G; ++k)
    q[base + k * inner] = static_cast<int8_t>(q_int8(ld1<DT>(x, base + k * inner) * inv));
}

// Groups along a non-last axis, tiled (inner % 8 == 0, 16-byte aligned x,
// 8-byte aligned q). A workgroup of NW waves covers kGtCols adjacent inner
// positions (64 lanes x 8) of one group: G = NW * rpt positions along len,
// wave w holding positions w, w + NW, ..., so each load instruction of a wave
// reads one contiguous 1 KiB (2-byte types) run of x. HOLD (rpt <= kGtHold):
// the group stays in registers between the max and the cast, so x is read
// once; otherwise the cast reads the tile again (L2 / Infinity Cache).
// TS (a workspace is given, ng > 1): inner tiles fastest, so the workgroups
// that run together read whole rows of x, and the scales go to group-major
// scratch [outer, ng, inner] (contiguous per workgroup); k_transpose_f32
// then writes the movedim order. Measured on MI355X, groups of 128 along
// axis 0 of [16384, 14336] bf16: the scattered 4-byte writes of the movedim
// order (each 128-byte line filled by 32 workgroups) took ~30 of ~150 us.
// Otherwise: logical workgroup index, after xcd_remap: g fastest, then the
// inner tile, then o, so the scales of neighbouring groups - adjacent in the
// movedim layout - are written from one XCD's L2.
constexpr int kGtCols = kWave * 8;
constexpr int kGtHold = 16;

template <int DT, int NW, bool HOLD, bool TS, int RPTC = 0>
__global__ __launch_bounds__(NW * kWave) void k_group_tile(
    const void* __restrict__ x, int64_t len, int64_t inner, int64_t G, int rpt, int64_t ng,
    int64_t tiles, int64_t nblocks, float eps, int8_t* __restrict__ q,
    float* __restrict__ scale) {
  int64_t g, ti, o;
  if constexpr (TS) {
    // inner tiles fastest: the workgroups running together read whole rows
    const int64_t b = blockIdx.x;
    ti = b % tiles; g = (b / tiles) % ng; o = b / (ng * tiles);
  } else {
    const int64_t b = xcd_remap(blockIdx.x, nblocks);
    g = b % ng; ti = (b / ng) % tiles; o = b / (ng * tiles);
  }
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int64_t i = ti * kGtCols + lane * 8;
  const bool act = i < inner;
  const int64_t base = (o * len + g * G + w) * inner + i;
  const int64_t rs = static_cast<int64_t>(NW) * inner;
  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  Raw8<DT> r[HOLD ? (RPTC > 0 ? RPTC : kGtHold) : 8];
  if constexpr (HOLD && RPTC > 0) {
    // compile-time count (rpt rounded up to a power of two): unguarded loads,
    // past rpt (and for lanes past inner) clamped to an in-bounds row and
    // left out of the maximum. Guarded loads made the compiler wait for every
    // outstanding load where the branches rejoin (groups of 128 along axis 0
    // of [16384, 14336] bf16: 136.6 us with them).
    const int64_t lb = act ? base : base - i;
#pragma unroll
    for (int k = 0; k < RPTC; ++k) r[k] = ld8<DT>(x, lb + min(k, rpt - 1) * rs);
#pragma unroll
    for (int k = 0; k < RPTC; ++k) {
      float f[8];
      cvt8<DT>(r[k], f);
      const bool use = act && k < rpt;
#pragma unroll
      for (int j = 0; j < 8; ++j) m[j] = use ? fmaxf(m[j], __builtin_fabsf(f[j])) : m[j];
    }
  } else if constexpr (HOLD) {
#pragma unroll
    for (int k = 0; k < kGtHold; ++k)
      if (k < rpt && act) r[k] = ld8<DT>(x, base + k * rs);
#pragma unroll
    for (int k = 0; k < kGtHold; ++k)
      if (k < rpt && act) {
        float f[8];
        cvt8<DT>(r[k], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = fmaxf(m[j], __builtin_fabsf(f[j]));
      }
  } else if (act) {
    for (int k0 = 0; k0 < rpt; k0 += 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < rpt) r[k] = ld8<DT>(x, base + (k0 + k) * rs);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < rpt) {
          float f[8];
          cvt8<DT>(r[k], f);
#pragma unroll
          for (int j = 0; j < 8; ++j) m[j] = fmaxf(m[j], __builtin_fabsf(f[j]));
        }
    }
  }
  if constexpr (NW > 1) {
    __shared__ float4 red[NW][kWave][2];
    red[w][lane][0] = make_float4(m[0], m[1], m[2], m[3]);
    red[w][lane][1] = make_float4(m[4], m[5], m[6], m[7]);
    __syncthreads();
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float4 a = red[v][lane][0], c = red[v][lane][1];
      m[0] = fmaxf(m[0], a.x); m[1] = fmaxf(m[1], a.y); m[2] = fmaxf(m[2], a.z);
      m[3] = fmaxf(m[3], a.w); m[4] = fmaxf(m[4], c.x); m[5] = fmaxf(m[5], c.y);
      m[6] = fmaxf(m[6], c.z); m[7] = fmaxf(m[7], c.w);
    }
  }
  if (!act) return;
  float inv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) inv[j] = inv_scale(m[j], eps, kQmaxInt8);
  if (w == 0) {
    if constexpr (TS) {
      // group-major scratch [outer, ng, inner]: 32 contiguous bytes per lane
      float4* d = reinterpret_cast<float4*>(scale + (o * ng + g) * inner + i);
      d[0] = make_float4(1.0f / inv[0], 1.0f / inv[1], 1.0f / inv[2], 1.0f / inv[3]);
      d[1] = make_float4(1.0f / inv[4], 1.0f / inv[5], 1.0f / inv[6], 1.0f / inv[7]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) scale[(o * inner + i + j) * ng + g] = 1.0f / inv[j];
    }
  }
  if constexpr (HOLD && RPTC > 0) {
#pragma unroll
    for (int k = 0; k < RPTC; ++k)
      if (k < rpt) {
        float f[8];
        reload_barrier<DT>(r[k]);
        cvt8<DT>(r[k], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= inv[j];
        stg8(q + base + k * rs, pack8_int8(f, 1.0f));
      }
  } else if constexpr (HOLD) {
#pragma unroll
    for (int k = 0; k < kGtHold; ++k)
      if (k < rpt) {
        float f[8];
        reload_barrier<DT>(r[k]);
        cvt8<DT>(r[k], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= inv[j];
        stg8(q + base + k * rs, pack8_int8(f, 1.0f));
      }
  } else {
    for (int k0 = 0; k0 < rpt; k0 += 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < rpt) r[k] = ld8<DT>(x, base + (k0 + k) * rs);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < rpt) {
          float f[8];
          cvt8<DT>(r[k], f);
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] *= inv[j];
          stg8(q + base + (k0 + k) * rs, pack8_int8(f, 1.0f));
        }
    }
  }
}

// Segment maxima for the N-D channel path when inner is long: x viewed as
// segs = outer * channels contiguous segments of inner elements; one wave per
// segment (grid-stride over waves), so partial is [outer, channels] and the
// channel maxima come from k_chan_finalize with inner = 1. vec: inner % 8 == 0
// and 16-byte aligned x; a wave then reads 1 KiB (2-byte types) per load.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_segmax(
    const void* __restrict__ x, int64_t segs, int64_t inner, int vec,
    float* __restrict__ partial) {
  constexpr int kWpb = kBlock / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWpb;
  for (int64_t sg = static_cast<int64_t>(blockIdx.x) * kWpb + threadIdx.x / kWave; sg < segs;
       sg += nwaves) {
    const int64_t e0 = sg * inner;
    float m = 0.0f;
    if (vec) {
      const int64_t n8 = inner >> 3;
      int64_t c = lane;
      for (; c + 3 * kWave < n8; c += 4 * kWave) {
        Raw8<DT> raw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) raw[u] = ld8<DT>(x, e0 + (c + u * kWave) * 8);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float f[8];
          cvt8<DT>(raw[u], f);
          m = absmax8(f, m);
        }
      }
      for (; c < n8; c += kWave) {
        float f[8];
        cvt8<DT>(ld8<DT>(x, e0 + c * 8), f);
        m = absmax8(f, m);
      }
    } else {
      for (int64_t e = lane; e < inner; e += kWave) m = fmaxf(m, __builtin_fabsf(ld1<DT>(x, e0 + e)));
    }
    m = group_max<kWave>(m);
    if (lane == 0) partial[sg] = m;
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
bool valid_dtype(int dt, bool allow_f32) {
  return dt == kF16 || dt == kBF16 || (allow_f32 && dt == kF32);
}

// Persistent grid shared by the amax and cast passes (one partial maximum per
// workgroup).
int64_t tensor_grid(int64_t n, bool vec) {
  const int64_t work = vec ? cdiv(n >> 3, static_cast<int64_t>(kU) * kBlock) : cdiv(n, kBlock);
  int64_t cap = static_cast<int64_t>(device_cus()) * kTensorWgPerCu;
  if (cap > kMaxTensorWg) cap = kMaxTensorWg;
  int64_t g = work < cap ? work : cap;
  return g < 1 ? 1 : g;
}

// Polls a one-launch wait makes before giving up: kFusedSpinLimit, or the
// CBQ_TENSOR_SPIN_LIMIT environment variable read at the first call, or the
// value set by cbq_set_tensor_spin_limit (a host switch that lets tests
// exercise the timeout path with every kernel still ending normally, and
// callers that share the GPU with long-running kernels pick their bound).
std::atomic<uint32_t>& spin_limit_var() {
  static std::atomic<uint32_t> v{[] {
    const char* e = getenv("CBQ_TENSOR_SPIN_LIMIT");
    if (!e || !*e) return kFusedSpinLimit;
    return static_cast<uint32_t>(strtoul(e, nullptr, 10));
  }()};
  return v;
}
uint32_t fused_spin_limit() { return spin_limit_var().load(std::memory_order_relaxed); }

// True if one workgroup of the one-launch kernel fits on a CU, i.e. a grid
// of one workgroup per CU is resident at once (cached per device and kernel).
template <int DT, bool FP8>
bool fused_fits() {
  static int cached[64];   // 0 unknown, 1 fits, 2 does not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (cached[dev] == 0) {
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &nb, reinterpret_cast<const void*>(&k_quant_tensor_1pass<DT, FP8>), kFusedBlock, 0);
    cached[dev] = (e == hipSuccess && nb >= 1) ? 1 : 2;
  }
  return cached[dev] == 1;
}

// Clears the sticky status word of a per-tensor control block (a kernel,
// not hipMemsetAsync, so that it is stream-ordered and safe under capture).
__global__ void k_clear_tensor_status(char* ctl) {
  __hip_atomic_store(reinterpret_cast<unsigned int*>(ctl + kCtlStatus), 0u, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT>
int tensor_quant_t(const void* x, int64_t n, float eps, float* partial, char* ctl, uint8_t* q,
                   float* scale, bool fp8, hipStream_t s) {
  const bool vec = aligned(x, 16) && aligned(q, 8);
  const char* what = fp8 ? "cbq_quant_fp8_tensor" : "cbq_quant_int8_tensor";
  if (vec && n >= kFusedMinElems && device_cus() <= kMaxFusedGrid &&
      (fp8 ? fused_fits<DT, true>() : fused_fits<DT, false>())) {
    // One workgroup per CU, or fewer when x has fewer 4096-chunk steps than
    // there are CUs (below 2^23 elements): the workgroups that would find no
    // chunk of x only lengthen the launch and the exchange. Measured on
    // MI355X (back-to-back launches): [1024, 4096] fp16 9.76 -> 8.67 us,
    // [1024, 1024] bf16 FP8 9.10 -> 8.21 us. Below 2^20 elements the two-pass
    // path's smaller workgroups spread a small x over more CUs: [16, 4096]
    // bf16 FP8 6.5 us against 7.6 us for one 1024-thread workgroup.
    const int64_t steps = cdiv(n >> 3, static_cast<int64_t>(kFusedBlock) * kFusedU);
    const dim3 g(static_cast<unsigned>(std::min<int64_t>(steps, device_cus()))), b(kFusedBlock);
    if (fp8)
      k_quant_tensor_1pass<DT, true><<<g, b, 0, s>>>(x, n, eps, q, scale, ctl, fused_spin_limit());
    else
      k_quant_tensor_1pass<DT, false><<<g, b, 0, s>>>(x, n, eps, q, scale, ctl, fused_spin_limit());
    return launch_status(what);
  }
  const int64_t grid = tensor_grid(n, vec);
  const dim3 g(static_cast<unsigned>(grid)), b(kBlock);
  k_amax_tensor<DT><<<g, b, 0, s>>>(x, n, vec ? 1 : 0, partial);
  if (fp8) {
    k_cast_tensor<DT, true><<<g, b, 0, s>>>(x, n, vec ? 1 : 0, partial, static_cast<int>(grid),
                                            eps, q, scale);
  } else {
    k_cast_tensor<DT, false><<<g, b, 0, s>>>(x, n, vec ? 1 : 0, partial, static_cast<int>(grid),
                                             eps, q, scale);
  }
  return launch_status(what);
}

constexpr size_t tensor_ws_bytes() { return CBQ_WS_CTRL_BYTES + sizeof(float) * kMaxTensorWg; }

int tensor_quant(const void* x, int dt, int64_t n, float eps, void* ws, size_t ws_bytes,
                 uint8_t* q, float* scale, bool fp8, hipStream_t s) {
  const char* what = fp8 ? "cbq_quant_fp8_tensor" : "cbq_quant_int8_tensor";
  CBQ_REQUIRE(valid_dtype(dt, !fp8), "%s: unsupported input dtype code %d", what, dt);
  CBQ_REQUIRE(n >= 0, "%s: negative element count", what);
  if (n == 0) return CBQ_OK;
  CBQ_REQUIRE(x && q && scale, "%s: null pointer", what);
  CBQ_REQUIRE(ws && ws_bytes >= tensor_ws_bytes() && aligned(ws, 16),
              "%s: workspace must be >= %zu bytes, 16-byte aligned", what, tensor_ws_bytes());
  char* ctl = static_cast<char*>(ws);
  float* partial = reinterpret_cast<float*>(ctl + CBQ_WS_CTRL_BYTES);
  switch (dt) {
    case kF16: return tensor_quant_t<kF16>(x, n, eps, partial, ctl, q, scale, fp8, s);
    case kBF16: return tensor_quant_t<kBF16>(x, n, eps, partial, ctl, q, scale, fp8, s);
    default: return tensor_quant_t<kF32>(x, n, eps, partial, ctl, q, scale, fp8, s);
  }
}

// Workgroup count for one-workgroup-per-row kernels (they stride over rows).
unsigned wg_rows_grid(int64_t rows) {
  const int64_t cap = 1 << 20;
  return static_cast<unsigned>(rows < cap ? rows : cap);
}

// Rows of length L (elements) -> fastest kernel shape that fits.
template <int DT, int LPR, int VPL>
void launch_rows_sub(const void* x, int64_t rows, float eps, int8_t* q, float* scale,
                     hipStream_t s) {
  constexpr int RI = (LPR * VPL >= 64) ? 2 : 4;
  constexpr int64_t rows_per_wg = static_cast<int64_t>(kBlock / kWave) * RI * (kWave / LPR);
  const int64_t grid = cdiv(rows, rows_per_wg);
  k_rows_sub<DT, LPR, VPL, RI><<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, s>>>(
      x, rows, eps, q, scale);
}

// The one-pass channel kernel (k_chan_wg) for channels of 256 to 8192
// chunks of 8 elements: 256 threads with up to 8 chunks each up to 2048
// chunks, else 512 threads with up to 16. It takes the N-D channel path
// (a middle axis of [outer, channels, inner]) and rows whose length has no
// fixed-shape kernel (outer = 1). Measured on MI355X, bf16, against the
// paths it replaced: [7, 4096, 8192] axis 1 201.7 -> 133.6 us; [2, 8192,
// 4096] 64.2 -> 41.9 us; rows [4096, 11008] 43.2 -> 29.6 us, [4096, 14336]
// 52.4 -> 34.4 us, [4096, 28672] 103.5 -> 63.1 us, [8192, 5120] 37.0 ->
// 30.2 us (k_rows_generic reads each row twice). 512 threads for every
// channel size: [8192, 5120] 37.0 us, [16, 4096, 512] 30.6 against 26.1 us.
constexpr int kChanWgThreads = 512;
constexpr int kChanWgMaxV = 16;
constexpr int kChanWgSmall = 2048;   // chunks: 256 threads up to here

bool chan_wg_applies(const void* x, const void* q, int64_t outer, int64_t inner) {
  const int64_t chunks = outer * (inner >> 3);
  return inner % 8 == 0 && aligned(x, 16) && aligned(q, 8) && chunks >= 256 &&
         chunks <= static_cast<int64_t>(kChanWgThreads) * kChanWgMaxV;
}

template <int DT>
int chan_wg_quant_t(const void* x, int64_t outer, int64_t channels, int64_t inner, float eps,
                    int8_t* q, float* scale, hipStream_t s, const char* what) {
  const int nchunks = static_cast<int>(outer * (inner >> 3));
  const dim3 g(static_cast<unsigned>(channels));
  if (nchunks <= kChanWgSmall) {
    const int v = static_cast<int>(cdiv(nchunks, 256));
    const dim3 b(256);
    if (v <= 2) k_chan_wg<DT, 2, 256><<<g, b, 0, s>>>(x, channels, inner, nchunks, eps, q, scale);
    else if (v <= 4) k_chan_wg<DT, 4, 256><<<g, b, 0, s>>>(x, channels, inner, nchunks, eps, q, scale);
    else k_chan_wg<DT, 8, 256><<<g, b, 0, s>>>(x, channels, inner, nchunks, eps, q, scale);
    return launch_status(what);
  }
  const int v = static_cast<int>(cdiv(nchunks, kChanWgThreads));
  const dim3 b(kChanWgThreads);
  if (v <= 8) k_chan_wg<DT, 8, kChanWgThreads><<<g, b, 0, s>>>(x, channels, inner, nchunks, eps, q, scale);
  else k_chan_wg<DT, kChanWgMaxV, kChanWgThreads><<<g, b, 0, s>>>(x, channels, inner, nchunks, eps, q, scale);
  return launch_status(what);
}

// Rows of cg < 512 chunks without a fixed-shape kernel: LPR lanes (a power
// of two, at most 64) x VPL chunks per row, the fewest slots that cover cg.
// Measured on MI355X, groups along the last axis of [16384, 14336] bf16,
// against k_rows_generic (a 256-thread workgroup per group, two reads):
// G = 56 3096.6 -> 114.4 us, G = 112 1624.7 -> 115.1 us, G = 224 869.6 ->
// 117.8 us, G = 896 285.0 -> 113.9 us, G = 1792 189.1 -> 113.5 us (G = 128:
// 112.7 us); G = 3584 117.5 us against 134.2 us in k_chan_wg, rows of 2056
// 24.7 against 35.5 us.
constexpr int kRowsAnyMaxChunks = 512;
template <int DT, int LPR, int VPL>
void launch_rows_sub_any(const void* x, int64_t rows, int cg, float eps, int8_t* q, float* scale,
                         hipStream_t s) {
  constexpr int RI = (LPR * VPL >= 64) ? 2 : 4;
  constexpr int64_t rows_per_wg = static_cast<int64_t>(kBlock / kWave) * RI * (kWave / LPR);
  k_rows_sub_any<DT, LPR, VPL, RI><<<dim3(static_cast<unsigned>(cdiv(rows, rows_per_wg))),
                                     dim3(kBlock), 0, s>>>(x, rows, cg, eps, q, scale);
}

template <int DT>
void rows_quant_any(const void* x, int64_t rows, int cg, float eps, int8_t* q, float* scale,
                    hipStream_t s) {
  if (cg <= 1) launch_rows_sub_any<DT, 1, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 2) launch_rows_sub_any<DT, 2, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 4) launch_rows_sub_any<DT, 4, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 8) launch_rows_sub_any<DT, 8, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 16) launch_rows_sub_any<DT, 16, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 32) launch_rows_sub_any<DT, 32, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 64) launch_rows_sub_any<DT, 64, 1>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 128) launch_rows_sub_any<DT, 64, 2>(x, rows, cg, eps, q, scale, s);
  else if (cg <= 256) launch_rows_sub_any<DT, 64, 4>(x, rows, cg, eps, q, scale, s);
  else launch_rows_sub_any<DT, 64, 8>(x, rows, cg, eps, q, scale, s);
}

template <int DT, int LPR, int VPL, int E>
void launch_rows_sub_any1(const void* x, int64_t rows, int L, float eps, int8_t* q, float* scale,
                          hipStream_t s) {
  constexpr int RI = VPL >= 16 ? 1 : 2;
  constexpr int64_t rows_per_wg = static_cast<int64_t>(kBlock / kWave) * RI * (kWave / LPR);
  k_rows_sub_any1<DT, LPR, VPL, RI, E><<<dim3(static_cast<unsigned>(cdiv(rows, rows_per_wg))),
                                         dim3(kBlock), 0, s>>>(x, rows, L, eps, q, scale);
}

constexpr int kRowsAny1Max = 2048;

template <int DT, int E>
void rows_quant_any1_e(const void* x, int64_t rows, int L, float eps, int8_t* q, float* scale,
                       hipStream_t s) {
  const int U = L / E;   // load units per row
  if (U <= 1) launch_rows_sub_any1<DT, 1, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 2) launch_rows_sub_any1<DT, 2, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 4) launch_rows_sub_any1<DT, 4, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 8) launch_rows_sub_any1<DT, 8, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 16) launch_rows_sub_any1<DT, 16, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 32) launch_rows_sub_any1<DT, 32, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 64) launch_rows_sub_any1<DT, 64, 1, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 128) launch_rows_sub_any1<DT, 64, 2, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 256) launch_rows_sub_any1<DT, 64, 4, E>(x, rows, L, eps, q, scale, s);
  else if (U <= 512) launch_rows_sub_any1<DT, 64, 8, E>(x, rows, L, eps, q, scale, s);
  else launch_rows_sub_any1<DT, 64, 16, E>(x, rows, L, eps, q, scale, s);
}

template <int DT>
void rows_quant_any1(const void* x, int64_t rows, int L, float eps, int8_t* q, float* scale,
                     hipStream_t s) {
  constexpr uintptr_t pair = DT == kF32 ? 8 : 4;
  if (L % 2 == 0 && aligned(x, pair) && aligned(q, 2))
    rows_quant_any1_e<DT, 2>(x, rows, L, eps, q, scale, s);
  else if (L <= 1024)
    rows_quant_any1_e<DT, 1>(x, rows, L, eps, q, scale, s);
  else
    launch_rows_sub_any1<DT, 64, 32, 1>(x, rows, L, eps, q, scale, s);
}

// Slices per row for the split-row path: enough workgroups for about four
// per CU, each slice at least kSplitMinChunks chunks; 1 (no split) when the
// one-workgroup-per-row kernels have enough rows. The split reads x twice,
// so it pays only where those kernels starve the CUs. Measured on MI355X,
// bf16, one workgroup per row -> split: [64, 2^20] 512.5 -> 63.6 us,
// [256, 262144] 146.7 -> 63.8 us, [8, 2^21] 1011.5 -> 21.1 us; against it
// [512, 65536] 24.2 -> 34.6 us and [255, 8200] 8.1 -> 10.3 us.
constexpr int64_t kSplitMinChunks = 1024;
constexpr int64_t kSplitMaxSlices = 256;

int64_t row_splits(int64_t rows, int64_t L) {
  if (L % 8 != 0 || rows <= 0 || rows > 65535) return 1;
  const int64_t n8 = L >> 3;
  const int64_t most = std::min<int64_t>(n8 / kSplitMinChunks, kSplitMaxSlices);
  if (most < 2) return 1;
  const int64_t cus = device_cus();
  const bool one_pass = n8 <= static_cast<int64_t>(kChanWgThreads) * kChanWgMaxV;
  if (rows >= 2 * cus || (one_pass && rows >= cus)) return 1;
  const int64_t sp = std::min(cdiv(4 * cus, rows), most);
  return sp >= 2 ? sp : 1;
}

size_t row_split_ws_bytes(int64_t rows, int64_t L) {
  const int64_t sp = row_splits(rows, L);
  return sp > 1 ? CBQ_WS_CTRL_BYTES + static_cast<size_t>(rows * sp) * 4 : CBQ_WS_CTRL_BYTES;
}

template <int DT>
int rows_split_quant_t(const void* x, int64_t rows, int64_t L, int64_t sp, float eps, void* ws,
                       int8_t* q, float* scale, hipStream_t s, const char* what) {
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + CBQ_WS_CTRL_BYTES);
  const int64_t sc = cdiv(L >> 3, sp);
  const dim3 g(static_cast<unsigned>(sp), static_cast<unsigned>(rows)), b(kBlock);
  k_rows_split_max<DT><<<g, b, 0, s>>>(x, L, sc, partial);
  k_rows_split_cast<DT><<<g, b, 0, s>>>(x, L, sc, partial, eps, q, scale);
  return launch_status(what);
}

template <int DT>
int rows_quant_t(const void* x, int64_t rows, int64_t L, float eps, int8_t* q, float* scale,
                 hipStream_t s, const char* what, void* ws = nullptr, size_t ws_bytes = 0) {
  CBQ_REQUIRE(rows <= 0x7fffffffLL, "%s: too many rows (%lld)", what, (long long)rows);
  const bool vec = (L % 8 == 0) && aligned(x, 16) && aligned(q, 8);
  if (vec && ws && aligned(ws, 16)) {
    // few long rows: slices of each row spread over the CUs
    const int64_t sp = row_splits(rows, L);
    if (sp > 1 && ws_bytes >= row_split_ws_bytes(rows, L))
      return rows_split_quant_t<DT>(x, rows, L, sp, eps, ws, q, scale, s, what);
  }
  if (vec) {
    switch (L) {
      case 8: launch_rows_sub<DT, 1, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 16: launch_rows_sub<DT, 2, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 32: launch_rows_sub<DT, 4, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 64: launch_rows_sub<DT, 8, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 128: launch_rows_sub<DT, 16, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 256: launch_rows_sub<DT, 32, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 512: launch_rows_sub<DT, 64, 1>(x, rows, eps, q, scale, s); return launch_status(what);
      case 1024: launch_rows_sub<DT, 64, 2>(x, rows, eps, q, scale, s); return launch_status(what);
      case 2048: launch_rows_sub<DT, 64, 4>(x, rows, eps, q, scale, s); return launch_status(what);
      case 4096:
        k_rows_wg<DT, 2><<<dim3(wg_rows_grid(rows)), dim3(kBlock), 0, s>>>(x, rows, eps, q, scale);
        return launch_status(what);
      case 8192:
        k_rows_wg<DT, 2, 512><<<dim3(wg_rows_grid(rows)), dim3(512), 0, s>>>(x, rows, eps, q, scale);
        return launch_status(what);
      case 16384:
        k_rows_wg<DT, 8><<<dim3(wg_rows_grid(rows)), dim3(kBlock), 0, s>>>(x, rows, eps, q, scale);
        return launch_status(what);
      default: break;
    }
    // other lengths: below 512 chunks several rows per wave, up to 8192 one
    // workgroup per row, in registers either way
    if ((L >> 3) < kRowsAnyMaxChunks) {
      rows_quant_any<DT>(x, rows, static_cast<int>(L >> 3), eps, q, scale, s);
      return launch_status(what);
    }
    if (chan_wg_applies(x, q, 1, L))
      return chan_wg_quant_t<DT>(x, 1, rows, L, eps, q, scale, s, what);
  } else if (L <= kRowsAny1Max) {
    // no 16-byte loads: several rows per wave with element loads
    rows_quant_any1<DT>(x, rows, static_cast<int>(L), eps, q, scale, s);
    return launch_status(what);
  }
  k_rows_generic<DT><<<dim3(wg_rows_grid(rows)), dim3(kBlock), 0, s>>>(
      x, rows, L, vec ? 1 : 0, eps, q, scale);
  return launch_status(what);
}

int rows_quant(const void* x, int dt, int64_t rows, int64_t L, float eps, int8_t* q, float* scale,
               hipStream_t s, const char* what, void* ws = nullptr, size_t ws_bytes = 0) {
  switch (dt) {
    case kF16: return rows_quant_t<kF16>(x, rows, L, eps, q, scale, s, what, ws, ws_bytes);
    case kBF16: return rows_quant_t<kBF16>(x, rows, L, eps, q, scale, s, what, ws, ws_bytes);
    default: return rows_quant_t<kF32>(x, rows, L, eps, q, scale, s, what, ws, ws_bytes);
  }
}

// Column quant geometry: the row-block count depends only on the shape so
// that the workspace size can be computed without a device.
struct ColGeom {
  int64_t col_blocks, nrb, RB;
  bool vec;
};

ColGeom col_geom(int64_t rows, int64_t cols, bool vec) {
  ColGeom g;
  g.vec = vec;
  g.col_blocks = vec ? cdiv(cdiv(cols, 8), kBlock) : cdiv(cols, kBlock);
  int64_t nrb = 1024 / (g.col_blocks > 0 ? g.col_blocks : 1);
  const int64_t max_nrb = cdiv(rows, 16);
  if (nrb > max_nrb) nrb = max_nrb;
  if (nrb > 65535) nrb = 65535;
  if (nrb < 1) nrb = 1;
  g.RB = cdiv(rows, nrb);
  g.nrb = cdiv(rows, g.RB);
  return g;
}

// Grid of the one-launch column quant (k_quant_cols_1pass) for x of rows x
// cols, or 0 when it does not apply: rows of 8192, 16384 or 32768 elements,
// at least kColsMinElems elements, a power-of-two grid of at most one
// workgroup per CU that splits the chunk-columns into slices of at most
// kColsMaxSlice.
int cols_1pass_grid(int64_t rows, int64_t cols) {
  if (cols != 8192 && cols != 16384 && cols != 32768) return 0;
  if (rows * cols < kColsMinElems) return 0;
  int g = 1;
  while (2 * g <= device_cus() && 2 * g <= kMaxFusedGrid) g *= 2;
  const int64_t c8 = cols / 8;
  if (c8 % g != 0 || c8 / g > kColsMaxSlice) return 0;
  return g;
}

// True if one workgroup of k_quant_cols_1pass<DT, CPT> fits on a CU, so that
// the whole grid is resident at once (cached per device and instantiation).
template <int DT, int CPT>
bool cols_1pass_fits() {
  static int cached[64];   // 0 unknown, 1 fits, 2 does not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (cached[dev] == 0) {
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &nb, reinterpret_cast<const void*>(&k_quant_cols_1pass<DT, CPT>), kFusedBlock, 0);
    cached[dev] = (e == hipSuccess && nb >= 1) ? 1 : 2;
  }
  return cached[dev] == 1;
}

size_t col_ws_bytes(int64_t rows, int64_t cols) {
  // The byte count does not depend on the vector path: nrb is computed for
  // the smaller (vector) column-block count, which never yields fewer row
  // blocks than the scalar path does. The one-launch path needs one [cols]
  // row of partial maxima per workgroup plus the [cols] multipliers.
  const ColGeom gv = col_geom(rows, cols, true);
  const ColGeom gs = col_geom(rows, cols, false);
  int64_t nrb = gv.nrb > gs.nrb ? gv.nrb : gs.nrb;
  const int64_t g1 = cols_1pass_grid(rows, cols);
  if (g1 > nrb) nrb = g1;
  return CBQ_WS_CTRL_BYTES + static_cast<size_t>(nrb) * cols * 4 + static_cast<size_t>(cols) * 4;
}

// Row blocking of the column cast (and of nothing else: the cast only needs
// the [cols] multipliers, so its geometry is independent of the partial
// maxima's). Short blocks keep many workgroups in flight; measured on
// MI355X at [28672, 8192] bf16: blocks of 4 rows (one batch of 4 loads per
// thread) 110.8 us, 2 rows 112.8, 8 rows 117.0, 16 rows 119.2, 1 row 127.9;
// walks of ~100 rows per thread lose ~25% of the bandwidth.
constexpr int64_t kCastRB = 4;
dim3 cast_grid(int64_t rows, int64_t col_blocks, int64_t& RB) {
  RB = kCastRB;
  if (cdiv(rows, RB) > 65535) RB = cdiv(rows, 65535);
  return dim3(static_cast<unsigned>(col_blocks), static_cast<unsigned>(cdiv(rows, RB)));
}

// Column path: per-column scales (inner == 1), or per-channel scales of the
// [rows, cols / inner, inner] view (inner adjacent columns per channel).
template <int DT>
int cols_quant_t(const void* x, int64_t rows, int64_t cols, int64_t inner, float eps, void* ws,
                 int8_t* q, float* scale, hipStream_t s, const char* what) {
  const bool vec = (cols % 8 == 0) && aligned(x, 16) && aligned(q, 8);
  if (vec && inner == 1 && rows * cols * elem_bytes<DT>() <= CBQ_COLS_1PASS_MAX_BYTES) {
    const int g1 = cols_1pass_grid(rows, cols);
    const int cpt = static_cast<int>(cols / 8192);
    if (g1 > 0 && (cpt == 1   ? cols_1pass_fits<DT, 1>()
                   : cpt == 2 ? cols_1pass_fits<DT, 2>()
                              : cols_1pass_fits<DT, 4>())) {
      char* ctl = static_cast<char*>(ws);
      float* part = reinterpret_cast<float*>(ctl + CBQ_WS_CTRL_BYTES);
      float* invs = part + static_cast<int64_t>(g1) * cols;
      const int64_t n8 = rows * cols / 8;
      const dim3 grid(static_cast<unsigned>(g1)), blk(kFusedBlock);
      if (cpt == 1)
        k_quant_cols_1pass<DT, 1><<<grid, blk, 0, s>>>(x, n8, eps, q, scale, ctl, part, invs,
                                                       fused_spin_limit());
      else if (cpt == 2)
        k_quant_cols_1pass<DT, 2><<<grid, blk, 0, s>>>(x, n8, eps, q, scale, ctl, part, invs,
                                                       fused_spin_limit());
      else
        k_quant_cols_1pass<DT, 4><<<grid, blk, 0, s>>>(x, n8, eps, q, scale, ctl, part, invs,
                                                       fused_spin_limit());
      return launch_status(what);
    }
  }
  const ColGeom g = col_geom(rows, cols, vec);
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + CBQ_WS_CTRL_BYTES);
  float* inv = partial + g.nrb * cols;
  const dim3 grid2(static_cast<unsigned>(g.col_blocks), static_cast<unsigned>(g.nrb));
  const int64_t u = cols >> 3;
  const bool narrow = vec && u <= kBlock / 2;
  const bool narrow1 = !vec && cols <= kBlock / 2;
  const int rpi = narrow ? kBlock / static_cast<int>(u)
                         : (narrow1 ? kBlock / static_cast<int>(cols) : 1);
  if (narrow1)
    k_colmax_narrow1<DT><<<grid2, dim3(kBlock), 0, s>>>(x, rows, cols, g.RB, rpi, partial);
  else if (narrow)
    k_colmax_narrow<DT><<<grid2, dim3(kBlock), 0, s>>>(x, rows, cols, g.RB, static_cast<int>(u),
                                                       rpi, partial);
  else
    k_colmax<DT><<<grid2, dim3(kBlock), 0, s>>>(x, rows, cols, g.RB, vec ? 1 : 0, partial);
  if (inner == 1)
    if (cols <= 1024)
      k_col_finalize<4><<<dim3(static_cast<unsigned>(cdiv(cols, 4))), dim3(kBlock), 0, s>>>(
          partial, g.nrb, cols, eps, inv, scale);
    else if (cols % 4 == 0)
      k_col_finalize4<<<dim3(static_cast<unsigned>(cdiv(cols, kFin4Cols))), dim3(kBlock), 0, s>>>(
          partial, g.nrb, cols, eps, inv, scale);
    else
      k_col_finalize<kFinCols><<<dim3(static_cast<unsigned>(cdiv(cols, kFinCols))), dim3(kBlock),
                                 0, s>>>(partial, g.nrb, cols, eps, inv, scale);
  else
    k_chan_finalize<<<dim3(static_cast<unsigned>(cols / inner)), dim3(kBlock), 0, s>>>(
        partial, g.nrb, cols, inner, eps, inv, scale);
  int64_t crb;
  if (narrow1) {
    // 2 kCastRB rows per thread, rpi threads per column
    crb = rpi * 2 * kCastRB;
    if (cdiv(rows, crb) > 65535) crb = cdiv(cdiv(rows, 65535), rpi) * rpi;
    k_cast_cols_narrow1<DT><<<dim3(1, static_cast<unsigned>(cdiv(rows, crb))), dim3(kBlock), 0,
                              s>>>(x, rows, cols, crb, rpi, inv, inner, q);
    return launch_status(what);
  }
  if (narrow) {
    // kCastRB rows per thread, rpi threads per column chunk
    crb = rpi * kCastRB;
    if (cdiv(rows, crb) > 65535) crb = cdiv(cdiv(rows, 65535), rpi) * rpi;
    k_cast_cols_narrow<DT><<<dim3(1, static_cast<unsigned>(cdiv(rows, crb))), dim3(kBlock), 0, s>>>(
        x, rows, cols, crb, static_cast<int>(u), rpi, inv, inner, q);
    return launch_status(what);
  }
  const dim3 cgrid = cast_grid(rows, g.col_blocks, crb);
  k_cast_cols<DT><<<cgrid, dim3(kBlock), 0, s>>>(x, rows, cols, crb, vec ? 1 : 0, inv, inner, q);
  return launch_status(what);
}

// Launch shape of k_group_tile for group size G: NW = the largest power of
// two <= 8 dividing G, rpt = G / NW positions per wave; 16 waves when 8 would
// hold more than kGtHold positions each (G > 128, G % 16 == 0), so that
// groups of up to 256 stay in registers. Measured on MI355X, groups of 256
// along axis 0 of [8192, 8192] bf16: 59.1 us with 16 waves, 65.8 us with 8
// (x read twice); at G = 128, 16 waves of 8 positions took 167.5 us against
// 128.3 us for 8 waves of 16.
int group_tile_waves(int64_t G) {
  if (G % 16 == 0 && G / 8 > kGtHold) return 16;
  return G % 8 == 0 ? 8 : G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
}

// Whether the tiled group path writes its scales through group-major
// scratch: ng > 1 (otherwise the movedim order is already contiguous) and
// 64 x 64 transpose tiles that fit a 32-bit grid.
bool group_scratch_applies(int64_t outer, int64_t ng, int64_t inner) {
  return ng > 1 && outer * cdiv(ng, static_cast<int64_t>(kTrTile)) *
                           cdiv(inner, static_cast<int64_t>(kTrTile)) < (1LL << 31);
}

template <int DT, int NW, bool TS>
void launch_group_tile_t(const void* x, int64_t outer, int64_t len, int64_t inner, int64_t G,
                         float eps, int8_t* q, float* scale, hipStream_t s) {
  const int64_t ng = len / G, tiles = cdiv(inner, kGtCols);
  const int64_t nblocks = outer * tiles * ng;
  const int rpt = static_cast<int>(G / NW);
  const dim3 grid(static_cast<unsigned>(nblocks)), block(NW * kWave);
  if (TS && NW >= 8 && rpt <= kGtHold) {
    // the scratch path of the usual group sizes (G % 8 == 0, G <= 128; with
    // 16 waves G <= 256): compile-time held count
    const int rc = rpt <= 1 ? 1 : rpt <= 2 ? 2 : rpt <= 4 ? 4 : rpt <= 8 ? 8 : 16;
    switch (rc) {
      case 1: k_group_tile<DT, NW, true, TS, 1><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles, nblocks, eps, q, scale); break;
      case 2: k_group_tile<DT, NW, true, TS, 2><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles, nblocks, eps, q, scale); break;
      case 4: k_group_tile<DT, NW, true, TS, 4><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles, nblocks, eps, q, scale); break;
      case 8: k_group_tile<DT, NW, true, TS, 8><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles, nblocks, eps, q, scale); break;
      default: k_group_tile<DT, NW, true, TS, 16><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles, nblocks, eps, q, scale); break;
    }
  } else if (rpt <= kGtHold)
    k_group_tile<DT, NW, true, TS><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles,
                                                          nblocks, eps, q, scale);
  else
    k_group_tile<DT, NW, false, TS><<<grid, block, 0, s>>>(x, len, inner, G, rpt, ng, tiles,
                                                           nblocks, eps, q, scale);
}

// tmp: group-major scratch of outer * ng * inner fp32, or null for direct
// scale writes.
template <int DT, int NW>
void launch_group_tile(const void* x, int64_t outer, int64_t len, int64_t inner, int64_t G,
                       float eps, int8_t* q, float* scale, float* tmp, hipStream_t s) {
  if (!tmp) {
    launch_group_tile_t<DT, NW, false>(x, outer, len, inner, G, eps, q, scale, s);
    return;
  }
  launch_group_tile_t<DT, NW, true>(x, outer, len, inner, G, eps, q, tmp, s);
  const int64_t ng = len / G;
  const int64_t gtiles = cdiv(ng, static_cast<int64_t>(kTrTile));
  const int64_t itiles = cdiv(inner, static_cast<int64_t>(kTrTile));
  k_transpose_f32<<<dim3(static_cast<unsigned>(outer * gtiles * itiles)), dim3(kBlock), 0, s>>>(
      tmp, ng, inner, gtiles, itiles, 1, (ng % 4 == 0 && aligned(scale, 16)) ? 1 : 0, scale);
}

template <int DT>
int group_strided_t(const void* x, int64_t outer, int64_t len, int64_t inner, int64_t G,
                    float eps, void* ws, size_t ws_bytes, int8_t* q, float* scale,
                    hipStream_t s, const char* what) {
  const int64_t ng = len / G;
  const bool tile = inner % 8 == 0 && aligned(x, 16) && aligned(q, 8) &&
                    outer * cdiv(inner, kGtCols) * ng < (1LL << 31);
  if (tile) {
    float* tmp = nullptr;
    if (ws && aligned(ws, 16) && group_scratch_applies(outer, ng, inner) &&
        ws_bytes >= CBQ_WS_CTRL_BYTES + static_cast<size_t>(outer * ng * inner) * 4)
      tmp = reinterpret_cast<float*>(static_cast<char*>(ws) + CBQ_WS_CTRL_BYTES);
    switch (group_tile_waves(G)) {
      case 16: launch_group_tile<DT, 16>(x, outer, len, inner, G, eps, q, scale, tmp, s); break;
      case 8: launch_group_tile<DT, 8>(x, outer, len, inner, G, eps, q, scale, tmp, s); break;
      case 4: launch_group_tile<DT, 4>(x, outer, len, inner, G, eps, q, scale, tmp, s); break;
      case 2: launch_group_tile<DT, 2>(x, outer, len, inner, G, eps, q, scale, tmp, s); break;
      default: launch_group_tile<DT, 1>(x, outer, len, inner, G, eps, q, scale, tmp, s); break;
    }
    return launch_status(what);
  }
  const int64_t threads = outer * ng * inner;
  k_group_strided<DT><<<dim3(static_cast<unsigned>(cdiv(threads, kBlock))), dim3(kBlock), 0, s>>>(
      x, outer, len, inner, G, eps, q, scale);
  return launch_status(what);
}

// N-D channel path, inner >= kSegInner: segment maxima (one wave per
// contiguous run of inner elements), channel maxima over outer, then the
// column cast with inner adjacent columns per channel. Shorter inner runs
// take the column path (column maxima per row block).
constexpr int64_t kSegInner = 512;
constexpr int64_t kSegMaxWg = 2048;

size_t seg_ws_bytes(int64_t outer, int64_t channels) {
  return CBQ_WS_CTRL_BYTES + static_cast<size_t>(outer * channels + channels) * 4;
}

size_t channel_nd_ws_bytes(int64_t outer, int64_t channels, int64_t inner) {
  return inner >= kSegInner ? seg_ws_bytes(outer, channels) : col_ws_bytes(outer, channels * inner);
}

template <int DT>
int seg_quant_t(const void* x, int64_t outer, int64_t channels, int64_t inner, float eps,
                void* ws, int8_t* q, float* scale, hipStream_t s, const char* what) {
  const int64_t segs = outer * channels, cols = channels * inner;
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + CBQ_WS_CTRL_BYTES);
  float* inv = partial + segs;
  const bool seg_vec = inner % 8 == 0 && aligned(x, 16);
  int64_t wg = cdiv(segs, kBlock / kWave);
  if (wg > kSegMaxWg) wg = kSegMaxWg;
  k_segmax<DT><<<dim3(static_cast<unsigned>(wg)), dim3(kBlock), 0, s>>>(x, segs, inner,
                                                                      seg_vec ? 1 : 0, partial);
  k_chan_finalize<<<dim3(static_cast<unsigned>(channels)), dim3(kBlock), 0, s>>>(
      partial, outer, channels, 1, eps, inv, scale);
  const bool vec = (cols % 8 == 0) && aligned(x, 16) && aligned(q, 8);
  const ColGeom g = col_geom(outer, cols, vec);
  int64_t crb;
  const dim3 cgrid = cast_grid(outer, g.col_blocks, crb);
  k_cast_cols<DT><<<cgrid, dim3(kBlock), 0, s>>>(x, outer, cols, crb, vec ? 1 : 0, inv, inner, q);
  return launch_status(what);
}

}  // namespace
}  // namespace cbq

// ---------------------------------------------------------------------------
// Scratch of cbq_quant_fp8_tensor_noalloc: the per-tensor workspace (control
// block + partial maxima) as device memory of the library, one copy per GPU,
// held until the process ends. Zero-initialised when the code object loads,
// which is the state the exchange protocol starts from; every call leaves it
// valid for the next (see k_quant_tensor_1pass), so nothing is cleared per
// call. Host code uses only the per-device address from hipGetSymbolAddress.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kNoAllocScratchBytes = 24576;
static_assert(cbq::tensor_ws_bytes() <= kNoAllocScratchBytes, "scratch too small");
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// Address of this device's copy of scratch (looked up once per device, with
// the device current).
int scratch_for_current_device(void** out, const char* what) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  CBQ_REQUIRE(e == hipSuccess && dev >= 0 && dev < 64, "%s: no current HIP device (%s)", what,
              hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t g = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (g != hipSuccess || !p) {
      cbq::set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                     hipGetErrorString(g));
      return CBQ_ELAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CBQ_OK;
}
}  // namespace

using namespace cbq;

extern "C" int cbq_quant_fp8_tensor_noalloc(const void* x, int dtype, int64_t n, float eps,
                                            uint8_t* q, float* scale, cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_quant_fp8_tensor_noalloc";
  // argument checks before any device call (as in tensor_quant)
  CBQ_REQUIRE(valid_dtype(dtype, false), "%s: unsupported input dtype code %d", what, dtype);
  CBQ_REQUIRE(n >= 0, "%s: negative element count", what);
  if (n == 0) return CBQ_OK;
  CBQ_REQUIRE(x && q && scale, "%s: null pointer", what);
  CBQ_REQUIRE(tensor_ws_bytes() <= kNoAllocScratchBytes,
              "%s: needs %zu bytes of scratch, the static array holds %zu", what,
              tensor_ws_bytes(), kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws, what);
  if (rc != CBQ_OK) return rc;
  return tensor_quant(x, dtype, n, eps, ws, kNoAllocScratchBytes, q, scale, true,
                      as_stream(stream));
}

extern "C" uint32_t cbq_set_tensor_spin_limit(uint32_t polls) {
  return spin_limit_var().exchange(polls, std::memory_order_relaxed);
}

extern "C" int cbq_tensor_quant_status(const void* ws, cbq_stream_t stream, int* status) {
  clear_error();
  const char* what = "cbq_tensor_quant_status";
  CBQ_REQUIRE(status, "%s: null status pointer", what);
  void* ctl = const_cast<void*>(ws);
  if (!ctl) {
    const int rc = scratch_for_current_device(&ctl, what);
    if (rc != CBQ_OK) return rc;
  }
  int32_t v = 0;
  const hipStream_t s = as_stream(stream);
  hipError_t e = hipMemcpyAsync(&v, static_cast<char*>(ctl) + kCtlStatus, sizeof(v),
                                hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    set_error("%s: reading the status word failed: %s", what, hipGetErrorString(e));
    return CBQ_ELAUNCH;
  }
  *status = v;
  return CBQ_OK;
}

extern "C" int cbq_tensor_quant_status_clear(void* ws, cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_tensor_quant_status_clear";
  void* ctl = ws;
  if (!ctl) {
    const int rc = scratch_for_current_device(&ctl, what);
    if (rc != CBQ_OK) return rc;
  }
  k_clear_tensor_status<<<dim3(1), dim3(1), 0, as_stream(stream)>>>(static_cast<char*>(ctl));
  return launch_status(what);
}

extern "C" int cbq_quant_fp8_tensor(const void* x, int dtype, int64_t n, float eps, void* ws,
                                    size_t ws_bytes, uint8_t* q, float* scale,
                                    cbq_stream_t stream) {
  clear_error();
  return tensor_quant(x, dtype, n, eps, ws, ws_bytes, q, scale, true, as_stream(stream));
}

extern "C" int cbq_quant_int8_tensor(const void* x, int dtype, int64_t n, float eps, void* ws,
                                     size_t ws_bytes, int8_t* q, float* scale,
                                     cbq_stream_t stream) {
  clear_error();
  return tensor_quant(x, dtype, n, eps, ws, ws_bytes, reinterpret_cast<uint8_t*>(q), scale, false,
                      as_stream(stream));
}

extern "C" size_t cbq_quant_tensor_ws_bytes(void) { return tensor_ws_bytes(); }

extern "C" size_t cbq_quant_int8_channel_ws_bytes(int64_t rows, int64_t cols, int axis) {
  if (rows <= 0 || cols <= 0) return CBQ_WS_CTRL_BYTES;
  return axis == 1 ? col_ws_bytes(rows, cols) : row_split_ws_bytes(rows, cols);
}

extern "C" int cbq_quant_int8_channel(const void* x, int dtype, int64_t rows, int64_t cols,
                                      int axis, float eps, void* ws, size_t ws_bytes, int8_t* q,
                                      float* scale, cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_quant_int8_channel";
  CBQ_REQUIRE(valid_dtype(dtype, true), "%s: unsupported input dtype code %d", what, dtype);
  CBQ_REQUIRE(axis == 0 || axis == 1, "%s: axis must be 0 or 1, got %d", what, axis);
  CBQ_REQUIRE(rows >= 0 && cols >= 0, "%s: negative shape", what);
  if (rows == 0 || cols == 0) return CBQ_OK;
  CBQ_REQUIRE(x && q && scale, "%s: null pointer", what);
  if (axis == 0)
    return rows_quant(x, dtype, rows, cols, eps, q, scale, as_stream(stream), what, ws, ws_bytes);
  const size_t need = col_ws_bytes(rows, cols);
  CBQ_REQUIRE(ws && ws_bytes >= need && aligned(ws, 16),
              "%s: axis 1 needs a 16-byte aligned workspace of %zu bytes, got %zu", what, need,
              ws_bytes);
  switch (dtype) {
    case kF16: return cols_quant_t<kF16>(x, rows, cols, 1, eps, ws, q, scale, as_stream(stream), what);
    case kBF16: return cols_quant_t<kBF16>(x, rows, cols, 1, eps, ws, q, scale, as_stream(stream), what);
    default: return cols_quant_t<kF32>(x, rows, cols, 1, eps, ws, q, scale, as_stream(stream), what);
  }
}

extern "C" size_t cbq_quant_int8_channel_nd_ws_bytes(int64_t outer, int64_t channels,
                                                     int64_t inner) {
  if (outer <= 0 || channels <= 0 || inner <= 0) return CBQ_WS_CTRL_BYTES;
  if (outer == 1) return row_split_ws_bytes(channels, inner);
  return channel_nd_ws_bytes(outer, channels, inner);
}

extern "C" int cbq_quant_int8_channel_nd(const void* x, int dtype, int64_t outer,
                                         int64_t channels, int64_t inner, float eps, void* ws,
                                         size_t ws_bytes, int8_t* q, float* scale,
                                         cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_quant_int8_channel_nd";
  CBQ_REQUIRE(valid_dtype(dtype, true), "%s: unsupported input dtype code %d", what, dtype);
  CBQ_REQUIRE(outer >= 0 && channels >= 0 && inner >= 0, "%s: negative shape", what);
  if (outer == 0 || channels == 0 || inner == 0) return CBQ_OK;
  CBQ_REQUIRE(x && q && scale, "%s: null pointer", what);
  if (outer == 1)   // channel axis leading: one row per channel
    return rows_quant(x, dtype, channels, inner, eps, q, scale, as_stream(stream), what, ws,
                      ws_bytes);
  const size_t need = channel_nd_ws_bytes(outer, channels, inner);
  CBQ_REQUIRE(ws && ws_bytes >= need && aligned(ws, 16),
              "%s: needs a 16-byte aligned workspace of %zu bytes, got %zu", what, need, ws_bytes);
  CBQ_REQUIRE(channels <= 0x7fffffffLL, "%s: too many channels (%lld)", what,
              (long long)channels);
  if (chan_wg_applies(x, q, outer, inner)) {
    switch (dtype) {
      case kF16: return chan_wg_quant_t<kF16>(x, outer, channels, inner, eps, q, scale, as_stream(stream), what);
      case kBF16: return chan_wg_quant_t<kBF16>(x, outer, channels, inner, eps, q, scale, as_stream(stream), what);
      default: return chan_wg_quant_t<kF32>(x, outer, channels, inner, eps, q, scale, as_stream(stream), what);
    }
  }
  const int64_t cols = channels * inner;
  if (inner >= kSegInner) {
    switch (dtype) {
      case kF16:
        return seg_quant_t<kF16>(x, outer, channels, inner, eps, ws, q, scale, as_stream(stream), what);
      case kBF16:
        return seg_quant_t<kBF16>(x, outer, channels, inner, eps, ws, q, scale, as_stream(stream), what);
      default:
        return seg_quant_t<kF32>(x, outer, channels, inner, eps, ws, q, scale, as_stream(stream), what);
    }
  }
  switch (dtype) {
    case kF16:
      return cols_quant_t<kF16>(x, outer, cols, inner, eps, ws, q, scale, as_stream(stream), what);
    case kBF16:
      return cols_quant_t<kBF16>(x, outer, cols, inner, eps, ws, q, scale, as_stream(stream), what);
    default:
      return cols_quant_t<kF32>(x, outer, cols, inner, eps, ws, q, scale, as_stream(stream), what);
  }
}

extern "C" int cbq_quant_int8_group(const void* x, int dtype, int64_t num_groups,
                                    int64_t group_size, float eps, int8_t* q, float* scale,
                                    cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_quant_int8_group";
  CBQ_REQUIRE(valid_dtype(dtype, true), "%s: unsupported input dtype code %d", what, dtype);
  CBQ_REQUIRE(group_size > 0 && group_size <= 4096, "%s: group_size must be in (0, 4096], got %lld",
              what, (long long)group_size);
  CBQ_REQUIRE(num_groups >= 0, "%s: negative group count", what);
  if (num_groups == 0) return CBQ_OK;
  CBQ_REQUIRE(x && q && scale, "%s: null pointer", what);
  return rows_quant(x, dtype, num_groups, group_size, eps, q, scale, as_stream(stream), what);
}

extern "C" size_t cbq_quant_int8_group_nd_ws_bytes(int64_t outer, int64_t len, int64_t inner,
                                                   int64_t group_size) {
  if (outer <= 0 || len <= 0 || inner <= 1 || group_size <= 0 || len % group_size != 0 ||
      inner % 8 != 0)
    return CBQ_WS_CTRL_BYTES;
  const int64_t ng = len / group_size;
  if (!group_scratch_applies(outer, ng, inner)) return CBQ_WS_CTRL_BYTES;
  return CBQ_WS_CTRL_BYTES + static_cast<size_t>(outer * ng * inner) * 4;
}

extern "C" int cbq_quant_int8_group_nd(const void* x, int dtype, int64_t outer, int64_t len,
                                       int64_t inner, int64_t group_size, float eps, void* ws,
                                       size_t ws_bytes, int8_t* q, float* scale,
                                       cbq_stream_t stream) {
  clear_error();
  const char* what = "cbq_quant_int8_group_nd";
  CBQ_REQUIRE(valid_dtype(dtype, true), "%s: unsupported input dtype code %d", what, dtype);
  CBQ_REQUIRE(group_size > 0 && group_size <= 4096, "%s: group_size must be in (0, 4096], got %lld",
              what, (long long)group_size);
  CBQ_REQUIRE(outer >= 0 && len >= 0 && inner >= 0, "%s: negative shape", what);
  CBQ_REQUIRE(len % group_size == 0, "%s: group_size %lld must divide the axis length %lld", what,
              (long long)group_size, (long long)len);
  if (outer == 0 || len == 0 || inner == 0) return CBQ_OK;
  CBQ_REQUIRE(x && q && scale, "%s: null pointer", what);
  CBQ_REQUIRE(cdiv(outer * (len / group_size) * inner, kBlock) < (1LL << 31),
              "%s: too many groups", what);
  if (inner == 1)   // groups along the last axis are contiguous rows
    return rows_quant(x, dtype, outer * (len / group_size), group_size, eps, q, scale,
                      as_stream(stream), what);
  switch (dtype) {
    case kF16: return group_strided_t<kF16>(x, outer, len, inner, group_size, eps, ws, ws_bytes, q, scale, as_stream(stream), what);
    case kBF16: return group_strided_t<kBF16>(x, outer, len, inner, group_size, eps, ws, ws_bytes, q, scale, as_stream(stream), what);
    default: return group_strided_t<kF32>(x, outer, len, inner, group_size, eps, ws, ws_bytes, q, scale, as_stream(stream), what);
  }
}
