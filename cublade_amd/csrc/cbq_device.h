// cbq_device.h - gfx950 device primitives shared by the quantization kernels.
//
// Element conversions, 8-element chunk loads/stores, the INT8 / FP8 E4M3
// encoders and wave64 cross-lane max reductions. Numerics restate the
// reference's shared headers:
//   kernels/cuda/quantization/fp8_pack.cuh:26-75  (exact widening to fp32,
//       round-to-nearest-even narrowing to fp16/bf16, FP8 -> 16-bit exact)
//   kernels/cuda/quantization/int8_pack.cuh:51-56 (round half to even, clamp
//       to [-127, 127])
//   kernels/cuda/quantization/quantize_per_tensor_fp8.cu:117,129 (E4M3 cast
//       with saturation to +-448, NaN kept)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbq {

enum : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

constexpr int kWave = 64;
constexpr int kBlock = 256;          // 4 waves per workgroup
constexpr float kQmaxInt8 = 127.0f;
constexpr float kQmaxFp8 = 448.0f;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Streaming loads and stores. Data read once (quantization inputs, codes to
// dequantize) is loaded non-temporally so it does not allocate in the
// Infinity Cache: measured on MI355X, 16-byte streaming reads reach ~6.8 TB/s
// that way against ~3.8 TB/s with ordinary loads once the cache holds dirty
// lines. Narrow outputs (8-byte code stores) are stored non-temporally too;
// wide outputs (16-byte dequantized stores) are faster as ordinary stores.
// The three switches are compile-time tuning knobs.
// ---------------------------------------------------------------------------
#ifndef CBQ_NT_LOADS
#define CBQ_NT_LOADS 1
#endif
#ifndef CBQ_NT_STORES_NARROW
#define CBQ_NT_STORES_NARROW 1
#endif
#ifndef CBQ_NT_STORES_WIDE
#define CBQ_NT_STORES_WIDE 0
#endif
// The per-tensor amax pass: its input is read again by the cast pass, so an
// ordinary (allocating) load can leave it in the Infinity Cache for the cast.
#ifndef CBQ_NT_LOADS_AMAX
#define CBQ_NT_LOADS_AMAX 1
#endif

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <bool NT = (CBQ_NT_LOADS != 0)>
__device__ __forceinline__ uint4 ldg16(const void* p) {
  u32x4 v;
  if constexpr (NT) v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  else v = *static_cast<const u32x4*>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 ldg8(const void* p) {
#if CBQ_NT_LOADS
  const u32x2 v = __builtin_nontemporal_load(static_cast<const u32x2*>(p));
#else
  const u32x2 v = *static_cast<const u32x2*>(p);
#endif
  return make_uint2(v.x, v.y);
}

__device__ __forceinline__ void stg8(void* p, uint2 v) {
#if CBQ_NT_STORES_NARROW
  __builtin_nontemporal_store(u32x2{v.x, v.y}, static_cast<u32x2*>(p));
#else
  *static_cast<u32x2*>(p) = u32x2{v.x, v.y};
#endif
}

__device__ __forceinline__ void stg16(void* p, uint4 v) {
#if CBQ_NT_STORES_WIDE
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, static_cast<u32x4*>(p));
#else
  *static_cast<u32x4*>(p) = u32x4{v.x, v.y, v.z, v.w};
#endif
}

// ---------------------------------------------------------------------------
// Raw 8-element chunks: one 16-byte load for 2-byte types, two for fp32.
// ---------------------------------------------------------------------------
template <int DT> struct Raw8 { uint4 a; };
template <> struct Raw8<kF32> { uint4 a, b; };

template <int DT> constexpr int elem_bytes() { return DT == kF32 ? 4 : 2; }

// Marks a held chunk as changed, so that a second conversion of it is
// recomputed from the raw words instead of keeping the first conversion's
// fp32 values live (which doubles the registers a held row or group needs).
template <int DT>
__device__ __forceinline__ void reload_barrier(Raw8<DT>& r) {
  asm volatile("" : "+v"(r.a.x), "+v"(r.a.y), "+v"(r.a.z), "+v"(r.a.w));
  if constexpr (DT == kF32) asm volatile("" : "+v"(r.b.x), "+v"(r.b.y), "+v"(r.b.z), "+v"(r.b.w));
}

template <int DT, bool NT = (CBQ_NT_LOADS != 0)>
__device__ __forceinline__ Raw8<DT> ld8(const void* base, int64_t elem) {
  Raw8<DT> r;
  const char* p = static_cast<const char*>(base) + elem * elem_bytes<DT>();
  r.a = ldg16<NT>(p);
  if constexpr (DT == kF32) r.b = ldg16<NT>(p + 16);
  return r;
}

__device__ __forceinline__ f32x2 bf16x2_to_f32(uint32_t w) {
  f32x2 f;
  f.x = __uint_as_float(w << 16);
  f.y = __uint_as_float(w & 0xffff0000u);
  return f;
}

__device__ __forceinline__ f32x2 f16x2_to_f32(uint32_t w) {
  return __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
}

template <int DT>
__device__ __forceinline__ f32x2 pair_to_f32(uint32_t w) {
  if constexpr (DT == kBF16) return bf16x2_to_f32(w);
  else return f16x2_to_f32(w);
}

template <int DT>
__device__ __forceinline__ void cvt8(const Raw8<DT>& r, float (&f)[8]) {
  if constexpr (DT == kF32) {
    f[0] = __uint_as_float(r.a.x); f[1] = __uint_as_float(r.a.y);
    f[2] = __uint_as_float(r.a.z); f[3] = __uint_as_float(r.a.w);
    f[4] = __uint_as_float(r.b.x); f[5] = __uint_as_float(r.b.y);
    f[6] = __uint_as_float(r.b.z); f[7] = __uint_as_float(r.b.w);
  } else {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f32x2 p = pair_to_f32<DT>(w[k]);
      f[2 * k] = p.x;
      f[2 * k + 1] = p.y;
    }
  }
}

// One element at an arbitrary index (scalar paths and tails).
template <int DT>
__device__ __forceinline__ float ld1(const void* base, int64_t i) {
  if constexpr (DT == kF32) {
    return static_cast<const float*>(base)[i];
  } else {
    const uint32_t h = static_cast<const uint16_t*>(base)[i];
    if constexpr (DT == kBF16) return __uint_as_float(h << 16);
    else return static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)h));
  }
}

// |x| max over a chunk. fmaxf returns the non-NaN operand, so NaN inputs are
// ignored exactly as the reference's fmaxf fold does.
__device__ __forceinline__ float absmax8(const float (&f)[8], float m) {
#pragma unroll
  for (int k = 0; k < 8; ++k) m = fmaxf(m, __builtin_fabsf(f[k]));
  return m;
}

// ---------------------------------------------------------------------------
// Output narrowing (round to nearest even).
// ---------------------------------------------------------------------------
template <int OUT>
__device__ __forceinline__ uint32_t pack2_out(float a, float b) {
  f32x2 v = {a, b};
  if constexpr (OUT == kBF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
}

// Scalar narrowing. The empty asm pins `a` as a finished fp32 value: without
// it the compiler folds a preceding multiply into v_fma_mixlo_f16 (a*b + 0,
// rounded once to fp16), which turns -0 into +0 and skips the fp32 rounding
// of the product that the reference performs.
template <int OUT>
__device__ __forceinline__ uint16_t out1(float a) {
  asm volatile("" : "+v"(a));
  return static_cast<uint16_t>(pack2_out<OUT>(a, 0.0f) & 0xffffu);
}

template <int OUT>
__device__ __forceinline__ uint4 pack8_out(const float (&f)[8]) {
  uint4 o;
  o.x = pack2_out<OUT>(f[0], f[1]);
  o.y = pack2_out<OUT>(f[2], f[3]);
  o.z = pack2_out<OUT>(f[4], f[5]);
  o.w = pack2_out<OUT>(f[6], f[7]);
  return o;
}

// ---------------------------------------------------------------------------
// INT8 encoder: round half to even, clamp to [-127, 127], NaN -> 0.
// ---------------------------------------------------------------------------
// Three VALU operations: v_rndne_f32 (ties to even), v_cvt_i32_f32 (the
// hardware conversion saturates out-of-range values and turns NaN into 0),
// and v_med3_i32 for the clamp. Same results as clamping in fp32 first.
__device__ __forceinline__ int q_int8(float v) {
  const float r = __builtin_rintf(v);
  int i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(r));
  return i < -127 ? -127 : (i > 127 ? 127 : i);
}

// Low bytes of four integers as one word, a in byte 0 (two v_perm_b32 and
// an or: selector nibbles 0-3 pick the second operand's bytes, 4-7 the
// first's, 0xc a zero byte).
__device__ __forceinline__ uint32_t pack4_low_bytes(int a, int b, int c, int d) {
  const uint32_t ab = __builtin_amdgcn_perm(static_cast<uint32_t>(b), static_cast<uint32_t>(a),
                                            0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(static_cast<uint32_t>(d), static_cast<uint32_t>(c),
                                            0x04000c0cu);
  return ab | cd;
}

__device__ __forceinline__ uint2 pack8_int8(const float (&f)[8], float inv) {
  uint32_t w[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    w[h] = pack4_low_bytes(q_int8(f[4 * h + 0] * inv), q_int8(f[4 * h + 1] * inv),
                           q_int8(f[4 * h + 2] * inv), q_int8(f[4 * h + 3] * inv));
  return make_uint2(w[0], w[1]);
}

// ---------------------------------------------------------------------------
// FP8 E4M3 (OCP e4m3fn) encoder. gfx950's v_cvt_pk_fp8_f32 rounds to nearest
// even; the explicit clamp gives the +-448 saturation and passes NaN through.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sat448(float v) {
  return __builtin_fabsf(v) > kQmaxFp8 ? __builtin_copysignf(kQmaxFp8, v) : v;
}

__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), w, true);
  return static_cast<uint32_t>(w);
}

__device__ __forceinline__ uint2 pack8_fp8(const float (&f)[8], float inv) {
  return make_uint2(pack4_fp8(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv),
                    pack4_fp8(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv));
}

__device__ __forceinline__ uint8_t q_fp8_1(float v) {
  return static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(sat448(v), 0.0f, 0, false) & 0xff);
}

// FP8 E4M3 -> fp32, exact (hardware conversion, OCP format on gfx950).
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float* f) {
  f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  f[0] = lo.x; f[1] = lo.y; f[2] = hi.x; f[3] = hi.y;
}

__device__ __forceinline__ void int8x4_to_f32(uint32_t w, float* f) {
  f[0] = static_cast<float>(static_cast<int8_t>(w & 0xffu));
  f[1] = static_cast<float>(static_cast<int8_t>((w >> 8) & 0xffu));
  f[2] = static_cast<float>(static_cast<int8_t>((w >> 16) & 0xffu));
  f[3] = static_cast<float>(static_cast<int8_t>(w >> 24));
}

// ---------------------------------------------------------------------------
// Cross-lane max over aligned groups of LPR lanes (LPR a power of two <= 64).
// Within a 16-lane DPP row: quad_perm xor-1, quad_perm xor-2, row_half_mirror,
// row_mirror; across rows: ds_bpermute shuffles. Every lane of a group ends
// with the group's maximum. All 64 lanes must be active.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int LPR>
__device__ __forceinline__ float group_max(float m) {
  static_assert(LPR >= 1 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "LPR");
  if constexpr (LPR >= 2) m = fmaxf(m, dpp_f32<0xB1>(m));   // quad_perm [1,0,3,2]
  if constexpr (LPR >= 4) m = fmaxf(m, dpp_f32<0x4E>(m));   // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) m = fmaxf(m, dpp_f32<0x141>(m));  // row_half_mirror
  if constexpr (LPR >= 16) m = fmaxf(m, dpp_f32<0x140>(m)); // row_mirror
  if constexpr (LPR >= 32) m = fmaxf(m, __shfl_xor(m, 16, kWave));
  if constexpr (LPR >= 64) m = fmaxf(m, __shfl_xor(m, 32, kWave));
  return m;
}

// Workgroup-wide max; every thread gets the result. `red` holds one slot per
// wave. Contains a barrier: call from uniform control flow only.
__device__ __forceinline__ float block_max(float m, float* red) {
  m = group_max<kWave>(m);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) red[wave] = m;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < static_cast<int>(blockDim.x) / kWave; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

// Workgroup order for grids whose neighbouring workgroups share cache lines
// (scales of adjacent groups): the dispatcher deals workgroups to the 8 XCDs
// round-robin, so hardware index b runs on XCD b % 8. The remap gives XCD k a
// contiguous run of logical indices; the last nb % 8 indices map to
// themselves.
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nb) {
  const int64_t per = nb >> 3;
  return b < (per << 3) ? (b & 7) * per + (b >> 3) : b;
}

// Per-channel values of 8 adjacent columns c .. c + 7 of a [rows, channels *
// inner] view (channel = column / inner) with at most one 64-bit division:
// inner == 1, every column its own channel; inner >= 8, at most one channel
// boundary among the 8. (Eight divisions per thread cost more than the
// loads they serve once a thread's row block is short.)
__device__ __forceinline__ void channel_vals8(const float* __restrict__ v, int64_t c,
                                              int64_t inner, float (&out)[8]) {
  if (inner == 1) {
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = v[c + k];
  } else if (inner >= 8) {
    const int64_t ch0 = c / inner, rem = c - ch0 * inner;
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = v[ch0 + (rem + k >= inner ? 1 : 0)];
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = v[(c + k) / inner];
  }
}

// fp32 transpose of outer stacked matrices, src [R, C] -> dst [C, R] each
// (the group scale orders: group-major [ng, inner] and the movedim order
// [inner, ng]): 64 x 64 tiles through LDS (row stride 65 floats: no bank
// conflicts on the transposed read), 256 threads. vld: 16-byte loads
// (C % 4 == 0, 16-byte aligned src); vst: 16-byte stores (R % 4 == 0,
// 16-byte aligned dst); else 4-byte accesses (4-byte accesses on both sides
// took 8.8 us, 16-byte ones 5.3 us, for the 7.3 MB of scales of groups of
// 128 along axis 0 of [16384, 14336] on MI355X). Workgroup b: the matrix,
// then the row tile, then the column tile fastest. (A kernel in a header:
// internal linkage, one copy per source that launches it.)
constexpr int kTrTile = 64;

namespace {
__global__ __launch_bounds__(kBlock) void k_transpose_f32(const float* __restrict__ src,
                                                          int64_t R, int64_t C, int64_t rtiles,
                                                          int64_t ctiles, int vld, int vst,
                                                          float* __restrict__ dst) {
  __shared__ float t[kTrTile][kTrTile + 1];
  const int64_t b = blockIdx.x;
  const int64_t ct = b % ctiles, rt = (b / ctiles) % rtiles, o = b / (ctiles * rtiles);
  const int64_t r0 = rt * kTrTile, c0 = ct * kTrTile;
  const float* sm = src + o * R * C;
  float* dm = dst + o * R * C;
  if (vld) {
    const int c4 = threadIdx.x % 16, q0 = threadIdx.x / 16;
#pragma unroll
    for (int k = 0; k < kTrTile / 16; ++k) {
      const int r = q0 + 16 * k;
      if (r0 + r < R && c0 + 4 * c4 < C) {
        const float4 v = *reinterpret_cast<const float4*>(sm + (r0 + r) * C + c0 + 4 * c4);
        t[r][4 * c4] = v.x; t[r][4 * c4 + 1] = v.y; t[r][4 * c4 + 2] = v.z; t[r][4 * c4 + 3] = v.w;
      }
    }
  } else {
    const int c = threadIdx.x % kTrTile, q0 = threadIdx.x / kTrTile;
#pragma unroll
    for (int k = 0; k < kTrTile / 4; ++k) {
      const int r = q0 + 4 * k;
      if (r0 + r < R && c0 + c < C) t[r][c] = sm[(r0 + r) * C + c0 + c];
    }
  }
  __syncthreads();
  if (vst) {
    const int r4 = threadIdx.x % 16, q0 = threadIdx.x / 16;
#pragma unroll
    for (int k = 0; k < kTrTile / 16; ++k) {
      const int c = q0 + 16 * k;   // a dst row
      if (c0 + c < C && r0 + 4 * r4 < R)
        *reinterpret_cast<float4*>(dm + (c0 + c) * R + r0 + 4 * r4) =
            make_float4(t[4 * r4][c], t[4 * r4 + 1][c], t[4 * r4 + 2][c], t[4 * r4 + 3][c]);
    }
  } else {
    const int r = threadIdx.x % kTrTile, q0 = threadIdx.x / kTrTile;
#pragma unroll
    for (int k = 0; k < kTrTile / 4; ++k) {
      const int c = q0 + 4 * k;
      if (c0 + c < C && r0 + r < R) dm[(c0 + c) * R + r0 + r] = t[r][c];
    }
  }
}
}  // namespace

// Raw buffer resources (gfx9 word 3: 32-bit dword data format) and the
// cache-policy argument of the buffer load / store builtins: kAuxNT marks an
// access non-temporal, kAuxSc1 gives it device (agent) scope, the bits the
// compiler uses for agent-scope atomic loads and stores on gfx950.
constexpr int kBufDword3 = 0x00020000;
constexpr int kAuxNT = 2;
constexpr int kAuxSc1 = 16;

// Reciprocal scale and stored scale, both correctly rounded fp32 divisions
// (quantize_int8.cu:120-126 computes them in double and narrows once, which
// is the same value; quantize_per_tensor_fp8.cu:99-102 intends the same).
__device__ __forceinline__ float inv_scale(float amax, float eps, float qmax) {
  return qmax / fmaxf(amax, eps);
}

}  // namespace cbq
