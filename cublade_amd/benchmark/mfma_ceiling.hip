// mfma_ceiling - the matrix-core rate this GPU sustains with nothing but
// MFMAs in flight: the ceiling the GEMM kernels' TFLOP/s are read against
// (the published dense peaks are 2.5 PFLOP/s fp16 / bf16 and 5.0 POP/s int8).
//
// Every wave of a full grid (one workgroup per CU, 1 or 2 waves per SIMD)
// runs a long chain of v_mfma_f32_32x32x16_{f16,bf16} or
// v_mfma_i32_32x32x32_i8 on operands held in registers, over 4 independent
// accumulators, and stores the accumulators at the end. The operands are
// random or all zero: the MFMA rate under load depends on the power the
// operand bits draw. Times are the median of 7 launches of about 300 us,
// HIP events around each.
//
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 mfma_ceiling.hip -o mfma_ceiling
//   ./mfma_ceiling
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x)                                                                  \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                            \
    }                                                                          \
  } while (0)

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef int i16x __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

namespace {

enum { kF16 = 0, kBF16 = 1, kI8 = 2 };
constexpr int kAcc = 4;   // independent accumulators per wave

template <int T>
__global__ __launch_bounds__(512) void k_mfma(const u32x4* __restrict__ src, int iters,
                                              float* __restrict__ out) {
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  const u32x4 a = src[(tid * 2) & 4095], b = src[(tid * 2 + 1) & 4095];
  if constexpr (T == kI8) {
    i16x acc[kAcc];
#pragma unroll
    for (int u = 0; u < kAcc; ++u) acc[u] = i16x{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int u = 0; u < kAcc; ++u)
        acc[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i4, a),
                                                       __builtin_bit_cast(i4, b), acc[u], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < kAcc; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += static_cast<float>(acc[u][r]);
    out[tid] = s;
  } else {
    f16x acc[kAcc];
#pragma unroll
    for (int u = 0; u < kAcc; ++u) acc[u] = f16x{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int u = 0; u < kAcc; ++u) {
        if constexpr (T == kF16)
          acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, a),
                                                          __builtin_bit_cast(h8, b), acc[u], 0, 0, 0);
        else
          acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8, a),
                                                           __builtin_bit_cast(b8, b), acc[u], 0, 0, 0);
      }
    }
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < kAcc; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[u][r];
    out[tid] = s;
  }
}

}  // namespace

int main() {
  int cus = 0;
  CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  // operands: random bit patterns that are finite, moderate fp16 / bf16
  // values (exponent bits kept in range), or zeros
  std::vector<unsigned> rnd(4096 * 4);
  unsigned st = 2024;
  for (auto& v : rnd) {
    st = st * 1664525u + 1013904223u;
    v = st & 0xbbffbbffu;   // clears a high exponent bit of each 16-bit half: finite values
  }
  u32x4 *src_r, *src_z;
  CK(hipMalloc(&src_r, rnd.size() * 4));
  CK(hipMalloc(&src_z, rnd.size() * 4));
  CK(hipMemcpy(src_r, rnd.data(), rnd.size() * 4, hipMemcpyHostToDevice));
  CK(hipMemset(src_z, 0, rnd.size() * 4));
  float* out;
  CK(hipMalloc(&out, static_cast<size_t>(cus) * 512 * 4));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  std::printf("# MFMA-only rate, one workgroup per CU (%d CUs), %d independent accumulators per wave,\n"
              "# median of 7 launches (HIP events); peak = published dense figure\n", cus, kAcc);
  std::printf("%-28s %-8s %-8s %9s %12s %7s\n", "instruction", "waves/SIMD", "operands", "us",
              "TFLOP(OP)/s", "frac");
  struct Case { int t; const char* name; double flop; double peak; };
  const Case cases[] = {{kF16, "v_mfma_f32_32x32x16_f16", 32.0 * 32 * 16 * 2, 2.5e15},
                        {kBF16, "v_mfma_f32_32x32x16_bf16", 32.0 * 32 * 16 * 2, 2.5e15},
                        {kI8, "v_mfma_i32_32x32x32_i8", 32.0 * 32 * 32 * 2, 5.0e15}};
  for (const Case& c : cases)
    for (int wps : {1, 2})
      for (int z = 0; z < 2; ++z) {
        const int threads = 256 * wps;
        const int iters = c.t == kI8 ? 1200 : 2400;   // about 300 us at the measured rates
        const u32x4* src = z ? src_z : src_r;
        auto launch = [&] {
          if (c.t == kF16) k_mfma<kF16><<<cus, threads>>>(src, iters, out);
          else if (c.t == kBF16) k_mfma<kBF16><<<cus, threads>>>(src, iters, out);
          else k_mfma<kI8><<<cus, threads>>>(src, iters, out);
        };
        launch();
        CK(hipDeviceSynchronize());
        std::vector<float> v;
        for (int rep = 0; rep < 7; ++rep) {
          CK(hipEventRecord(e0));
          launch();
          CK(hipEventRecord(e1));
          CK(hipEventSynchronize(e1));
          float ms;
          CK(hipEventElapsedTime(&ms, e0, e1));
          v.push_back(ms * 1000.0f);
        }
        std::sort(v.begin(), v.end());
        const double us = v[v.size() / 2];
        const double waves = static_cast<double>(cus) * 4 * wps;
        const double rate = waves * iters * kAcc * c.flop / (us * 1e-6);
        std::printf("%-28s %-10d %-8s %9.2f %12.1f %7.3f\n", c.name, wps, z ? "zero" : "random", us,
                    rate / 1e12, rate / c.peak);
        std::fflush(stdout);
      }
  return 0;
}
