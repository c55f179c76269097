// stream_ceiling - bare HBM stream rates on this GPU for the access mixes of
// the quant / dequant kernels, as the ceilings their roofline fractions are
// read against. No arithmetic: each kernel only moves bytes.
//
//   quant mix    16-byte loads, 8-byte stores (2 bytes in per byte out)
//   dequant mix  8-byte loads, 16-byte stores
//   read only    16-byte loads (the amax / column-max passes)
//
// First the timing floor: an event pair with nothing between and an empty
// kernel, after the same sweep. Each stream is timed as a one-shot grid (one
// 16-byte chunk per thread and step, U steps per thread, all loads issued
// first) and as a persistent grid-stride
// loop, with non-temporal or ordinary stores, after a read-only ("clean") and
// a write ("dirty") 512 MiB sweep that evicts the 256 MB Infinity Cache. Sizes:
// BASELINE configs 1 (16 Mi bf16 elements), 2 (64 Mi fp16 elements) and 3
// (28672 x 8192 bf16).
// Fractions are of 8 TB/s over the bytes moved.
//
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 stream_ceiling.hip -o stream_ceiling
//   ./stream_ceiling
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

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

namespace {

template <bool NT>
__device__ __forceinline__ void st8(u32x2* p, u32x2 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <bool NT>
__device__ __forceinline__ void st16(u32x4* p, u32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// quant mix, one-shot: thread t of workgroup b takes chunks b*256*U + t + u*256
template <int U, bool NTS>
__global__ __launch_bounds__(256) void k_q1(const u32x4* __restrict__ x, long n16,
                                            u32x2* __restrict__ q) {
  const long b0 = static_cast<long>(blockIdx.x) * 256 * U + threadIdx.x;
  u32x4 r[U];
#pragma unroll
  for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(x + std::min(b0 + u * 256, n16 - 1));
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (b0 + u * 256 < n16) st8<NTS>(q + b0 + u * 256, u32x2{r[u].x ^ r[u].y, r[u].z ^ r[u].w});
}

// quant mix, persistent grid-stride
template <int U, bool NTS>
__global__ __launch_bounds__(256) void k_qp(const u32x4* __restrict__ x, long n16,
                                            u32x2* __restrict__ q) {
  const long step = static_cast<long>(gridDim.x) * 256 * U;
  for (long b0 = static_cast<long>(blockIdx.x) * 256 * U + threadIdx.x; b0 < n16; b0 += step) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(x + std::min(b0 + u * 256, n16 - 1));
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (b0 + u * 256 < n16) st8<NTS>(q + b0 + u * 256, u32x2{r[u].x ^ r[u].y, r[u].z ^ r[u].w});
  }
}

// dequant mix, one-shot
template <int U, bool NTS>
__global__ __launch_bounds__(256) void k_d1(const u32x2* __restrict__ q, long n8,
                                            u32x4* __restrict__ y) {
  const long b0 = static_cast<long>(blockIdx.x) * 256 * U + threadIdx.x;
  u32x2 r[U];
#pragma unroll
  for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(q + std::min(b0 + u * 256, n8 - 1));
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (b0 + u * 256 < n8) st16<NTS>(y + b0 + u * 256, u32x4{r[u].x, r[u].y, r[u].x ^ 1u, r[u].y ^ 1u});
}

// read only, one-shot; the xor keeps the loads alive
template <int U>
__global__ __launch_bounds__(256) void k_r1(const u32x4* __restrict__ x, long n16,
                                            unsigned* __restrict__ sink) {
  const long b0 = static_cast<long>(blockIdx.x) * 256 * U + threadIdx.x;
  unsigned h = 0;
  u32x4 r[U];
#pragma unroll
  for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(x + std::min(b0 + u * 256, n16 - 1));
#pragma unroll
  for (int u = 0; u < U; ++u) h ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
  if (h == 0x9e3779b9u) sink[0] = h;
}

// near-empty kernel: the event / dispatch floor of a single timed launch
template <int B>
__global__ __launch_bounds__(B) void k_empty(unsigned* sink, int never) {
  if (static_cast<int>(blockIdx.x) == never) sink[0] = threadIdx.x;
}

__global__ void k_sweep_read(const u32x4* p, long n16, unsigned* sink) {
  unsigned h = 0;
  for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<long>(gridDim.x) * 256)
    h ^= p[i].x;
  if (h == 0x9e3779b9u) sink[0] = h;
}

__global__ void k_sweep_write(u32x4* p, long n16) {
  for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<long>(gridDim.x) * 256)
    p[i] = u32x4{static_cast<unsigned>(i), 1u, 2u, 3u};
}

}  // namespace

int main() {
  int cus = 0;
  CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  const size_t sweep_bytes = size_t(512) << 20;
  void* sw;
  CK(hipMalloc(&sw, sweep_bytes));
  CK(hipMemset(sw, 1, sweep_bytes));
  unsigned* sink;
  CK(hipMalloc(&sink, 64));
  const size_t max_in = size_t(28672) * 8192 * 2;   // C3 bf16
  void *in, *out;
  CK(hipMalloc(&in, max_in));
  CK(hipMalloc(&out, max_in));
  CK(hipMemset(in, 3, max_in));
  CK(hipMemset(out, 0, max_in));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  auto sweep = [&](bool dirty) {
    if (dirty) k_sweep_write<<<cus * 8, 256>>>(static_cast<u32x4*>(sw), sweep_bytes / 16);
    else k_sweep_read<<<cus * 8, 256>>>(static_cast<const u32x4*>(sw), sweep_bytes / 16, sink);
  };
  auto timeit = [&](bool dirty, auto launch) {
    std::vector<float> v;
    for (int it = 0; it < 23; ++it) {
      sweep(dirty);
      CK(hipEventRecord(e0));
      launch();
      CK(hipEventRecord(e1));
      CK(hipEventSynchronize(e1));
      float ms;
      CK(hipEventElapsedTime(&ms, e0, e1));
      if (it >= 3) v.push_back(ms * 1000.0f);
    }
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
  };
  struct Size { const char* name; size_t elems; };
  const Size sizes[] = {{"C1 16Mi x 2B", size_t(4096) * 4096}, {"C2 64Mi x 2B", size_t(8192) * 8192},
                        {"C3 28672x8192 x 2B", size_t(28672) * 8192}};
  std::printf("# timing floor of one launch between two events after a sweep (median of 20)\n");
  std::printf("%-44s %9.2f us\n", "event pair, nothing between", timeit(false, [&] {}));
  std::printf("%-44s %9.2f us\n", "empty kernel, 256 x 1024 threads",
              timeit(false, [&] { k_empty<1024><<<256, 1024>>>(sink, -1); }));
  std::printf("%-44s %9.2f us\n", "empty kernel, 8192 x 256 threads",
              timeit(false, [&] { k_empty<256><<<8192, 256>>>(sink, -1); }));
  std::printf("# bare streams, median of 20 launches after a 512 MiB sweep; frac = bytes / time / 8 TB/s\n");
  std::printf("%-20s %-34s %-6s %9s %9s %6s\n", "size", "kernel", "sweep", "us", "GB/s", "frac");
  for (const Size& sz : sizes) {
    const long n16 = static_cast<long>(sz.elems * 2 / 16);   // 16-byte input chunks
    const long n8 = static_cast<long>(sz.elems / 8);         // 8-byte code chunks
    const double qbytes = 3.0 * sz.elems, rbytes = 2.0 * sz.elems;
    const auto* x16 = static_cast<const u32x4*>(in);
    auto* q8 = static_cast<u32x2*>(out);
    const auto* c8 = static_cast<const u32x2*>(in);
    auto* y16 = static_cast<u32x4*>(out);
    auto row = [&](const char* kern, bool dirty, double bytes, float us) {
      std::printf("%-20s %-34s %-6s %9.2f %9.1f %6.3f\n", sz.name, kern, dirty ? "dirty" : "clean", us,
                  bytes / us / 1e3, bytes / us / 8e6);
      std::fflush(stdout);
    };
    for (int d = 0; d < 2; ++d) {
      const bool dirty = d == 1;
      row("quant mix one-shot U4 NT stores", dirty, qbytes, timeit(dirty, [&] {
            k_q1<4, true><<<static_cast<unsigned>((n16 + 1023) / 1024), 256>>>(x16, n16, q8); }));
      row("quant mix one-shot U4 stores", dirty, qbytes, timeit(dirty, [&] {
            k_q1<4, false><<<static_cast<unsigned>((n16 + 1023) / 1024), 256>>>(x16, n16, q8); }));
      row("quant mix one-shot U2 NT stores", dirty, qbytes, timeit(dirty, [&] {
            k_q1<2, true><<<static_cast<unsigned>((n16 + 511) / 512), 256>>>(x16, n16, q8); }));
      row("quant mix persistent 8/CU U4 NT", dirty, qbytes, timeit(dirty, [&] {
            k_qp<4, true><<<cus * 8, 256>>>(x16, n16, q8); }));
      row("dequant mix one-shot U2 stores", dirty, qbytes, timeit(dirty, [&] {
            k_d1<2, false><<<static_cast<unsigned>((n8 + 511) / 512), 256>>>(c8, n8, y16); }));
      row("dequant mix one-shot U2 NT stores", dirty, qbytes, timeit(dirty, [&] {
            k_d1<2, true><<<static_cast<unsigned>((n8 + 511) / 512), 256>>>(c8, n8, y16); }));
      row("read only one-shot U4", dirty, rbytes, timeit(dirty, [&] {
            k_r1<4><<<static_cast<unsigned>((n16 + 1023) / 1024), 256>>>(x16, n16, sink); }));
    }
  }
  return 0;
}
