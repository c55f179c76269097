// cbq_common.hip - error reporting, launch checks and device queries behind
// the C ABI of libcublade_quant.so.
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "cbq_host.h"

namespace cbq {

namespace {
thread_local char g_err[512] = {0};
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices] = {0};
std::mutex g_cus_mu;
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return CBQ_ELAUNCH;
  }
  return CBQ_OK;
}

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> lk(g_cus_mu);
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

}  // namespace cbq

extern "C" const char* cbq_last_error(void) { return cbq::g_err; }

extern "C" int cbq_abi_version(void) { return 200; }
