// cbq_host.h - host-side helpers shared by the C-ABI entry points: the
// thread-local error slot, launch-status checking and device queries.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cublade_quant.h"

namespace cbq {

// Records a printf-style message for cbq_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// CBQ_OK if the launches since the last call succeeded, else records the HIP
// error under `what` and returns CBQ_ELAUNCH.
int launch_status(const char* what);

// Compute units of the current device (cached per device).
int device_cus();

inline hipStream_t as_stream(cbq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace cbq

#define CBQ_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::cbq::set_error(__VA_ARGS__);  \
      return CBQ_EINVAL;              \
    }                                 \
  } while (0)
