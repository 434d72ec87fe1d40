// Validation helpers shared by the C-ABI translation units (capi*.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsplat {

// Records a failed HIP call for tsplat_last_hip_error(); kOk or kErrLaunch.
int note(hipError_t e);
// kOk when [p, p + bytes) lies inside one device (or managed) allocation of
// the current device; kErrNull / kErrPointer otherwise.
int check_dev(const void* p, int64_t bytes);
bool aligned16(const void* p);
// Waits for the null stream (the blocking reference-named entry points).
int sync_null_stream();

}  // namespace tsplat

#define TSPLAT_CHECK(expr)        \
  do {                            \
    const int st_ = (expr);       \
    if (st_ != kOk) return st_;   \
  } while (0)
