// Validation helpers shared by the C-ABI translation units (capi*.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsplat {

// Records a failed HIP call for tsplat_last_hip_error(); kOk or kErrLaunch.
int note(hipError_t e);
// The pointer checks of one C-ABI call.  check(p, bytes) is kOk when
// [p, p + bytes) lies inside one device (or managed) allocation of the
// current device, kErrNull / kErrPointer otherwise: a wrong pointer becomes a
// status code instead of a GPU memory fault.  Each runtime query costs about
// 0.1 us of host time and a call checks 3-11 pointers, so the current device
// is read once per call, and a range inside an allocation that an earlier
// check of the same call validated is accepted without a query (torch's
// caching allocator carves many tensors out of one segment).
class DeviceRanges {
 public:
  int check(const void* p, int64_t bytes);

 private:
  static constexpr int kMaxRanges = 12;
  int device_ = -1;
  int count_ = 0;
  uintptr_t lo_[kMaxRanges];
  uintptr_t hi_[kMaxRanges];
};
bool aligned16(const void* p);
// Bytes of one bf16 weight plane of a [K, N] weight: k-blocked
// [ceil(K / 32), N, 32] (tsplat_nf24_bf16_planes_async).
inline int64_t planes_bytes(int K, int N) { return (int64_t)((K + 31) / 32) * N * 64; }
// Waits for the null stream (the blocking reference-named entry points).
int sync_null_stream();
// Argument checks of the SDPA entry points, then launch_sdpa on `stream`;
// scratch / scratch_bytes as SdpaParams (null: the stream's workspace).
int sdpa_checked(const float* q, const float* k, const float* v, const float* bias, float* out,
                 int B, int H, int Lq, int Lk, int D, int has_bias, int bias_len,
                 int64_t bias_head_stride, int kv_packed, int Lkp, int out_blhd,
                 hipStream_t stream, int precision, float* scratch, size_t scratch_bytes);

}  // namespace tsplat

#define TSPLAT_CHECK(expr)        \
  do {                            \
    const int st_ = (expr);       \
    if (st_ != kOk) return st_;   \
  } while (0)
