// The exact SDPA entry point for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc): tsplat_sdpa_precision_async with the key-split partials kept in
// a file-scope device array instead of the library's per-stream workspace.
//
// Scratch bound.  A launch splits the keys only for the partial last round
// of query tiles: its tiles (tiles mod CUs of them) become pieces of at most
// 16 key ranges each, every piece writing kBQ <= 512 query rows of 64
// outputs + (max, sum) in fp32, and the plan keeps all pieces within
// 2 * CUs - 1, so on a 256-CU MI355X a plan needs at most 511 * 512 * 66 * 4
// = 69,074,944 bytes.  The array holds 66 MiB (69,206,016 bytes): every plan
// of a 256-CU device fits; a call whose plan needs more (a device with more
// CUs) returns -8 before any launch.
//
// Sharing.  One array per GPU, shared by every call on that GPU, whatever the
// stream.  Nothing in it has to start at zero (each partial row is written
// before the merge reads it), but calls that overlap in time on one GPU --
// on different streams, or a graph replay beside an eager call -- race on
// its contents.  Order them.

#include <hip/hip_runtime.h>

#include <mutex>

#include "capi_internal.h"
#include "tsplat_common.h"
#include "tsplat_launch.h"
#include "../../include/tsplat_hip.h"

namespace tsplat {
namespace {

constexpr size_t kScratchBytes = 66u << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (each GPU holds its own copy),
// looked up once per device with that device current.  In host code the
// array's name is only a stand-in; this address is what kernels get.
float* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
      (void)note(hipGetLastError());
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return static_cast<float*>(g_scratch_ptr[dev]);
}

}  // namespace
}  // namespace tsplat

extern "C" int tsplat_sdpa_noalloc_async(const float* q, const float* k, const float* v,
                                         const float* key_bias_or_null, float* out, int B, int H,
                                         int Lq, int Lk, int D, int has_key_bias, int key_bias_len,
                                         int64_t bias_head_stride, int kv_packed, int Lkp,
                                         int out_blhd, int precision, void* stream) {
  using namespace tsplat;
  float* ws = device_scratch();
  if (ws == nullptr) return kErrLaunch;
  return sdpa_checked(q, k, v, key_bias_or_null, out, B, H, Lq, Lk, D, has_key_bias, key_bias_len,
                      bias_head_stride, kv_packed, Lkp, out_blhd,
                      static_cast<hipStream_t>(stream), precision, ws, kScratchBytes);
}
