// Per-stream device workspaces for kernels that need scratch memory (split-K
// partial sums, the QKV projection between the GEMM and the postprocess).
//
// One grow-only buffer per (device, stream, slot), zero-filled when
// allocated.  Calls on one stream are ordered by the stream, so they may
// share its buffer; calls on different streams get different buffers.
// Growing waits for the stream before the old buffer is released.  Buffers
// live until the process ends.

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <tuple>

#include "tsplat_launch.h"

namespace tsplat {
namespace {

struct Buffer {
  void* ptr = nullptr;
  size_t bytes = 0;
};

std::mutex g_mu;
std::map<std::tuple<int, hipStream_t, int>, Buffer>* g_buffers = nullptr;

}  // namespace

void* stream_workspace(hipStream_t stream, size_t bytes, int slot) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_buffers == nullptr) g_buffers = new std::map<std::tuple<int, hipStream_t, int>, Buffer>();
  Buffer& b = (*g_buffers)[std::make_tuple(dev, stream, slot)];
  if (b.bytes >= bytes && b.ptr != nullptr) return b.ptr;
  if (b.ptr != nullptr) {
    if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
    (void)hipFree(b.ptr);
    b.ptr = nullptr;
    b.bytes = 0;
  }
  const size_t want = bytes < 256 ? 256 : bytes;
  if (hipMalloc(&b.ptr, want) != hipSuccess) {
    (void)hipGetLastError();
    b.ptr = nullptr;
    return nullptr;
  }
  // New buffers start zeroed (counters kept in a workspace rely on it); the
  // fill is ordered on the stream that will use the buffer.
  if (hipMemsetAsync(b.ptr, 0, want, stream) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(b.ptr);
    b.ptr = nullptr;
    return nullptr;
  }
  b.bytes = want;
  return b.ptr;
}

}  // namespace tsplat
