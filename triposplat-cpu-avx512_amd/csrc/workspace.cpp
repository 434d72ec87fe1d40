// Per-stream device workspaces for kernels that need scratch memory: the
// split-K partial sums of the few-row GEMM and the key-split partials of the
// SDPA tail.  Every user overwrites the part it reads, so buffers are not
// cleared.
//
// One grow-only buffer per (device, stream, slot).  Calls on one stream are
// ordered by the stream, so they may share its buffer; calls on different
// streams get different buffers.  Growing waits for the stream before the
// old buffer is released.  A stream under HIP-graph capture cannot allocate
// or wait, so a call there that needs a larger buffer fails (the caller
// returns -5); one eager call of the same or a larger shape on that stream
// beforehand provides the buffer.  Buffers live until the process ends.

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
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (capture != hipStreamCaptureStatusNone) return nullptr;
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
  b.bytes = want;
  return b.ptr;
}

}  // namespace tsplat
