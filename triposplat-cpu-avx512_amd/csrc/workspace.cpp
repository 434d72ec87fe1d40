// Per-stream device workspaces for kernels that need scratch memory: the
// split-K partial sums of the few-row GEMM, the key-split partials of the
// SDPA tail and the pre-split K/V tiles of the bf16 SDPA modes.  Every user
// overwrites the part it reads, so buffers are not cleared.  The grow / free / retire policy is WorkspacePool's
// (workspace_pool.h); this file supplies the HIP operations and a lock.

#include <hip/hip_runtime.h>

#include <chrono>
#include <mutex>

#include "tsplat_launch.h"
#include "workspace_pool.h"

namespace tsplat {
namespace {

// The pool clears the error a failed call leaves (clear_error), so the
// caller's next hipGetLastError() check sees only its own launch.
struct HipOps {
  void* alloc(size_t bytes) {
    void* p = nullptr;
    return hipMalloc(&p, bytes) == hipSuccess ? p : nullptr;
  }
  bool free(void* p) { return hipFree(p) == hipSuccess; }
  bool sync(hipStream_t s) { return hipStreamSynchronize(s) == hipSuccess; }
  void clear_error() { (void)hipGetLastError(); }
  StreamState state(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
      (void)hipGetLastError();
      return StreamState::kGone;
    }
    return st == hipStreamCaptureStatusNone ? StreamState::kIdle : StreamState::kCapturing;
  }
  uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
  }
};

using Pool = WorkspacePool<hipStream_t, HipOps>;
static_assert(kSlotSdpaPartial < Pool::kSlots && kSlotGemmTail < Pool::kSlots &&
                  kSlotSdpaPlanes < Pool::kSlots,
              "workspace slot out of range");

std::mutex g_mu;
// Never destroyed: retired buffers stay valid for graphs until the process
// ends, and the HIP runtime may be gone by the time static destructors run.
Pool* g_pool = nullptr;

Pool& pool() {
  if (g_pool == nullptr) g_pool = new Pool(HipOps{});
  return *g_pool;
}

}  // namespace

void* stream_workspace(hipStream_t stream, size_t bytes, int slot) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  return pool().acquire(dev, stream, slot, bytes, capture != hipStreamCaptureStatusNone);
}

void release_workspace(int slot) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  pool().release(dev, slot);
}

void workspace_stats(int slot, uint64_t* allocations, uint64_t* live_bytes,
                     uint64_t* retired_bytes) {
  std::lock_guard<std::mutex> lock(g_mu);
  const WorkspaceSlotStats s = pool().stats(slot);
  if (allocations) *allocations = s.allocations;
  if (live_bytes) *live_bytes = s.live_bytes;
  if (retired_bytes) *retired_bytes = s.retired_bytes;
}

void workspace_timing(int slot, uint64_t* alloc_ns, uint64_t* free_ns) {
  std::lock_guard<std::mutex> lock(g_mu);
  const WorkspaceSlotStats s = pool().stats(slot);
  if (alloc_ns) *alloc_ns = s.alloc_ns;
  if (free_ns) *free_ns = s.free_ns;
}

}  // namespace tsplat
