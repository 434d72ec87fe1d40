// Grow-only device scratch buffers keyed by (device, stream, slot): the
// bookkeeping, free of HIP so that the policy is testable on the host (the
// device operations come in through `Ops`).
//
// Policy
//   - A request that fits the key's current buffer reuses it.  When the
//     stream is under graph capture, the buffer is marked `captured`: the
//     graph holds its address for as long as the graph exists.
//   - A request that does not fit, on a stream under capture, fails (a
//     capture can neither allocate nor wait).  One eager call of the same or
//     a larger shape on that stream beforehand provides the buffer.
//   - A request that does not fit, eagerly, allocates a larger buffer
//     (rounded up to a power of two, at least kMinBytes, so that a sequence
//     of growing requests allocates O(log) times).  The old buffer is freed
//     after the stream has finished with it -- unless a capture recorded it:
//     then it is retired (kept allocated until the process ends), because a
//     graph replayed later still writes to it.
//   - release() frees, after its stream, every buffer of a slot on the
//     current device whose stream is idle (not under capture), and retires
//     the others: buffers a capture recorded, buffers of a stream under
//     capture right now (waiting on such a stream would end its capture),
//     and buffers of a stream that no longer exists (it cannot be waited
//     on).  A destroyed stream's buffer is therefore reclaimed only by a
//     release() made before the stream is destroyed.
// Calls on one stream are ordered by the stream and share its buffer; a
// graph must be replayed on the stream it was captured on (or ordered with
// that stream's eager work), since both use the same buffer.  Streams are
// keyed by handle: a new stream that reuses a destroyed stream's handle
// value takes over its buffers, which is safe because the runtime releases
// a stream's handle only once the work queued on it has finished.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <tuple>
#include <vector>

namespace tsplat {

struct WorkspaceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool captured = false;  // handed to a stream under graph capture
};

struct WorkspaceSlotStats {
  uint64_t allocations = 0;     // buffers allocated for the slot
  uint64_t live_bytes = 0;      // bytes of the current buffers
  uint64_t retired_bytes = 0;   // superseded buffers a capture may still use
  uint64_t alloc_ns = 0;        // host time in alloc
  uint64_t free_ns = 0;         // host time waiting for streams and in free
};

// What a stream is doing when release() looks at it.
enum class StreamState { kIdle, kCapturing, kGone };

// Ops: void* alloc(size_t); bool free(void*); bool sync(Stream);
//      StreamState state(Stream); void clear_error(); uint64_t now_ns();
// alloc / free / sync report failure by null / false and may leave a
// runtime error pending; the pool clears it (clear_error) right away, so a
// caller that checks the runtime's last error after its own launch sees only
// that launch's.  Stream must be ordered (operator<): it is part of the map key.
template <class Stream, class Ops>
class WorkspacePool {
 public:
  static constexpr size_t kMinBytes = 64 * 1024;
  static constexpr int kSlots = 4;

  explicit WorkspacePool(Ops ops) : ops_(ops) {}

  static size_t round_up(size_t bytes) {
    size_t n = kMinBytes;
    while (n < bytes) n <<= 1;
    return n;
  }

  // The buffer for (device, stream, slot) with at least `bytes`, or null.
  void* acquire(int device, Stream stream, int slot, size_t bytes, bool capturing) {
    if (slot < 0 || slot >= kSlots) return nullptr;
    WorkspaceBuffer& b = buffers_[std::make_tuple(device, stream, slot)];
    if (b.ptr != nullptr && b.bytes >= bytes) {
      if (capturing) b.captured = true;
      return b.ptr;
    }
    if (capturing) return nullptr;
    const size_t want = round_up(bytes);
    const uint64_t t0 = ops_.now_ns();
    void* fresh = ops_.alloc(want);
    stats_[slot].alloc_ns += ops_.now_ns() - t0;
    if (fresh == nullptr) {
      ops_.clear_error();
      return nullptr;
    }
    if (b.ptr != nullptr && !drop(b, stream, slot)) {
      if (!ops_.free(fresh)) ops_.clear_error();
      return nullptr;
    }
    b.ptr = fresh;
    b.bytes = want;
    b.captured = false;
    stats_[slot].allocations += 1;
    stats_[slot].live_bytes += want;
    return fresh;
  }

  // Frees (after its stream) or retires every buffer of `slot` on `device`;
  // buffers of streams that are capturing or gone are retired, never waited on.
  void release(int device, int slot) {
    if (slot < 0 || slot >= kSlots) return;
    for (auto it = buffers_.begin(); it != buffers_.end();) {
      if (std::get<0>(it->first) != device || std::get<2>(it->first) != slot) {
        ++it;
        continue;
      }
      WorkspaceBuffer& b = it->second;
      const Stream stream = std::get<1>(it->first);
      if (b.ptr != nullptr && !b.captured && ops_.state(stream) != StreamState::kIdle) b.captured = true;
      if (b.ptr == nullptr || drop(b, stream, slot))
        it = buffers_.erase(it);
      else
        ++it;
    }
  }

  WorkspaceSlotStats stats(int slot) const {
    return (slot >= 0 && slot < kSlots) ? stats_[slot] : WorkspaceSlotStats{};
  }
  const std::vector<void*>& retired() const { return retired_; }

 private:
  // Gives up b's memory: retired when a capture holds it, else freed once
  // the stream no longer uses it.  False if the stream wait failed (b kept).
  bool drop(WorkspaceBuffer& b, Stream stream, int slot) {
    if (b.captured) {
      retired_.push_back(b.ptr);
      stats_[slot].retired_bytes += b.bytes;
    } else {
      const uint64_t t0 = ops_.now_ns();
      const bool ok = ops_.sync(stream);
      if (ok && !ops_.free(b.ptr)) ops_.clear_error();
      stats_[slot].free_ns += ops_.now_ns() - t0;
      if (!ok) {
        ops_.clear_error();
        return false;
      }
    }
    stats_[slot].live_bytes -= b.bytes;
    b.ptr = nullptr;
    b.bytes = 0;
    b.captured = false;
    return true;
  }

  Ops ops_;
  std::map<std::tuple<int, Stream, int>, WorkspaceBuffer> buffers_;
  std::vector<void*> retired_;
  WorkspaceSlotStats stats_[kSlots];
};

}  // namespace tsplat
