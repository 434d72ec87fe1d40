// Host check of the device-workspace policy (csrc/workspace_pool.h) with
// fake device operations: every alloc / free / stream wait is logged, and
// the scenarios below assert what the policy must do.  Built and run by
// tests/test_workspace_pool.py; prints "ok" and exits 0 when every check
// holds, else names the failed check and exits 1.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <string>
#include <vector>

#include "workspace_pool.h"

namespace {

struct Log {
  std::vector<std::string> events;
  std::set<void*> live;
  int next = 1;
  bool fail_sync = false;
  bool fail_alloc = false;
  bool fail_free = false;
  bool pending_error = false;  // what a failed runtime call leaves behind
  std::set<int> capturing, gone;
  uint64_t clock = 0;
};

struct FakeOps {
  Log* log;
  void* alloc(size_t bytes) {
    if (log->fail_alloc) {
      log->pending_error = true;
      return nullptr;
    }
    void* p = reinterpret_cast<void*>((uintptr_t)(log->next++) << 32);
    log->live.insert(p);
    log->events.push_back("alloc " + std::to_string(bytes));
    return p;
  }
  bool free(void* p) {
    if (!log->live.count(p)) {
      std::printf("FAIL: free of a pointer that is not live\n");
      std::exit(1);
    }
    if (log->fail_free) {
      log->pending_error = true;
      return false;
    }
    log->live.erase(p);
    log->events.push_back("free");
    return true;
  }
  bool sync(int stream) {
    if (log->capturing.count(stream) || log->gone.count(stream)) {
      std::printf("FAIL: wait on a stream that is capturing or gone\n");
      std::exit(1);
    }
    log->events.push_back("sync " + std::to_string(stream));
    if (log->fail_sync) log->pending_error = true;
    return !log->fail_sync;
  }
  tsplat::StreamState state(int stream) {
    if (log->gone.count(stream)) return tsplat::StreamState::kGone;
    return log->capturing.count(stream) ? tsplat::StreamState::kCapturing : tsplat::StreamState::kIdle;
  }
  void clear_error() { log->pending_error = false; }
  uint64_t now_ns() { return log->clock += 10; }
};

using Pool = tsplat::WorkspacePool<int, FakeOps>;

int failures = 0;
void check(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAIL: %s\n", what);
    ++failures;
  }
}

}  // namespace

int main() {
  const size_t kMin = Pool::kMinBytes;
  check(Pool::round_up(1) == kMin && Pool::round_up(kMin) == kMin &&
            Pool::round_up(kMin + 1) == 2 * kMin && Pool::round_up(5 * kMin) == 8 * kMin,
        "round_up gives powers of two >= kMinBytes");

  {  // eager growth frees the old buffer only after its stream
    Log log;
    Pool pool(FakeOps{&log});
    void* a = pool.acquire(0, 7, 1, 1000, false);
    check(a != nullptr && log.events.size() == 1, "first request allocates");
    check(pool.acquire(0, 7, 1, kMin, false) == a, "a fitting request reuses the buffer");
    check(log.events.size() == 1, "reuse allocates nothing");
    void* b = pool.acquire(0, 7, 1, 3 * kMin, false);
    check(b != nullptr && b != a, "a larger request gets a new buffer");
    check(log.events.size() == 4 && log.events[1] == "alloc " + std::to_string(4 * kMin) &&
              log.events[2] == "sync 7" && log.events[3] == "free",
          "uncaptured old buffer: new alloc, wait for its stream, then free");
    check(!log.live.count(a) && log.live.count(b), "old freed, new live");
    check(pool.retired().empty(), "nothing retired without a capture");
    const tsplat::WorkspaceSlotStats s = pool.stats(1);
    check(s.allocations == 2 && s.live_bytes == 4 * kMin && s.retired_bytes == 0,
          "stats after growth");
    check(s.alloc_ns > 0 && s.free_ns > 0, "timing accumulates");
  }

  {  // a buffer recorded by a capture is never freed
    Log log;
    Pool pool(FakeOps{&log});
    void* a = pool.acquire(0, 3, 0, kMin, false);
    check(pool.acquire(0, 3, 0, kMin / 2, true) == a, "capture reuses a fitting buffer");
    check(pool.acquire(0, 3, 0, 2 * kMin, true) == nullptr,
          "capture cannot grow: the request fails");
    check(log.live.count(a) == 1, "failed capture request keeps the buffer");
    const size_t before = log.events.size();
    void* b = pool.acquire(0, 3, 0, 2 * kMin, false);
    check(b != nullptr && b != a, "eager growth after a capture gets a new buffer");
    check(log.live.count(a) == 1, "captured buffer stays allocated (retired)");
    bool freed = false, synced = false;
    for (size_t i = before; i < log.events.size(); ++i) {
      freed |= log.events[i] == "free";
      synced |= log.events[i].rfind("sync", 0) == 0;
    }
    check(!freed && !synced, "retiring needs no free and no wait");
    check(pool.retired().size() == 1 && pool.retired()[0] == a, "retired list holds it");
    check(pool.stats(0).retired_bytes == kMin && pool.stats(0).live_bytes == 2 * kMin,
          "retired bytes accounted");
    // the new buffer starts uncaptured: growing again frees it normally
    void* c = pool.acquire(0, 3, 0, 4 * kMin, false);
    check(c != nullptr && !log.live.count(b) && log.live.count(a), "new buffer freed, old kept");
  }

  {  // keys are independent: streams, devices, slots
    Log log;
    Pool pool(FakeOps{&log});
    void* s1 = pool.acquire(0, 1, 0, kMin, false);
    void* s2 = pool.acquire(0, 2, 0, kMin, false);
    void* d1 = pool.acquire(1, 1, 0, kMin, false);
    void* o1 = pool.acquire(0, 1, 1, kMin, false);
    std::set<void*> all{s1, s2, d1, o1};
    check(all.size() == 4, "distinct buffers per (device, stream, slot)");
    check(pool.acquire(0, 1, Pool::kSlots, kMin, false) == nullptr &&
              pool.acquire(0, 1, -1, kMin, false) == nullptr,
          "slot out of range is rejected");
  }

  {  // release: frees uncaptured (after the stream), retires captured
    Log log;
    Pool pool(FakeOps{&log});
    void* a = pool.acquire(0, 1, 1, kMin, false);
    void* b = pool.acquire(0, 2, 1, kMin, false);
    void* other_dev = pool.acquire(1, 1, 1, kMin, false);
    void* other_slot = pool.acquire(0, 1, 0, kMin, false);
    check(pool.acquire(0, 2, 1, kMin, true) == b, "capture on stream 2");
    pool.release(0, 1);
    check(!log.live.count(a) && log.live.count(b), "released: uncaptured freed, captured kept");
    check(log.live.count(other_dev) && log.live.count(other_slot),
          "release touches only its device and slot");
    check(pool.retired().size() == 1 && pool.retired()[0] == b, "captured buffer retired");
    check(pool.stats(1).live_bytes == kMin, "only the other device's buffer is live");
    void* again = pool.acquire(0, 1, 1, kMin, false);
    check(again != nullptr && again != a, "a request after release allocates again");
  }

  {  // failures leave the pool consistent
    Log log;
    Pool pool(FakeOps{&log});
    void* a = pool.acquire(0, 1, 0, kMin, false);
    log.fail_sync = true;
    check(pool.acquire(0, 1, 0, 2 * kMin, false) == nullptr, "failed stream wait fails the request");
    check(log.live.count(a) == 1 && log.live.size() == 1, "old kept, the fresh buffer freed");
    check(!log.pending_error, "a failed stream wait leaves no runtime error for the next launch check");
    log.fail_sync = false;
    log.fail_alloc = true;
    check(pool.acquire(0, 1, 0, 2 * kMin, false) == nullptr, "failed alloc fails the request");
    check(log.live.count(a) == 1, "old kept after a failed alloc");
    check(!log.pending_error, "a failed alloc leaves no runtime error");
    log.fail_alloc = false;
    check(pool.acquire(0, 1, 0, kMin, false) == a, "the old buffer still serves fitting requests");
    log.fail_free = true;
    void* b = pool.acquire(0, 1, 0, 2 * kMin, false);
    check(b != nullptr && b != a, "growth succeeds when the old buffer's free fails");
    check(!log.pending_error, "a failed free leaves no runtime error");
    log.fail_free = false;
  }

  {  // release never waits on a stream under capture or one that is gone
    Log log;
    Pool pool(FakeOps{&log});
    void* idle = pool.acquire(0, 1, 1, kMin, false);
    void* cap = pool.acquire(0, 2, 1, kMin, false);
    void* gone = pool.acquire(0, 3, 1, kMin, false);
    log.capturing.insert(2);
    log.gone.insert(3);
    pool.release(0, 1);
    check(!log.live.count(idle), "idle stream: buffer freed after its stream");
    check(log.live.count(cap) && log.live.count(gone), "capturing / gone streams: buffers kept");
    check(pool.retired().size() == 2, "both retired");
    check(pool.stats(1).live_bytes == 0 && pool.stats(1).retired_bytes == 2 * kMin,
          "retired bytes accounted");
    log.capturing.clear();
    void* again = pool.acquire(0, 2, 1, kMin, false);
    check(again != nullptr && again != cap, "the stream gets a fresh buffer after release");
  }

  if (failures == 0) std::printf("ok\n");
  return failures == 0 ? 0 : 1;
}
