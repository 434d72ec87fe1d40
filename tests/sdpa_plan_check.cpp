// Host check of the exact SDPA's launch plan (csrc/sdpa_plan.h): for every
// head count and query-tile count up to a bound, with full and partial last
// query tiles, several key lengths and the kernels' tile shapes, on a
// 256-CU device, the plan must
//   - run every query tile exactly once: whole, or as key ranges that cover
//     [0, Lk) once each (ranges a multiple of the key tile, none empty);
//   - keep all pieces within 2 * CUs - 1;
//   - need at most the no-allocation entry point's 66 MiB of scratch;
//   - refuse a caller scratch one byte smaller than it needs.
// Built and run by tests/test_sdpa_plan.py; prints "ok <plans checked>" and
// exits 0, else names the first failed check and exits 1.
#include <cstdio>
#include <cstdlib>

#include "sdpa_plan.h"

namespace {

using tsplat::sdpa::TilePlan;

int failures = 0;
void check(bool ok, const char* what, long bh, int Lq, int Lk, int bq, int bkv) {
  if (!ok && failures++ < 10)
    std::printf("FAIL: %s (B*H=%ld Lq=%d Lk=%d kBQ=%d kBKV=%d)\n", what, bh, Lq, Lk, bq, bkv);
}

// Key ranges of `splits` x `kps` keys cover [0, Lk) once, none empty.
bool ranges_ok(int Lk, int kps, int splits, int bkv) {
  if (splits == 1) return kps >= Lk;
  return kps % bkv == 0 && (int64_t)(splits - 1) * kps < Lk && (int64_t)splits * kps >= Lk;
}

}  // namespace

int main() {
  constexpr int kCus = 256, kD = 64;
  constexpr size_t kNoAllocScratch = 66u << 20;
  const int bqs[] = {128, 256, 512};
  const int bkvs[] = {32, 64, 128};
  const int lks[] = {1, 63, 64, 65, 320, 1000, 2048, 8194, 12294, 16384, 16385};
  long plans = 0;
  size_t worst = 0;
  for (int bq : bqs)
    for (int bkv : bkvs)
      for (long bh = 1; bh <= 64; bh = bh < 20 ? bh + 1 : bh * 2)
        for (int qt = 1; qt <= 96; ++qt)
          for (int part = 0; part < 2; ++part) {
            const int Lq = qt * bq - (part ? bq / 2 + 1 : 0);
            for (int Lk : lks) {
              TilePlan pl;
              const bool ok = tsplat::sdpa::plan_tiles(1, bh, Lq, Lk, bq, bkv, kD, kCus, pl);
              ++plans;
              check(ok, "plan refused", bh, Lq, Lk, bq, bkv);
              if (!ok) continue;
              check(pl.tiles == bh * qt, "tile count", bh, Lq, Lk, bq, bkv);
              check(pl.pieces <= 2 * kCus - 1, "pieces within 2 * CUs - 1", bh, Lq, Lk, bq, bkv);
              if (pl.pieces == 0) {
                check(pl.full_tiles == pl.tiles && pl.scratch_bytes == 0, "no split: all tiles whole",
                      bh, Lq, Lk, bq, bkv);
                continue;
              }
              const int64_t tail = pl.tiles - pl.full_tiles;
              const int64_t tail_full = pl.splits >= 2 ? pl.pieces_full / pl.splits : 0;
              check(pl.pieces_full == tail_full * pl.splits, "full tail tiles split evenly", bh, Lq, Lk,
                    bq, bkv);
              check(pl.pieces - pl.pieces_full == (tail - tail_full) * pl.splits_p,
                    "partial tail tiles split evenly", bh, Lq, Lk, bq, bkv);
              check(tail > 0 && tail <= pl.tiles % kCus, "tail within the last round", bh, Lq, Lk, bq,
                    bkv);
              check(part || tail_full == tail, "partial tiles only when Lq is ragged", bh, Lq, Lk, bq, bkv);
              if (tail_full > 0)
                check(ranges_ok(Lk, pl.keys_per_split, pl.splits, bkv), "full tiles' key ranges", bh, Lq,
                      Lk, bq, bkv);
              if (tail > tail_full)
                check(ranges_ok(Lk, pl.keys_per_split_p, pl.splits_p, bkv), "partial tiles' key ranges",
                      bh, Lq, Lk, bq, bkv);
              check(pl.scratch_bytes == (size_t)pl.pieces * bq * (kD + 2) * 4, "scratch bytes", bh, Lq, Lk,
                    bq, bkv);
              check(pl.scratch_bytes <= kNoAllocScratch, "fits the 66 MiB static scratch", bh, Lq, Lk, bq,
                    bkv);
              check(tsplat::sdpa::scratch_fits(pl, pl.scratch_bytes) &&
                        !tsplat::sdpa::scratch_fits(pl, pl.scratch_bytes - 1),
                    "a scratch one byte short is refused", bh, Lq, Lk, bq, bkv);
              if (pl.scratch_bytes > worst) worst = pl.scratch_bytes;
            }
          }
  // the bound the comments state: (2 * CUs - 1) pieces of 512 rows x 66 floats
  check(worst <= (size_t)(2 * kCus - 1) * 512 * (kD + 2) * 4, "worst plan within the stated bound", 0, 0, 0,
        0, 0);
  {
    TilePlan pl;
    check(!tsplat::sdpa::plan_tiles(1, 0, 16, 16, 512, 64, kD, kCus, pl), "no tiles: refused", 0, 16, 16, 512,
          64);
    check(tsplat::sdpa::plan_tiles(1, 16, 16384, 16384, 512, 64, kD, 0, pl) && pl.pieces == 0,
          "cus = 0: no split", 16, 16384, 16384, 512, 64);
  }
  if (failures == 0) std::printf("ok %ld\n", plans);
  return failures == 0 ? 0 : 1;
}
