// Launch plan of the exact SDPA's query tiles: which tiles run whole and
// how the tiles of a partial last round are split along the keys.  Host
// arithmetic only, free of HIP, so that the plan is checked on the host
// (tests/sdpa_plan_check.cpp); the launcher in sdpa_common.h runs it.
//
// Query tiles of kBQ queries, B * H * ceil(Lq / kBQ) of them, one workgroup
// per CU.  When the tiles leave a partial last round (tiles % cus != 0), its
// tiles are cut into key ranges (multiples of the key tile kBKV) so that the
// round fills every CU; each range ("piece") writes its kBQ unnormalised
// output rows and (max, sum) to scratch, and a merge kernel combines them.
// Partial query tiles (Lq % kBQ != 0, one per head, numbered after the full
// tiles) take a split of their own.  Every plan keeps the pieces within
// 2 * cus - 1, so the scratch a plan needs is at most
// (2 * cus - 1) * kBQ * (kD + 2) * 4 bytes.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace tsplat {
namespace sdpa {

// Key ranges for the tiles of a partial last round.  Modelled in units of
// one full tile over all keys: `full` full tiles split s ways make
// ceil(full * s / cus) rounds of 1/s each, plus a fixed cost per piece (its
// prologue, Q load and partial store) of 2 % of a tile.  The `partial` query
// tiles (numbered last; their few live waves still stream every key tile, at
// a few us each) take the slots left after the full tiles' pieces and are
// split by the same model into s_p ranges of their own.  All pieces together
// stay within 2 * cus - 1; s, s_p <= 16.
inline int choose_splits(int64_t full, int64_t reserve, int cus) {
  int best = 1;
  double best_t = 1e30;
  for (int s = 1; s <= 16 && full * s + reserve <= 2 * (int64_t)cus - 1; ++s) {
    const double t = (double)((full * s + cus - 1) / cus) * (1.0 / s + 0.02);
    if (t < best_t - 1e-9) {
      best_t = t;
      best = s;
    }
  }
  return best;
}

// Keys per range (a multiple of the key tile) and the resulting range count.
inline void key_ranges(int Lk, int kBKV, int s0, int& kps, int& splits) {
  kps = ((Lk + s0 - 1) / s0 + kBKV - 1) / kBKV * kBKV;
  splits = (Lk + kps - 1) / kps;
}

struct TilePlan {
  int64_t tiles = 0;       // query tiles over all (b, h)
  int64_t full_tiles = 0;  // tiles [0, full_tiles) run whole; the rest are pieces
  int splits = 1, keys_per_split = 0;      // the full tail tiles' key ranges
  int64_t pieces_full = 0;                 // their pieces (0 when they do not split)
  int splits_p = 1, keys_per_split_p = 0;  // the partial query tiles' key ranges
  int64_t pieces = 0;                      // all pieces (0: no split)
  size_t scratch_bytes = 0;                // partial rows + (max, sum) of the pieces
  int64_t grid() const { return full_tiles + pieces; }
};

// The plan of B * H heads of Lq queries over Lk keys with kBQ-query tiles,
// kBKV-key tiles and head dim kD on `cus` CUs (0: never split).  False when
// the tile count is out of range (none, or more than a grid holds).
inline bool plan_tiles(int64_t B, int64_t H, int Lq, int Lk, int kBQ, int kBKV, int kD, int cus,
                       TilePlan& pl) {
  pl = TilePlan{};
  pl.tiles = B * H * ((Lq + kBQ - 1) / kBQ);
  if (pl.tiles <= 0 || pl.tiles > 0x7fffffff) return false;
  pl.full_tiles = pl.tiles;
  pl.keys_per_split = Lk;
  pl.keys_per_split_p = Lk;
  const int64_t rest = cus > 0 ? pl.tiles % cus : 0;
  if (cus <= 0 || pl.tiles < cus || rest == 0) return true;
  const int64_t partial_all = (Lq % kBQ != 0) ? B * H : 0;
  const int64_t partial = partial_all < rest ? partial_all : rest;
  const int64_t full = rest - partial;
  int kps = Lk, splits = 1, kps_p = Lk, splits_p = 1;
  if (full > 0) key_ranges(Lk, kBKV, choose_splits(full, partial, cus), kps, splits);
  const int64_t pieces_full = splits >= 2 ? full * splits : 0;
  if (partial > 0) key_ranges(Lk, kBKV, choose_splits(partial, pieces_full, cus), kps_p, splits_p);
  // Tail tiles: the `full` ones when they split, then the partial ones when
  // either kind splits (a partial tile kept whole is one piece).
  const int64_t tail_tiles = (splits >= 2 ? full : 0) + ((splits >= 2 || splits_p >= 2) ? partial : 0);
  if (tail_tiles == 0) return true;
  pl.full_tiles = pl.tiles - tail_tiles;
  pl.splits = splits;
  pl.keys_per_split = kps;
  pl.pieces_full = pieces_full;
  pl.splits_p = splits_p;
  pl.keys_per_split_p = kps_p;
  pl.pieces = pieces_full + partial * splits_p;
  pl.scratch_bytes = (size_t)pl.pieces * kBQ * (kD + 2) * sizeof(float);
  return true;
}

// Whether a caller-provided scratch of `have` bytes holds the plan's pieces
// (the no-allocation entry point's static array; a plan needing more is
// refused before any launch).
inline bool scratch_fits(const TilePlan& pl, size_t have) { return pl.scratch_bytes <= have; }

}  // namespace sdpa
}  // namespace tsplat
