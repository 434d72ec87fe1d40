// Pieces shared by the fp32 SDPA kernel (sdpa.hip) and its bf16-MFMA
// precision modes (sdpa_bf16.hip): the kernel arguments, the half-wave pair
// reductions, the merge of key-split partial results and the launch plan
// that splits the last, partial round of query tiles along the keys.
#pragma once

#include "sdpa_plan.h"
#include "tsplat_common.h"
#include "tsplat_launch.h"

namespace tsplat {
namespace sdpa {

constexpr int kD = 64;
constexpr float kLog2e = 1.4426950408889634f;

struct SdpaArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* bias;
  float* out;
  int B, H, Lq, Lk, Lkp;  // Lkp: key stride of a key-contiguous operand
  int64_t bias_head_stride;
  int out_blhd;
  // Tail split: workgroups [0, full_tiles) each own one query tile over all
  // keys; the rest are pieces, each one key range of a tail tile, writing
  // the unnormalised output rows and (max, sum) to part_o / part_ml (piece
  // j: rows j * kBQ ..), which sdpa_combine_kernel merges.  The first
  // pieces_full pieces split their tiles into `splits` ranges of
  // keys_per_split keys (a multiple of the key tile); the pieces after them
  // split the partial query tiles (numbered last) into splits_p ranges of
  // keys_per_split_p keys.
  int full_tiles, splits, keys_per_split;
  int pieces_full, splits_p, keys_per_split_p;
  float* part_o;   // [split item][query][64]
  float* part_ml;  // [split item][query][2]
};

inline SdpaArgs make_args(const SdpaParams& p) {
  return SdpaArgs{p.q,   p.k,  p.v,  p.bias, p.out, p.B, p.H, p.Lq, p.Lk, p.Lkp, p.bias_head_stride,
                  p.out_blhd, 0, 1, p.Lk, 0, 1, p.Lk, nullptr, nullptr};
}

namespace {

// max / sum of a value with the same register of lane l ^ 32.  Both lanes of
// a pair obtain the identical result (the swap returns both halves).
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One float4 staging unit of a K or V tile (keys key0 .. key0 + kBKV - 1)
// of one (b, h), base pointing at that (b, h).  [Lk, 64] operand (kPacked
// false): unit idx = dims 4c..4c+3 of key row; key-contiguous [64, Lkp]
// operand: keys 4c..4c+3 of dim row.  Keys past Lk read as zeros.
template <bool kPacked, int kBKV>
__device__ __forceinline__ floatx4 fetch_unit(const SdpaArgs& a, const float* base, int idx, int key0) {
  if constexpr (!kPacked) {
    const int row = idx / (kD / 4), c = idx % (kD / 4);
    const int key = key0 + row;
    const bool ok = key < a.Lk;
    const int64_t off = (int64_t)(ok ? key : 0) * kD + 4 * c;
    return ok ? *reinterpret_cast<const floatx4*>(base + off) : floatx4{0, 0, 0, 0};
  } else {
    const int row = idx / (kBKV / 4), c = idx % (kBKV / 4);
    const int key = key0 + 4 * c;
    const bool ok = key < a.Lk;
    const int64_t off = (int64_t)row * a.Lkp + (ok ? key : 0);
    floatx4 x = ok ? *reinterpret_cast<const floatx4*>(base + off) : floatx4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (key + e >= a.Lk) x[e] = 0.0f;
    return x;
  }
}

// Both [Lk, 64] operands' unit idx at once (one shared offset).
template <int kBKV>
__device__ __forceinline__ void fetch_units_kv(const SdpaArgs& a, const float* kbase, const float* vbase,
                                               int idx, int key0, floatx4& kx, floatx4& vx) {
  const int row = idx / (kD / 4), c = idx % (kD / 4);
  const int key = key0 + row;
  const bool ok = key < a.Lk;
  const int64_t off = (int64_t)(ok ? key : 0) * kD + 4 * c;
  kx = ok ? *reinterpret_cast<const floatx4*>(kbase + off) : floatx4{0, 0, 0, 0};
  vx = ok ? *reinterpret_cast<const floatx4*>(vbase + off) : floatx4{0, 0, 0, 0};
}

// (b*H + h, query block) of query tile `tile`.  When Lq is not a multiple of
// kBQ, each head's last, partial tile is numbered after all the full tiles:
// its waves past Lq skip the arithmetic, so partial tiles are cheap, and this
// order puts them in the launch's last (key-split) round instead of among the
// full tiles of the first rounds.
__device__ __forceinline__ void tile_coords(const SdpaArgs& a, int tile, int kBQ, int& bh, int& qb) {
  const int qblocks = (a.Lq + kBQ - 1) / kBQ;
  if (a.Lq % kBQ == 0) {
    bh = tile / qblocks;
    qb = tile % qblocks;
    return;
  }
  const int full = a.B * a.H * (qblocks - 1);
  if (tile < full) {
    bh = tile / (qblocks - 1);
    qb = tile % (qblocks - 1);
  } else {
    bh = tile - full;
    qb = qblocks - 1;
  }
}

// Query tile and key range of this workgroup (see SdpaArgs).
struct TileWork {
  int tile, part, k_begin, k_end;
};
__device__ __forceinline__ TileWork tile_work(const SdpaArgs& a) {
  TileWork w{0, -1, 0, a.Lk};
  if ((int)blockIdx.x < a.full_tiles) {
    w.tile = xcd_tile_index(blockIdx.x, a.full_tiles);
  } else if ((int)blockIdx.x - a.full_tiles < a.pieces_full) {  // tail: a key range of a tile
    w.part = blockIdx.x - a.full_tiles;
    w.tile = a.full_tiles + w.part / a.splits;
    w.k_begin = (w.part % a.splits) * a.keys_per_split;
    w.k_end = min(a.Lk, w.k_begin + a.keys_per_split);
  } else {  // tail: a key range of a partial query tile
    w.part = blockIdx.x - a.full_tiles;
    const int pp = w.part - a.pieces_full;
    w.tile = a.full_tiles + a.pieces_full / a.splits + pp / a.splits_p;
    w.k_begin = (pp % a.splits_p) * a.keys_per_split_p;
    w.k_end = min(a.Lk, w.k_begin + a.keys_per_split_p);
  }
  return w;
}

// Final store of a wave's 32 queries: o[db][r] holds O^T[db*32 + 8*(r/4) +
// 4*g + r%4][query] (the 32x32 MFMA accumulator layout), m_run / l_run the
// lane's running max and partial sum.  Split parts write the unnormalised
// rows and (max, sum) for the combine kernel.  The tile indices are
// recomputed here from the launch state rather than kept live across the
// key loop (fewer registers held through it).
template <int kBQ>
__device__ __forceinline__ void store_rows(const SdpaArgs& a, const floatx16 (&o)[2], float m_run,
                                           float l_run) {
  const TileWork w = tile_work(a);
  int bh, qb;
  tile_coords(a, w.tile, kBQ, bh, qb);
  const int b = bh / a.H, h = bh % a.H, part = w.part;
  const int wave = threadIdx.x >> 6, g = (threadIdx.x >> 5) & 1, l32 = threadIdx.x & 31;
  const int qrow = qb * kBQ + wave * 32 + l32;
  if (qrow >= a.Lq) return;  // lanes l and l ^ 32 share the query: both leave or neither
  const float lsum = pair_sum(l_run);
  if (part >= 0) {
    const int64_t row = (int64_t)part * kBQ + wave * 32 + l32;
    float* po = a.part_o + row * kD;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        floatx4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = o[db][4 * r4 + e];
        *reinterpret_cast<floatx4*>(po + db * 32 + 8 * r4 + 4 * g) = y;
      }
    if (g == 0) {
      a.part_ml[2 * row] = m_run;
      a.part_ml[2 * row + 1] = lsum;
    }
    return;
  }
  const float inv = 1.0f / lsum;
  float* dst = a.out_blhd ? a.out + (((int64_t)b * a.Lq + qrow) * a.H + h) * kD
                          : a.out + ((int64_t)bh * a.Lq + qrow) * kD;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      floatx4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = o[db][4 * r4 + e] * inv;
      *reinterpret_cast<floatx4*>(dst + db * 32 + 8 * r4 + 4 * g) = y;
    }
}

// Merge of the tail's key-range partials, one thread per (query, dim):
// m = max m_s, w_s = exp2(m_s - m), out = (sum_s o_s w_s) * (1 / sum_s l_s w_s).
constexpr int kCombineThreads = 256;
__global__ __launch_bounds__(kCombineThreads) void sdpa_combine_kernel(SdpaArgs a, int q_per_tile,
                                                                       int64_t rows) {
  const int64_t i = (int64_t)blockIdx.x * kCombineThreads + threadIdx.x;
  if (i >= rows * kD) return;
  const int d = (int)(i % kD);
  const int64_t r = i / kD;  // (tail tile, query in tile)
  const int ptile = (int)(r / q_per_tile), qi = (int)(r % q_per_tile);
  const int tile = a.full_tiles + ptile;
  int bh, qb;
  tile_coords(a, tile, q_per_tile, bh, qb);
  const int qrow = qb * q_per_tile + qi;
  if (qrow >= a.Lq) return;
  const int tail_full = a.pieces_full / a.splits;  // tail tiles split `splits` ways
  const int nsplit = ptile < tail_full ? a.splits : a.splits_p;
  const int64_t piece0 = ptile < tail_full ? (int64_t)ptile * a.splits
                                           : a.pieces_full + (int64_t)(ptile - tail_full) * a.splits_p;
  const int64_t base = piece0 * q_per_tile + qi;
  // Unrolled so that the loads of eight ranges are in flight together (the
  // sums keep their order: the same result as the rolled loops).
  float m = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) m = fmaxf(m, a.part_ml[2 * (base + (int64_t)s * q_per_tile)]);
  float l = 0.0f, o = 0.0f;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) {
    const int64_t row = base + (int64_t)s * q_per_tile;
    const float w = __builtin_amdgcn_exp2f(a.part_ml[2 * row] - m);
    l = fmaf(a.part_ml[2 * row + 1], w, l);
    o = fmaf(a.part_o[row * kD + d], w, o);
  }
  const int b = bh / a.H, h = bh % a.H;
  float* dst = a.out_blhd ? a.out + (((int64_t)b * a.Lq + qrow) * a.H + h) * kD
                          : a.out + ((int64_t)bh * a.Lq + qrow) * kD;
  dst[d] = o * (1.0f / l);
}

// Launches `main(grid, args)` over the query tiles of kBQ queries.  A last
// round that would leave CUs idle (tiles % CUs workgroups of a
// one-workgroup-per-CU shape) is split along the keys instead, so that the
// tail fills every CU; the partial results are merged by a second kernel.
// cus = 0 disables the split.
template <class Main>
int launch_tiles(SdpaArgs a, const SdpaParams& p, int kBQ, int kBKV, int cus, hipStream_t stream,
                 Main&& main) {
  TilePlan pl;
  if (!plan_tiles(p.B, p.H, p.Lq, p.Lk, kBQ, kBKV, kD, cus, pl)) return kErrDims;
  note_sdpa_query_tile(kBQ);
  a.full_tiles = (int)pl.full_tiles;
  a.splits = pl.splits;
  a.keys_per_split = pl.keys_per_split;
  a.pieces_full = (int)pl.pieces_full;
  a.splits_p = pl.splits_p;
  a.keys_per_split_p = pl.keys_per_split_p;
  if (pl.pieces > 0) {
    float* ws;
    if (p.scratch != nullptr) {
      if (!scratch_fits(pl, p.scratch_bytes)) return kErrScratch;
      ws = p.scratch;
    } else {
      ws = static_cast<float*>(stream_workspace(stream, pl.scratch_bytes, kSlotSdpaPartial));
      if (ws == nullptr) return kErrWorkspace;
    }
    a.part_o = ws;
    a.part_ml = ws + (size_t)pl.pieces * kBQ * kD;
  }
  const int64_t grid_n = pl.grid();
  main(dim3((unsigned)grid_n), a);
  if (hipGetLastError() != hipSuccess) return kErrLaunch;
  if (pl.full_tiles < pl.tiles) {
    const int64_t rows = (pl.tiles - pl.full_tiles) * (int64_t)kBQ;
    hipLaunchKernelGGL(sdpa_combine_kernel,
                       dim3((unsigned)((rows * kD + kCombineThreads - 1) / kCombineThreads)),
                       dim3(kCombineThreads), 0, stream, a, kBQ, rows);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  return kOk;
}

}  // namespace
}  // namespace sdpa
}  // namespace tsplat
