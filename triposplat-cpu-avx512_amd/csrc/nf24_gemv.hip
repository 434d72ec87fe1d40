// NF24 GEMM for few rows (M <= 32): the HBM-bound case (timestep / adaLN /
// camera rows), where the 3 bytes per weight dominate and the arithmetic
// intensity is ~0.66*M FLOP/B.
//
// Same semantics as nf24_gemm.hip (scripts/gemm_nf24_i16_avx512.c:26-197):
// out[m, c] = bias[n] + sum_k x[m, k] * w[k, n] with the weight decoded in
// registers exactly as decode16 does.  Layout of the work:
//   * a lane owns two adjacent columns (one 32-bit code01 load and one 16-bit
//     q2 load per k row: a wave reads 256 B + 128 B contiguous per row);
//   * a workgroup (W waves) owns 128 columns and a K range, split into W
//     consecutive parts, one per wave; x for that range is staged in LDS and
//     read as broadcasts;
//   * K is also split across workgroups so that every CU streams weights; the
//     per-wave partial sums are combined in LDS in wave order; each split
//     writes its partial to a per-stream workspace and a second kernel sums
//     the partials in split order, so the result is deterministic.  (A
//     last-workgroup reduction inside one kernel needs agent-scope fences,
//     which write back L2 and measured 3x slower on gfx950.)
// Per output the order is: sequential fma over each wave's rows, then the
// fixed-order sums.

#include "tsplat_common.h"
#include "tsplat_launch.h"

#include <algorithm>

namespace tsplat {
namespace {

constexpr int kReduceThreads = 256;
constexpr int kCols = 128;  // columns per workgroup

struct GemvArgs {
  const float* x;
  const int16_t* code01;
  const int8_t* q2;
  const float* scale;
  const float* bias;
  float* out;
  float* partial;   // [splits][M][count] when splits > 1
  int M, K, N, n_start, n_count, stride_x, stride_out;
  int k_per_split;  // rows of K per workgroup (multiple of 4)
  int splits;
};

template <int MT, int W>
__global__ __launch_bounds__(W * 64) void nf24_gemv_kernel(GemvArgs a) {
  constexpr int kThreads = W * 64;
  extern __shared__ float smem[];  // x tile [MT][k_per_split], then wave partials
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cgroups = (a.n_count + kCols - 1) / kCols;
  const int cg = blockIdx.x % cgroups;
  const int split = blockIdx.x / cgroups;
  const int k0 = split * a.k_per_split;
  const int k1 = min(a.K, k0 + a.k_per_split);
  const int kn = k1 - k0;

  // Stage x[k0..k1)[m] k-major, so the MT values of one row are contiguous
  // (read as 128-bit broadcasts); rows past M and K are zero.
  float* xs = smem;
  for (int i = tid; i < MT * a.k_per_split; i += kThreads) {
    const int m = i / a.k_per_split, kk = i % a.k_per_split;
    xs[kk * MT + m] = (m < a.M && kk < kn) ? a.x[(int64_t)m * a.stride_x + k0 + kk] : 0.0f;
  }
  __syncthreads();

  const int lc = cg * kCols + 2 * lane;  // local column of this lane's first column
  const bool ok0 = lc < a.n_count, ok1 = lc + 1 < a.n_count;
  const int n = a.n_start + lc;
  const float s0 = ok0 ? a.scale[n] : 0.0f;
  const float s1 = ok1 ? a.scale[n + 1] : 0.0f;
  const bool vec = ((a.N | a.n_start) & 1) == 0;

  // This wave's 1/W of the split's rows.
  const int q = (kn + W - 1) / W;
  const int r0 = wave * q, r1 = min(kn, r0 + q);

  float acc0[MT], acc1[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc0[m] = acc1[m] = 0.0f;

  auto load_row = [&](int r, uint32_t& c, uint32_t& qq) {
    const int64_t off = (int64_t)(k0 + r) * a.N + n;
    c = 0;
    qq = 0;
    if (vec) {
      if (ok0) {
        c = *reinterpret_cast<const uint32_t*>(a.code01 + off);
        qq = *reinterpret_cast<const uint16_t*>(a.q2 + off);
      }
    } else {
      if (ok0) { c = (uint16_t)a.code01[off]; qq = (uint8_t)a.q2[off]; }
      if (ok1) { c |= (uint32_t)(uint16_t)a.code01[off + 1] << 16; qq |= (uint32_t)(uint8_t)a.q2[off + 1] << 8; }
    }
  };
  auto consume = [&](int r, uint32_t c, uint32_t qq) {
    const float w0 = (float)((int32_t)(int16_t)(c & 0xffffu) * 256 + (int32_t)(int8_t)(qq & 0xffu)) * s0;
    const float w1 = (float)((int32_t)(int16_t)(c >> 16) * 256 + (int32_t)(int8_t)((qq >> 8) & 0xffu)) * s1;
    const float* xr = xs + r * MT;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float xv = xr[m];
      acc0[m] = fmaf(xv, w0, acc0[m]);
      acc1[m] = fmaf(xv, w1, acc1[m]);
    }
  };
  // Rows in groups of 8: all eight loads are issued before any is consumed.
  constexpr int kU = 8;
  int r = r0;
  for (; r + kU <= r1; r += kU) {
    uint32_t c[kU], qq[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) load_row(r + u, c[u], qq[u]);
#pragma unroll
    for (int u = 0; u < kU; ++u) consume(r + u, c[u], qq[u]);
  }
  for (; r < r1; ++r) {
    uint32_t c, qq;
    load_row(r, c, qq);
    consume(r, c, qq);
  }

  // Combine the W waves in wave order through LDS.
  __syncthreads();
  float* part = smem;  // [W][MT][kCols]
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    part[(wave * MT + m) * kCols + 2 * lane] = acc0[m];
    part[(wave * MT + m) * kCols + 2 * lane + 1] = acc1[m];
  }
  __syncthreads();
  for (int i = tid; i < MT * kCols; i += kThreads) {
    const int m = i / kCols, c = i % kCols;
    const int col = cg * kCols + c;
    if (m >= a.M || col >= a.n_count) continue;
    float v = part[m * kCols + c];
#pragma unroll
    for (int w = 1; w < W; ++w) v += part[(w * MT + m) * kCols + c];
    if (a.splits > 1) {
      a.partial[((int64_t)split * a.M + m) * a.n_count + col] = v;
    } else {
      a.out[(int64_t)m * a.stride_out + col] = a.bias[a.n_start + col] + v;
    }
  }
}

// out[m, c] = bias + sum over splits (in split order) of the partials.
__global__ __launch_bounds__(kReduceThreads) void nf24_gemv_reduce_kernel(
    const float* partial, const float* bias, float* out, int M, int count, int n_start,
    int stride_out, int splits) {
  const int64_t i = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;
  if (i >= (int64_t)M * count) return;
  const int m = (int)(i / count), c = (int)(i % count);
  float v = partial[i];
  for (int s = 1; s < splits; ++s) v += partial[(int64_t)s * M * count + i];
  out[(int64_t)m * stride_out + c] = bias[n_start + c] + v;
}

// ---------------------------------------------------------------------------
// Wide form for M <= 16 with 8-aligned columns: a lane owns 8 adjacent columns
// (one 128-bit code01 and one 64-bit q2 load per row: a wave reads 1 KB + 512 B
// of one row), a wave owns 16 (or 8) consecutive rows and issues all of
// their loads before consuming any (one HBM round trip), x comes through the
// scalar cache (a wave's row is uniform), and a workgroup of 4 waves owns 512
// columns x 64 (or 32) rows.  The 4 wave partials are added in wave order in
// LDS; splits along K go to the workspace and nf24_gemv_merge_kernel adds
// them in split order.
constexpr int kWideWaves = 4;
constexpr int kWideCols = 512;

template <int MT, int kRows>
__global__ __launch_bounds__(kWideWaves * 64) void nf24_gemv_wide_kernel(GemvArgs a) {
  constexpr int rows_per_wave = kRows;
  constexpr int kRedM = MT < 8 ? MT : 8;  // rows of x reduced per LDS pass
  __shared__ float red[kWideWaves - 1][kRedM][kWideCols];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slabs = (a.n_count + kWideCols - 1) / kWideCols;
  const int slab = blockIdx.x % slabs;
  const int split = blockIdx.x / slabs;
  const int lc = slab * kWideCols + 8 * lane;        // first local column of this lane
  const bool live = lc < a.n_count;                   // n_count % 8 == 0: all 8 or none
  const int r0 = split * a.k_per_split + wave * rows_per_wave;
  const int r1 = min(min(a.K, (split + 1) * a.k_per_split), r0 + rows_per_wave);
  const int nr = max(0, r1 - r0);

  // Issue every load of this wave's rows, then consume.  Loads are
  // unconditional (rows past the range re-read a valid row, columns past
  // n_count the first column) so they can all be in flight at once; such
  // rows are multiplied by x = 0 and such columns get scale 0.
  uint4 c[kRows];
  uint2 q[kRows];
  const int64_t col = a.n_start + (live ? lc : 0);
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t off = (int64_t)min(r0 + i, a.K - 1) * a.N + col;
    c[i] = *reinterpret_cast<const uint4*>(a.code01 + off);
    q[i] = *reinterpret_cast<const uint2*>(a.q2 + off);
  }
  float sc[8];
  {
    const floatx4 s0 = *reinterpret_cast<const floatx4*>(a.scale + col);
    const floatx4 s1 = *reinterpret_cast<const floatx4*>(a.scale + col + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc[e] = live ? s0[e] : 0.0f;
      sc[4 + e] = live ? s1[e] : 0.0f;
    }
  }
  float acc[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.0f;
  // acc[m] += x[m][row] * w[row] over the wave's rows.  Rows of x past M
  // read row M - 1 (those sums are never stored), so every x load is
  // unconditional; only rows past the split's range (the last wave of a
  // ragged split, nr < kRows: uniform) are masked, by x = 0, on a separate
  // path -- a select on a loaded value is compiled into a branch and a wait
  // per load, which would serialise the x loads of the common case.
  auto decode = [&](int i, float (&w)[8]) {
    const uint32_t cw[4] = {c[i].x, c[i].y, c[i].z, c[i].w};
    const uint32_t qw[2] = {q[i].x, q[i].y};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int32_t code = (int32_t)(int16_t)((cw[e >> 1] >> (16 * (e & 1))) & 0xffffu);
      const int32_t res = (int32_t)(int8_t)((qw[e >> 2] >> (8 * (e & 3))) & 0xffu);
      w[e] = (float)(code * 256 + res) * sc[e];
    }
  };
  const float* xrow = a.x + r0;
  if (nr == kRows) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      float w[8];
      decode(i, w);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float xv = xrow[(int64_t)min(m, a.M - 1) * a.stride_x + i];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = fmaf(xv, w[e], acc[m][e]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      float w[8];
      decode(i, w);
      const int row = min(r0 + i, a.K - 1);
      const bool row_ok = i < nr;  // uniform over the wave
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float xv = row_ok ? a.x[(int64_t)min(m, a.M - 1) * a.stride_x + row] : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = fmaf(xv, w[e], acc[m][e]);
      }
    }
  }

  // Waves 1..3 hand their sums to wave 0, which adds them in wave order
  // (kRedM rows of x per pass through LDS).
#pragma unroll
  for (int m0 = 0; m0 < MT; m0 += kRedM) {
    if (m0 > 0) __syncthreads();  // wave 0 has read the previous pass
    if (wave > 0) {
#pragma unroll
      for (int m = 0; m < kRedM; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wave - 1][m][8 * lane + e] = acc[m0 + m][e];
    }
    __syncthreads();
    if (wave != 0 || !live) continue;
#pragma unroll
    for (int m = m0; m < m0 + kRedM; ++m) {
      if (m >= a.M) break;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = acc[m][e];
#pragma unroll
        for (int w = 0; w < kWideWaves - 1; ++w) v[e] += red[w][m - m0][8 * lane + e];
      }
      if (a.splits > 1) {
        float* dst = a.partial + ((int64_t)split * a.M + m) * a.n_count + lc;
        *reinterpret_cast<floatx4*>(dst) = floatx4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<floatx4*>(dst + 4) = floatx4{v[4], v[5], v[6], v[7]};
      } else {
        float* dst = a.out + (int64_t)m * a.stride_out + lc;
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = a.bias[col + e] + v[e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA form for 4 <= M <= 16 (columns, column offset and N multiples of kCols,
// 16-byte aligned codes, scales and x rows): one workgroup owns kCols
// columns over the whole K range, so no partial sums leave the chip and no
// second kernel runs.  Each wave takes consecutive 32-row chunks of K
// (kWaves equal ranges); per chunk every lane loads 8 columns of one row
// (a 128-bit code01 and a 64-bit q2 load: a wave instruction covers whole
// rows of the slab) and 8 values of one x row, decodes the weights exactly
// as decode16 and stores them transposed into the wave's own LDS tile
// ([col][k], [row][k]); v_mfma_f32_16x16x4_f32 then accumulates x rows
// 0..15 against 16-column blocks, the k inside each 16-slice permuted
// identically for both operands so every lane reads 4 consecutive k with one
// ds_read_b128.  The loads of kPass chunks are issued before any is used.
// (Rows a wave does not own are multiplied by x = 0.)
// The wave sums are added in wave order through LDS.  Rows of x past M read
// row M - 1; their sums are never stored.  With a.splits > 1 the K range is
// also split across workgroups (workgroup (split, slab) runs waves split *
// kWaves .. of a.k_per_split rows each) and each writes its sums to
// a.partial[split][M][n_count] for nf24_gemv_merge_kernel, which adds the
// bias and the splits in split order.
constexpr int kMfmaRows = 32;            // K rows per chunk
constexpr int kMfmaS = kMfmaRows + 4;    // LDS row stride in floats

template <int kCols, int kWaves, int kPass>
__global__ __launch_bounds__(kWaves * 64) void nf24_gemv_mfma_kernel(GemvArgs a) {
  constexpr int kLanesPerRow = kCols / 8;              // 8 columns per lane
  constexpr int kRowsPerLoad = 64 / kLanesPerRow;      // rows per wave instruction
  constexpr int kLoads = kMfmaRows / kRowsPerLoad;     // instructions per chunk
  constexpr int kBlocks = kCols / 16;
  __shared__ __attribute__((aligned(16))) float ws[kWaves][kCols * kMfmaS];
  __shared__ __attribute__((aligned(16))) float xs[kWaves][16 * kMfmaS];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Neighbouring slabs share cache lines (a 32-column slab is half a 128-byte
  // line of code01 and a quarter of one of q2): each XCD takes a contiguous
  // run of slabs so that a line is fetched into one L2, not up to four.
  // Tiles are split-major, so an XCD's run holds neighbouring slabs of one split.
  const int slabs = gridDim.x / a.splits;
  const int tile = xcd_tile_index(blockIdx.x, gridDim.x);
  const int split = tile / slabs;
  const int c0 = (tile % slabs) * kCols;             // first local column of the slab
  const int cg = lane % kLanesPerRow, lr = lane / kLanesPerRow;
  const int64_t ncol = a.n_start + c0 + 8 * cg;      // this lane's first column
  const int kw0 = (split * kWaves + wave) * a.k_per_split;  // k_per_split: rows per wave
  const int kw1 = min(a.K, kw0 + a.k_per_split);
  const int xm = min(lane >> 2, a.M - 1);            // x row this lane stages
  const int xk = 8 * (lane & 3);                     // its 8 k within a chunk

  float sc[8];
  {
    const floatx4 s0 = *reinterpret_cast<const floatx4*>(a.scale + ncol);
    const floatx4 s1 = *reinterpret_cast<const floatx4*>(a.scale + ncol + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc[e] = s0[e];
      sc[4 + e] = s1[e];
    }
  }
  floatx4 acc[kBlocks];
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) acc[b] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  float* wsw = ws[wave];
  float* xsw = xs[wave];

  for (int kb = kw0; kb < kw1; kb += kPass * kMfmaRows) {
    uint4 c[kPass][kLoads];
    uint2 q[kPass][kLoads];
    floatx4 xv[kPass][2];
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      const int kc = kb + p * kMfmaRows;
      // Code loads are unconditional (rows past K re-read row K - 1) so that
      // all of them are in flight at once; rows outside the wave's range
      // meet x = 0 below, and every decoded weight is finite.
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int kr = min(kc + i * kRowsPerLoad + lr, a.K - 1);
        const int64_t off = (int64_t)kr * a.N + ncol;
        c[p][i] = *reinterpret_cast<const uint4*>(a.code01 + off);
        q[p][i] = *reinterpret_cast<const uint2*>(a.q2 + off);
      }
      const float* xr = a.x + (int64_t)xm * a.stride_x + kc + xk;
      if (kc + kMfmaRows <= kw1) {  // uniform over the wave
        xv[p][0] = *reinterpret_cast<const floatx4*>(xr);
        xv[p][1] = *reinterpret_cast<const floatx4*>(xr + 4);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[p][e >> 2][e & 3] = (kc + xk + e < kw1) ? xr[e] : 0.0f;
      }
    }
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const uint32_t cw[4] = {c[p][i].x, c[p][i].y, c[p][i].z, c[p][i].w};
        const uint32_t qw[2] = {q[p][i].x, q[p][i].y};
        const int kl = i * kRowsPerLoad + lr;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int32_t code = (int32_t)(int16_t)((cw[e >> 1] >> (16 * (e & 1))) & 0xffffu);
          const int32_t res = (int32_t)(int8_t)((qw[e >> 2] >> (8 * (e & 3))) & 0xffu);
          wsw[(8 * cg + e) * kMfmaS + kl] = (float)(code * 256 + res) * sc[e];
        }
      }
      *reinterpret_cast<floatx4*>(&xsw[(lane >> 2) * kMfmaS + xk]) = xv[p][0];
      *reinterpret_cast<floatx4*>(&xsw[(lane >> 2) * kMfmaS + xk + 4]) = xv[p][1];
      // The tile is this wave's alone: LDS runs one wave's instructions in
      // order, so a wave-scope fence (which keeps the compiler from moving
      // the reads above the stores) is all the ordering needed.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int kk = 0; kk < kMfmaRows / 16; ++kk) {
        const int koff = 16 * kk + 4 * (lane >> 4);
        const floatx4 af = *reinterpret_cast<const floatx4*>(&xsw[(lane & 15) * kMfmaS + koff]);
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
          const floatx4 bf =
              *reinterpret_cast<const floatx4*>(&wsw[(16 * b + (lane & 15)) * kMfmaS + koff]);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[t], bf[t], acc[b], 0, 0, 0);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // Wave sums in wave order.  Lane l of block b holds rows 4*(l/16) + i,
  // column 16 b + l % 16.
  __syncthreads();
  float* red = &ws[0][0];  // [kWaves][kBlocks][64 lanes][4]
#pragma unroll
  for (int b = 0; b < kBlocks; ++b)
    *reinterpret_cast<floatx4*>(&red[((wave * kBlocks + b) * 64 + lane) * 4]) = acc[b];
  __syncthreads();
  for (int i = tid; i < kBlocks * 64 * 4; i += kWaves * 64) {
    float v = red[i];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += red[w * kBlocks * 256 + i];
    const int b = i / 256, l = (i / 4) % 64, r = i % 4;
    const int row = 4 * (l >> 4) + r, col = c0 + 16 * b + (l & 15);
    if (row >= a.M) continue;
    if (a.splits == 1)
      a.out[(int64_t)row * a.stride_out + col] = a.bias[a.n_start + col] + v;
    else
      a.partial[((int64_t)split * a.M + row) * a.n_count + col] = v;
  }
}

// out[m, c] = bias + sum over splits (in split order) of the partials, for
// up to kMergeMaxSplits splits.  A workgroup owns 16 columns of one row m;
// its 16 threads per column each load every 16th split -- all of a thread's
// loads are issued before any is used, so the partials arrive in one memory
// round trip -- and stage them in LDS, where one thread per column adds them
// in split order.  (16 columns per workgroup gives 4x the workgroups of a
// 64-column chunk; the merge is latency-bound, not bandwidth-bound.)
constexpr int kMergeCols = 16;
constexpr int kMergeLanes = kReduceThreads / kMergeCols;  // threads per column
constexpr int kMergeMaxSplits = 128;
__global__ __launch_bounds__(kReduceThreads) void nf24_gemv_merge_kernel(
    const float* partial, const float* bias, float* out, int M, int count, int n_start,
    int stride_out, int splits) {
  __shared__ float part[kMergeMaxSplits][kMergeCols + 1];
  const int chunks = (count + kMergeCols - 1) / kMergeCols;
  const int m = blockIdx.x / chunks;
  const int c0 = (blockIdx.x % chunks) * kMergeCols;
  const int c = threadIdx.x % kMergeCols, j = threadIdx.x / kMergeCols;
  const bool ok = c0 + c < count;
  constexpr int kPer = kMergeMaxSplits / kMergeLanes;
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int sp = j + kMergeLanes * i;
    v[i] = (ok && sp < splits) ? partial[((int64_t)sp * M + m) * count + c0 + c] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int sp = j + kMergeLanes * i;
    if (sp < splits) part[sp][c] = v[i];
  }
  __syncthreads();
  if (j != 0 || !ok) return;
  float acc = part[0][c];
  for (int sp = 1; sp < splits; ++sp) acc += part[sp][c];
  out[(int64_t)m * stride_out + c0 + c] = bias[n_start + c0 + c] + acc;
}

// Second kernel of a split call: the merge above, or for more splits than it
// stages, one thread per output (same order, same result).
int launch_merge(const float* partial, const float* bias, float* out, int M, int count, int n_start,
                 int stride_out, int splits, hipStream_t stream) {
  if (splits <= kMergeMaxSplits) {
    const int chunks = (count + kMergeCols - 1) / kMergeCols;
    hipLaunchKernelGGL(nf24_gemv_merge_kernel, dim3((unsigned)(M * chunks)), dim3(kReduceThreads), 0,
                       stream, partial, bias, out, M, count, n_start, stride_out, splits);
  } else {
    const int64_t total = (int64_t)M * count;
    hipLaunchKernelGGL(nf24_gemv_reduce_kernel,
                       dim3((unsigned)((total + kReduceThreads - 1) / kReduceThreads)),
                       dim3(kReduceThreads), 0, stream, partial, bias, out, M, count, n_start,
                       stride_out, splits);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <int MT>
int launch_wide(GemvArgs a, hipStream_t stream) {
  const dim3 grid((unsigned)(((a.n_count + kWideCols - 1) / kWideCols) * a.splits));
  if (a.k_per_split == kWideWaves * 16)
    hipLaunchKernelGGL((nf24_gemv_wide_kernel<MT, 16>), grid, dim3(kWideWaves * 64), 0, stream, a);
  else
    hipLaunchKernelGGL((nf24_gemv_wide_kernel<MT, 8>), grid, dim3(kWideWaves * 64), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <int MT, int W>
int launch_mt(GemvArgs a, int cgroups, int splits, hipStream_t stream) {
  const size_t x_bytes = (size_t)MT * a.k_per_split * 4;
  const size_t p_bytes = (size_t)W * MT * kCols * 4;
  const size_t lds = x_bytes > p_bytes ? x_bytes : p_bytes;
  if (lds > 64 * 1024) return kErrDims;
  hipLaunchKernelGGL((nf24_gemv_kernel<MT, W>), dim3(cgroups * splits), dim3(W * 64), lds, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace

// Workgroups of W waves (16 for M <= 4, 8 for M <= 8, else 4: the LDS of the
// in-workgroup reduction is W * M * 128 floats) own 128 columns and split
// their K range W ways.  K is split across workgroups only when the column
// groups alone leave most CUs idle (fewer than 64 groups), so that ~256
// workgroups stream the weights, at most until each wave keeps 16 rows and
// the partial sums (splits * M * count * 8 bytes) stay under half the weight
// bytes; a split costs a second, small kernel.
namespace {
// The MFMA form, 8 waves, all loads of up to 4 chunks in flight, slabs of 32
// columns when that gives at least 192 workgroups, else of 16 (N = 3072:
// 192 slabs of 16).  Measured against the K-split wide kernel (cold weights,
// HIP-graph replay, per call; M = 16 / 8 / 4): N = 3072, K = 1024: 8.4 /
// 8.3 / ~8.2 us (16-column slabs; 32-column: 9.9 / 9.6) against 16.3 / 11.4 /
// 9.1 us; N = 6144: 10.5 / 10.2 / ~10.2 us (32-column; 16-column: 13.9 /
// 13.4) against 22.0 / 14.9 / 11.3 us.  With fewer than 192 slabs of 16
// (N = 1024, K = 4096) too few CUs stream, and at M <= 2 the split kernel
// is faster (7.2-9.5 us), so those stay on it.  64-column slabs and 4 or 16
// waves measured slower.
constexpr int kMfmaWaves = 8;
constexpr int kMfmaMinRows = 4;
constexpr int kMfmaMinWorkgroups = 192;
// Fewer slabs than that (N = 1024): the K range is split too, so that about
// kMfmaSplitTarget workgroups stream the weights, each wave keeping at least
// one 32-row chunk; the partial sums (splits * M * N * 8 bytes moved, 0.5 MB
// at K = 4096, N = 1024, M = 16, four splits) are a few percent of the
// weight bytes, and nf24_gemv_merge_kernel adds them in split order.
constexpr int kMfmaSplitTarget = 256;

template <int kCols>
int launch_mfma_form(const GemmParams& p, int splits, hipStream_t stream) {
  const int waves = kMfmaWaves * splits;
  const int per_wave = ((p.K + waves * kMfmaRows - 1) / (waves * kMfmaRows)) * kMfmaRows;
  // Splits left with no rows after the rounding to whole chunks are dropped.
  splits = (p.K + kMfmaWaves * per_wave - 1) / (kMfmaWaves * per_wave);
  GemvArgs a{p.x, p.code01, p.q2, p.scale, p.bias, p.out, nullptr, p.M, p.K, p.N,
             p.n_start, p.n_count, p.stride_x, p.stride_out, per_wave, splits};
  if (splits > 1) {
    a.partial = static_cast<float*>(
        stream_workspace(stream, (size_t)splits * p.M * p.n_count * 4, kSlotGemvPartial));
    if (a.partial == nullptr) return kErrWorkspace;
  }
  // Chunks in flight per wave: 4, or as many as a wave owns when that is
  // fewer (a K split can leave a wave one 32-row chunk: the out-projection's
  // 6-row tail at K = 1024, whose chunks 2-4 were loaded, decoded and
  // multiplied by x = 0; 12294 x 1024 x 1024 212.0 -> 208.7 us, the same
  // bits).
  const int chunks = per_wave / kMfmaRows;
  const dim3 grid((unsigned)(p.n_count / kCols * splits)), block(kMfmaWaves * 64);
  if (chunks >= 4)
    hipLaunchKernelGGL((nf24_gemv_mfma_kernel<kCols, kMfmaWaves, 4>), grid, block, 0, stream, a);
  else if (chunks >= 2)
    hipLaunchKernelGGL((nf24_gemv_mfma_kernel<kCols, kMfmaWaves, 2>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((nf24_gemv_mfma_kernel<kCols, kMfmaWaves, 1>), grid, block, 0, stream, a);
  if (hipGetLastError() != hipSuccess) return kErrLaunch;
  if (splits == 1) return kOk;
  return launch_merge(a.partial, p.bias, p.out, p.M, p.n_count, p.n_start, p.stride_out, splits, stream);
}
}  // namespace

int launch_nf24_gemv(const GemmParams& p, hipStream_t stream) {
  if (p.M < 1 || p.M > 32) return kErrDims;
  const bool mfma_shape = p.M >= kMfmaMinRows && p.M <= 16 && ((p.N | p.n_start | p.n_count) % 16) == 0 &&
                          (p.stride_x & 3) == 0 && (reinterpret_cast<uintptr_t>(p.x) & 15) == 0 &&
                          (reinterpret_cast<uintptr_t>(p.code01) & 15) == 0 &&
                          (reinterpret_cast<uintptr_t>(p.q2) & 15) == 0 &&
                          (reinterpret_cast<uintptr_t>(p.scale) & 15) == 0;
  if (mfma_shape) {
    const int slabs16 = p.n_count / 16;
    if (slabs16 >= kMfmaMinWorkgroups) {
      if (((p.N | p.n_start | p.n_count) % 32) == 0 && p.n_count / 32 >= kMfmaMinWorkgroups)
        return launch_mfma_form<32>(p, 1, stream);
      return launch_mfma_form<16>(p, 1, stream);
    }
    const int splits = std::min((kMfmaSplitTarget + slabs16 - 1) / slabs16, p.K / (kMfmaWaves * kMfmaRows));
    if (splits >= 2 && splits <= kMergeMaxSplits && slabs16 * splits >= kMfmaMinWorkgroups)
      return launch_mfma_form<16>(p, splits, stream);
  }
  const bool wide = p.M <= 16 && ((p.N | p.n_start | p.n_count) & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.code01) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.q2) & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.scale) & 15) == 0;
  if (wide) {
    // 16 rows per wave (64 per workgroup); 8 when that leaves fewer than 128
    // workgroups (one K split per 64 or 32 rows).
    const int slabs = (p.n_count + kWideCols - 1) / kWideCols;
    int kps = kWideWaves * 16;
    if ((int64_t)slabs * ((p.K + kps - 1) / kps) < 128) kps /= 2;
    const int splits = (p.K + kps - 1) / kps;
    if (splits <= kMergeMaxSplits) {
      GemvArgs a{p.x, p.code01, p.q2, p.scale, p.bias, p.out, nullptr, p.M, p.K, p.N,
                 p.n_start, p.n_count, p.stride_x, p.stride_out, kps, splits};
      if (splits > 1) {
        a.partial = static_cast<float*>(
            stream_workspace(stream, (size_t)splits * p.M * p.n_count * 4, kSlotGemvPartial));
        if (a.partial == nullptr) return kErrWorkspace;
      }
      int st;
      switch (p.M <= 1 ? 1 : p.M <= 2 ? 2 : p.M <= 4 ? 4 : p.M <= 8 ? 8 : 16) {
        case 1: st = launch_wide<1>(a, stream); break;
        case 2: st = launch_wide<2>(a, stream); break;
        case 4: st = launch_wide<4>(a, stream); break;
        case 8: st = launch_wide<8>(a, stream); break;
        default: st = launch_wide<16>(a, stream); break;
      }
      if (st != kOk || splits == 1) return st;
      return launch_merge(a.partial, p.bias, p.out, p.M, p.n_count, p.n_start, p.stride_out, splits,
                          stream);
    }
  }
  const int mt = p.M <= 1 ? 1 : p.M <= 2 ? 2 : p.M <= 4 ? 4 : p.M <= 8 ? 8 : p.M <= 16 ? 16 : 32;
  const int w = mt <= 4 ? 16 : mt <= 8 ? 8 : 4;
  const int cgroups = (p.n_count + kCols - 1) / kCols;
  int splits = 1;
  if (cgroups < 64) {
    splits = (256 + cgroups - 1) / cgroups;
    const int by_rows = p.K / (16 * w) > 1 ? p.K / (16 * w) : 1;
    const double by_traffic = 0.1875 * (double)p.K / (double)p.M;
    if (splits > by_rows) splits = by_rows;
    if (splits > by_traffic) splits = by_traffic < 1.0 ? 1 : (int)by_traffic;
    if (splits < 1) splits = 1;
  }
  int kps = (((p.K + splits - 1) / splits) + 3) & ~3;
  while ((size_t)mt * kps * 4 > 64 * 1024) {  // keep the x tile within 64 KB of LDS
    ++splits;
    kps = (((p.K + splits - 1) / splits) + 3) & ~3;
  }
  splits = (p.K + kps - 1) / kps;

  GemvArgs a{p.x, p.code01, p.q2, p.scale, p.bias, p.out, nullptr, p.M, p.K, p.N,
             p.n_start, p.n_count, p.stride_x, p.stride_out, kps, splits};
  if (splits > 1) {
    a.partial = static_cast<float*>(
        stream_workspace(stream, (size_t)splits * p.M * p.n_count * 4, kSlotGemvPartial));
    if (a.partial == nullptr) return kErrWorkspace;
  }
  int st;
  switch (mt) {
    case 1: st = launch_mt<1, 16>(a, cgroups, splits, stream); break;
    case 2: st = launch_mt<2, 16>(a, cgroups, splits, stream); break;
    case 4: st = launch_mt<4, 16>(a, cgroups, splits, stream); break;
    case 8: st = launch_mt<8, 8>(a, cgroups, splits, stream); break;
    case 16: st = launch_mt<16, 4>(a, cgroups, splits, stream); break;
    default: st = launch_mt<32, 4>(a, cgroups, splits, stream); break;
  }
  if (st != kOk || splits == 1) return st;
  return launch_merge(a.partial, p.bias, p.out, p.M, p.n_count, p.n_start, p.stride_out, splits, stream);
}

}  // namespace tsplat
