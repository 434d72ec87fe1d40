// NF24 packed-weight GEMM for gfx950: out = bias + X * decode(W).
//
// Reference semantics: scripts/gemm_nf24_i16_avx512.c:26-33 (decode16) and
// :35-197 (kernel_mx16 / range API).  Each weight is decoded exactly as the
// reference does -- fp32((int32)q01 * 256 + q2) * scale[n], one rounding --
// in registers, right after the packed codes arrive from HBM; no fp32
// weight copy ever exists in HBM.  The products are accumulated with fp32
// MFMA (v_mfma_f32_32x32x2_f32), so only the summation order differs from
// the reference's sequential fmaf chain.
//
// Tiling: a workgroup computes a BM x BN output tile with WM x WN waves; a
// wave owns (BM/WM) x (BN/WN) = MB x NB blocks of 32x32.  Per K step of BK,
// the X tile (fp32) and the decoded W tile (fp32) are staged in LDS, both
// stored k-contiguous ([row][k] and [col][k]) so that every lane fetches
// four consecutive k of its row/column with one ds_read_b128.  The K index
// inside an 8-wide slice is permuted: MFMA step t of slice kk reads
// k = 8*kk + 4*(lane/32) + t, the same permutation for A and B, which keeps
// the dot product exact while turning 4 scalar LDS reads into one.
// The next K step's codes and X are fetched into registers while the MFMAs
// of the current step run (double-buffered LDS, one barrier per step).

#include "nf24_gemm_common.h"

#include <atomic>


namespace tsplat {
namespace {

using namespace nf24;

template <int BM_, int BN_, int BK_, int WM_, int WN_, int kMinWaves_ = 1, int kProducers_ = 0,
          bool kDefer_ = false>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  // kDefer: the last k-slice of each K step is read into registers before the
  // step's barrier and multiplied after it, overlapping the next step's first
  // LDS reads (same per-accumulator order, so the same result).
  static constexpr bool kDefer = kDefer_;
  static constexpr int kMinWaves = kMinWaves_;  // waves per SIMD the register budget must allow
  // kProducers > 0: that many extra waves only stage tiles (load, decode,
  // store to LDS) while the WM x WN waves only run MFMAs; 0: every wave does both.
  static constexpr int kProducers = kProducers_;
  static constexpr int kComputeWaves = WM * WN;
  static constexpr int kThreads = (kComputeWaves + kProducers) * 64;
  static constexpr int kLoadThreads = kProducers > 0 ? kProducers * 64 : kThreads;
  static constexpr int kTM = BM / WM, kTN = BN / WN;
  static constexpr int kMB = kTM / 32, kNB = kTN / 32;
  static constexpr int kS = BK + 4;  // LDS row stride in floats (bank spread)
  // X tile: BM x BK as float4 units; W tile: (column pair, kWK consecutive k)
  // units, kWK = 4 unless that leaves loading threads idle.
  static constexpr int kXUnits = BM * BK / 4;
  static constexpr int kWK = ((BN / 2) * (BK / 4) >= kLoadThreads) ? 4 : 2;
  static constexpr int kWUnits = (BN / 2) * (BK / kWK);
  static constexpr int kXIter = (kXUnits + kLoadThreads - 1) / kLoadThreads;
  static constexpr int kWIter = (kWUnits + kLoadThreads - 1) / kLoadThreads;
  static_assert(kTM % 32 == 0 && kTN % 32 == 0, "wave tile must be 32-aligned");
  static_assert(BK % 8 == 0 && BN % 2 == 0, "BK must be a multiple of 8, BN even");
  static_assert(kThreads <= 1024, "at most 1024 threads per workgroup");
};

// Moves one K step of the X tile (fp32) and the W tile (packed codes, decoded
// to fp32) from global memory through registers into LDS, both stored
// k-contiguous ([row][k], [col][k], row stride kS).  Thread t of the
// C::kLoadThreads loading threads owns fixed X float4 units and W units
// (column pair, kWK consecutive k).  kVec: x rows 16-byte aligned with
// K % 4 == 0, and N, n_start, n_count even (a column pair is one 32-bit /
// 16-bit access), the code planes and the tile's x rows each below 2^31
// bytes (vec_buffers_fit).  The kVec path loads through buffer resources --
// x from the tile's first row, the code planes from their start -- with
// fixed per-thread byte offsets: rows past M and columns past n_count carry
// kBufOob, code rows past K lie past the end of the planes, so every bound
// reads 0 without a branch in the K loop (measured against guarded 64-bit
// pointer loads: configs[0] 207 -> 198 us, 16384 x 4096 x 1024 1084 -> 1036
// us, 12294 x 4096 x 1024 1078 -> 937 us, bit-identical).
template <class C, bool kVec>
struct TileLoader {
  int t;
  int m0;
  int w_pair[C::kWIter], w_kq[C::kWIter], w_nabs[C::kWIter];
  bool w_ok0[C::kWIter], w_ok1[C::kWIter], w_live[C::kWIter];
  float w_sc0[C::kWIter], w_sc1[C::kWIter];
  floatx4 xr[C::kXIter];
  uint32_t cr[C::kWIter][C::kWK];  // two int16 codes (columns lc, lc+1)
  uint32_t qr[C::kWIter][C::kWK];  // two int8 codes in the low 16 bits
  __amdgpu_buffer_rsrc_t rx, rc, rq;  // kVec: x tile rows, code01 plane, q2 plane
  uint32_t x_off[C::kXIter];          // byte offset of the x unit at k0 = 0, or kBufOob
  uint32_t c_off[C::kWIter], q_off[C::kWIter];  // byte offsets of the code row kWK*w_kq at k0 = 0

  // The column pairs and their scales are fixed for the whole K loop.
  __device__ __forceinline__ void init(const GemmArgs& a, int t_, int m0_, int c0) {
    t = t_;
    m0 = m0_;
#pragma unroll
    for (int j = 0; j < C::kWIter; ++j) {
      const int u = t + j * C::kLoadThreads;
      w_live[j] = u < C::kWUnits;
      w_pair[j] = u % (C::BN / 2);
      w_kq[j] = u / (C::BN / 2);
      const int lc = c0 + 2 * w_pair[j];
      w_ok0[j] = w_live[j] && lc < a.n_count;
      w_ok1[j] = w_live[j] && lc + 1 < a.n_count;
      w_nabs[j] = a.n_start + lc;
      w_sc0[j] = w_ok0[j] ? a.scale[w_nabs[j]] : 0.0f;
      w_sc1[j] = w_ok1[j] ? a.scale[w_nabs[j] + 1] : 0.0f;
    }
    if constexpr (kVec) {
      // x: rows m0 .. m0 + rows - 1, the last one K floats long
      const int rows = min(C::BM, a.M - m0);
      rx = buffer_rsrc(a.x + (int64_t)m0 * a.stride_x, ((int64_t)(rows - 1) * a.stride_x + a.K) * 4);
      rc = buffer_rsrc(a.code01, (int64_t)a.K * a.N * 2);
      rq = buffer_rsrc(a.q2, (int64_t)a.K * a.N);
#pragma unroll
      for (int j = 0; j < C::kXIter; ++j) {
        const int idx = t + j * C::kLoadThreads;
        const int row = idx / (C::BK / 4);
        const int kc = idx % (C::BK / 4);
        const bool live = (C::kXUnits % C::kLoadThreads == 0) || idx < C::kXUnits;
        x_off[j] = (live && row < rows) ? (uint32_t)(row * a.stride_x + 4 * kc) * 4u : kBufOob;
      }
#pragma unroll
      for (int j = 0; j < C::kWIter; ++j) {
        // w_ok1 == w_ok0 here: n_start and n_count are even
        const uint32_t e = (uint32_t)(C::kWK * w_kq[j] * a.N + w_nabs[j]);
        c_off[j] = w_ok0[j] ? 2u * e : kBufOob;
        q_off[j] = w_ok0[j] ? e : kBufOob;
      }
    }
  }

  __device__ __forceinline__ void load(const GemmArgs& a, int k0) {
    if constexpr (kVec) {
#pragma unroll
      for (int j = 0; j < C::kXIter; ++j) {
        // K % 4 == 0: a float4 unit lies wholly inside or past the row's K floats
        const int kc = (t + j * C::kLoadThreads) % (C::BK / 4);
        const uint32_t off = (k0 + 4 * kc < a.K) ? x_off[j] + 4u * (uint32_t)k0 : kBufOob;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
        xr[j] = floatx4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                        __uint_as_float(v[3])};
      }
#pragma unroll
      for (int j = 0; j < C::kWIter; ++j) {
#pragma unroll
        for (int i = 0; i < C::kWK; ++i) {
          // code rows k0 + i + kWK*w_kq >= K lie past the end of the planes: they read 0
          const uint32_t e = (uint32_t)(k0 + i) * (uint32_t)a.N;
          cr[j][i] = __builtin_amdgcn_raw_buffer_load_b32(rc, (int)(c_off[j] + 2u * e), 0, 0);
          qr[j][i] = __builtin_amdgcn_raw_buffer_load_b16(rq, (int)(q_off[j] + e), 0, 0);
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < C::kXIter; ++j) {
      const int idx = t + j * C::kLoadThreads;
      const int row = idx / (C::BK / 4);
      const int kc = idx % (C::BK / 4);
      const int gm = m0 + row;
      const int gk = k0 + 4 * kc;
      const bool live = (C::kXUnits % C::kLoadThreads == 0) || idx < C::kXUnits;
      const float* src = a.x + (int64_t)gm * a.stride_x + gk;
#pragma unroll
      for (int e = 0; e < 4; ++e) xr[j][e] = (live && gm < a.M && gk + e < a.K) ? src[e] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < C::kWIter; ++j) {
#pragma unroll
      for (int i = 0; i < C::kWK; ++i) {
        const int gk = k0 + C::kWK * w_kq[j] + i;
        const int64_t off = (int64_t)gk * a.N + w_nabs[j];
        const bool k_ok = gk < a.K;
        const uint32_t c_lo = (k_ok && w_ok0[j]) ? (uint16_t)a.code01[off] : 0u;
        const uint32_t c_hi = (k_ok && w_ok1[j]) ? (uint16_t)a.code01[off + 1] : 0u;
        const uint32_t q_lo = (k_ok && w_ok0[j]) ? (uint8_t)a.q2[off] : 0u;
        const uint32_t q_hi = (k_ok && w_ok1[j]) ? (uint8_t)a.q2[off + 1] : 0u;
        cr[j][i] = c_lo | (c_hi << 16);
        qr[j][i] = q_lo | (q_hi << 8);
      }
    }
  }

  // Decodes w = fp32((int32)q01 * 256 + q2) * scale (the reference's
  // decode16, one rounding) and stores both tiles.
  __device__ __forceinline__ void store(float* xs, float* ws) {
#pragma unroll
    for (int j = 0; j < C::kXIter; ++j) {
      const int idx = t + j * C::kLoadThreads;
      if ((C::kXUnits % C::kLoadThreads) != 0 && idx >= C::kXUnits) continue;
      const int row = idx / (C::BK / 4);
      const int kc = idx % (C::BK / 4);
      *reinterpret_cast<floatx4*>(&xs[row * C::kS + 4 * kc]) = xr[j];
    }
#pragma unroll
    for (int j = 0; j < C::kWIter; ++j) {
      if ((C::kWUnits % C::kLoadThreads) != 0 && !w_live[j]) continue;
      typedef float wvec __attribute__((ext_vector_type(C::kWK)));
      wvec w0, w1;
#pragma unroll
      for (int e = 0; e < C::kWK; ++e) {
        const uint32_t c = cr[j][e];
        const uint32_t q = qr[j][e];
        const int32_t qa = (int32_t)(int16_t)(c & 0xffffu) * 256 + (int32_t)(int8_t)(q & 0xffu);
        const int32_t qb = (int32_t)(int16_t)(c >> 16) * 256 + (int32_t)(int8_t)((q >> 8) & 0xffu);
        w0[e] = (float)qa * w_sc0[j];
        w1[e] = (float)qb * w_sc1[j];
      }
      *reinterpret_cast<wvec*>(&ws[(2 * w_pair[j]) * C::kS + C::kWK * w_kq[j]]) = w0;
      *reinterpret_cast<wvec*>(&ws[(2 * w_pair[j] + 1) * C::kS + C::kWK * w_kq[j]]) = w1;
    }
  }
};

// One K step of MFMAs of a wave over the staged tiles xb / wb.  The K index
// inside each 8-slice is permuted identically for A and B (step t reads
// k = 8kk + 4*(lane/32) + t), so every lane fetches 4 consecutive k with one
// ds_read_b128 and the dot product is unchanged.
template <class C>
__device__ __forceinline__ void mfma_step(const float* xb, const float* wb, int wm, int wn, int g,
                                          int l32, floatx16 (&acc)[C::kMB][C::kNB]) {
#pragma unroll
  for (int kk = 0; kk < C::BK / 8; ++kk) {
    floatx4 af[C::kMB], bf[C::kNB];
#pragma unroll
    for (int mb = 0; mb < C::kMB; ++mb)
      af[mb] = *reinterpret_cast<const floatx4*>(
          &xb[(wm * C::kTM + mb * 32 + l32) * C::kS + 8 * kk + 4 * g]);
#pragma unroll
    for (int nb = 0; nb < C::kNB; ++nb)
      bf[nb] = *reinterpret_cast<const floatx4*>(
          &wb[(wn * C::kTN + nb * 32 + l32) * C::kS + 8 * kk + 4 * g]);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
        for (int nb = 0; nb < C::kNB; ++nb)
          acc[mb][nb] = mfma32x32x2(af[mb][t], bf[nb][t], acc[mb][nb]);
  }
}

// Fragments of k-slice kk of a staged step, and their 16 MFMA k-steps.
template <class C>
struct Frags {
  floatx4 af[C::kMB], bf[C::kNB];
};
template <class C>
__device__ __forceinline__ void read_slice(const float* xb, const float* wb, int kk, int wm, int wn,
                                           int g, int l32, Frags<C>& f) {
#pragma unroll
  for (int mb = 0; mb < C::kMB; ++mb)
    f.af[mb] = *reinterpret_cast<const floatx4*>(
        &xb[(wm * C::kTM + mb * 32 + l32) * C::kS + 8 * kk + 4 * g]);
#pragma unroll
  for (int nb = 0; nb < C::kNB; ++nb)
    f.bf[nb] = *reinterpret_cast<const floatx4*>(
        &wb[(wn * C::kTN + nb * 32 + l32) * C::kS + 8 * kk + 4 * g]);
}
template <class C>
__device__ __forceinline__ void mfma_slice(const Frags<C>& f, floatx16 (&acc)[C::kMB][C::kNB]) {
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < C::kNB; ++nb)
        acc[mb][nb] = mfma32x32x2(f.af[mb][t], f.bf[nb][t], acc[mb][nb]);
}

template <class C, bool kVec, int kEpi>
__global__ __launch_bounds__(C::kThreads) __attribute__((amdgpu_waves_per_eu(C::kMinWaves)))
void nf24_gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[2][C::BM * C::kS];
  __shared__ __attribute__((aligned(16))) float ws[2][C::BN * C::kS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int l32 = lane & 31;

  const int tiles_n = (a.n_count + C::BN - 1) / C::BN;
  int tm, tn;
  xcd_grid(blockIdx.x, gridDim.x / tiles_n, tiles_n, a.xcd_pm, a.xcd_pn, tm, tn);
  const int m0 = tm * C::BM;
  const int c0 = tn * C::BN;
  const int nk = (a.K + C::BK - 1) / C::BK;

  if (C::kProducers > 0 && wave >= C::kComputeWaves) {
    // Producer waves: stage K step kt + 1 into the other buffer while the
    // MFMA waves consume step kt; one barrier per step, as the consumers.
    TileLoader<C, kVec> ld;
    ld.init(a, tid - C::kComputeWaves * 64, m0, c0);
    ld.load(a, 0);
    ld.store(xs[0], ws[0]);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) {
        ld.load(a, (kt + 1) * C::BK);
        ld.store(xs[(kt & 1) ^ 1], ws[(kt & 1) ^ 1]);
      }
      __syncthreads();
    }
    return;
  }

  const int wm = wave / C::WN, wn = wave % C::WN;
  // Accumulators start at the bias, as the reference's chain does.
  floatx16 acc[C::kMB][C::kNB];
#pragma unroll
  for (int nb = 0; nb < C::kNB; ++nb) {
    const int col = c0 + wn * C::kTN + nb * 32 + l32;
    const float bv = col < a.n_count ? a.bias[a.n_start + col] : 0.0f;
#pragma unroll
    for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = bv;
  }

  if constexpr (C::kProducers > 0) {
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      mfma_step<C>(xs[kt & 1], ws[kt & 1], wm, wn, g, l32, acc);
      __syncthreads();
    }
  } else if constexpr (C::kDefer) {
    TileLoader<C, kVec> ld;
    ld.init(a, tid, m0, c0);
    ld.load(a, 0);
    ld.store(xs[0], ws[0]);
    __syncthreads();
    Frags<C> last;
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      Frags<C> f0;
      read_slice<C>(xs[buf], ws[buf], 0, wm, wn, g, l32, f0);
      if (kt > 0) mfma_slice<C>(last, acc);  // the previous step's deferred slice
      if (kt + 1 < nk) ld.load(a, (kt + 1) * C::BK);
      mfma_slice<C>(f0, acc);
#pragma unroll
      for (int kk = 1; kk + 1 < C::BK / 8; ++kk) {
        Frags<C> f;
        read_slice<C>(xs[buf], ws[buf], kk, wm, wn, g, l32, f);
        mfma_slice<C>(f, acc);
      }
      read_slice<C>(xs[buf], ws[buf], C::BK / 8 - 1, wm, wn, g, l32, last);
      if (kt + 1 < nk) ld.store(xs[buf ^ 1], ws[buf ^ 1]);
      __syncthreads();
    }
    mfma_slice<C>(last, acc);
  } else {
    // Every wave stages: the next K step's codes and X are fetched into
    // registers while the MFMAs of the current step run (double-buffered
    // LDS, one barrier per step).
    TileLoader<C, kVec> ld;
    ld.init(a, tid, m0, c0);
    ld.load(a, 0);
    ld.store(xs[0], ws[0]);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      if (kt + 1 < nk) ld.load(a, (kt + 1) * C::BK);
      mfma_step<C>(xs[buf], ws[buf], wm, wn, g, l32, acc);
      if (kt + 1 < nk) ld.store(xs[buf ^ 1], ws[buf ^ 1]);
      __syncthreads();
    }
  }

  if constexpr (kEpi == kEpiQkv) {
    qkv_epilogue<C>(a, acc, m0 + wm * C::kTM, c0 + wn * C::kTN, g, l32);
    return;
  }
  store_result<C::kMB, C::kNB, kEpi>(a, acc, m0 + wm * C::kTM, c0 + wn * C::kTN, g, l32);
}

// The XCD rectangles (xcd_grid) that minimise the bytes of x rows and
// codes each XCD's L2 must fetch for its tiles, or pm = pn = 0 when the grid
// does not divide into 8 equal rectangles or the contiguous runs of
// xcd_tile_index fetch as little.
inline bool g_xcd_blocking = true;
void xcd_blocking(int tiles_m, int tiles_n, int bm, int bn, int K, int& pm, int& pn) {
  pm = pn = 0;
  if (!g_xcd_blocking || (tiles_m * tiles_n) % 8 != 0) return;
  auto bytes = [&](double rows, double cols) { return rows * bm * K * 4.0 + cols * bn * K * 3.0; };
  // contiguous runs: tiles/8 consecutive tiles, row-major
  const int run = tiles_m * tiles_n / 8;
  const int run_rows = (run + tiles_n - 1) / tiles_n + (run % tiles_n != 0 ? 1 : 0);
  const int run_cols = run >= tiles_n ? tiles_n : run;
  double best = bytes(run_rows, run_cols);
  for (int m = 1; m <= 8; m *= 2) {
    const int n = 8 / m;
    if (tiles_m % m != 0 || tiles_n % n != 0) continue;
    const double b = bytes((double)tiles_m / m, (double)tiles_n / n);
    if (b < best) {
      best = b;
      pm = m;
      pn = n;
    }
  }
}

// Tile configuration of the scalar-load path for configuration C (C itself
// unless specialised below).
template <class C>
struct ScalarPathCfg {
  using type = C;
};

template <class C, int kEpi = kEpiStore>
int launch_cfg(const GemmParams& p, hipStream_t stream, const QkvArgs& e = QkvArgs{},
               const GemmEpilogueParams& ep = GemmEpilogueParams{kEpilogueStore, nullptr, 0, 1},
               int row0 = 0) {
  GemmArgs a{p.x, p.code01, p.q2, p.scale, p.bias, p.out,
             p.M, p.K, p.N, p.n_start, p.n_count, p.stride_x, p.stride_out, e,
             ep.gate, ep.gate_stride, ep.rows_per_batch, row0, 0, 0};
  const int tiles_m = (p.M + C::BM - 1) / C::BM, tiles_n = (p.n_count + C::BN - 1) / C::BN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  if (tiles <= 0 || tiles > 0x7fffffff) return kErrDims;
  xcd_blocking(tiles_m, tiles_n, C::BM, C::BN, p.K, a.xcd_pm, a.xcd_pn);
  const bool vec = (reinterpret_cast<uintptr_t>(p.x) % 16 == 0) && (p.stride_x % 4 == 0) &&
                   (p.K % 4 == 0) && (p.N % 2 == 0) && (p.n_start % 2 == 0) &&
                   (p.n_count % 2 == 0) && (reinterpret_cast<uintptr_t>(p.code01) % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(p.q2) % 2 == 0) &&
                   vec_buffers_fit(p, C::BM, C::BK);
  // The scalar path's configuration covers the same tiles, possibly with
  // another K step or wave layout (and so another workgroup size).
  using S = typename ScalarPathCfg<C>::type;
  static_assert(S::BM == C::BM && S::BN == C::BN, "the scalar path must cover the same tiles");
  dim3 grid((unsigned)tiles);
  if (vec)
    hipLaunchKernelGGL((nf24_gemm_kernel<C, true, kEpi>), grid, dim3(C::kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((nf24_gemm_kernel<S, false, kEpi>), grid, dim3(S::kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Epilogue of the row-tail rows (M <= kTailRows, see tail_rows): `raw`
// holds bias + x W of those rows ([M, n_count], from the few-row kernels);
// each wave loads a 32 x 64 block of it into the MFMA accumulator layout and
// runs the same epilogue code as the tile kernels (one head per wave for
// the QKV epilogue), so the tail rows get the same elementwise arithmetic.
template <class C, int kEpi>
__global__ __launch_bounds__(64) void tail_epilogue_kernel(GemmArgs a, const float* raw) {
  static_assert(C::kMB == 1 && C::kNB == 2, "one 32 x 64 block per wave");
  const int lane = threadIdx.x;
  const int g = lane >> 5, l32 = lane & 31;
  const int colw = blockIdx.x * 64;
  floatx16 acc[1][2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int col = colw + nb * 32 + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 8 * (r / 4) + 4 * g + (r % 4);
      acc[0][nb][r] = (row < a.M && col < a.n_count) ? raw[(int64_t)row * a.n_count + col] : 0.0f;
    }
  }
  if constexpr (kEpi == kEpiQkv)
    qkv_epilogue<C>(a, acc, 0, colw, g, l32);
  else
    store_result<1, 2, kEpi>(a, acc, 0, colw, g, l32);
}

// Packed k/v tokens L..Lpad-1 of every (b, h, dim) row are zero.
constexpr int kTailThreads = 256;
__global__ __launch_bounds__(kTailThreads) void packed_tail_zero_kernel(float* pk, float* pv,
                                                                        int64_t rows, int L,
                                                                        int Lpad) {
  const int tail = Lpad - L;
  const int64_t i = (int64_t)blockIdx.x * kTailThreads + threadIdx.x;
  if (i >= rows * tail) return;
  const int64_t off = (i / tail) * Lpad + L + i % tail;
  pk[off] = 0.0f;
  pv[off] = 0.0f;
}

// Tile configurations and the rates they sustain on MI355X when the grid is
// many rounds deep (fp32 TFLOP/s, measured over M = 16384..32768 shapes; the
// order of the rates is what the choices rest on: where 256 x 256 and
// 256 x 192 both fill whole rounds, 256 x 256 is 2-3 % faster, e.g.
// 16384 x 1024 x 3072 754 against 775 us).
// The launcher picks the one with the smallest modelled time: full rounds of
// CUs * wgs_per_cu tiles cost wgs_per_cu * BM * BN / rate each; a partial
// last round costs ceil(rest / CUs) tiles' worth, 25 % more when a 4-wave
// workgroup then runs alone on its CU (one wave per SIMD hides less latency).
// Against measurement (M = 2048..32768, N = 1024..4096) the model picks the
// fastest configuration or one within 3 % of it.  The 256 x 128 rate (119)
// is fitted to its one-round calls against 128 x 128 (M = 2048..8192), the
// 128 x 64 rate (100) to M = 512..8192 at N = 1024..4096.
// 16 waves, 1 workgroup / CU, K steps of 32 with the deferred last slice
// (since the buffer-resource loads left room: 16384 x 4096 x 1024 1033 ->
// 990 us against K steps of 16; two live-range values spill once per
// workgroup, outside the K loop)
using CfgLarge = GemmCfg<256, 256, 32, 4, 4, 1, 0, true>;
// 12 waves, 1 workgroup / CU, K steps of 32, the last k-slice of each step
// multiplied after its barrier (measured at configs[0]: BK 16 -> 32 -5 %,
// deferral a further -3 %; with deferral the 256 x 256 tile is 4 % slower)
using CfgWide = GemmCfg<256, 192, 32, 4, 3, 1, 0, true>;
// 12 waves, 1 workgroup / CU, the 256 x 192 tile's loop transposed: for
// row counts whose 256-row bands leave CUs idle but 192-row bands fill whole
// rounds (the reference's L = 12294 at N = 1024: 196 tiles of 256 x 256 on
// 256 CUs, against 256 tiles of 192 x 256 plus the 6-row tail launch)
using CfgTall = GemmCfg<192, 256, 32, 3, 4, 1, 0, true>;
using CfgSmall = GemmCfg<128, 128, 16, 2, 2, 3>; // 4 waves, 3 workgroups / CU
// 8 waves (two per SIMD), 1 workgroup / CU: for calls whose 256 x 256 /
// 256 x 192 tiles leave CUs idle and whose 128 x 128 tiles would share CUs
// two or three to one (the compressed negative branch's 8192 x 1024 GEMMs:
// 256 tiles, one per CU; 152 -> 141 us at K = 1024, 568 -> 533 us at
// K = 4096 against 512 tiles of 128 x 128)
using CfgHalf = GemmCfg<256, 128, 32, 4, 2, 1, 0, true>;
// 4 waves of 32 x 64, 2 workgroups / CU: for calls too small to fill the
// chip with the larger tiles (the 2048-row remainder of the single-stream
// graph's 18432 rows: 2048 x 1024 x 1024 90 -> 51 us, 2048 x 4096 x 1024
// 344 -> 188 us, 4096 x 1024 x 1024 91 -> 81 us, 3000 x 1024 x 1024 93 ->
// 81 us, against 128 x 128 tiles that left half the CUs idle)
using CfgNarrow = GemmCfg<128, 64, 32, 4, 1, 2, 0, true>;
// The scalar-load path (unaligned or odd operands) runs the 256 x 256 tile at
// K steps of 16: the guarded per-element loads need the registers that the
// 32-deep step and its deferred slice take, and spill inside the K loop.
// Same tile, same per-output order: the same results.
template <>
struct ScalarPathCfg<CfgLarge> {
  using type = GemmCfg<256, 256, 16, 4, 4>;
};
using CfgSkinny = GemmCfg<32, 128, 32, 1, 4>;
// Accumulator layout of tail_epilogue_kernel: one 32 x 64 block per wave
// (64 columns: a head, for the QKV epilogue).
using CfgTail = GemmCfg<32, 128, 32, 1, 2>;

struct Choice {
  int bm, bn, wgs_per_cu, waves;
  double rate;
};
constexpr Choice kChoices[] = {
    {256, 256, 1, 16, 126.0}, {256, 192, 1, 12, 125.0}, {128, 128, 3, 4, 111.0}, {192, 256, 1, 12, 125.0},
    {256, 128, 1, 8, 119.0},  {128, 64, 2, 4, 100.0}};
constexpr int kNumChoices = sizeof(kChoices) / sizeof(kChoices[0]);

// Modelled time of configuration i (kChoices) over M x n_count outputs.
double model_time(int i, int M, int n_count) {
  const int cus = compute_units();
  const Choice& c = kChoices[i];
  const int64_t tiles = (int64_t)((M + c.bm - 1) / c.bm) * ((n_count + c.bn - 1) / c.bn);
  const int64_t slots = (int64_t)cus * c.wgs_per_cu;
  const int64_t full = tiles / slots;
  const int64_t rest = tiles - full * slots;
  const double tile_t = (double)c.bm * c.bn / c.rate;
  double t = (double)full * c.wgs_per_cu * tile_t;
  if (rest > 0) {
    const int64_t k = (rest + cus - 1) / cus;
    t += (double)k * tile_t * ((k == 1 && c.waves == 4) ? 1.25 : 1.0);
  }
  return t;
}

// Index into kChoices of the configuration with the smallest modelled time.
int pick_config(int M, int n_count) {
  int best = 0;
  for (int i = 1; i < kNumChoices; ++i)
    if (model_time(i, M, n_count) < model_time(best, M, n_count)) best = i;
  return best;
}

// Rows to run as a first launch of 256 x 256 tiles that fill whole rounds
// of CUs, the rest going to a second launch with its own best shape -- or 0
// when one launch is modelled as fast (within 3 %).  E.g. the single-stream
// graph's M = 18432 rows: 16384 rows of 256 x 256 tiles plus 2048 rows of
// 128 x 128 tiles model 8-9 % faster at N = 3072 / 4096 than any one shape,
// whose last round would be mostly idle.  Every tile shape sums each output
// in the same order, so the split changes no result bit.
int round_split_rows(int M, int n_count) {
  const int cus = compute_units();
  const int bands = (n_count + 255) / 256;  // 256 x 256 tiles per 256 rows
  int g = cus, r = bands;                   // rows of whole rounds: multiples of
  while (r != 0) {                          // 256 * cus / gcd(cus, bands)
    const int t = g % r;
    g = r;
    r = t;
  }
  const int64_t unit = 256LL * (cus / g);
  const int64_t m1 = (int64_t)M / unit * unit;
  if (m1 == 0 || m1 == M) return 0;
  const double one = model_time(pick_config(M, n_count), M, n_count);
  const int rest = M - (int)m1;
  const double two = model_time(0, (int)m1, n_count) + model_time(pick_config(rest, n_count), rest, n_count);
  return two < 0.97 * one ? (int)m1 : 0;
}

// Rows past the last multiple of 256 that number at most kTailRows, when
// they would occupy a whole extra round of 256-row tiles (e.g. M = 16385:
// 1040 tiles = 4 rounds + 16 one-row tiles, ~270 us at K = 1024), run on the
// few-row kernels instead (launch_tail_rows: the K range split over the
// whole chip, partial sums merged in a fixed order).  When they fit in the
// last round the main launch already has (e.g. M = 2818, N = 3072: 12 bands
// of 256 x 192 tiles, one round either way), they stay in it: the partial
// tile costs nothing there, while a second launch would add its own time.
// The tile shapes all sum each output in one order; the few-row kernels sum
// in another (deterministic) one, so a tail row equals the same row of a
// call over exactly the tail rows, bit for bit, and a row inside a tile to
// within the fp32 summation-order bound.
constexpr int kTailRows = 32;

GemmParams rows_slice(const GemmParams& p, int first, int count) {
  GemmParams q = p;
  q.x = p.x + (int64_t)first * p.stride_x;
  if (q.out != nullptr) q.out = p.out + (int64_t)first * p.stride_out;
  q.M = count;
  return q;
}

int tail_rows(int M, int n_count) {
  const int rem = M % 256;
  if (M <= 256 || rem == 0 || rem > kTailRows) return 0;
  const double with_tail = model_time(pick_config(M, n_count), M, n_count);
  const double without = model_time(pick_config(M - rem, n_count), M - rem, n_count);
  return with_tail > without ? rem : 0;
}

}  // namespace

int compute_units() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  // A failed query falls back to MI355X's 256 CUs (the count only shapes the
  // launch plan) and leaves no error behind for the caller's next check.
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = 256;
    }
    if (n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int launch_nf24_gemm(const GemmParams& p, hipStream_t stream) {
  if (p.precision != kPrecisionFp32 && p.M > 32)
    return launch_gemm_bf16(p, kEpiStore, QkvArgs{},
                            GemmEpilogueParams{kEpilogueStore, nullptr, 0, 1}, 0, stream);
  // Few rows: the weight stream is the cost; the MFMA skinny tile only wins
  // for 9..32 rows over a short K (measured at K = 256).
  if (p.M <= 32) {
    if (p.M > 8 && p.K <= 256) return launch_cfg<CfgSkinny>(p, stream);
    return launch_nf24_gemv(p, stream);
  }
  // The row tail goes first: its workspace is the only thing that can fail
  // (e.g. under graph capture), and then nothing has been enqueued.
  if (const int rem = tail_rows(p.M, p.n_count)) {
    // the tail rows take the path of a call over exactly those rows
    const int st = launch_nf24_gemm(rows_slice(p, p.M - rem, rem), stream);
    return st != kOk ? st : launch_nf24_gemm(rows_slice(p, 0, p.M - rem), stream);
  }
  if (const int m1 = round_split_rows(p.M, p.n_count)) {
    const int st = launch_nf24_gemm(rows_slice(p, 0, m1), stream);
    return st != kOk ? st : launch_nf24_gemm(rows_slice(p, m1, p.M - m1), stream);
  }
  const int best = pick_config(p.M, p.n_count);
  if (best == 0) return launch_cfg<CfgLarge>(p, stream);
  if (best == 1) return launch_cfg<CfgWide>(p, stream);
  if (best == 3) return launch_cfg<CfgTall>(p, stream);
  if (best == 4) return launch_cfg<CfgHalf>(p, stream);
  if (best == 5) return launch_cfg<CfgNarrow>(p, stream);
  return launch_cfg<CfgSmall>(p, stream);
}

namespace {
// At most kTailRows rows t (token index of its row 0 row0) of an epilogue
// GEMM -- a whole call of that size or the row tail of a larger one: bias +
// x W of its rows as a plain call over exactly them computes it (the
// few-row kernels, or the 32-row tile for 9-32 rows over K <= 256) into the
// per-stream workspace, then tail_epilogue_kernel.  So few rows with an
// epilogue equal the plain GEMM of those rows followed by the elementwise
// step, bit for bit, wherever they sit.
template <int kEpi>
int launch_tail_rows(const GemmParams& t, const GemmEpilogueParams& e, const QkvArgs& q, int row0,
                     hipStream_t stream) {
  float* raw = static_cast<float*>(
      stream_workspace(stream, (size_t)t.M * t.n_count * sizeof(float), kSlotGemmTail));
  if (raw == nullptr) return kErrWorkspace;
  GemmParams r = t;
  r.out = raw;
  r.stride_out = t.n_count;
  r.precision = kPrecisionFp32;
  const int st = launch_nf24_gemm(r, stream);
  if (st != kOk) return st;
  GemmArgs a{t.x, t.code01, t.q2, t.scale, t.bias, t.out,
             t.M, t.K, t.N, t.n_start, t.n_count, t.stride_x, t.stride_out, q,
             e.gate, e.gate_stride, e.rows_per_batch, row0, 0, 0};
  hipLaunchKernelGGL((tail_epilogue_kernel<CfgTail, kEpi>), dim3((unsigned)((t.n_count + 63) / 64)),
                     dim3(64), 0, stream, a, raw);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <int kEpi>
int launch_epi_kind(const GemmParams& p, const GemmEpilogueParams& e, hipStream_t stream,
                    const QkvArgs& q = QkvArgs{}, int row0 = 0) {
  if (p.precision != kPrecisionFp32 && p.M > 32) return launch_gemm_bf16(p, kEpi, q, e, row0, stream);
  // The row tail first (as in launch_nf24_gemm: only its workspace can fail).
  if (const int rem = tail_rows(p.M, p.n_count)) {
    const int st = launch_tail_rows<kEpi>(rows_slice(p, p.M - rem, rem), e, q, row0 + p.M - rem, stream);
    return st != kOk ? st : launch_epi_kind<kEpi>(rows_slice(p, 0, p.M - rem), e, stream, q, row0);
  }
  // Few rows: the plain few-row path, then the epilogue (a single 32-row
  // tile would run one chain of K/2 MFMAs per wave: 39-41 us at K = 1024).
  if (p.M <= 32) return launch_tail_rows<kEpi>(p, e, q, row0, stream);
  if (const int m1 = round_split_rows(p.M, p.n_count)) {
    const int st = launch_epi_kind<kEpi>(rows_slice(p, 0, m1), e, stream, q, row0);
    return st != kOk ? st : launch_epi_kind<kEpi>(rows_slice(p, m1, p.M - m1), e, stream, q, row0 + m1);
  }
  const int best = pick_config(p.M, p.n_count);
  if (best == 0) return launch_cfg<CfgLarge, kEpi>(p, stream, q, e, row0);
  if (best == 1) return launch_cfg<CfgWide, kEpi>(p, stream, q, e, row0);
  if (best == 3) return launch_cfg<CfgTall, kEpi>(p, stream, q, e, row0);
  if (best == 4) return launch_cfg<CfgHalf, kEpi>(p, stream, q, e, row0);
  if (best == 5) return launch_cfg<CfgNarrow, kEpi>(p, stream, q, e, row0);
  return launch_cfg<CfgSmall, kEpi>(p, stream, q, e, row0);
}
}  // namespace

int nf24::launch_strict_tail(const GemmParams& p, int epi, const QkvArgs& e,
                             const GemmEpilogueParams& ep, int row0, hipStream_t stream) {
  GemmParams s = p;
  s.precision = kPrecisionFp32;
  if (s.M < 1 || s.M > kTailRows) return kErrDims;
  switch (epi) {
    case kEpiStore: return launch_nf24_gemm(s, stream);
    case kEpiQkv: return launch_tail_rows<kEpiQkv>(s, ep, e, row0, stream);
    case kEpilogueGelu: return launch_tail_rows<kEpilogueGelu>(s, ep, e, row0, stream);
    case kEpilogueGated: return launch_tail_rows<kEpilogueGated>(s, ep, e, row0, stream);
    case kEpilogueAdd: return launch_tail_rows<kEpilogueAdd>(s, ep, e, row0, stream);
    default: return kErrDims;
  }
}

int launch_nf24_gemm_epilogue(const GemmParams& p, const GemmEpilogueParams& e,
                              hipStream_t stream) {
  switch (e.kind) {
    case kEpilogueStore: return launch_nf24_gemm(p, stream);
    case kEpilogueGelu: return launch_epi_kind<kEpilogueGelu>(p, e, stream);
    case kEpilogueGated:
      if (e.gate == nullptr || e.rows_per_batch <= 0) return kErrDims;
      return launch_epi_kind<kEpilogueGated>(p, e, stream);
    case kEpilogueAdd: return launch_epi_kind<kEpilogueAdd>(p, e, stream);
    default: return kErrDims;
  }
}

int launch_nf24_gemm_qkv(const QkvFusedParams& p, hipStream_t stream) {
  const GemmParams& gp = p.gemm;
  if (gp.n_start != 0 || gp.n_count != gp.N || gp.N != 3 * p.H * 64 ||
      (int64_t)p.B * p.L != gp.M || p.L_padded < p.L)
    return kErrDims;
  const QkvArgs e{p.freqs, p.q_gamma, p.k_gamma, p.q, p.packed_k, p.packed_v,
                  p.L, p.H, p.L_padded, p.freq_batches, p.kv_bhld, p.kv_round};
  const GemmEpilogueParams none{kEpilogueStore, nullptr, 0, 1};
  const int st = launch_epi_kind<kEpiQkv>(gp, none, stream, e);
  if (st != kOk) return st;
  // tokens L .. Lpad - 1 of the packed k / v (disjoint from what the GEMM writes)
  if (!p.kv_bhld && p.L_padded > p.L) {
    const int64_t rows = (int64_t)p.B * p.H * 64;
    const int64_t n = rows * (p.L_padded - p.L);
    hipLaunchKernelGGL(packed_tail_zero_kernel,
                       dim3((unsigned)((n + kTailThreads - 1) / kTailThreads)), dim3(kTailThreads),
                       0, stream, p.packed_k, p.packed_v, rows, p.L, p.L_padded);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  return kOk;
}

}  // namespace tsplat
