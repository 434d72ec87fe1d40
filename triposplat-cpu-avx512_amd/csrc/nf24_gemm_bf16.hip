// NF24 packed-weight GEMM on the bf16 matrix cores: the opt-in precision
// modes kPrecisionBf16 and kPrecisionBf16x3 of tsplat_launch.h.
//
// Same operation as nf24_gemm.hip -- out = bias + X * decode(W), each weight
// decoded as the reference does (scripts/gemm_nf24_i16_avx512.c:26-33:
// fp32((int32)q01 * 256 + q2) * scale[n]) in registers, no weight copy in
// HBM -- but the products run on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation:
//   kPrecisionBf16:   bf16(x) * bf16(w)
//   kPrecisionBf16x3: xh*wh + xh*wl + xl*wh with xh = bf16(x), xl = bf16(x - xh),
//                     wh = bf16(w), wl = bf16(fma(p, s, -wh))
// where bf16() rounds the fp32 value to nearest even (v_cvt_pk_bf16_f32,
// the rounding torch's float32 -> bfloat16 conversion uses), w = fp32(p * s)
// is the decoded weight of payload p = q01 * 256 + q2 and scale s, and the
// FMA takes the exact product minus wh, rounded once.  x - xh is exact in
// fp32, so xh + xl holds 16 significant bits of x (wh + wl likewise of
// p * s); the dropped xl*wl term and the rounding of xl leave a product
// error near 2^-16 relative, against 2^-8 for bf16 alone.  Products of two bf16 values are
// exact in fp32, so the only other difference from a float64 sum of the same
// terms is the fp32 accumulation order.
//
// Tiling: BM x BN workgroup tile, WM x WN waves, a wave owns MB x NB blocks
// of 32x32 (the accumulator layout of the fp32 kernel, so the epilogues of
// nf24_gemm_common.h serve both).  K advances 32 per step, two MFMA k-slices
// of 16.  x (converted on the way in) and the decoded W are staged in LDS as
// bf16, k-contiguous: a row of the tile is 64 bytes, four 16-byte chunks of
// 8 k, their order within the row swizzled.  Lane l of an MFMA reads row
// l%32, chunk 2s + l/32 of slice s, the same k assignment for A and B.
// gfx950 serves a 128-bit LDS read in four 16-lane groups (one half-wave,
// the 4-lane quads whose index -- lane bits 2..4 -- has one parity: lanes
// 0-3, 12-15, 20-23, 24-27 form the first) over 64 banks of 4 bytes, and an
// LDS write in a fixed ~8 cycles per 64-bit store unless one bank takes more
// than ~8 of its 128 dwords.  Three terms (kSwz): chunk c of row r sits at
// position c ^ ((r >> 2) & 3) -- the quads of a read group differ in
// (r >> 2) & 3, so its 16 rows fill the 16 bank slots once -- and W tile
// column r is kept in LDS row w_row(r), so that the 64 columns of one
// staging store reach 16 bank slots instead of 4 (6x fewer bank-conflict
// cycles, 2-3 % faster).  One term keeps position c ^ (((r >> 1) ^ (r >> 3))
// & 3) and unpermuted rows: the same change there needs registers the
// two-stage fetch has not got (it spills and runs 6-9 % slower).  LDS is
// double-buffered with one barrier per step; codes and x are fetched into
// registers two steps ahead (bf16) or one step ahead (bf16x3, whose extra
// fragments leave no registers for a second set).

#include "nf24_gemm_common.h"

#include <type_traits>

namespace tsplat {
namespace nf24 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

template <int BM_, int BN_, int WM_, int WN_, int WK_ = 4>
struct Bf16Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int WK = WK_;  // k rows of a W staging unit
  static constexpr int BK = 32;
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int kTM = BM / WM, kTN = BN / WN;
  static constexpr int kMB = kTM / 32, kNB = kTN / 32;
  // x: float4 units (row, 4 k); W: units of 4 columns x WK k.  A last
  // iteration that not every thread has covers whole waves (the threads
  // past the units skip it).
  static_assert(WK == 2 || WK == 4, "W units are 2 or 4 k rows deep");
  static constexpr int kXUnits = BM * BK / 4, kWUnits = (BN / 4) * (BK / WK);
  static constexpr int kXIter = (kXUnits + kThreads - 1) / kThreads;
  static constexpr int kWIter = (kWUnits + kThreads - 1) / kThreads;
  static_assert(kXUnits % 64 == 0 && kWUnits % 64 == 0, "a partial iteration must cover whole waves");
  static_assert(kTM % 32 == 0 && kTN % 32 == 0, "wave tile must be 32-aligned");
  // unit j of this thread exists (uniform over a wave)
  __device__ static constexpr bool x_unit(int tid, int j) {
    return kXUnits % kThreads == 0 || j + 1 < kXIter || tid + j * kThreads < kXUnits;
  }
  __device__ static constexpr bool w_unit(int tid, int j) {
    return kWUnits % kThreads == 0 || j + 1 < kWIter || tid + j * kThreads < kWUnits;
  }
};

using Bf16Large = Bf16Cfg<256, 256, 2, 4>;  // 8 waves, 128 x 64 per wave
// 12 waves, 64 x 64 per wave; 2-deep W units give every thread one, so the
// decode is spread over all twelve waves (4-deep units would leave it to six,
// two on each of two SIMDs and one on each of the others)
using Bf16Wide = Bf16Cfg<256, 192, 4, 3, 2>;
using Bf16Small = Bf16Cfg<128, 128, 2, 2>;  // 4 waves, 64 x 64 per wave
// Where the larger tiles leave CUs idle (measured, bf16x3 / bf16, gated
// epilogue): 12 waves of 64 x 64 over 192 rows -- the reference's 12288
// rows at N = 1024, 256 tiles: 114 -> 92 / 77 -> 64 us; 256 x 128 (as 8
// waves of 64 x 64) -- 8192 x 1024: 79 -> 69 / 56 -> 52 us; 4 waves of
// 32 x 64, two workgroups per CU -- 2048 x 1024: 74 -> 38 / 52 -> 35 us.
using Bf16Tall = Bf16Cfg<192, 256, 3, 4, 2>;
using Bf16Half = Bf16Cfg<256, 128, 8, 2, 2>;
using Bf16Narrow = Bf16Cfg<128, 64, 4, 1, 2>;
// 16 waves (four per SIMD) where the accumulators allow them: the 256 x 128
// tile as 16 waves of 32 x 64 (above; against 8 of 64 x 64, gated: 8192 x
// 1024 x 1024 69 -> 63 / 57 -> 51 us, 8192 x 4096 x 1024 217 -> 202 / 149 ->
// 136 us), the 256 x 192 tile as 16 waves of 32 x 96 for every epilogue but
// QKV (a head per wave): configs[0] in the bench 78.4 -> 75.5 us bf16x3,
// 48.0 -> 47.6 us bf16.  The kernel is VALU-bound; the fourth wave of a
// SIMD overlaps more of the decode with the MFMAs.  (192 x 256 as 16 waves
// of 96 x 32, time -3.5 % at K = 1024 and +0.6 % at 4096: not kept; 256 x
// 256: 64 accumulators per wave at 16 waves spill.)  Bit-identical: one
// order per output.
using Bf16Wide16 = Bf16Cfg<256, 192, 8, 2, 2>;

// bf16 element offset of (row r, chunk c) in a 32-k tile row.
template <bool kSwz>
__device__ __forceinline__ int chunk_offset(int r, int c) {
  if constexpr (kSwz) return r * 32 + ((c ^ ((r >> 2) & 3)) << 3);
  return r * 32 + ((c ^ (((r >> 1) ^ (r >> 3)) & 3)) << 3);
}

// LDS row of W tile column r: the low two bits XOR bits 4 and 6 of r, so the
// 64 columns 4l + e of one staging store (l = lane) land on 16 bank slots; a
// 4-row quad stays a quad, which keeps the fragment reads conflict-free, and
// w_row(r + 32) = w_row(r) + 32 for the 32-column blocks of a wave.
template <bool kSwz>
__device__ __forceinline__ int w_row(int r) {
  if constexpr (kSwz) return r ^ (((r >> 4) & 1) | ((r >> 5) & 2));
  return r;
}

template <bool kSwz>
__device__ __forceinline__ bf16x8 lds_frag(const __bf16* base, int r, int c) {
  return *reinterpret_cast<const bf16x8*>(base + chunk_offset<kSwz>(r, c));
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef unsigned uintx2 __attribute__((ext_vector_type(2)));
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));

// hi = bf16(v); lo = bf16(v - hi) (only with three terms).  Pairs go
// through one v_cvt_pk_bf16_f32 each; the hi values come back to fp32 by a
// shift / mask of the packed pair.
template <int kTerms>
__device__ __forceinline__ void split4(const floatx4& v, bf16x4& hi, bf16x4& lo) {
  unsigned h[2], l[2] = {0, 0};
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float a = v[2 * p], b = v[2 * p + 1];
    h[p] = __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{a, b}, bf16x2));
    if constexpr (kTerms == 3) {
      const float ha = __uint_as_float(h[p] << 16), hb = __uint_as_float(h[p] & 0xffff0000u);
      l[p] = __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{a - ha, b - hb}, bf16x2));
    }
  }
  hi = __builtin_bit_cast(bf16x4, uintx2{h[0], h[1]});
  if constexpr (kTerms == 3) lo = __builtin_bit_cast(bf16x4, uintx2{l[0], l[1]});
}

// Integer payload (int32)q01 * 256 + q2 of column e of a staged unit row, as
// fp32 (exact: its magnitude is below 2^24), codes packed as loaded (two
// int16 codes per word, four int8 codes per word).
__device__ __forceinline__ float w_payload(const uint32_t (&c)[2], uint32_t q, int e) {
  const int32_t code = (int32_t)(int16_t)(c[e >> 1] >> (16 * (e & 1)));
  const int32_t q2 = (int32_t)(int8_t)(q >> (8 * e));
  return (float)(code * 256 + q2);
}

// WK weights w = fp32(p * s) of one column -- the reference's decode
// (scripts/gemm_nf24_i16_avx512.c:26-33) -- split into bf16 pairs: hi =
// bf16(w), and with three terms lo = bf16 of fma(p, s, -hi), the exact
// p * s minus hi rounded once to fp32.  Spelled out so that the result does
// not depend on whether the compiler contracts w - hi with the product
// that made w.
template <int kTerms, int WK>
__device__ __forceinline__ void split_w(const float (&p)[WK], float s, unsigned (&h)[WK / 2],
                                        unsigned (&l)[WK / 2]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int q = 0; q < WK / 2; ++q) {
    const float w0 = p[2 * q] * s, w1 = p[2 * q + 1] * s;
    h[q] = __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{w0, w1}, bf16x2));
    if constexpr (kTerms == 3) {
      const float h0 = __uint_as_float(h[q] << 16), h1 = __uint_as_float(h[q] & 0xffff0000u);
      l[q] = __builtin_bit_cast(unsigned, __builtin_convertvector(
                                              floatx2{__builtin_fmaf(p[2 * q], s, -h0),
                                                      __builtin_fmaf(p[2 * q + 1], s, -h1)},
                                              bf16x2));
    }
  }
}

// WK / 2 bf16 pairs stored at dst (8- or 4-byte aligned).
template <int NW>
__device__ __forceinline__ void store_pairs(__bf16* dst, const unsigned (&w)[NW]) {
  if constexpr (NW == 2) *reinterpret_cast<uintx2*>(dst) = uintx2{w[0], w[1]};
  else *reinterpret_cast<unsigned*>(dst) = w[0];
}

__device__ __forceinline__ floatx16 mfma_bf16(const bf16x8& a, const bf16x8& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// kVec: x rows 16-byte aligned with K % 4 == 0; N, n_start, n_count
// multiples of 4 with code01 8-byte and q2 4-byte aligned (four columns of
// one k row per 64-bit / 32-bit load).
// kPl: W from the bf16 planes a.w_hi / a.w_lo (kVec only) instead of the
// codes.  The planes are k-blocked, [ceil(K / 32), N, 32]: the 32 k of a
// step of one column are 64 contiguous bytes and the columns of a step
// follow each other, so the units -- (tile column, 8-k chunk), four lanes
// per column -- make one 16-byte load and one 16-byte LDS store per plane,
// and a wave reads 1 KB in one run; no decode and no split in the K loop.
// The planes hold the values the decode path computes, stored where it
// stores them, so both paths give the same result bit for bit.
template <class C, int kTerms, bool kVec, int kEpi, bool kPl>
__global__ __launch_bounds__(C::kThreads) void nf24_gemm_bf16_kernel(GemmArgs a) {
  static_assert(!kPl || kVec, "the planes path loads through buffer resources");
  constexpr int kPlanes = kTerms == 3 ? 2 : 1;
  constexpr bool kSwz = kTerms == 3;
  __shared__ __attribute__((aligned(16))) __bf16 xs[2][kPlanes][C::BM * C::BK];
  __shared__ __attribute__((aligned(16))) __bf16 ws[2][kPlanes][C::BN * C::BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int g = lane >> 5;
  const int l32 = lane & 31;

  const int tiles_n = (a.n_count + C::BN - 1) / C::BN;
  const int tile = xcd_tile_index(blockIdx.x, gridDim.x);
  const int m0 = (tile / tiles_n) * C::BM;
  const int c0 = (tile % tiles_n) * C::BN;

  // W units of this thread: columns w_col .. w_col+3 of the tile, k rows
  // w_k .. w_k+WK-1 of each step; the columns and their scales are fixed.
  int w_col[C::kWIter], w_k[C::kWIter];
  float w_sc[C::kWIter][4];
  bool w_ok[C::kWIter][4];
#pragma unroll
  for (int j = 0; j < (kPl ? 0 : C::kWIter); ++j) {
    const int u = tid + j * C::kThreads;
    w_col[j] = 4 * (u % (C::BN / 4));
    w_k[j] = C::WK * (u / (C::BN / 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int lc = c0 + w_col[j] + e;
      w_ok[j][e] = C::w_unit(tid, j) && lc < a.n_count;
      w_sc[j][e] = w_ok[j][e] ? a.scale[a.n_start + lc] : 0.0f;
    }
  }

  // kStages register sets: the codes and x of step k arrive in set
  // k % kStages while the kStages steps before it run.  Two stages for one
  // term; three terms have no registers for a second set.
  constexpr int kStages = kTerms == 3 ? 1 : 2;
  floatx4 xr[kStages][C::kXIter];
  uint32_t cr[kStages][C::kWIter][C::WK][2];  // k row i: int16 codes of columns 0,1 | 2,3
  uint32_t qr[kStages][C::kWIter][C::WK];     // k row i: int8 codes of columns 0..3

  // kPl: this thread's plane units j (tile column p_col, chunk p_ch) and the
  // byte offset of the unit at k0 = 0, or kBufOob past n_count.
  static_assert(C::BK == 32, "the planes are blocked by 32 k");
  constexpr int kPUnits = C::BN * (C::BK / 8);
  constexpr int kPIter = (kPUnits + C::kThreads - 1) / C::kThreads;
  static_assert(kPUnits % 64 == 0, "a partial iteration must cover whole waves");
  auto p_unit = [&](int j) {
    return kPUnits % C::kThreads == 0 || j + 1 < kPIter || tid + j * C::kThreads < kPUnits;
  };
  int p_col[kPIter], p_ch[kPIter];
  uint32_t p_off[kPIter];
  uintx4 phr[kStages][kPIter], plr[kStages][kPIter];
  __amdgpu_buffer_rsrc_t rph, rpl;
  if constexpr (kPl) {
    const int64_t bytes = (int64_t)((a.K + 31) / 32) * a.N * 64;
    rph = buffer_rsrc(a.w_hi, bytes);
    if constexpr (kTerms == 3) rpl = buffer_rsrc(a.w_lo, bytes);
#pragma unroll
    for (int j = 0; j < kPIter; ++j) {
      const int u = tid + j * C::kThreads;
      p_col[j] = u / (C::BK / 8);
      p_ch[j] = u % (C::BK / 8);
      const int lc = c0 + p_col[j];
      p_off[j] = (p_unit(j) && lc < a.n_count) ? (uint32_t)(((a.n_start + lc) * 32 + 8 * p_ch[j]) * 2)
                                                 : kBufOob;
    }
  }

  // kVec: buffer-resource loads from per-thread byte offsets, as in the
  // strict kernel's TileLoader -- rows past M and columns past n_count carry
  // kBufOob, code rows past K lie past the end of the planes.
  __amdgpu_buffer_rsrc_t rx, rc, rq;
  uint32_t x_off[C::kXIter], c_off[C::kWIter], q_off[C::kWIter];
  if constexpr (kVec) {
    const int rows = min(C::BM, a.M - m0);
    rx = buffer_rsrc(a.x + (int64_t)m0 * a.stride_x, ((int64_t)(rows - 1) * a.stride_x + a.K) * 4);
    if constexpr (!kPl) {
      rc = buffer_rsrc(a.code01, (int64_t)a.K * a.N * 2);
      rq = buffer_rsrc(a.q2, (int64_t)a.K * a.N);
    }
#pragma unroll
    for (int j = 0; j < C::kXIter; ++j) {
      const int idx = tid + j * C::kThreads;
      const int row = idx / (C::BK / 4);
      x_off[j] = row < rows ? (uint32_t)(row * a.stride_x + 4 * (idx % (C::BK / 4))) * 4u : kBufOob;
    }
#pragma unroll
    for (int j = 0; j < (kPl ? 0 : C::kWIter); ++j) {
      // all four columns are valid with the first: n_start and n_count are multiples of 4
      const uint32_t e = (uint32_t)(w_k[j] * a.N + a.n_start + c0 + w_col[j]);
      c_off[j] = w_ok[j][0] ? 2u * e : kBufOob;
      q_off[j] = w_ok[j][0] ? e : kBufOob;
    }
  }

  auto load_tile = [&](auto set_c, int k0) {
    constexpr int S = decltype(set_c)::value;
    if constexpr (kVec) {
#pragma unroll
      for (int j = 0; j < C::kXIter; ++j) {
        if (!C::x_unit(tid, j)) continue;
        // K % 4 == 0: a float4 unit lies wholly inside or past the row's K floats
        const int kc = (tid + j * C::kThreads) % (C::BK / 4);
        const uint32_t off = (k0 + 4 * kc < a.K) ? x_off[j] + 4u * (uint32_t)k0 : kBufOob;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
        xr[S][j] = floatx4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                           __uint_as_float(v[3])};
      }
      if constexpr (kPl) {
#pragma unroll
        for (int j = 0; j < kPIter; ++j) {
          if (!p_unit(j)) continue;
          // block k0 / 32 starts N * 64 bytes after the previous one; k past K
          // up to the block's end reads the planes' zero padding
          const uint32_t off = p_off[j] + 2u * (uint32_t)k0 * (uint32_t)a.N;
          phr[S][j] = __builtin_bit_cast(uintx4, __builtin_amdgcn_raw_buffer_load_b128(rph, (int)off, 0, 0));
          if constexpr (kTerms == 3)
            plr[S][j] = __builtin_bit_cast(uintx4, __builtin_amdgcn_raw_buffer_load_b128(rpl, (int)off, 0, 0));
        }
        return;
      }
#pragma unroll
      for (int j = 0; j < C::kWIter; ++j) {
        if (!C::w_unit(tid, j)) continue;
#pragma unroll
        for (int i = 0; i < C::WK; ++i) {
          const uint32_t e = (uint32_t)(k0 + i) * (uint32_t)a.N;
          const auto c = __builtin_amdgcn_raw_buffer_load_b64(rc, (int)(c_off[j] + 2u * e), 0, 0);
          cr[S][j][i][0] = c[0];
          cr[S][j][i][1] = c[1];
          qr[S][j][i] = __builtin_amdgcn_raw_buffer_load_b32(rq, (int)(q_off[j] + e), 0, 0);
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < C::kXIter; ++j) {
      if (!C::x_unit(tid, j)) continue;
      const int idx = tid + j * C::kThreads;
      const int row = idx / (C::BK / 4);
      const int gm = m0 + row;
      const int gk = k0 + 4 * (idx % (C::BK / 4));
      const float* src = a.x + (int64_t)gm * a.stride_x + gk;
      if (kVec) {
        xr[S][j] = (gm < a.M && gk < a.K) ? *reinterpret_cast<const floatx4*>(src)
                                          : floatx4{0, 0, 0, 0};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[S][j][e] = (gm < a.M && gk + e < a.K) ? src[e] : 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < C::kWIter; ++j) {
      if (!C::w_unit(tid, j)) continue;
#pragma unroll
      for (int i = 0; i < C::WK; ++i) {
        const int gk = k0 + w_k[j] + i;
        const int64_t off = (int64_t)gk * a.N + a.n_start + c0 + w_col[j];
        if (kVec) {
          const bool ok = w_ok[j][0] && gk < a.K;
          const uint2 c = ok ? *reinterpret_cast<const uint2*>(a.code01 + off) : uint2{0u, 0u};
          cr[S][j][i][0] = c.x;
          cr[S][j][i][1] = c.y;
          qr[S][j][i] = ok ? *reinterpret_cast<const uint32_t*>(a.q2 + off) : 0u;
        } else {
          uint32_t c[4], q = 0u;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool ok = w_ok[j][e] && gk < a.K;
            c[e] = ok ? (uint16_t)a.code01[off + e] : 0u;
            q |= (ok ? (uint32_t)(uint8_t)a.q2[off + e] : 0u) << (8 * e);
          }
          cr[S][j][i][0] = c[0] | (c[1] << 16);
          cr[S][j][i][1] = c[2] | (c[3] << 16);
          qr[S][j][i] = q;
        }
      }
    }
  };

  auto store_tile = [&](auto set_c, auto buf_c) {
    constexpr int S = decltype(set_c)::value;
    constexpr int buf = decltype(buf_c)::value;
#pragma unroll
    for (int j = 0; j < C::kXIter; ++j) {
      if (!C::x_unit(tid, j)) continue;
      const int idx = tid + j * C::kThreads;
      const int row = idx / (C::BK / 4);
      const int kc = idx % (C::BK / 4);  // 4-k unit: chunk kc/2, half kc%2
      bf16x4 hi, lo;
      split4<kTerms>(xr[S][j], hi, lo);
      const int off = chunk_offset<kSwz>(row, kc >> 1) + 4 * (kc & 1);
      *reinterpret_cast<bf16x4*>(&xs[buf][0][off]) = hi;
      if constexpr (kTerms == 3) *reinterpret_cast<bf16x4*>(&xs[buf][kPlanes - 1][off]) = lo;
    }
    if constexpr (kPl) {
#pragma unroll
      for (int j = 0; j < kPIter; ++j) {
        if (!p_unit(j)) continue;
        const int off = chunk_offset<kSwz>(w_row<kSwz>(p_col[j]), p_ch[j]);
        *reinterpret_cast<uintx4*>(&ws[buf][0][off]) = phr[S][j];
        if constexpr (kTerms == 3) *reinterpret_cast<uintx4*>(&ws[buf][kPlanes - 1][off]) = plr[S][j];
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < C::kWIter; ++j) {
      if (!C::w_unit(tid, j)) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pw[C::WK];
#pragma unroll
        for (int i = 0; i < C::WK; ++i) pw[i] = w_payload(cr[S][j][i], qr[S][j][i], e);
        unsigned hi[C::WK / 2], lo[C::WK / 2];
        split_w<kTerms, C::WK>(pw, w_sc[j][e], hi, lo);
        const int off = chunk_offset<kSwz>(w_row<kSwz>(w_col[j] + e), w_k[j] >> 3) + (w_k[j] & 7);
        store_pairs(&ws[buf][0][off], hi);
        if constexpr (kTerms == 3) store_pairs(&ws[buf][kPlanes - 1][off], lo);
      }
    }
  };

  // Accumulators start at the bias.
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

  const int nk = (a.K + C::BK - 1) / C::BK;
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  load_tile(Set0{}, 0);
  store_tile(Set0{}, Set0{});
  if (kStages == 2 && nk > 1) load_tile(std::integral_constant<int, kStages - 1>{}, C::BK);
  __syncthreads();

  const int arow = wm * C::kTM + l32;
  const int bcol = wn * C::kTN + l32;
  // Step kt reads LDS buffer P = kt % 2, fetches step kt + kStages into
  // register set kt % kStages (free: its previous step was stored into LDS
  // one step earlier) and stores step kt + 1 from set (kt + 1) % kStages into
  // buffer 1 - P (read in step kt - 1, done before the last barrier).
  auto step = [&](auto p_c, int kt) {
    constexpr int P = decltype(p_c)::value;
    if (kt + kStages < nk) load_tile(std::integral_constant<int, P % kStages>{}, (kt + kStages) * C::BK);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int ch = 2 * s + g;
      bf16x8 ah[C::kMB], bh[C::kNB];
#pragma unroll
      for (int mb = 0; mb < C::kMB; ++mb) ah[mb] = lds_frag<kSwz>(xs[P][0], arow + mb * 32, ch);
#pragma unroll
      for (int nb = 0; nb < C::kNB; ++nb) bh[nb] = lds_frag<kSwz>(ws[P][0], w_row<kSwz>(bcol + nb * 32), ch);
#pragma unroll
      for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
        for (int nb = 0; nb < C::kNB; ++nb) acc[mb][nb] = mfma_bf16(ah[mb], bh[nb], acc[mb][nb]);
      if constexpr (kTerms == 3) {
        bf16x8 al[C::kMB], bl[C::kNB];
#pragma unroll
        for (int nb = 0; nb < C::kNB; ++nb) bl[nb] = lds_frag<kSwz>(ws[P][1], w_row<kSwz>(bcol + nb * 32), ch);
#pragma unroll
        for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
          for (int nb = 0; nb < C::kNB; ++nb)
            acc[mb][nb] = mfma_bf16(ah[mb], bl[nb], acc[mb][nb]);
#pragma unroll
        for (int mb = 0; mb < C::kMB; ++mb) al[mb] = lds_frag<kSwz>(xs[P][1], arow + mb * 32, ch);
#pragma unroll
        for (int mb = 0; mb < C::kMB; ++mb)
#pragma unroll
          for (int nb = 0; nb < C::kNB; ++nb)
            acc[mb][nb] = mfma_bf16(al[mb], bh[nb], acc[mb][nb]);
      }
    }
    if (kt + 1 < nk)
      store_tile(std::integral_constant<int, (P + 1) % kStages>{}, std::integral_constant<int, 1 - P>{});
    __syncthreads();
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(Set0{}, kt);
    if (kt + 1 < nk) step(Set1{}, kt + 1);
  }

  if constexpr (kEpi == kEpiQkv) {
    qkv_epilogue<C>(a, acc, m0 + wm * C::kTM, c0 + wn * C::kTN, g, l32);
  } else {
    store_result<C::kMB, C::kNB, kEpi>(a, acc, m0 + wm * C::kTM, c0 + wn * C::kTN, g, l32);
  }
}

template <class C, int kTerms, bool kVec, bool kPl>
int launch_terms(const GemmArgs& a, int epi, hipStream_t stream) {
  const int64_t tiles = (int64_t)((a.M + C::BM - 1) / C::BM) * ((a.n_count + C::BN - 1) / C::BN);
  if (tiles <= 0 || tiles > 0x7fffffff) return kErrDims;
  const dim3 grid((unsigned)tiles), block(C::kThreads);
  switch (epi) {
    case kEpiStore:
      hipLaunchKernelGGL((nf24_gemm_bf16_kernel<C, kTerms, kVec, kEpiStore, kPl>), grid, block, 0, stream, a);
      break;
    case kEpiQkv:
      // the QKV epilogue takes one head (64 columns) per wave
      if constexpr (C::kTN == 64 && C::kNB == 2)
        hipLaunchKernelGGL((nf24_gemm_bf16_kernel<C, kTerms, kVec, kEpiQkv, kPl>), grid, block, 0, stream, a);
      else
        return kErrDims;
      break;
    case kEpilogueGelu:
      hipLaunchKernelGGL((nf24_gemm_bf16_kernel<C, kTerms, kVec, kEpilogueGelu, kPl>), grid, block, 0, stream, a);
      break;
    case kEpilogueGated:
      hipLaunchKernelGGL((nf24_gemm_bf16_kernel<C, kTerms, kVec, kEpilogueGated, kPl>), grid, block, 0, stream, a);
      break;
    case kEpilogueAdd:
      hipLaunchKernelGGL((nf24_gemm_bf16_kernel<C, kTerms, kVec, kEpilogueAdd, kPl>), grid, block, 0, stream, a);
      break;
    default:
      return kErrDims;
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <class C, bool kVec, bool kPl = false>
int launch_shape(const GemmArgs& a, int terms, int epi, hipStream_t stream) {
  return terms == 3 ? launch_terms<C, 3, kVec, kPl>(a, epi, stream)
                    : launch_terms<C, 1, kVec, kPl>(a, epi, stream);
}

// The vector path's tile shapes with or without the planes.
template <class C>
int launch_vec(const GemmArgs& a, int terms, int epi, bool planes, hipStream_t stream) {
  return planes ? launch_shape<C, true, true>(a, terms, epi, stream)
                : launch_shape<C, true, false>(a, terms, epi, stream);
}

// The tile shapes the launch model chooses from: a round of the chip
// (CUs x wgs_per_cu workgroups) costs `round` units, measured at K = 1024
// for three terms (bf16x3) and one (bf16); the model is rounds x cost.  The
// VALU- and power-bound kernels gain little from a round left part-empty,
// so a partial round costs a whole one.
struct Bf16Choice {
  int bm, bn, wgs_per_cu, round3, round1;
};
constexpr Bf16Choice kBf16Choices[] = {
    {256, 256, 1, 113, 74}, {256, 192, 1, 82, 57}, {192, 256, 1, 92, 63},
    {256, 128, 1, 60, 45},  {128, 64, 2, 40, 35}};
constexpr int kNumBf16Choices = sizeof(kBf16Choices) / sizeof(kBf16Choices[0]);

int64_t bf16_model_time(int i, int M, int n_count, int terms) {
  const Bf16Choice& c = kBf16Choices[i];
  const int64_t tiles = (int64_t)((M + c.bm - 1) / c.bm) * ((n_count + c.bn - 1) / c.bn);
  const int64_t slots = (int64_t)compute_units() * c.wgs_per_cu;
  return (tiles + slots - 1) / slots * (terms == 3 ? c.round3 : c.round1);
}

// Index into kBf16Choices with the smallest modelled time (a tie keeps the
// earlier entry, 256 x 256 first).
int bf16_pick(int M, int n_count, int terms) {
  int best = 0;
  for (int i = 1; i < kNumBf16Choices; ++i)
    if (bf16_model_time(i, M, n_count, terms) < bf16_model_time(best, M, n_count, terms)) best = i;
  return best;
}

// Rows [first, first + count) of the call as their own launch.
GemmArgs rows_of(GemmArgs a, int first, int count) {
  a.x += (int64_t)first * a.stride_x;
  if (a.out != nullptr) a.out += (int64_t)first * a.stride_out;
  a.M = count;
  a.row0 += first;
  return a;
}

}  // namespace

int launch_gemm_bf16(const GemmParams& p, int epi, const QkvArgs& e, const GemmEpilogueParams& ep,
                     int row0, hipStream_t stream) {
  const int terms = p.precision == kPrecisionBf16x3 ? 3 : 1;
  GemmArgs a{p.x, p.code01, p.q2, p.scale, p.bias, p.out,
             p.M, p.K, p.N, p.n_start, p.n_count, p.stride_x, p.stride_out, e,
             ep.gate, ep.gate_stride, ep.rows_per_batch, row0};
  a.w_hi = p.w_hi;
  a.w_lo = p.w_lo;
  const bool vec = (reinterpret_cast<uintptr_t>(p.x) % 16 == 0) && (p.stride_x % 4 == 0) &&
                   (p.K % 4 == 0) && (p.N % 4 == 0) && (p.n_start % 4 == 0) &&
                   (p.n_count % 4 == 0) && (reinterpret_cast<uintptr_t>(p.code01) % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(p.q2) % 4 == 0) &&
                   vec_buffers_fit(p, Bf16Large::BM, Bf16Large::BK);
  // The planes replace the codes in the K loop on the vector path when they
  // are 16-byte aligned; otherwise the kernels decode the codes (same result).
  const bool planes = vec && p.w_hi != nullptr &&
                      reinterpret_cast<uintptr_t>(p.w_hi) % 16 == 0 &&
                      (terms == 1 || (p.w_lo != nullptr && reinterpret_cast<uintptr_t>(p.w_lo) % 16 == 0));
  if (!vec) return launch_shape<Bf16Small, false>(a, terms, epi, stream);
  if (p.M < 256 || p.n_count < 256) return launch_vec<Bf16Small>(a, terms, epi, planes, stream);
  // Rows past the last multiple of 256 that number at most 32 stay in the
  // grid when they add no modelled time (M = 2818, N = 3072: 12 row bands
  // of 256 x 192 tiles, one round either way), else they run on the strict
  // few-row path (launch_strict_tail, first: its workspace is the only thing
  // that can fail), as whole calls of that size do in every mode: fp32 rows,
  // e.g. 12294 x 1024 x 4096's 6 rows in ~15 us where 128-row bf16 tiles
  // over 32 column bands took ~50 us.  Every tile shape sums each output in
  // the same order.
  const int rem = p.M % 256;
  const bool split = rem != 0 && rem <= 32 &&
                     bf16_model_time(bf16_pick(p.M, p.n_count, terms), p.M, p.n_count, terms) >
                         bf16_model_time(bf16_pick(p.M - rem, p.n_count, terms), p.M - rem, p.n_count,
                                         terms);
  const int rows = split ? p.M - rem : p.M;
  if (split) {
    GemmParams t = p;
    t.x = p.x + (int64_t)rows * p.stride_x;
    t.out = p.out != nullptr ? p.out + (int64_t)rows * p.stride_out : nullptr;
    t.M = rem;
    const int st = launch_strict_tail(t, epi, e, ep, row0 + rows, stream);
    if (st != kOk) return st;
  }
  const GemmArgs m = rows_of(a, 0, rows);
  switch (bf16_pick(rows, p.n_count, terms)) {
    case 0: return launch_vec<Bf16Large>(m, terms, epi, planes, stream);
    case 1:
      if (epi == kEpiQkv) return launch_vec<Bf16Wide>(m, terms, epi, planes, stream);
      return launch_vec<Bf16Wide16>(m, terms, epi, planes, stream);
    case 2: return launch_vec<Bf16Tall>(m, terms, epi, planes, stream);
    case 3: return launch_vec<Bf16Half>(m, terms, epi, planes, stream);
    default: return launch_vec<Bf16Narrow>(m, terms, epi, planes, stream);
  }
}

}  // namespace nf24

namespace {

// The bf16 planes of a packed weight, as split_w forms them in the K loop:
// w = fp32((int32)q01 * 256 + q2) * scale (one rounding, no contraction),
// hi = bf16(w), lo = bf16(fma(p, scale, -hi)); k-blocked [ceil(K / 32), N,
// 32] with zeros past K.  64 x 64 tiles through LDS: the codes [K, N] are
// read along n, the planes written along k.
constexpr int kPlaneTile = 64;
template <int kTerms>
__global__ __launch_bounds__(256) void nf24_bf16_planes_kernel(const int16_t* code01, const int8_t* q2,
                                                               const float* scale, int K, int N,
                                                               uint16_t* w_hi, uint16_t* w_lo) {
  __shared__ uint16_t th[kPlaneTile][kPlaneTile + 2];
  __shared__ uint16_t tl[kTerms == 3 ? kPlaneTile : 1][kPlaneTile + 2];
  const int n0 = blockIdx.x * kPlaneTile, k0 = blockIdx.y * kPlaneTile;
  const int tx = threadIdx.x % kPlaneTile, ty = threadIdx.x / kPlaneTile;
  for (int kk = ty; kk < kPlaneTile; kk += 256 / kPlaneTile) {
    const int k = k0 + kk, n = n0 + tx;
    uint16_t h = 0, l = 0;
    if (k < K && n < N) {
#pragma clang fp contract(off)
      const int64_t off = (int64_t)k * N + n;
      const float p = (float)((int32_t)code01[off] * 256 + (int32_t)q2[off]);
      const float s = scale[n];
      const float w = p * s;
      const __bf16 hb = (__bf16)w;
      h = __builtin_bit_cast(uint16_t, hb);
      if constexpr (kTerms == 3) l = __builtin_bit_cast(uint16_t, (__bf16)__builtin_fmaf(p, s, -(float)hb));
    }
    th[tx][kk] = h;
    if constexpr (kTerms == 3) tl[tx][kk] = l;
  }
  __syncthreads();
  const int k32 = (K + 31) / 32 * 32;
  for (int nn = ty; nn < kPlaneTile; nn += 256 / kPlaneTile) {
    const int n = n0 + nn, k = k0 + tx;
    if (n < N && k < k32) {
      const int64_t off = ((int64_t)(k / 32) * N + n) * 32 + k % 32;
      w_hi[off] = th[nn][tx];
      if constexpr (kTerms == 3) w_lo[off] = tl[nn][tx];
    }
  }
}

}  // namespace

int launch_nf24_bf16_planes(const int16_t* code01, const int8_t* q2, const float* scale, int K, int N,
                            int precision, uint16_t* w_hi, uint16_t* w_lo, hipStream_t stream) {
  if (K <= 0 || N <= 0 || (K + kPlaneTile - 1) / kPlaneTile > 65535) return kErrDims;
  // the tiles cover the zero padding of the last 32-k block as well
  const dim3 grid((unsigned)((N + kPlaneTile - 1) / kPlaneTile), (unsigned)((K + kPlaneTile - 1) / kPlaneTile));
  if (precision == kPrecisionBf16x3)
    hipLaunchKernelGGL(nf24_bf16_planes_kernel<3>, grid, dim3(256), 0, stream, code01, q2, scale, K, N, w_hi,
                       w_lo);
  else if (precision == kPrecisionBf16)
    hipLaunchKernelGGL(nf24_bf16_planes_kernel<1>, grid, dim3(256), 0, stream, code01, q2, scale, K, N, w_hi,
                       w_lo);
  else
    return kErrDims;
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace tsplat
