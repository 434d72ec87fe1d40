// Operands and epilogues shared by the NF24 GEMM kernels (the fp32-MFMA
// kernel of nf24_gemm.hip and the bf16-MFMA kernel of nf24_gemm_bf16.hip).
// Both keep the 32x32 MFMA accumulator layout: register r of lane l holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32 of a 32x32 block, so the
// epilogues below serve both.
#pragma once

#include "tsplat_common.h"
#include "tsplat_ew.h"
#include "tsplat_launch.h"

#include <utility>

namespace tsplat {
namespace nf24 {

// f(std::integral_constant<int, i>) for i = 0 .. N-1, expanded at compile time.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Fused QKV epilogue operands (kEpiQkv): rows are tokens b*L + l, columns
// [q | k | v] with H heads of 64 each.
struct QkvArgs {
  const float* freqs;  // [fb, L, H, 64] interleaved (cos, sin)
  const float* qg;     // [H, 64]
  const float* kg;     // [H, 64]
  float* q;            // [B, H, L, 64]
  float* pk;           // [B, H, 64, Lpad], or [B, H, L, 64] with kv_bhld
  float* pv;           // same layout as pk
  int L, H, Lpad, fb;
  int kv_bhld;         // 1: k and v stored [B, H, L, 64] like q
  int kv_round;        // bit 0: k, bit 1: v stored rounded to bf16
};

struct GemmArgs {
  const float* x;
  const int16_t* code01;
  const int8_t* q2;
  const float* scale;
  const float* bias;
  float* out;
  int M, K, N, n_start, n_count, stride_x, stride_out;
  QkvArgs e;
  // kEpilogueGated: gate row of batch (row0 + m) / rows_per_batch
  const float* gate;
  int64_t gate_stride;
  int rows_per_batch;
  int row0;  // global index of row 0 of x / out (the epilogues' token mapping)
  // XCD blocking of the tile grid (xcd_grid): 0, or pm x pn = 8 rectangles
  int xcd_pm, xcd_pn;
  // bf16 planes of the weights (GemmParams::w_hi / w_lo), or null
  const uint16_t* w_hi = nullptr;
  const uint16_t* w_lo = nullptr;
};

// Tile (row band, column band) of workgroup `id` in a grid of tiles_m x
// tiles_n tiles.  Workgroup i runs on XCD i % 8.  With pm x pn = 8 the grid
// is cut into pm x pn rectangles, one per XCD, so that each XCD's L2 holds
// the x rows of tiles_m / pm bands and the codes of tiles_n / pn bands
// instead of every band of one operand; within a rectangle the XCD's
// workgroups take tiles row by row in dispatch order.  Otherwise each XCD
// gets a contiguous run of tile indices (xcd_tile_index).
__device__ __forceinline__ void xcd_grid(int id, int tiles_m, int tiles_n, int pm, int pn,
                                         int& tm, int& tn) {
  if (pm > 0) {
    const int xcd = id & 7, j = id >> 3;
    const int rw = tiles_n / pn, rh = tiles_m / pm;
    tm = (xcd / pn) * rh + j / rw;
    tn = (xcd % pn) * rw + j % rw;
    return;
  }
  const int tile = xcd_tile_index(id, tiles_m * tiles_n);
  tm = tile / tiles_n;
  tn = tile % tiles_n;
}

// kEpilogue* of tsplat_launch.h, plus the fused QKV epilogue.
enum Epilogue : int { kEpiStore = kEpilogueStore, kEpiQkv = 1 };

// ||y||^2 of one head row whose dims d and 32+d sit in lane d (r0, r1) of a
// half-wave, summed in the reference's order (native_qkv_postprocess_v2_avx512.c:3-24):
// the AVX-512 lane j chains fma over dims j, 16+j, 32+j, 48+j, then the
// _mm512_reduce_add_ps tree.  Lanes j < 16 of the half gather the two dims
// they lack from lane j+16; every lane receives the sum.
__device__ __forceinline__ float head_sumsq_ref(float r0, float r1, int g, int l32) {
#pragma clang fp contract(off)
  const int src = (g << 5) | ((l32 + 16) & 31);
  const float rb = __shfl(r0, src);
  const float rd = __shfl(r1, src);
  float acc = fmaf(r0, r0, 0.0f);
  acc = fmaf(rb, rb, acc);
  acc = fmaf(r1, r1, acc);
  acc = fmaf(rd, rd, acc);
  return __shfl(reduce_add16(acc), g << 5);
}

// QKV epilogue of one wave: its 64 columns are one head of q, k or v
// (colw = first column, a multiple of 64); lane l32 holds dims l32 and
// 32 + l32 of rows 8*(r/4) + 4*g + r%4 of each 32-row block.  q and k get
// RoPE (the partner of dim 2i / 2i+1 is the neighbouring lane) then
// y * 8 / max(||y||, 1e-12) * gamma with ||y||^2 in the reference's order;
// q is stored [B, H, L, 64], k and v key-contiguous [B, H, 64, Lpad] (four
// consecutive tokens per 128-bit store when L % 4 == 0) or, with kv_bhld,
// [B, H, L, 64] like q.  Same arithmetic as
// qkv_postprocess.hip, so GEMM + this epilogue equals GEMM + postprocess
// bit for bit.
template <class C>
__device__ __forceinline__ void qkv_epilogue(const GemmArgs& a, floatx16 (&acc)[C::kMB][C::kNB],
                                             int row_base, int colw, int g, int l32) {
  static_assert(C::kTN == 64 && C::kNB == 2, "the QKV epilogue needs one head per wave");
  if (colw >= a.n_count) return;
  const QkvArgs& e = a.e;
  const int width = e.H * 64;
  const int sec = colw / width;  // 0 q, 1 k, 2 v
  const int h = (colw - sec * width) >> 6;
  const bool odd = (l32 & 1) != 0;
  float g0 = 1.0f, g1 = 1.0f;
  if (sec < 2) {
    const float* gp = (sec == 0 ? e.qg : e.kg) + h * 64;
    g0 = gp[l32];
    g1 = gp[32 + l32];
  }
  // Row blocks are expanded at compile time: a pragma-unrolled loop over
  // four of them exceeds the unroller's size limit and sends acc to scratch.
  static_for<C::kMB>([&](auto mb_c) {
    constexpr int mb = decltype(mb_c)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row0 = row_base + mb * 32 + 8 * j + 4 * g;
      floatx4 y0, y1;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float v0 = acc[mb][0][4 * j + t];
        float v1 = acc[mb][1][4 * j + t];
        if (sec < 2) {  // uniform over the wave
          const int row = row0 + t;
          const bool valid = row < a.M;  // uniform over the half-wave
          const int tok = a.row0 + row;  // token index b * L + l
          const int b = valid ? tok / e.L : 0;
          const int l = valid ? tok - b * e.L : 0;
          const float* fr =
              e.freqs + (((int64_t)(e.fb == 1 ? 0 : b) * e.L + l) * e.H + h) * 64;
          const float f0 = valid ? fr[l32] : 0.0f;
          const float f1 = valid ? fr[32 + l32] : 0.0f;
          const float p0 = __shfl_xor(v0, 1), p1 = __shfl_xor(v1, 1);
          const float fp0 = __shfl_xor(f0, 1), fp1 = __shfl_xor(f1, 1);
          const float r0 = odd ? fmaf(p0, f0, v0 * fp0) : fmaf(v0, f0, -(p0 * fp0));
          const float r1 = odd ? fmaf(p1, f1, v1 * fp1) : fmaf(v1, f1, -(p1 * fp1));
          const float ss = head_sumsq_ref(r0, r1, g, l32);
          const float fac = 8.0f / fmaxf(sqrtf(ss), 1.0e-12f);
          v0 = (r0 * fac) * g0;
          v1 = (r1 * fac) * g1;
        }
        y0[t] = v0;
        y1[t] = v1;
      }
      if (sec > 0 && ((e.kv_round >> (sec - 1)) & 1)) {  // uniform over the wave
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          y0[t] = bf16_roundtrip(y0[t]);
          y1[t] = bf16_roundtrip(y1[t]);
        }
      }
      if (sec == 0 || e.kv_bhld) {
        float* base = sec == 0 ? e.q : (sec == 1 ? e.pk : e.pv);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int row = row0 + t;
          if (row >= a.M) continue;
          const int tok = a.row0 + row;
          const int b = tok / e.L, l = tok - b * e.L;
          float* dst = base + (((int64_t)b * e.H + h) * e.L + l) * 64;
          dst[l32] = y0[t];
          dst[32 + l32] = y1[t];
        }
      } else {
        float* base = sec == 1 ? e.pk : e.pv;
        const int64_t dim_stride = (int64_t)32 * e.Lpad;
        if (((e.L | a.row0) & 3) == 0) {  // the four rows are four tokens of one sequence
          if (row0 < a.M) {
            const int tok = a.row0 + row0;
            const int b = tok / e.L, l = tok - b * e.L;
            const int64_t off = (((int64_t)b * e.H + h) * 64 + l32) * e.Lpad + l;
            *reinterpret_cast<floatx4*>(base + off) = y0;
            *reinterpret_cast<floatx4*>(base + off + dim_stride) = y1;
          }
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int row = row0 + t;
            if (row >= a.M) continue;
            const int tok = a.row0 + row;
            const int b = tok / e.L, l = tok - b * e.L;
            const int64_t off = (((int64_t)b * e.H + h) * 64 + l32) * e.Lpad + l;
            base[off] = y0[t];
            base[off + dim_stride] = y1[t];
          }
        }
      }
    }
  });
}

// Stores a wave's MB x NB blocks of 32x32 (rows from row_base, columns from
// col_base, both within the launch's output range) with the plain-store
// epilogue kinds of tsplat_launch.h.
template <int kMB, int kNB, int kEpi>
__device__ __forceinline__ void store_result(const GemmArgs& a, floatx16 (&acc)[kMB][kNB],
                                             int row_base, int col_base, int g, int l32) {
  if constexpr (kEpi == kEpilogueGated || kEpi == kEpilogueAdd) {
    // Read-modify-write epilogues: each 32 x 32 block reads all of its old
    // values (and, when its 32 rows lie in one gate batch, its gate value
    // once) before it stores any, so that the loads are in flight together;
    // element by element, every load would wait behind the previous store,
    // which might alias it.  The same arithmetic per element.
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) {
        const int col = col_base + nb * 32 + l32;
        const int rb = row_base + mb * 32;
        if (col >= a.n_count || rb >= a.M) continue;
        float* dst = a.out + (int64_t)rb * a.stride_out + col;
        float old[16], gt[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 8 * (r / 4) + 4 * g + (r % 4);
          old[r] = rb + dr < a.M ? dst[(int64_t)dr * a.stride_out] : 0.0f;
        }
        if constexpr (kEpi == kEpilogueGated) {
          const int t0 = a.row0 + rb;
          const int b0 = t0 / a.rows_per_batch;
          if (b0 == (t0 + 31) / a.rows_per_batch) {  // uniform over the wave
            const float gv = a.gate[(int64_t)b0 * a.gate_stride + a.n_start + col];
#pragma unroll
            for (int r = 0; r < 16; ++r) gt[r] = gv;
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int dr = 8 * (r / 4) + 4 * g + (r % 4);
              gt[r] = rb + dr < a.M
                          ? a.gate[(int64_t)((t0 + dr) / a.rows_per_batch) * a.gate_stride +
                                   a.n_start + col]
                          : 0.0f;
            }
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 8 * (r / 4) + 4 * g + (r % 4);
          if (rb + dr >= a.M) continue;
          if constexpr (kEpi == kEpilogueGated)
            // h = acc * gate, x = x + h: two roundings, as the reference's
            // native_block_elementwise_avx512.c:24-35
            dst[(int64_t)dr * a.stride_out] = gated_residual_ref(old[r], acc[mb][nb][r], gt[r]);
          else
            dst[(int64_t)dr * a.stride_out] = old[r] + acc[mb][nb][r];
        }
      }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const int col = col_base + nb * 32 + l32;
      if (col >= a.n_count) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row_base + mb * 32 + 8 * (r / 4) + 4 * g + (r % 4);
        if (row >= a.M) continue;
        float* dst = a.out + (int64_t)row * a.stride_out + col;
        const float v = acc[mb][nb][r];
        if constexpr (kEpi == kEpilogueGelu) {
          *dst = gelu_tanh_ref(v);
        } else {
          *dst = v;
        }
      }
    }
}

// The buffer-resource loads of the kernels' vector paths address the code
// planes (rows up to K + bk) and a tile's bm rows of x with 32-bit byte
// offsets that must stay below 2^31 (kBufOob); larger operands take the
// scalar paths.
inline bool vec_buffers_fit(const GemmParams& p, int bm, int bk) {
  constexpr int64_t kLimit = 0x7fffffffLL;
  return ((int64_t)p.K + bk) * p.N * 2 < kLimit &&
         ((int64_t)(bm - 1) * p.stride_x + p.K + bk) * 4 < kLimit;
}

// bf16-MFMA GEMM (nf24_gemm_bf16.hip) for p.precision kPrecisionBf16 /
// kPrecisionBf16x3 and M > 32: epilogue kind epi (kEpi* / kEpilogue*), QKV
// operands e, gate operands ep, token index of row 0 row0.
int launch_gemm_bf16(const GemmParams& p, int epi, const QkvArgs& e, const GemmEpilogueParams& ep,
                     int row0, hipStream_t stream);

// A row tail (at most 32 rows, token index of its row 0 row0) split off a
// bf16-mode call, on the strict few-row path (nf24_gemm.hip) with epilogue
// kind epi: as whole calls of at most 32 rows in every mode, the weight
// stream is the cost there and fp32 is free.
int launch_strict_tail(const GemmParams& p, int epi, const QkvArgs& e, const GemmEpilogueParams& ep,
                       int row0, hipStream_t stream);

}  // namespace nf24
}  // namespace tsplat
