// Opt-in bf16-MFMA precision modes of the exact SDPA (SdpaParams.precision).
//
// Same operation and softmax as sdpa.hip -- out[q] = sum_j softmax_j(q.k_j
// * 0.125 + bias[j]) v_j over all keys, online (max, sum) merge, no Lq x Lk
// matrix -- with the two products on v_mfma_f32_32x32x16_bf16 and fp32
// accumulation:
//   kPrecisionBf16:   S = qh.kh,                  O += ph vh
//   kPrecisionBf16x3: S = qh.kh + qh.kl + ql.kh,  O += ph vh + ph vl + pl vh
// where q is first scaled by 0.125 * log2(e) in fp32 (the scores come out in
// log2 units, as in the fp32 kernel), p = exp2(s - m) is the unnormalised
// exponential of the running max m, and xh = bf16(x), xl = bf16(x - xh)
// with bf16() the nearest-even rounding of the fp32 value (v_cvt_pk_bf16_f32).
// xh + xl holds 16 significant bits of x, so each bf16x3 product is within
// about 3 * 2^-18 of the exact one (the dropped xl*yl term and the rounding
// of xl, yl); bf16 alone is within 2^-8.  The max, exp2, sums, rescaling and
// normalisation are the fp32 kernel's.
//
// Mapping (same roles as sdpa.hip): a wave owns 32 queries and computes
// S^T = K Q^T, so each lane holds 16 keys of one query per 32-key block
// (accumulator register r: key 8*(r/4) + 4*(lane/32) + r%4) and reduces
// the max / sum in-lane plus one half-wave swap.  The 16-deep k-slices of
// the bf16 MFMA take lane l's 8 values at k = 8*(l/32) + i:
//   QK: k runs over the head dimension, dims 16c + 8*(l/32) + i of slice c,
//       for both K (A operand) and Q (B operand, held in registers);
//   PV: slice c of a 32-key block uses the accumulator registers 8c + i of
//       P^T (B operand) -- keys 16c + 8*(i/4) + 4*(l/32) + i%4 -- so V^T
//       (A operand) must supply those keys at the same k: V^T rows are
//       stored with bits 2 and 3 of the key index (mod 16) swapped, which
//       makes the 8 keys of each lane contiguous.
// K and V are converted (and split) once per tile on their way into LDS,
// as bf16 rows of 72 (K: 64 dims + 8) or kBKV + 8 (V^T) elements: 8
// consecutive rows read at one column fall in distinct 16-byte bank groups.

#include "sdpa_common.h"

namespace tsplat {
namespace sdpa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx16 mfma_bf16(const bf16x8& a, const bf16x8& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Position of tile key k in a V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vt_pos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef unsigned uintx2 __attribute__((ext_vector_type(2)));
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));

// Packed bf16 pairs: hi = (bf16(a), bf16(b)), lo = bf16 of the residuals
// a - bf16(a), b - bf16(b) (exact in fp32).  One v_cvt_pk_bf16_f32 per pair
// and, for lo, two bit operations, two subtractions and a second conversion.
template <bool kLo>
__device__ __forceinline__ void split2(float a, float b, unsigned& hi, unsigned& lo) {
  hi = __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{a, b}, bf16x2));
  if constexpr (kLo) {
    const float ha = __uint_as_float(hi << 16), hb = __uint_as_float(hi & 0xffff0000u);
    lo = __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{a - ha, b - hb}, bf16x2));
  }
}

template <bool kLo>
__device__ __forceinline__ void split4(const floatx4& v, bf16x4& hi, bf16x4& lo) {
  unsigned h0, h1, l0 = 0, l1 = 0;
  split2<kLo>(v[0], v[1], h0, l0);
  split2<kLo>(v[2], v[3], h1, l1);
  hi = __builtin_bit_cast(bf16x4, uintx2{h0, h1});
  if constexpr (kLo) lo = __builtin_bit_cast(bf16x4, uintx2{l0, l1});
}

// Elements 8c..8c+7 of an accumulator block, split.
template <bool kLo>
__device__ __forceinline__ void split8(const floatx16& s, int c, bf16x8& hi, bf16x8& lo) {
  unsigned h[4], l[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 4; ++e) split2<kLo>(s[8 * c + 2 * e], s[8 * c + 2 * e + 1], h[e], l[e]);
  hi = __builtin_bit_cast(bf16x8, uintx4{h[0], h[1], h[2], h[3]});
  if constexpr (kLo) lo = __builtin_bit_cast(bf16x8, uintx4{l[0], l[1], l[2], l[3]});
}

// kLayout: 0 = k and v [B, H, Lk, 64] (v is transposed on its way into
// LDS); 1 = both key-contiguous [B, H, 64, Lkp] (k is transposed).  kWaves
// waves of 32 queries share each K/V tile of kBKV keys; kGB 32-key blocks
// per softmax step (1 keeps 16 score registers live).  kTerms: 1 (bf16) or
// 3 (bf16x3).
template <int kLayout, bool kBias, int kWaves, int kBKV, int kGB, int kTerms>
__global__ __launch_bounds__(kWaves * 64) void sdpa_bf16_kernel(SdpaArgs a) {
  constexpr int kThreads = kWaves * 64;
  constexpr int kBQ = kWaves * 32;
  constexpr int kNKB = kBKV / 32;
  constexpr bool kLo = kTerms == 3;
  constexpr int kKS = kD + 8;    // bf16 per K row (one key)
  constexpr int kVS = kBKV + 8;  // bf16 per V^T row (one dim)
  constexpr int kUnits = kBKV * kD / 4;  // float4 of K (and of V) per tile
  constexpr int kLoads = kUnits / kThreads;
  static_assert(kLoads * kThreads == kUnits, "tile split");
  static_assert(kThreads >= kBKV, "bias row load");
  static_assert(kNKB % kGB == 0, "softmax groups");
  __shared__ __attribute__((aligned(16))) __bf16 khi[2][kBKV * kKS];
  __shared__ __attribute__((aligned(16))) __bf16 klo[2][kLo ? kBKV * kKS : 8];
  __shared__ __attribute__((aligned(16))) __bf16 vhi[2][kD * kVS];
  __shared__ __attribute__((aligned(16))) __bf16 vlo[2][kLo ? kD * kVS : 8];
  __shared__ __attribute__((aligned(16))) float bbuf[2][kBKV];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int l32 = lane & 31;

  const TileWork w = tile_work(a);
  int bh, qb;
  tile_coords(a, w.tile, kBQ, bh, qb);
  // A wave whose 32 queries all lie past Lq only helps stage K/V.
  const bool wave_live = qb * kBQ + wave * 32 < a.Lq;
  const int h = bh % a.H;
  const int qrow = qb * kBQ + wave * 32 + l32;
  const bool q_ok = qrow < a.Lq;

  // Q slices in registers: dims 16c + 8g + i of the scaled query, split.
  const float c1 = 0.125f * kLog2e;
  bf16x8 qh[4], ql[4];
  {
    const float* qp = a.q + ((int64_t)bh * a.Lq + (q_ok ? qrow : 0)) * kD + 8 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        floatx4 x = q_ok ? *reinterpret_cast<const floatx4*>(qp + 16 * c + 4 * half)
                         : floatx4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // q' = fp32(q * c1) is split, not the exact product: no contraction
          // of v - hv with the multiply.
#pragma clang fp contract(off)
          const float v = x[e] * c1;
          const __bf16 hv = (__bf16)v;
          qh[c][4 * half + e] = hv;
          if constexpr (kLo) ql[c][4 * half + e] = (__bf16)(v - (float)hv);
        }
      }
  }

  constexpr bool kKP = kLayout == 1;  // k key-contiguous
  constexpr bool kVP = kLayout != 0;  // v key-contiguous
  const float* kbase = a.k + (int64_t)bh * (kKP ? (int64_t)kD * a.Lkp : (int64_t)a.Lk * kD);
  const float* vbase = a.v + (int64_t)bh * (kVP ? (int64_t)kD * a.Lkp : (int64_t)a.Lk * kD);
  const float* brow = kBias ? a.bias + (int64_t)h * a.bias_head_stride : nullptr;

  floatx4 kr[kLoads], vr[kLoads];
  float br = 0.0f;
  auto load = [&](int key0) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int idx = tid + j * kThreads;
      if constexpr (!kKP && !kVP) {
        fetch_units_kv<kBKV>(a, kbase, vbase, idx, key0, kr[j], vr[j]);
      } else {
        kr[j] = fetch_unit<kKP, kBKV>(a, kbase, idx, key0);
        vr[j] = fetch_unit<kVP, kBKV>(a, vbase, idx, key0);
      }
    }
    if (kBias && tid < kBKV) {
      const int key = key0 + tid;
      br = key < a.Lk ? brow[key] * kLog2e : 0.0f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int idx = tid + j * kThreads;
      bf16x4 kh, kl, vh, vl;
      split4<kLo>(kr[j], kh, kl);
      split4<kLo>(vr[j], vh, vl);
      if constexpr (!kKP) {  // key row, dims 4c..4c+3: one 8-byte store per plane
        const int row = idx / (kD / 4), c = idx % (kD / 4);
        *reinterpret_cast<bf16x4*>(&khi[buf][row * kKS + 4 * c]) = kh;
        if constexpr (kLo) *reinterpret_cast<bf16x4*>(&klo[buf][row * kKS + 4 * c]) = kl;
      } else {  // dim row, keys 4c..4c+3: transposed element by element
        const int row = idx / (kBKV / 4), c = idx % (kBKV / 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          khi[buf][(4 * c + e) * kKS + row] = kh[e];
          if constexpr (kLo) klo[buf][(4 * c + e) * kKS + row] = kl[e];
        }
      }
      if constexpr (!kVP) {  // key row, dims 4c..4c+3: transposed element by element
        const int row = idx / (kD / 4), c = idx % (kD / 4);
        const int p = vt_pos(row);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vhi[buf][(4 * c + e) * kVS + p] = vh[e];
          if constexpr (kLo) vlo[buf][(4 * c + e) * kVS + p] = vl[e];
        }
      } else {  // dim row, keys 4c..4c+3 (contiguous in V^T: vt_pos keeps bits 0-1)
        const int row = idx / (kBKV / 4), c = idx % (kBKV / 4);
        *reinterpret_cast<bf16x4*>(&vhi[buf][row * kVS + vt_pos(4 * c)]) = vh;
        if constexpr (kLo) *reinterpret_cast<bf16x4*>(&vlo[buf][row * kVS + vt_pos(4 * c)]) = vl;
      }
    }
    if (kBias && tid < kBKV) bbuf[buf][tid] = br;
  };

  floatx16 o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const int ntiles = (w.k_end - w.k_begin + kBKV - 1) / kBKV;
  load(w.k_begin);
  store(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const int key0 = w.k_begin + t * kBKV;
    if (t + 1 < ntiles) load(key0 + kBKV);
    const __bf16* kh_ = khi[buf];
    const __bf16* kl_ = klo[buf];
    const __bf16* vh_ = vhi[buf];
    const __bf16* vl_ = vlo[buf];
    const bool tail = key0 + kBKV > a.Lk;

    if (wave_live) {
#pragma unroll
    for (int kb0 = 0; kb0 < kNKB; kb0 += kGB) {
      // The key bias (in log2 units) is the accumulators' starting value, so
      // it is summed with the score terms and needs no registers of its own
      // (the order of an fp32 sum of the terms and the bias, as bounded).
      floatx16 s[kGB];
#pragma unroll
      for (int i = 0; i < kGB; ++i) {
        if constexpr (kBias) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const floatx4 bb =
                *reinterpret_cast<const floatx4*>(&bbuf[buf][(kb0 + i) * 32 + 8 * r4 + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e) s[i][4 * r4 + e] = bb[e];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) s[i][r] = 0.0f;
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < kGB; ++i) {
          const int off = ((kb0 + i) * 32 + l32) * kKS + 16 * c + 8 * g;
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kh_ + off);
          s[i] = mfma_bf16(kf, qh[c], s[i]);
          if constexpr (kLo) {
            const bf16x8 kfl = *reinterpret_cast<const bf16x8*>(kl_ + off);
            s[i] = mfma_bf16(kf, ql[c], s[i]);
            s[i] = mfma_bf16(kfl, qh[c], s[i]);
          }
        }

      if (tail) {
        const int valid = a.Lk - key0 - 4 * g;
#pragma unroll
        for (int i = 0; i < kGB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if ((kb0 + i) * 32 + 8 * (r / 4) + (r % 4) >= valid) s[i][r] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < kGB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[i][r]);
      mx = pair_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float ls = 0.0f;
#pragma unroll
      for (int i = 0; i < kGB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pr = __builtin_amdgcn_exp2f(s[i][r] - m_new);
          s[i][r] = pr;
          ls += pr;
        }
      l_run = fmaf(l_run, alpha, ls);
      if (__builtin_amdgcn_ballot_w64(m_new != m_run) != 0) {
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
      m_run = m_new;

      // O^T[d][query] += V^T P^T, two 16-key slices per 32-key block.
#pragma unroll
      for (int i = 0; i < kGB; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          bf16x8 ph, pl;
          split8<kLo>(s[i], c, ph, pl);
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const int off = (db * 32 + l32) * kVS + (kb0 + i) * 32 + 16 * c + 8 * g;
            const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vh_ + off);
            o[db] = mfma_bf16(vf, ph, o[db]);
            if constexpr (kLo) {
              const bf16x8 vfl = *reinterpret_cast<const bf16x8*>(vl_ + off);
              o[db] = mfma_bf16(vf, pl, o[db]);
              o[db] = mfma_bf16(vfl, ph, o[db]);
            }
          }
        }
    }
    }  // wave_live

    if (t + 1 < ntiles) store(buf ^ 1);
    __syncthreads();
  }

  store_rows<kBQ>(a, o, m_run, l_run);
}

template <int kLayout, bool kBias, int kTerms, int kWaves>
int launch_shape(const SdpaParams& p, hipStream_t stream, int cus) {
  return launch_tiles(make_args(p), p, kWaves * 32, 64, cus, stream, [&](dim3 grid, const SdpaArgs& a) {
    hipLaunchKernelGGL((sdpa_bf16_kernel<kLayout, kBias, kWaves, 64, 1, kTerms>), grid, dim3(kWaves * 64), 0,
                       stream, a);
  });
}

// Small grids: 4 waves.  Wide grids: 16 waves, except bf16x3 with packed
// k/v, which spills 148-160 bytes per lane at 16 waves (6.0 ms at
// configs[1]) and none at 8 (3.5 ms).
template <int kLayout, bool kBias, int kTerms>
int launch_sized(const SdpaParams& p, hipStream_t stream) {
  const int cus = compute_units();
  const int64_t wide_tiles = (int64_t)p.B * p.H * ((p.Lq + 511) / 512);
  if (wide_tiles < cus) return launch_shape<kLayout, kBias, kTerms, 4>(p, stream, 0);
  constexpr int kWide = (kLayout == 1 && kTerms == 3) ? 8 : 16;
  return launch_shape<kLayout, kBias, kTerms, kWide>(p, stream, cus);
}

template <int kLayout, bool kBias>
int launch_terms(const SdpaParams& p, hipStream_t stream) {
  return p.precision == kPrecisionBf16x3 ? launch_sized<kLayout, kBias, 3>(p, stream)
                                         : launch_sized<kLayout, kBias, 1>(p, stream);
}

}  // namespace
}  // namespace sdpa

int launch_sdpa_bf16(const SdpaParams& p, hipStream_t stream) {
  using namespace sdpa;
  if (p.precision != kPrecisionBf16 && p.precision != kPrecisionBf16x3) return kErrDims;
  const bool bias = p.bias != nullptr;
  if (p.kv_packed) return bias ? launch_terms<1, true>(p, stream) : launch_terms<1, false>(p, stream);
  return bias ? launch_terms<0, true>(p, stream) : launch_terms<0, false>(p, stream);
}

}  // namespace tsplat
