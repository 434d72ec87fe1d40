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
//
// Wide launches without a caller scratch first run sdpa_bf16_presplit_kernel,
// which stages every 64-key tile of every (b, h) once, through the same
// fetch / split / placement code, and writes the tile's LDS contents to
// memory (its bf16 planes without the row padding, then the key-bias row in
// log2 units); the main kernel (kPre) then copies the planes into LDS with
// 16-byte loads and stores, and the bias row with one direct-to-LDS load,
// instead of converting, splitting and transposing the tile in each of the
// Lq / 512 query tiles that read it.  The LDS contents, and so the results,
// are the same bit for bit.

#include "sdpa_common.h"

namespace tsplat {
namespace sdpa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx16 mfma_bf16(const bf16x8& a, const bf16x8& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// s_waitcnt operand: vector-memory count 0, export and LDS/scalar counts
// left at their maxima (not waited on).
constexpr int kWaitVmcnt0 = 0x0f70;

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

// LDS image of one K/V tile of kBKV == kD keys: bf16 planes of kPlaneElems
// elements, 0 = K hi, 1 = V^T hi, 2 = K lo, 3 = V^T lo (bf16x3 only); K rows
// (one key) and V^T rows (one dim) both of kRowElems = 72.
constexpr int kTileKeys = 64;
constexpr int kRowElems = kTileKeys + 8;
constexpr int kPlaneElems = kTileKeys * kRowElems;
static_assert(kTileKeys == kD, "K rows and V^T rows share one stride");

// Fetches thread tid's kLoads float4 units of K and V for the tile at key0.
// kLayout: 0 = k and v [B, H, Lk, 64]; 1 = both key-contiguous [B, H, 64, Lkp].
template <int kLayout, int kThreads, int kLoads>
__device__ __forceinline__ void fetch_kv(const SdpaArgs& a, const float* kbase, const float* vbase, int tid,
                                         int key0, floatx4 (&kr)[kLoads], floatx4 (&vr)[kLoads]) {
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int idx = tid + j * kThreads;
    if constexpr (kLayout == 0) {
      fetch_units_kv<kTileKeys>(a, kbase, vbase, idx, key0, kr[j], vr[j]);
    } else {
      kr[j] = fetch_unit<true, kTileKeys>(a, kbase, idx, key0);
      vr[j] = fetch_unit<true, kTileKeys>(a, vbase, idx, key0);
    }
  }
}

// Splits the fetched units and places them in the LDS planes at `planes`:
// K as key rows, V transposed to dim rows with its keys at vt_pos.
template <int kLayout, bool kLo, int kThreads, int kLoads>
__device__ __forceinline__ void place_kv(int tid, const floatx4 (&kr)[kLoads], const floatx4 (&vr)[kLoads],
                                         __bf16* planes) {
  // (without kLo the lo planes do not exist and are never stored to)
  __bf16* khi = planes;
  __bf16* vhi = planes + kPlaneElems;
  __bf16* klo = kLo ? planes + 2 * kPlaneElems : planes;
  __bf16* vlo = kLo ? planes + 3 * kPlaneElems : planes;
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int idx = tid + j * kThreads;
    bf16x4 kh, kl, vh, vl;
    split4<kLo>(kr[j], kh, kl);
    split4<kLo>(vr[j], vh, vl);
    if constexpr (kLayout == 0) {
      // key row, dims 4c..4c+3: one 8-byte store per K plane, V transposed
      // element by element
      const int row = idx / (kD / 4), c = idx % (kD / 4);
      *reinterpret_cast<bf16x4*>(&khi[row * kRowElems + 4 * c]) = kh;
      if constexpr (kLo) *reinterpret_cast<bf16x4*>(&klo[row * kRowElems + 4 * c]) = kl;
      const int p = vt_pos(row);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vhi[(4 * c + e) * kRowElems + p] = vh[e];
        if constexpr (kLo) vlo[(4 * c + e) * kRowElems + p] = vl[e];
      }
    } else {
      // dim row, keys 4c..4c+3: K transposed element by element, V one
      // 8-byte store per plane (contiguous in V^T: vt_pos keeps bits 0-1)
      const int row = idx / (kTileKeys / 4), c = idx % (kTileKeys / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        khi[(4 * c + e) * kRowElems + row] = kh[e];
        if constexpr (kLo) klo[(4 * c + e) * kRowElems + row] = kl[e];
      }
      *reinterpret_cast<bf16x4*>(&vhi[row * kRowElems + vt_pos(4 * c)]) = vh;
      if constexpr (kLo) *reinterpret_cast<bf16x4*>(&vlo[row * kRowElems + vt_pos(4 * c)]) = vl;
    }
  }
}

// Global image of the staged tiles: per (b*H + h, tile of 64 keys), the LDS
// planes (kPlanes x 64 rows x 64 bf16, the rows without their padding), then
// with a key bias the tile's 64 bias values in log2 units (zero past Lk).
template <int kTerms, bool kBias>
constexpr int kImageTileBytes = (kTerms == 3 ? 4 : 2) * kTileKeys * kTileKeys * 2 + (kBias ? kTileKeys * 4 : 0);
constexpr int kPreThreads = 256;

template <int kLayout, int kTerms, bool kBias>
__global__ __launch_bounds__(kPreThreads) void sdpa_bf16_presplit_kernel(SdpaArgs a, uintx4* out,
                                                                         int ntiles) {
  constexpr bool kLo = kTerms == 3;
  constexpr int kPlanes = kLo ? 4 : 2;
  constexpr int kLoads = kTileKeys * kD / 4 / kPreThreads;
  constexpr int kUnits = kPlanes * kTileKeys * kTileKeys / 8;  // 16-byte units of the planes
  __shared__ __attribute__((aligned(16))) __bf16 lds[kPlanes * kPlaneElems];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x / ntiles, tile = blockIdx.x % ntiles;
  const int64_t head = kLayout == 1 ? (int64_t)kD * a.Lkp : (int64_t)a.Lk * kD;
  floatx4 kr[kLoads], vr[kLoads];
  fetch_kv<kLayout, kPreThreads, kLoads>(a, a.k + bh * head, a.v + bh * head, tid, tile * kTileKeys, kr, vr);
  place_kv<kLayout, kLo, kPreThreads, kLoads>(tid, kr, vr, lds);
  __syncthreads();
  uintx4* dst = out + (int64_t)blockIdx.x * (kImageTileBytes<kTerms, kBias> / 16);
#pragma unroll
  for (int j = 0; j < kUnits / kPreThreads; ++j) {
    const int u = tid + j * kPreThreads;
    const int p = u / (kUnits / kPlanes), r = (u / 8) % kTileKeys, ch = u % 8;
    dst[u] = *reinterpret_cast<const uintx4*>(&lds[p * kPlaneElems + r * kRowElems + 8 * ch]);
  }
  if (kBias && tid < kTileKeys) {
    const int key = tile * kTileKeys + tid;
    const float* brow = a.bias + (int64_t)(bh % a.H) * a.bias_head_stride;
    reinterpret_cast<float*>(dst + kUnits)[tid] = key < a.Lk ? brow[key] * kLog2e : 0.0f;
  }
}

// kLayout: 0 = k and v [B, H, Lk, 64] (v is transposed on its way into
// LDS); 1 = both key-contiguous [B, H, 64, Lkp] (k is transposed).  kWaves
// waves of 32 queries share each K/V tile of kBKV keys; kGB 32-key blocks
// per softmax step (1 keeps 16 score registers live).  kTerms: 1 (bf16) or
// 3 (bf16x3).  kPre: the tiles come from sdpa_bf16_presplit_kernel's image
// `pre` (kLayout is then unused).
template <int kLayout, bool kBias, int kWaves, int kBKV, int kGB, int kTerms, bool kPre>
__global__ __launch_bounds__(kWaves * 64) void sdpa_bf16_kernel(SdpaArgs a, const uintx4* pre) {
  constexpr int kThreads = kWaves * 64;
  constexpr int kBQ = kWaves * 32;
  constexpr int kNKB = kBKV / 32;
  constexpr bool kLo = kTerms == 3;
  constexpr int kPlanes = kLo ? 4 : 2;
  constexpr int kKS = kRowElems;  // bf16 per K row (one key)
  constexpr int kVS = kRowElems;  // bf16 per V^T row (one dim)
  constexpr int kUnits = kBKV * kD / 4;  // float4 of K (and of V) per tile
  constexpr int kLoads = kPre ? 1 : kUnits / kThreads;
  constexpr int kPUnits = kPlanes * kBKV * kD / 8;  // 16-byte units of a tile's image planes
  constexpr int kPLoads = kPre ? kPUnits / kThreads : 1;
  static_assert(kBKV == kTileKeys, "tile image");
  static_assert(kPre ? kPLoads * kThreads == kPUnits : kLoads * kThreads == kUnits, "tile split");
  static_assert(kThreads >= kBKV, "bias row load");
  static_assert(kNKB % kGB == 0, "softmax groups");
  __shared__ __attribute__((aligned(16))) __bf16 kvl[2][kPlanes * kPlaneElems];
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

  const int64_t head = kLayout == 1 ? (int64_t)kD * a.Lkp : (int64_t)a.Lk * kD;
  const float* kbase = a.k + (int64_t)bh * head;
  const float* vbase = a.v + (int64_t)bh * head;
  const float* brow = kBias ? a.bias + (int64_t)h * a.bias_head_stride : nullptr;
  constexpr int kTileBytes = kImageTileBytes<kTerms, kBias>;
  const char* pbase =
      kPre ? reinterpret_cast<const char*>(pre) + (int64_t)bh * ((a.Lk + kBKV - 1) / kBKV) * kTileBytes : nullptr;

  floatx4 kr[kLoads], vr[kLoads];
  uintx4 pr[kPLoads];
  float br = 0.0f;
  // load(key0, buf): kPre fetches thread tid's 16-byte units of the tile's
  // image planes into registers, and the last wave copies the bias row
  // straight into LDS buffer buf (direct-to-LDS, no register); otherwise
  // the fp32 units and the bias value are fetched into registers.
  // store(buf) places the units in LDS buffer buf (kPre: and waits for the
  // bias copy), before the barrier that publishes it.
  auto load = [&](int key0, int buf) {
    if constexpr (kPre) {
      const char* src = pbase + (int64_t)(key0 / kBKV) * kTileBytes;
#pragma unroll
      for (int j = 0; j < kPLoads; ++j) pr[j] = reinterpret_cast<const uintx4*>(src)[tid + j * kThreads];
      if (kBias && __builtin_amdgcn_readfirstlane(wave) == kWaves - 1)
        __builtin_amdgcn_global_load_lds(src + kPUnits * 16 + lane * 4,
                                         (__attribute__((address_space(3))) void*)(&bbuf[buf][0]), 4, 0, 0);
    } else {
      fetch_kv<kLayout, kThreads, kLoads>(a, kbase, vbase, tid, key0, kr, vr);
      if (kBias && tid < kBKV) {
        const int key = key0 + tid;
        br = key < a.Lk ? brow[key] * kLog2e : 0.0f;
      }
    }
  };
  auto store = [&](int buf) {
    if constexpr (kPre) {
#pragma unroll
      for (int j = 0; j < kPLoads; ++j) {
        const int u = tid + j * kThreads;
        const int p = u / (kPUnits / kPlanes), r = (u / 8) % kBKV, ch = u % 8;
        *reinterpret_cast<uintx4*>(&kvl[buf][p * kPlaneElems + r * kRowElems + 8 * ch]) = pr[j];
      }
      if constexpr (kBias) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    } else {
      place_kv<kLayout, kLo, kThreads, kLoads>(tid, kr, vr, kvl[buf]);
      if (kBias && tid < kBKV) bbuf[buf][tid] = br;
    }
  };

  floatx16 o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const int ntiles = (w.k_end - w.k_begin + kBKV - 1) / kBKV;
  load(w.k_begin, 0);
  store(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const int key0 = w.k_begin + t * kBKV;
    if (t + 1 < ntiles) load(key0 + kBKV, buf ^ 1);
    const __bf16* kh_ = kvl[buf];
    const __bf16* vh_ = kvl[buf] + kPlaneElems;
    const __bf16* kl_ = kLo ? kvl[buf] + 2 * kPlaneElems : kh_;
    const __bf16* vl_ = kLo ? kvl[buf] + 3 * kPlaneElems : vh_;
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

template <int kLayout, bool kBias, int kTerms, int kWaves, bool kPre>
int launch_shape(const SdpaParams& p, hipStream_t stream, int cus, const uintx4* pre) {
  return launch_tiles(make_args(p), p, kWaves * 32, 64, cus, stream, [&](dim3 grid, const SdpaArgs& a) {
    hipLaunchKernelGGL((sdpa_bf16_kernel<kLayout, kBias, kWaves, 64, 1, kTerms, kPre>), grid,
                       dim3(kWaves * 64), 0, stream, a, pre);
  });
}

// Largest pre-split image (as large as the fp32 K and V it replaces, in
// bf16x3) the library allocates for one call; larger calls stage in the
// kernel rather than grow a stream's workspace further.
constexpr size_t kPreMaxImageBytes = size_t(2) << 30;

// Stages every K/V tile once into the stream's pre-split workspace.  Null
// (and st untouched) when the image would exceed kPreMaxImageBytes or the
// workspace is not available -- allocation failure, or a graph capture that
// would need it to grow -- so the caller stages in the main kernel instead;
// st = kErrLaunch on a failed launch.
template <int kLayout, int kTerms, bool kBias>
const uintx4* presplit(const SdpaParams& p, hipStream_t stream, int& st) {
  const int64_t ntiles = (p.Lk + kTileKeys - 1) / kTileKeys;
  const int64_t blocks = (int64_t)p.B * p.H * ntiles;
  if (blocks <= 0 || blocks > 0x7fffffff) return nullptr;
  const size_t bytes = (size_t)blocks * kImageTileBytes<kTerms, kBias>;
  if (bytes > kPreMaxImageBytes) return nullptr;
  auto* img = static_cast<uintx4*>(stream_workspace(stream, bytes, kSlotSdpaPlanes));
  if (img == nullptr) return nullptr;
  hipLaunchKernelGGL((sdpa_bf16_presplit_kernel<kLayout, kTerms, kBias>), dim3((unsigned)blocks),
                     dim3(kPreThreads), 0, stream, make_args(p), img, (int)ntiles);
  if (hipGetLastError() != hipSuccess) {
    st = kErrLaunch;
    return nullptr;
  }
  return img;
}

// Query tiles of 512 per head from which the pre-split pass is used: it
// reads K / V once and writes their bf16 image once (46 us for 16 heads x
// 16384 keys in bf16x3), and each query tile then saves the conversion and
// transposition of every K/V tile.  Measured break-even: 8-12 tiles with
// [Lk, 64] k/v (configs[1]: 2.81 -> 2.69 ms in bf16x3, 1.29 -> 1.24 ms in
// bf16; 2 tiles: 1.43 -> 1.73 ms), 4-8 with key-contiguous k/v, whose
// in-kernel staging transposes K element by element.
template <int kLayout>
constexpr int kPreMinQueryTiles = kLayout == 1 ? 6 : 12;

// Small grids: 4 waves.  Wide grids: 16 waves, on the pre-split tiles when
// the call may allocate (no caller scratch) and enough query tiles share
// each K/V tile, else staging in the kernel.  Both wide forms run the same
// tile plan, so they give the same bits.
template <int kLayout, bool kBias, int kTerms>
int launch_sized(const SdpaParams& p, hipStream_t stream) {
  const int cus = compute_units();
  const int64_t wide_tiles = (int64_t)p.B * p.H * ((p.Lq + 511) / 512);
  if (wide_tiles < cus) return launch_shape<kLayout, kBias, kTerms, 4, false>(p, stream, 0, nullptr);
  if (p.scratch == nullptr && (p.Lq + 511) / 512 >= kPreMinQueryTiles<kLayout>) {
    int st = kOk;
    const uintx4* img = presplit<kLayout, kTerms, kBias>(p, stream, st);
    if (st != kOk) return st;
    if (img != nullptr) return launch_shape<0, kBias, kTerms, 16, true>(p, stream, cus, img);
  }
  return launch_shape<kLayout, kBias, kTerms, 16, false>(p, stream, cus, nullptr);
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
