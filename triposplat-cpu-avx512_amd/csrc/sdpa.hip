// Exact online-softmax SDPA for gfx950 (head dim 64, fp32 throughout).
//
// Reference semantics: scripts/native_sdpa_avx512_exact_q8t512.c:137-332 and
// the packed/BLHD variant scripts/native_sdpa_avx512_exact_q8t512_packed.c:3-158:
// out[q] = sum_j softmax_j(q.k_j * 0.125 + bias[j]) v_j, exact, with a
// running (max, sum) merged tile by tile; no Lq x Lk matrix, no pruning.
//
// Mapping.  A workgroup owns 32 queries per wave (16 waves = 512 queries for
// large grids, 4 waves otherwise) of one (b, h), Q resident in registers.
// Keys stream through LDS in double-buffered tiles of 64 (K and V, plus the
// bias row), shared by all waves of the workgroup.  Each wave
// computes the transposed score block S^T = K Q^T with
// v_mfma_f32_32x32x2_f32, which leaves every lane holding 32 keys of ONE
// query (its own column): the row max and row sum are in-lane reductions
// plus one v_permlane32_swap with the partner half-wave, and the
// exponentiated block is already laid out as the B operand of the second
// MFMA, O^T += V^T P^T, so P never leaves registers.  The head dimension
// inside each 8-wide slice is permuted (step t of slice hh reads
// d = 8*hh + 4*(lane/32) + t) identically for Q and K, so K fragments load
// as ds_read_b128.
//
// Scores are kept in log2 units: x = (q * 0.125 * log2 e) . k + bias * log2 e
// (Q is scaled once, in registers), p = exp2(x - m) with v_exp_f32.  This is
// the reference's exp(s - m) up to fp32 rounding of the scaled operands and
// of the argument; the maximal key still gets p = 1 exactly.  The merge is
// the usual rescale by exp2(m_old - m_new), skipped when no lane's maximum
// moved (alpha = 1 exactly).

#include "sdpa_common.h"

namespace tsplat {
namespace sdpa {
namespace {

// kLayout: 0 = k and v [B, H, Lk, 64]; 1 = both key-contiguous [B, H, 64,
// Lkp] (as the reference's packed kernel takes them).  Each operand keeps
// its orientation in LDS.
// kWaves waves of 32 queries each share every K/V tile of kBKV keys.
// kSplit: run scores -> softmax -> PV per 32-key block of the tile (16 score
// registers live instead of kBKV/2), for configurations short of registers.
template <int kLayout, bool kBias, int kWaves, int kBKV, bool kSplit>
__global__ __launch_bounds__(kWaves * 64) void sdpa_kernel(SdpaArgs a) {
  constexpr int kThreads = kWaves * 64;
  constexpr int kBQ = kWaves * 32;
  constexpr int kNKB = kBKV / 32;              // 32-key blocks per tile
  constexpr bool kKP = kLayout == 1;           // k key-contiguous
  constexpr bool kVP = kLayout != 0;           // v key-contiguous
  // LDS: K [key][64 + 4] or [d][kBKV + 4]; V [key][64] or [d][kBKV + 4].
  constexpr int kKS = kKP ? kBKV + 4 : kD + 4;
  constexpr int kVS = kVP ? kBKV + 4 : kD;
  constexpr int kKRowUnits = kKP ? kBKV / 4 : kD / 4;  // float4 per LDS row
  constexpr int kVRowUnits = kVP ? kBKV / 4 : kD / 4;
  constexpr int kUnits = kBKV * kD / 4;
  constexpr int kLoads = kUnits / kThreads;    // float4 of K (and of V) per thread
  static_assert(kLoads * kThreads == kUnits, "tile split");
  static_assert(kThreads >= kBKV, "bias row load");
  __shared__ __attribute__((aligned(16))) float kbuf[2][(kKP ? kD : kBKV) * kKS];
  __shared__ __attribute__((aligned(16))) float vbuf[2][(kVP ? kD : kBKV) * kVS];
  __shared__ __attribute__((aligned(16))) float bbuf[2][kBKV];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int l32 = lane & 31;

  const TileWork w = tile_work(a);
  const int k_begin = w.k_begin, k_end = w.k_end;
  int bh, qb;
  tile_coords(a, w.tile, kBQ, bh, qb);
  const int h = bh % a.H;
  const int qrow = qb * kBQ + wave * 32 + l32;
  const bool q_ok = qrow < a.Lq;
  // A wave whose 32 queries all lie past Lq only helps stage K/V.
  const bool wave_live = qb * kBQ + wave * 32 < a.Lq;

  // Q fragment for this lane's query, pre-scaled into log2 units:
  // qf[hh][t] = q[8*hh + 4*g + t] * 0.125 * log2(e), so the MFMA yields the
  // scores x = (q . k) / 8 * log2(e) directly.
  const float c1 = 0.125f * kLog2e;
  floatx4 qf[8];
  {
    const float* qp = a.q + ((int64_t)bh * a.Lq + (q_ok ? qrow : 0)) * kD + 4 * g;
#pragma unroll
    for (int hh = 0; hh < 8; ++hh) {
      qf[hh] = q_ok ? *reinterpret_cast<const floatx4*>(qp + 8 * hh) : floatx4{0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < 4; ++t) qf[hh][t] *= c1;
    }
  }

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
      *reinterpret_cast<floatx4*>(&kbuf[buf][(idx / kKRowUnits) * kKS + 4 * (idx % kKRowUnits)]) = kr[j];
      *reinterpret_cast<floatx4*>(&vbuf[buf][(idx / kVRowUnits) * kVS + 4 * (idx % kVRowUnits)]) = vr[j];
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

  const int ntiles = (k_end - k_begin + kBKV - 1) / kBKV;
  load(k_begin);
  store(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const int key0 = k_begin + t * kBKV;
    if (t + 1 < ntiles) load(key0 + kBKV);
    const float* kb_ = kbuf[buf];
    const float* vb_ = vbuf[buf];

    // One pass per group of kGB 32-key blocks: scores S^T[key][query] for keys
    // key0 + 32*kb + (8*(r/4) + 4*g + r%4), running max, exponentials, PV.
    constexpr int kGB = kSplit ? 1 : kNKB;
    constexpr int kGroupUnroll = kSplit ? 1 : kNKB;
    const bool tail = key0 + kBKV > a.Lk;
    if (wave_live) {
#pragma unroll kGroupUnroll
    for (int kb0 = 0; kb0 < kNKB; kb0 += kGB) {
      floatx16 s[kGB];
#pragma unroll
      for (int i = 0; i < kGB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[i][r] = 0.0f;
#pragma unroll
      for (int hh = 0; hh < 8; ++hh) {
        floatx4 kf[kGB];
#pragma unroll
        for (int i = 0; i < kGB; ++i) {
          const int kb = kb0 + i;
          if (!kKP) {
            kf[i] = *reinterpret_cast<const floatx4*>(&kb_[(kb * 32 + l32) * kKS + 8 * hh + 4 * g]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) kf[i][e] = kb_[(8 * hh + 4 * g + e) * kKS + kb * 32 + l32];
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < kGB; ++i) s[i] = mfma32x32x2(kf[i][e], qf[hh][e], s[i]);
      }

      // Scores in log2 units (+ bias * log2 e).  Keys past Lk are masked only
      // in a tile that reaches past Lk (a wave-uniform branch around the
      // index compares).
#pragma unroll
      for (int i = 0; i < kGB; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int kb = kb0 + i;
          floatx4 bb = {0, 0, 0, 0};
          if (kBias) bb = *reinterpret_cast<const floatx4*>(&bbuf[buf][kb * 32 + 8 * r4 + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * r4 + e;
            if (kBias) s[i][r] += bb[e];
          }
        }
      if (tail) {
        const int valid = a.Lk - key0 - 4 * g;  // key index within the tile, minus 4*g
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
      // alpha is exactly 1 where the max did not move; the rescale is skipped
      // when that holds for every lane of the wave.
      if (__builtin_amdgcn_ballot_w64(m_new != m_run) != 0) {
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
      m_run = m_new;

      // O^T[d][query] += V^T P^T over these keys.
#pragma unroll
      for (int i = 0; i < kGB; ++i)
#pragma unroll
        for (int hh = 0; hh < 4; ++hh) {
          const int kb = kb0 + i;
          floatx4 vf[2];
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            if (!kVP) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                vf[db][e] = vb_[(kb * 32 + 8 * hh + 4 * g + e) * kVS + db * 32 + l32];
            } else {
              vf[db] = *reinterpret_cast<const floatx4*>(
                  &vb_[(db * 32 + l32) * kVS + kb * 32 + 8 * hh + 4 * g]);
            }
          }
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int db = 0; db < 2; ++db) o[db] = mfma32x32x2(vf[db][e], s[i][4 * hh + e], o[db]);
        }
    }
    }  // wave_live

    if (t + 1 < ntiles) store(buf ^ 1);
    __syncthreads();
  }

  store_rows<kBQ>(a, o, m_run, l_run);
}

template <int kLayout, bool kBias, int kWaves, int kBKV, bool kSplit>
int launch_shape(const SdpaParams& p, hipStream_t stream, int cus) {
  return launch_tiles(make_args(p), p, kWaves * 32, kBKV, cus, stream, [&](dim3 grid, const SdpaArgs& a) {
    hipLaunchKernelGGL((sdpa_kernel<kLayout, kBias, kWaves, kBKV, kSplit>), grid, dim3(kWaves * 64), 0,
                       stream, a);
  });
}

// Grids too small to give every CU one 512-query workgroup use 4 waves;
// larger grids whose tile count is not a multiple of the CU count split the
// remainder's keys (launch_tiles).  A key bias runs the per-32-key-block
// softmax (kSplit).
template <int kLayout, bool kBias>
int launch_sized(const SdpaParams& p, hipStream_t stream) {
  const int cus = compute_units();
  const int64_t wide_tiles = (int64_t)p.B * p.H * ((p.Lq + 511) / 512);
  if (wide_tiles < cus) return launch_shape<kLayout, kBias, 4, 64, false>(p, stream, 0);
  return launch_shape<kLayout, kBias, 16, 64, kBias>(p, stream, cus);
}

}  // namespace

}  // namespace sdpa

// Shapes measured on MI355X at B=1, H=16, L=16384 (fp32 TFLOP/s): 16 waves x
// 64-key tiles 140 (unpacked) / 135 (packed) without a bias, the same tile
// split per 32-key block 134.7 with a key bias (unsplit 124: it spills), 16 x
// 128 split 130-134, 8 x 64 135-137, 4 x 64 121-123.  Storing the operand
// that arrives key-major for V (or dim-major for K) transposed in LDS, so all
// fragments are 128-bit reads, costs 2-4 %: the wider fragments push the
// 16-wave kernels into spills.
int launch_sdpa(const SdpaParams& p, hipStream_t stream) {
  using namespace sdpa;
  if (p.precision != kPrecisionFp32) return launch_sdpa_bf16(p, stream);
  const bool bias = p.bias != nullptr;
  if (p.kv_packed) return bias ? launch_sized<1, true>(p, stream) : launch_sized<1, false>(p, stream);
  return bias ? launch_sized<0, true>(p, stream) : launch_sized<0, false>(p, stream);
}

}  // namespace tsplat
