// QKV postprocess for gfx950: RoPE then per-head RMSNorm on q and k, layout
// change to q [B, H, Lq, 64] and key-contiguous packed k/v [B, H, 64, Lkp].
//
// Reference semantics (bit-identical): scripts/native_qkv_postprocess_v2_avx512.c
// :3-24 (transform_q64), :45-105 (the full-sequence entry) and :107-191 (the
// selected-rows entry, queries taking their frequency row from an index
// list), with rope16 of native_qkv_postprocess_avx512.c:16-21:
//   rope:  y[2i]   = fma(x[2i], cos_i, -(x[2i+1] * sin_i))
//          y[2i+1] = fma(x[2i], sin_i,   x[2i+1] * cos_i)
//   norm:  y * (8 / max(||y||, 1e-12)) * gamma[h]
//   v:     copied; packed tail tokens Lk..Lkp-1 are zero.
//
// A 64-wide head row is held by a 16-lane group the way the reference's
// 16-lane vectors hold it: lane j owns dims j, 16+j, 32+j, 48+j.  The RoPE
// partner of a dim is the neighbouring lane; ||y||^2 is lane j's fma chain
// over its four dims followed by the _mm512_reduce_add_ps tree.  A
// workgroup handles 64 tokens of one (b, h): query tiles store q rows
// directly, key tiles transpose k and v through LDS into the packed layout.

#include "tsplat_common.h"
#include "tsplat_ew.h"
#include "tsplat_launch.h"

namespace tsplat {
namespace {

constexpr int kD = 64;
constexpr int kTok = 64;
constexpr int kThreads = 256;

struct PostArgs {
  const float* q_src;      // row (b, t): q_src + (b*Lq + t) * q_stride + h*64
  const float* k_src;      // row (b, t): k_src + (b*Lk + t) * kv_stride + h*64
  const float* v_src;      // same stride as k_src
  int64_t q_stride, kv_stride;
  const int64_t* sel;      // null: query t uses frequency row t; else row sel[t]
  const float* freqs;      // [fb, Lk, H, 64]
  const float* qg;
  const float* kg;
  float* q;                // [B, H, Lq, 64]
  float* pk;               // [B, H, 64, Lkp]
  float* pv;
  int B, Lq, Lk, H, Lkp, fb;
  int q_tiles;             // blocks [0, B*H*q_tiles) do queries, the rest keys
  int kv_round;            // bit 0: k, bit 1: v stored rounded to bf16
};

// RoPE + RMSNorm of the head row held as x[c] = dim 16c + j by lane j of a
// 16-lane group (all 16 lanes must call it together).
__device__ __forceinline__ void rope_rmsnorm_row(float (&x)[4], const float (&f)[4],
                                                 const float (&g)[4], bool odd) {
#pragma clang fp contract(off)
  float y[4];
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float px = __shfl_xor(x[c], 1);
    const float pf = __shfl_xor(f[c], 1);
    y[c] = odd ? fmaf(px, f[c], x[c] * pf) : fmaf(x[c], f[c], -(px * pf));
    acc = fmaf(y[c], y[c], acc);
  }
  const float norm = sqrtf(reduce_add16(acc));
  const float factor = 8.0f / fmaxf(norm, 1.0e-12f);
#pragma unroll
  for (int c = 0; c < 4; ++c) x[c] = (y[c] * factor) * g[c];
}

__global__ __launch_bounds__(kThreads) void qkv_postprocess_kernel(PostArgs a) {
  __shared__ float kl[kTok][kD + 1];
  __shared__ float vl[kTok][kD + 1];

  const int tid = threadIdx.x;
  const int j = tid & 15;        // lane within the 16-lane group
  const int grp = tid >> 4;      // 16 groups, one token each per pass
  const bool odd = (j & 1) != 0;
  const bool query_tile = (int64_t)blockIdx.x < (int64_t)a.B * a.H * a.q_tiles;
  const int64_t blk = query_tile ? blockIdx.x : blockIdx.x - (int64_t)a.B * a.H * a.q_tiles;
  const int tiles = query_tile ? a.q_tiles : (a.Lkp + kTok - 1) / kTok;
  const int64_t bh = blk / tiles;
  const int t0 = (int)(blk % tiles) * kTok;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int fbi = a.fb == 1 ? 0 : b;
  const float* gsrc = (query_tile ? a.qg : a.kg) + h * kD;
  float g[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) g[c] = gsrc[16 * c + j];

  if (query_tile) {
#pragma unroll
    for (int pass = 0; pass < kTok / 16; ++pass) {
      const int t = t0 + pass * 16 + grp;
      if (t >= a.Lq) continue;  // uniform over the 16-lane group
      int64_t frow = t;
      if (a.sel != nullptr) {
        frow = a.sel[t];
        if (frow < 0 || frow >= a.Lk) frow = -1;  // invalid index: the row is written as zeros
      }
      float x[4], f[4];
      const float* src = a.q_src + ((int64_t)b * a.Lq + t) * a.q_stride + h * kD;
      const float* fr = a.freqs + (((int64_t)fbi * a.Lk + (frow < 0 ? 0 : frow)) * a.H + h) * kD;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        x[c] = src[16 * c + j];
        f[c] = fr[16 * c + j];
      }
      rope_rmsnorm_row(x, f, g, odd);
      float* dst = a.q + (bh * a.Lq + t) * kD;
#pragma unroll
      for (int c = 0; c < 4; ++c) dst[16 * c + j] = frow < 0 ? 0.0f : x[c];
    }
    return;
  }

#pragma unroll
  for (int pass = 0; pass < kTok / 16; ++pass) {
    const int tl = pass * 16 + grp;
    const int t = t0 + tl;
    float x[4] = {0, 0, 0, 0}, v[4] = {0, 0, 0, 0};
    if (t < a.Lk) {  // uniform over the 16-lane group
      const int64_t row = ((int64_t)b * a.Lk + t) * a.kv_stride + h * kD;
      const float* fr = a.freqs + (((int64_t)fbi * a.Lk + t) * a.H + h) * kD;
      float f[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        x[c] = a.k_src[row + 16 * c + j];
        v[c] = a.v_src[row + 16 * c + j];
        f[c] = fr[16 * c + j];
      }
      rope_rmsnorm_row(x, f, g, odd);
    }
    if (a.kv_round & 1)
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = bf16_roundtrip(x[c]);
    if (a.kv_round & 2)
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = bf16_roundtrip(v[c]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kl[tl][16 * c + j] = x[c];
      vl[tl][16 * c + j] = v[c];
    }
  }
  __syncthreads();

  // Key-contiguous stores: 64 dims x 16 float4 of tokens (zeros past Lk).
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = tid + it * kThreads;
    const int d = idx >> 4;
    const int c = idx & 15;
    const int t = t0 + 4 * c;
    if (t >= a.Lkp) continue;
    floatx4 kk, vv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kk[e] = kl[4 * c + e][d];
      vv[e] = vl[4 * c + e][d];
    }
    const int64_t off = (bh * kD + d) * a.Lkp + t;
    *reinterpret_cast<floatx4*>(a.pk + off) = kk;
    *reinterpret_cast<floatx4*>(a.pv + off) = vv;
  }
}

int launch_post(const PostArgs& a, hipStream_t stream) {
  const int64_t kv_tiles = (a.Lkp + kTok - 1) / kTok;
  const int64_t blocks = (int64_t)a.B * a.H * (a.q_tiles + kv_tiles);
  if (blocks <= 0 || blocks > 0x7fffffff) return kErrDims;
  hipLaunchKernelGGL(qkv_postprocess_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace

int launch_qkv_postprocess(const QkvPostParams& p, hipStream_t stream) {
  const int64_t C = (int64_t)p.H * kD;
  PostArgs a{p.qkv, p.qkv + C, p.qkv + 2 * C, 3 * C, 3 * C, nullptr, p.freqs, p.q_gamma,
             p.k_gamma, p.q, p.packed_k, p.packed_v, p.B, p.L, p.L, p.H, p.L_padded,
             p.freq_batches, (p.L + kTok - 1) / kTok, p.kv_round};
  return launch_post(a, stream);
}

int launch_qkv_selected_postprocess(const QkvSelectedParams& p, hipStream_t stream) {
  const int64_t C = (int64_t)p.H * kD;
  PostArgs a{p.q, p.kv, p.kv + C, C, 2 * C, p.selected, p.freqs, p.q_gamma, p.k_gamma,
             p.q_out, p.packed_k, p.packed_v, p.B, p.Lq, p.Lk, p.H, p.Lk_padded,
             p.freq_batches, (p.Lq + kTok - 1) / kTok, p.kv_round};
  return launch_post(a, stream);
}

}  // namespace tsplat
