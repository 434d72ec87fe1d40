// QKV postprocess for gfx950: RoPE then per-head RMSNorm on q and k, layout
// change to q [B, H, L, 64] and key-contiguous packed k/v [B, H, 64, Lpad].
//
// Reference semantics: scripts/native_qkv_postprocess_v2_avx512.c:3-105 and
// the epilogue of scripts/gemm_nf24_qkv_direct_avx512.c:11-85:
//   rope:  y[2i]   = x[2i]*cos_i - x[2i+1]*sin_i
//          y[2i+1] = x[2i]*sin_i + x[2i+1]*cos_i   (freq row = (cos, sin) pairs)
//   norm:  y * 8 / max(||y||_2, 1e-12) * gamma[h]   (RoPE first, then RMSNorm)
//   v:     copied; packed tail tokens L..Lpad-1 are zero.
//
// One workgroup handles 64 tokens of one (b, h).  Sixteen lanes own one
// token row (a float4 each), so the norm is a 16-lane shuffle reduction;
// q rows go straight to HBM, k/v rows are transposed through LDS so the
// packed stores are key-contiguous.

#include "tsplat_common.h"
#include "tsplat_launch.h"

namespace tsplat {
namespace {

constexpr int kD = 64;
constexpr int kTok = 64;
constexpr int kThreads = 256;

struct PostArgs {
  const float* qkv;
  const float* freqs;
  const float* qg;
  const float* kg;
  float* q;
  float* pk;
  float* pv;
  int B, L, H, Lpad, fb;
};

__device__ __forceinline__ floatx4 rope4(floatx4 x, floatx4 f) {
  floatx4 y;
  y[0] = fmaf(x[0], f[0], -(x[1] * f[1]));
  y[1] = fmaf(x[0], f[1], x[1] * f[0]);
  y[2] = fmaf(x[2], f[2], -(x[3] * f[3]));
  y[3] = fmaf(x[2], f[3], x[3] * f[2]);
  return y;
}

__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

__global__ __launch_bounds__(kThreads) void qkv_postprocess_kernel(PostArgs a) {
  __shared__ float kl[kTok][kD + 1];
  __shared__ float vl[kTok][kD + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tiles = (a.Lpad + kTok - 1) / kTok;
  const int bh = blockIdx.x / tiles;
  const int t0 = (blockIdx.x % tiles) * kTok;
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int fbi = a.fb == 1 ? 0 : b;
  const int64_t C = (int64_t)a.H * kD;
  const int d4 = lane & 15;

  const floatx4 gq = *reinterpret_cast<const floatx4*>(a.qg + h * kD + 4 * d4);
  const floatx4 gk = *reinterpret_cast<const floatx4*>(a.kg + h * kD + 4 * d4);

#pragma unroll
  for (int pass = 0; pass < kTok / 16; ++pass) {
    const int tl = pass * 16 + wave * 4 + (lane >> 4);
    const int tok = t0 + tl;
    floatx4 yk = {0, 0, 0, 0}, v4 = {0, 0, 0, 0};
    if (tok < a.L) {  // uniform across each 16-lane group
      const float* src = a.qkv + ((int64_t)b * a.L + tok) * 3 * C + h * kD + 4 * d4;
      const floatx4 q4 = *reinterpret_cast<const floatx4*>(src);
      const floatx4 k4 = *reinterpret_cast<const floatx4*>(src + C);
      v4 = *reinterpret_cast<const floatx4*>(src + 2 * C);
      const floatx4 f4 = *reinterpret_cast<const floatx4*>(
          a.freqs + (((int64_t)fbi * a.L + tok) * a.H + h) * kD + 4 * d4);
      const floatx4 rq = rope4(q4, f4);
      const floatx4 rk = rope4(k4, f4);
      const float sq = sum16(rq[0] * rq[0] + rq[1] * rq[1] + rq[2] * rq[2] + rq[3] * rq[3]);
      const float sk = sum16(rk[0] * rk[0] + rk[1] * rk[1] + rk[2] * rk[2] + rk[3] * rk[3]);
      const float fq = 8.0f / fmaxf(sqrtf(sq), 1.0e-12f);
      const float fk = 8.0f / fmaxf(sqrtf(sk), 1.0e-12f);
      floatx4 yq;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        yq[e] = (rq[e] * fq) * gq[e];
        yk[e] = (rk[e] * fk) * gk[e];
      }
      *reinterpret_cast<floatx4*>(a.q + ((int64_t)bh * a.L + tok) * kD + 4 * d4) = yq;
    } else {
      // keep the shuffle participation uniform: the group is inactive as a whole
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kl[tl][4 * d4 + e] = yk[e];
      vl[tl][4 * d4 + e] = v4[e];
    }
  }
  __syncthreads();

  // Transposed, key-contiguous stores: 64 dims x 16 float4 of tokens.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = tid + j * kThreads;
    const int d = idx >> 4;
    const int c = idx & 15;
    const int tok = t0 + 4 * c;
    if (tok >= a.Lpad) continue;
    floatx4 kk, vv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kk[e] = kl[4 * c + e][d];
      vv[e] = vl[4 * c + e][d];
    }
    const int64_t off = ((int64_t)bh * kD + d) * a.Lpad + tok;
    *reinterpret_cast<floatx4*>(a.pk + off) = kk;
    *reinterpret_cast<floatx4*>(a.pv + off) = vv;
  }
}

}  // namespace

int launch_qkv_postprocess(const QkvPostParams& p, hipStream_t stream) {
  PostArgs a{p.qkv, p.freqs, p.q_gamma, p.k_gamma, p.q, p.packed_k, p.packed_v,
             p.B, p.L, p.H, p.L_padded, p.freq_batches};
  const int64_t blocks = (int64_t)p.B * p.H * ((p.L_padded + kTok - 1) / kTok);
  if (blocks <= 0 || blocks > 0x7fffffff) return kErrDims;
  hipLaunchKernelGGL(qkv_postprocess_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace tsplat
