// NF24 weight packer for gfx950: fp32 W [out, in] -> code01_t int16 [in, out],
// q2_t int8 [in, out], scale fp32 [out].
//
// Reference semantics: scripts/native_linear_rnf8_avx512_patch.py:14-87
// (quantize_nf24_per_output_channel / _i16), every step in fp32 with one
// rounding per operation, as torch's CPU elementwise kernels do:
//   base  = max(max_k |w[n,k]|, FLT_MIN) / 127
//   q0    = alphabet[#{mid < w/base}]        (bucketize, ties to the lower level)
//   r1    = w - q0*base;        q1 = clamp(floor(r1/(base/4)    + 0.5), -128, 127)
//   r2    = r1 - q1*(base/4);   q2 = clamp(floor(r2/(base/1024) + 0.5), -128, 127)
//   code01 = 4*q0 + q1,  scale = base/1024.
// Contraction is disabled so that no multiply is fused into a subtraction.

#include <float.h>

#include "tsplat_common.h"
#include "tsplat_launch.h"

namespace tsplat {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxAlphabet = 256;

__global__ __launch_bounds__(kThreads) void nf24_rowscale_kernel(const float* w, int in_f,
                                                                 float* base_out,
                                                                 float* scale_out) {
#pragma clang fp contract(off)
  __shared__ float red[kThreads / 64];
  const int n = blockIdx.x;
  const float* row = w + (int64_t)n * in_f;
  float m = 0.0f;
  for (int k = threadIdx.x; k < in_f; k += kThreads) m = fmaxf(m, fabsf(row[k]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kThreads / 64; ++i) m = fmaxf(m, red[i]);
    m = fmaxf(red[0], m);
    const float base = fmaxf(m, FLT_MIN) / 127.0f;
    base_out[n] = base;
    scale_out[n] = base / 1024.0f;
  }
}

// 32 output rows x 64 input columns per block; codes are transposed through
// LDS so both the fp32 reads and the [in, out] code writes are coalesced.
__global__ __launch_bounds__(kThreads) void nf24_quantize_kernel(
    const float* w, const float* base_in, const float* alphabet, int alphabet_len, int out_f,
    int in_f, int16_t* code01_t, int8_t* q2_t) {
#pragma clang fp contract(off)
  __shared__ float alpha[kMaxAlphabet];
  __shared__ float mid[kMaxAlphabet];
  __shared__ int16_t c01[64][33];
  __shared__ int8_t c2[64][33];
  for (int i = threadIdx.x; i < alphabet_len; i += kThreads) alpha[i] = alphabet[i];
  __syncthreads();
  for (int i = threadIdx.x; i + 1 < alphabet_len; i += kThreads)
    mid[i] = (alpha[i] + alpha[i + 1]) * 0.5f;
  __syncthreads();

  const int tiles_k = (in_f + 63) / 64;
  const int n0 = (blockIdx.x / tiles_k) * 32;
  const int k0 = (blockIdx.x % tiles_k) * 64;
  const int nmid = alphabet_len - 1;

  for (int e = threadIdx.x; e < 32 * 64; e += kThreads) {
    const int nl = e / 64, kl = e % 64;
    const int n = n0 + nl, k = k0 + kl;
    int16_t code = 0;
    int8_t q2c = 0;
    if (n < out_f && k < in_f) {
      const float x = w[(int64_t)n * in_f + k];
      const float base = base_in[n];
      const float v = x / base;
      int lo = 0, hi = nmid;  // first index with v <= mid[index]
      while (lo < hi) {
        const int m = (lo + hi) >> 1;
        if (mid[m] < v) lo = m + 1; else hi = m;
      }
      const float q0 = alpha[lo];
      const float p0 = q0 * base;
      const float r1 = x - p0;
      const float s1 = base / 4.0f;
      const float q1 = fminf(fmaxf(floorf(r1 / s1 + 0.5f), -128.0f), 127.0f);
      const float p1 = q1 * s1;
      const float r2 = r1 - p1;
      const float fs = base / 1024.0f;
      const float q2 = fminf(fmaxf(floorf(r2 / fs + 0.5f), -128.0f), 127.0f);
      code = (int16_t)((int)q0 * 4 + (int)q1);
      q2c = (int8_t)(int)q2;
    }
    c01[kl][nl] = code;
    c2[kl][nl] = q2c;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 32 * 64; e += kThreads) {
    const int kl = e / 32, nl = e % 32;
    const int n = n0 + nl, k = k0 + kl;
    if (n < out_f && k < in_f) {
      code01_t[(int64_t)k * out_f + n] = c01[kl][nl];
      q2_t[(int64_t)k * out_f + n] = c2[kl][nl];
    }
  }
}

// Exact decode (scripts/native_linear_nf24_prepacked.py:17-36): w = fp32(256 *
// q01 + q2) * scale[n] (the integer is exact in fp32, one rounding in the
// multiply), written [in, out] like the codes or transposed to [out, in]
// through a 64 x 64 LDS tile so both sides stay coalesced.
template <bool kTransposed>
__global__ __launch_bounds__(kThreads) void nf24_decode_kernel(const int16_t* code01_t,
                                                               const int8_t* q2_t,
                                                               const float* scale, float* out,
                                                               int in_f, int out_f) {
#pragma clang fp contract(off)
  __shared__ float tile[64][65];
  const int tiles_n = (out_f + 63) / 64;
  const int k0 = (blockIdx.x / tiles_n) * 64;
  const int n0 = (blockIdx.x % tiles_n) * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += kThreads) {
    const int kl = e / 64, nl = e % 64;
    const int k = k0 + kl, n = n0 + nl;
    if (k < in_f && n < out_f) {
      const int64_t i = (int64_t)k * out_f + n;
      const float w = (float)((int32_t)code01_t[i] * 256 + (int32_t)q2_t[i]) * scale[n];
      if (kTransposed)
        tile[nl][kl] = w;
      else
        out[i] = w;
    }
  }
  if (!kTransposed) return;
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += kThreads) {
    const int nl = e / 64, kl = e % 64;
    const int k = k0 + kl, n = n0 + nl;
    if (k < in_f && n < out_f) out[(int64_t)n * in_f + k] = tile[nl][kl];
  }
}

}  // namespace

int launch_nf24_decode(const int16_t* code01_t, const int8_t* q2_t, const float* scale, float* out,
                       int in_f, int out_f, int transposed, hipStream_t stream) {
  if (in_f <= 0 || out_f <= 0) return kErrDims;
  const int64_t blocks = (int64_t)((in_f + 63) / 64) * ((out_f + 63) / 64);
  if (blocks > 0x7fffffff) return kErrDims;
  if (transposed)
    hipLaunchKernelGGL((nf24_decode_kernel<true>), dim3((unsigned)blocks), dim3(kThreads), 0,
                       stream, code01_t, q2_t, scale, out, in_f, out_f);
  else
    hipLaunchKernelGGL((nf24_decode_kernel<false>), dim3((unsigned)blocks), dim3(kThreads), 0,
                       stream, code01_t, q2_t, scale, out, in_f, out_f);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int launch_nf24_pack(const float* w, int out_f, int in_f, const float* alphabet, int alphabet_len,
                     float* base_tmp, int16_t* code01_t, int8_t* q2_t, float* scale,
                     hipStream_t stream) {
  if (alphabet_len < 2 || alphabet_len > kMaxAlphabet) return kErrDims;
  hipLaunchKernelGGL(nf24_rowscale_kernel, dim3(out_f), dim3(kThreads), 0, stream, w, in_f,
                     base_tmp, scale);
  const int64_t blocks = (int64_t)((out_f + 31) / 32) * ((in_f + 63) / 64);
  if (blocks > 0x7fffffff) return kErrDims;
  hipLaunchKernelGGL(nf24_quantize_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, w,
                     base_tmp, alphabet, alphabet_len, out_f, in_f, code01_t, q2_t);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace tsplat
