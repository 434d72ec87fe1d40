// Scalar device forms of the reference's AVX-512 elementwise arithmetic.
//
// Each function performs the same fp32 operations, in the same order and
// with the same fused multiply-adds, as one lane of the reference kernel it
// cites, so the device results are bit-identical to the reference build.
// Contraction is switched off inside each body: a fused multiply-add appears
// only where the reference has one (an explicit _mm512_fmadd_ps, or one GCC
// forms at -O3 -mfma, where noted).  Division and sqrtf are correctly
// rounded on gfx950 (hipcc's default), as vdivps / vsqrtps are.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsplat {

// Cephes-style exp: scripts/native_gelu_avx512.c:9-31 (the same polynomial as
// native_sdpa_avx512_exact_q8t512.c:102-131 and native_silu_avx512_extra.c).
// The clamps keep x86 minps/maxps semantics (the second operand on NaN).
__device__ __forceinline__ float exp_cephes(float x) {
#pragma clang fp contract(off)
  x = (x < 88.3762626647949f) ? x : 88.3762626647949f;
  x = (x > -88.3762626647949f) ? x : -88.3762626647949f;
  const float fx = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
  x = fmaf(-fx, 0.693359375f, x);
  x = fmaf(-fx, -2.12194440e-4f, x);
  const float z = x * x;
  float y = 1.9875691500e-4f;
  y = fmaf(y, x, 1.3981999507e-3f);
  y = fmaf(y, x, 8.3334519073e-3f);
  y = fmaf(y, x, 4.1665795894e-2f);
  y = fmaf(y, x, 1.6666665459e-1f);
  y = fmaf(y, x, 5.0000001201e-1f);
  y = fmaf(y, z, x) + 1.0f;
  const int32_t e = ((int32_t)fx + 0x7f) << 23;
  return y * __int_as_float(e);
}

// GELU, tanh form: native_gelu_avx512.c:33-68.  GCC contracts
// x + 0.044715 * (x^2 * x) into one fma at -O3 -mfma (checked against the
// reference build); tanh(u) = sign(u) * (1 - 2 / (exp(2|u|) + 1)), 0 at u = 0.
__device__ __forceinline__ float gelu_tanh_ref(float x) {
#pragma clang fp contract(off)
  const float x2 = x * x;
  const float s = fmaf(0.044715f, x2 * x, x);
  const float inner = 0.7978845608028654f * s;
  const float e = exp_cephes(2.0f * fabsf(inner));
  float t = 1.0f - 2.0f / (e + 1.0f);
  t = copysignf(t, inner);
  if (inner == 0.0f) t = 0.0f;
  return (0.5f * x) * (1.0f + t);
}

// SiLU: native_silu_avx512_extra.c: x / (1 + exp(0 - x)).
__device__ __forceinline__ float silu_ref(float x) {
#pragma clang fp contract(off)
  return x / (1.0f + exp_cephes(0.0f - x));
}

// Gated residual of native_block_elementwise_avx512.c:24-35 for one element:
// h = delta * gate (rounded), then base + h -- never one fma.
__device__ __forceinline__ float gated_residual_ref(float base, float delta, float gate) {
#pragma clang fp contract(off)
  const float h = delta * gate;
  return base + h;
}

// Horizontal sum of the 16 lanes of an aligned 16-lane group in the order of
// GCC's _mm512_reduce_add_ps (lane i + lane i^8, then ^4, ^2, ^1); every lane
// of the group receives the sum.
__device__ __forceinline__ float reduce_add16(float v) {
#pragma clang fp contract(off)
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

}  // namespace tsplat
