// C-ABI of the flow-block and sampler kernels (block_ops.hip) and of the
// NF24 GEMM with an elementwise epilogue.
//
// The reference-named symbols keep the reference's signatures and status
// codes (scripts/native_norm_rope_avx512.c, native_block_elementwise_avx512.c,
// native_gelu_avx512.c, native_silu_avx512_extra.c, native_sampler_avx512.c):
// pointers are device pointers, `threads` is ignored, the work runs on the
// null stream and the call returns when it is done.  The tsplat_*_async
// forms take a hipStream_t and return after the launch.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "capi_internal.h"
#include "tsplat_common.h"
#include "tsplat_launch.h"
#include "../../include/tsplat_hip.h"

using namespace tsplat;

namespace {

int launched(int st) {
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

int blocking(int st) { return st == kOk ? sync_null_stream() : st; }

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int layernorm_checked(const float* input, const float* weight, const float* bias, float* output,
                      int64_t rows, int cols, float eps, int has_affine, const float* scale,
                      const float* shift, int64_t mod_batch_stride, int64_t rows_per_batch,
                      hipStream_t stream) {
  if (!input || !output) return kErrNull;
  if (rows <= 0 || cols <= 0 || !(eps >= 0.0f)) return kErrDims;
  if (has_affine && (!weight || !bias)) return kErrRange;
  const bool modulate = scale != nullptr || shift != nullptr;
  if (modulate && (!scale || !shift || rows_per_batch <= 0 || mod_batch_stride < cols))
    return kErrRange;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(input, rows * cols * 4));
  TSPLAT_CHECK(ptrs.check(output, rows * cols * 4));
  if (has_affine) {
    TSPLAT_CHECK(ptrs.check(weight, (int64_t)cols * 4));
    TSPLAT_CHECK(ptrs.check(bias, (int64_t)cols * 4));
  }
  if (modulate) {
    const int64_t batches = (rows + rows_per_batch - 1) / rows_per_batch;
    TSPLAT_CHECK(ptrs.check(scale, ((batches - 1) * mod_batch_stride + cols) * 4));
    TSPLAT_CHECK(ptrs.check(shift, ((batches - 1) * mod_batch_stride + cols) * 4));
  }
  LayerNormParams p{input, weight, bias, output, rows, cols, eps, has_affine ? 1 : 0,
                    modulate ? 1 : 0, scale, shift, mod_batch_stride,
                    modulate ? rows_per_batch : 1};
  return launched(launch_layernorm(p, stream));
}

int head_rmsnorm_checked(const float* input, int64_t in_token_stride, const float* gamma,
                         float* output, int B, int L, int H, int dim, float eps, int out_bhld,
                         int normalize, hipStream_t stream) {
  if (!input || !output || (normalize && !gamma)) return kErrNull;
  if (B <= 0 || L <= 0 || H <= 0 || dim <= 0 || !(eps >= 0.0f)) return kErrDims;
  if (in_token_stride < (int64_t)H * dim) return kErrRange;
  const int64_t tokens = (int64_t)B * L;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(input, ((tokens - 1) * in_token_stride + (int64_t)H * dim) * 4));
  TSPLAT_CHECK(ptrs.check(output, tokens * H * dim * 4));
  if (normalize) TSPLAT_CHECK(ptrs.check(gamma, (int64_t)H * dim * 4));
  HeadNormParams p{input, gamma, output, B, L, H, dim, in_token_stride, eps, out_bhld ? 1 : 0,
                   normalize ? 1 : 0};
  return launched(launch_head_rmsnorm(p, stream));
}

int rope_checked(const float* input, const float* freqs, float* output, int64_t vectors, int dim,
                 hipStream_t stream) {
  if (!input || !freqs || !output) return kErrNull;
  if (vectors <= 0 || dim <= 0 || (dim & 1) != 0) return kErrDims;
  const uintptr_t mis = reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(freqs) |
                        reinterpret_cast<uintptr_t>(output);
  if ((mis & 7u) != 0) return kErrAlign;
  const int64_t n = vectors * dim;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(input, n * 4));
  TSPLAT_CHECK(ptrs.check(freqs, n * 4));
  TSPLAT_CHECK(ptrs.check(output, n * 4));
  return launched(launch_rope_complex(input, freqs, output, n / 2, stream));
}

int rows_op_checked(bool gated, float* x, float* y, const float* a, const float* b, int batch,
                    int rows, int cols, hipStream_t stream) {
  if (!x || !a || (gated ? !y : !b)) return kErrNull;
  if (batch <= 0 || rows <= 0 || cols <= 0) return kErrDims;
  const int64_t n = (int64_t)batch * rows * cols;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(x, n * 4));
  TSPLAT_CHECK(ptrs.check(a, (int64_t)batch * cols * 4));
  if (gated) {
    TSPLAT_CHECK(ptrs.check(y, n * 4));
    return launched(launch_gated_residual(x, y, a, batch, rows, cols, stream));
  }
  TSPLAT_CHECK(ptrs.check(b, (int64_t)batch * cols * 4));
  return launched(launch_modulate(x, a, b, batch, rows, cols, stream));
}

int unary_checked(int op, const float* input, float* output, int64_t count, hipStream_t stream) {
  if (!input || !output) return kErrNull;
  if (count <= 0) return kErrDims;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(input, count * 4));
  TSPLAT_CHECK(ptrs.check(output, count * 4));
  switch (op) {
    case 0: return launched(launch_add(output, input, count, stream));
    case 1: return launched(launch_gelu_tanh(input, output, count, stream));
    default: return launched(launch_silu(input, output, count, stream));
  }
}

// op 0: cfg (x = positive, a = negative, s0 = guidance); 1: euler (x = sample,
// a = prediction, s0 = dt); 2: ab2 (+ p = previous prediction, s1 = previous dt).
int sampler_checked(int op, float* x, const float* a, const float* p, const float* s0,
                    const float* s1, int batch, int64_t per_batch, hipStream_t stream) {
  if (!x || !a || !s0 || (op == 2 && (!p || !s1))) return kErrNull;
  if (batch <= 0 || per_batch <= 0) return kErrDims;
  const int64_t n = (int64_t)batch * per_batch;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(x, n * 4));
  TSPLAT_CHECK(ptrs.check(a, n * 4));
  TSPLAT_CHECK(ptrs.check(s0, (int64_t)batch * 4));
  if (op == 0) return launched(launch_cfg_combine(x, a, s0, batch, per_batch, stream));
  if (op == 1) return launched(launch_euler_update(x, a, s0, batch, per_batch, stream));
  TSPLAT_CHECK(ptrs.check(p, n * 4));
  TSPLAT_CHECK(ptrs.check(s1, (int64_t)batch * 4));
  return launched(launch_ab2_update(x, a, p, s0, s1, batch, per_batch, stream));
}

// The NF24 GEMM entries' checks and launch; w_hi / w_lo: the bf16 planes
// of the weights (tsplat_nf24_bf16_planes_async) or null.
int gemm_precision_checked(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                           const float* scale, const float* bias, float* out, int M, int K, int N,
                           int output_start, int output_count, int stride_x, int stride_out,
                           int epilogue, const float* gate, int64_t gate_stride,
                           int rows_per_batch, int precision, const uint16_t* w_hi,
                           const uint16_t* w_lo, hipStream_t stream) {
  if (!x || !code01_t || !q2_t || !scale || !bias || !out) return kErrNull;
  if (M <= 0 || K <= 0 || N <= 0 || output_start < 0 || output_count <= 0) return kErrDims;
  if (output_start + output_count > N || stride_x < K || stride_out < output_count)
    return kErrRange;
  if (epilogue != kEpilogueStore && epilogue != kEpilogueGelu && epilogue != kEpilogueGated &&
      epilogue != kEpilogueAdd)
    return kErrDims;
  if (precision != kPrecisionFp32 && precision != kPrecisionBf16 && precision != kPrecisionBf16x3)
    return kErrDims;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(x, ((int64_t)(M - 1) * stride_x + K) * 4));
  TSPLAT_CHECK(ptrs.check(code01_t, (int64_t)K * N * 2));
  TSPLAT_CHECK(ptrs.check(q2_t, (int64_t)K * N));
  TSPLAT_CHECK(ptrs.check(scale, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(bias, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(out, ((int64_t)(M - 1) * stride_out + output_count) * 4));
  if (epilogue == kEpilogueGated) {
    if (!gate) return kErrNull;
    if (rows_per_batch <= 0 || gate_stride < N) return kErrRange;
    const int64_t batches = ((int64_t)M + rows_per_batch - 1) / rows_per_batch;
    TSPLAT_CHECK(ptrs.check(gate, ((batches - 1) * gate_stride + N) * 4));
  }
  if (w_hi) {
    TSPLAT_CHECK(ptrs.check(w_hi, planes_bytes(K, N)));
    if (precision == kPrecisionBf16x3) TSPLAT_CHECK(ptrs.check(w_lo, planes_bytes(K, N)));
  }
  GemmParams p{x, code01_t, q2_t, scale, bias, out, M, K, N, output_start, output_count,
               stride_x, stride_out, precision};
  p.w_hi = w_hi;
  p.w_lo = precision == kPrecisionBf16x3 ? w_lo : nullptr;
  GemmEpilogueParams e{epilogue, gate, gate_stride, rows_per_batch > 0 ? rows_per_batch : 1};
  return launched(launch_nf24_gemm_epilogue(p, e, stream));
}

}  // namespace

extern "C" {

// ------------------------------------------------------- reference-named
int triposplat_layernorm_f32_avx512(const float* input, const float* weight, const float* bias,
                                    float* output, int64_t rows, int cols, float eps,
                                    int has_affine, int threads) {
  (void)threads;
  return blocking(layernorm_checked(input, weight, bias, output, rows, cols, eps, has_affine,
                                    nullptr, nullptr, 0, 1, nullptr));
}

int triposplat_multihead_rmsnorm_f32_avx512(const float* input, const float* gamma, float* output,
                                            int64_t outer, int heads, int dim, float eps,
                                            int threads) {
  (void)threads;
  if (!input || !gamma || !output) return kErrNull;
  if (outer <= 0 || outer > 0x7fffffff || heads <= 0 || dim <= 0 || !(eps >= 0.0f))
    return kErrDims;
  return blocking(head_rmsnorm_checked(input, (int64_t)heads * dim, gamma, output, 1, (int)outer,
                                       heads, dim, eps, 0, 1, nullptr));
}

int triposplat_rope_complex_f32_avx512(const float* input, const float* freqs_interleaved,
                                       float* output, int64_t vectors, int dim, int threads) {
  (void)threads;
  return blocking(rope_checked(input, freqs_interleaved, output, vectors, dim, nullptr));
}

int triposplat_modulate_inplace_f32_avx512(float* h, const float* scale, const float* shift,
                                           int batch, int rows, int cols, int threads) {
  (void)threads;
  if (!h || !scale || !shift) return kErrNull;
  return blocking(rows_op_checked(false, h, nullptr, scale, shift, batch, rows, cols, nullptr));
}

int triposplat_gated_residual_inplace_f32_avx512(float* base, float* delta, const float* gate,
                                                 int batch, int rows, int cols, int threads) {
  (void)threads;
  if (!base || !delta || !gate) return kErrNull;
  return blocking(rows_op_checked(true, base, delta, gate, nullptr, batch, rows, cols, nullptr));
}

int triposplat_add_inplace_f32_avx512(float* base, const float* delta, int64_t count,
                                      int threads) {
  (void)threads;
  if (!base || !delta) return kErrNull;
  return blocking(unary_checked(0, delta, base, count, nullptr));
}

int triposplat_gelu_tanh_f32_avx512(const float* input, float* output, int64_t count,
                                    int threads) {
  (void)threads;
  return blocking(unary_checked(1, input, output, count, nullptr));
}

int triposplat_silu_f32_avx512(const float* input, float* output, int64_t count, int threads) {
  (void)threads;
  return blocking(unary_checked(2, input, output, count, nullptr));
}

int triposplat_cfg_combine_inplace_f32_avx512(float* positive, const float* negative,
                                              const float* guidance, int batch,
                                              int64_t elements_per_batch, int threads) {
  (void)threads;
  return blocking(sampler_checked(0, positive, negative, nullptr, guidance, nullptr, batch,
                                  elements_per_batch, nullptr));
}

int triposplat_euler_update_inplace_f32_avx512(float* sample, const float* prediction,
                                               const float* dt, int batch,
                                               int64_t elements_per_batch, int threads) {
  (void)threads;
  return blocking(sampler_checked(1, sample, prediction, nullptr, dt, nullptr, batch,
                                  elements_per_batch, nullptr));
}

int triposplat_ab2_update_inplace_f32_avx512(float* sample, const float* prediction,
                                             const float* previous_prediction, const float* dt,
                                             const float* previous_dt, int batch,
                                             int64_t elements_per_batch, int threads) {
  (void)threads;
  return blocking(sampler_checked(2, sample, prediction, previous_prediction, dt, previous_dt,
                                  batch, elements_per_batch, nullptr));
}

// ---------------------------------------------------------------- async
int tsplat_layernorm_modulate_async(const float* input, const float* weight, const float* bias,
                                    float* output, int64_t rows, int cols, float eps,
                                    int has_affine, const float* scale, const float* shift,
                                    int64_t mod_batch_stride, int64_t rows_per_batch,
                                    void* stream) {
  return layernorm_checked(input, weight, bias, output, rows, cols, eps, has_affine, scale, shift,
                           mod_batch_stride, rows_per_batch, as_stream(stream));
}

int tsplat_head_rmsnorm_async(const float* input, int64_t in_token_stride, const float* gamma,
                              float* output, int B, int L, int H, int dim, float eps,
                              int out_bhld, int normalize, void* stream) {
  return head_rmsnorm_checked(input, in_token_stride, gamma, output, B, L, H, dim, eps, out_bhld,
                              normalize, as_stream(stream));
}

int tsplat_rope_complex_async(const float* input, const float* freqs_interleaved, float* output,
                              int64_t vectors, int dim, void* stream) {
  return rope_checked(input, freqs_interleaved, output, vectors, dim, as_stream(stream));
}

int tsplat_modulate_async(float* h, const float* scale, const float* shift, int batch, int rows,
                          int cols, void* stream) {
  if (!h || !scale || !shift) return kErrNull;
  return rows_op_checked(false, h, nullptr, scale, shift, batch, rows, cols, as_stream(stream));
}

int tsplat_gated_residual_async(float* base, float* delta, const float* gate, int batch, int rows,
                                int cols, void* stream) {
  if (!base || !delta || !gate) return kErrNull;
  return rows_op_checked(true, base, delta, gate, nullptr, batch, rows, cols, as_stream(stream));
}

int tsplat_add_async(float* base, const float* delta, int64_t count, void* stream) {
  if (!base || !delta) return kErrNull;
  return unary_checked(0, delta, base, count, as_stream(stream));
}

int tsplat_gelu_tanh_async(const float* input, float* output, int64_t count, void* stream) {
  return unary_checked(1, input, output, count, as_stream(stream));
}

int tsplat_silu_async(const float* input, float* output, int64_t count, void* stream) {
  return unary_checked(2, input, output, count, as_stream(stream));
}

int tsplat_cfg_combine_async(float* positive, const float* negative, const float* guidance,
                             int batch, int64_t elements_per_batch, void* stream) {
  return sampler_checked(0, positive, negative, nullptr, guidance, nullptr, batch,
                         elements_per_batch, as_stream(stream));
}

int tsplat_euler_update_async(float* sample, const float* prediction, const float* dt, int batch,
                              int64_t elements_per_batch, void* stream) {
  return sampler_checked(1, sample, prediction, nullptr, dt, nullptr, batch, elements_per_batch,
                         as_stream(stream));
}

int tsplat_ab2_update_async(float* sample, const float* prediction,
                            const float* previous_prediction, const float* dt,
                            const float* previous_dt, int batch, int64_t elements_per_batch,
                            void* stream) {
  return sampler_checked(2, sample, prediction, previous_prediction, dt, previous_dt, batch,
                         elements_per_batch, as_stream(stream));
}

int tsplat_nf24_gemm_planes_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                  const float* scale, const float* bias, float* out, int M, int K,
                                  int N, int output_start, int output_count, int stride_x,
                                  int stride_out, int epilogue, const float* gate,
                                  int64_t gate_stride, int rows_per_batch, int precision,
                                  const uint16_t* w_hi, const uint16_t* w_lo, void* stream) {
  if (!w_hi || (precision == kPrecisionBf16x3 && !w_lo)) return kErrNull;
  return gemm_precision_checked(x, code01_t, q2_t, scale, bias, out, M, K, N, output_start,
                                output_count, stride_x, stride_out, epilogue, gate, gate_stride,
                                rows_per_batch, precision, w_hi, w_lo, as_stream(stream));
}

int tsplat_nf24_gemm_precision_async(const float* x, const int16_t* code01_t,
                                     const int8_t* q2_t, const float* scale, const float* bias,
                                     float* out, int M, int K, int N, int output_start,
                                     int output_count, int stride_x, int stride_out, int epilogue,
                                     const float* gate, int64_t gate_stride, int rows_per_batch,
                                     int precision, void* stream) {
  return gemm_precision_checked(x, code01_t, q2_t, scale, bias, out, M, K, N, output_start,
                                output_count, stride_x, stride_out, epilogue, gate, gate_stride,
                                rows_per_batch, precision, nullptr, nullptr, as_stream(stream));
}

int tsplat_nf24_gemm_epilogue_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                    const float* scale, const float* bias, float* out, int M,
                                    int K, int N, int output_start, int output_count,
                                    int stride_x, int stride_out, int epilogue, const float* gate,
                                    int64_t gate_stride, int rows_per_batch, void* stream) {
  return tsplat_nf24_gemm_precision_async(x, code01_t, q2_t, scale, bias, out, M, K, N,
                                          output_start, output_count, stride_x, stride_out,
                                          epilogue, gate, gate_stride, rows_per_batch,
                                          kPrecisionFp32, stream);
}

}  // extern "C"
