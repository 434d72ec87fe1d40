// Flow-block and sampler elementwise kernels for gfx950: LayerNorm (+ adaLN
// modulation), multi-head RMSNorm (+ the [B,L,H,D] -> [B,H,L,D] permute),
// complex RoPE, modulation, gated residual, add, GELU-tanh, SiLU, and the
// CFG / Euler / AB2 sampler updates.
//
// Reference semantics (bit-identical per element; see tsplat_ew.h):
//   scripts/native_norm_rope_avx512.c:13-119,
//   scripts/native_block_elementwise_avx512.c:9-46,
//   scripts/native_gelu_avx512.c:44-68, scripts/native_silu_avx512_extra.c,
//   scripts/native_sampler_avx512.c:19-160.
// The reductions follow the reference's lane order: a row is read by a
// 16-lane group, lane j owning columns j, j+16, j+32, ... (the j-th lane of
// the AVX-512 accumulator), summed sequentially, then combined in
// _mm512_reduce_add_ps order.  All of these kernels are HBM-bound.

#include "tsplat_common.h"
#include "tsplat_ew.h"
#include "tsplat_launch.h"

#pragma clang fp contract(off)

namespace tsplat {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 16;
constexpr int kMaxChunks = 64;  // rows up to 1024 columns stay in registers

// LayerNorm of one row per 16-lane group (native_norm_rope_avx512.c:13-49),
// optionally followed by the modulation h * (1 + scale[b]) + shift[b]
// (native_block_elementwise_avx512.c:9-22, fused by GCC into one fma).
// The variance sums (x - mean)^2 over every lane of every 16-column chunk,
// so a partial last chunk adds mean^2 per masked lane, as the reference does.
__global__ __launch_bounds__(kThreads) void layernorm_kernel(LayerNormParams a) {
  const int tid = threadIdx.x;
  const int j = tid & 15;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (tid >> 4);
  const bool live = row < a.rows;  // uniform over the 16-lane group
  const float* src = a.input + (live ? row : 0) * (int64_t)a.cols;
  const int nch = (a.cols + 15) >> 4;

  float v[kMaxChunks];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    if (i < nch) {
      const int c = 16 * i + j;
      v[i] = (live && c < a.cols) ? src[c] : 0.0f;
      sum += v[i];
    }
  }
  for (int i = kMaxChunks; i < nch; ++i) {
    const int c = 16 * i + j;
    sum += (live && c < a.cols) ? src[c] : 0.0f;
  }
  const float mean = reduce_add16(sum) / (float)a.cols;

  float var = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    if (i < nch) {
      const float d = v[i] - mean;
      var = fmaf(d, d, var);
    }
  }
  for (int i = kMaxChunks; i < nch; ++i) {
    const int c = 16 * i + j;
    const float d = ((live && c < a.cols) ? src[c] : 0.0f) - mean;
    var = fmaf(d, d, var);
  }
  const float inv_std = 1.0f / sqrtf(reduce_add16(var) / (float)a.cols + a.eps);
  if (!live) return;

  float* dst = a.output + row * (int64_t)a.cols;
  const int64_t b = a.modulate ? row / a.rows_per_batch : 0;
  const float* sc = a.modulate ? a.scale + b * a.mod_batch_stride : nullptr;
  const float* sh = a.modulate ? a.shift + b * a.mod_batch_stride : nullptr;
  auto emit = [&](int c, float x) {
    float y = (x - mean) * inv_std;
    if (a.affine) y = fmaf(y, a.weight[c], a.bias[c]);
    if (a.modulate) y = fmaf(y, 1.0f + sc[c], sh[c]);
    dst[c] = y;
  };
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = 16 * i + j;
    if (i < nch && c < a.cols) emit(c, v[i]);
  }
  for (int i = kMaxChunks; i < nch; ++i) {
    const int c = 16 * i + j;
    if (c < a.cols) emit(c, src[c]);
  }
}

// layernorm_kernel for rows of at most kVecMaxCols columns, a multiple of 4,
// with 16-byte aligned operands.  A 16-lane group stages its row in LDS from
// 128-bit loads (256 contiguous bytes per instruction and group), all issued
// before the first is used; reads it back in the reference's lane order
// (lane j: columns j, j + 16, ...) for the two sums; and writes the result
// with 128-bit stores, half a row at a time with that half's column
// parameters loaded first.  The same per-element arithmetic and summation
// order as layernorm_kernel, so the same bits.  Rows are padded in LDS by 16
// floats so that the four groups of a wave read 64 distinct banks.
// (Measured against a resident-workgroup form that walks the rows with the
// next row prefetched into registers: that one is 1.8-2x slower.)
constexpr int kVecMaxCols = 1024;
constexpr int kVecRowStride = kVecMaxCols + 16;
constexpr int kVecIters = kVecMaxCols / 64;  // float4 units per lane of a full row
__global__ __launch_bounds__(kThreads) void layernorm_vec_kernel(LayerNormParams a) {
  __shared__ __attribute__((aligned(16))) float rows_lds[kRowsPerBlock * kVecRowStride];
  const int tid = threadIdx.x;
  const int j = tid & 15;
  const int grp = tid >> 4;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + grp;
  const bool live = row < a.rows;  // uniform over the 16-lane group
  float* lrow = rows_lds + grp * kVecRowStride;
  const int nch = (a.cols + 15) >> 4;
  const int nf4 = a.cols >> 2;
  // Units past the row re-read unit 0 and rows past the end row 0, so no
  // select waits on a load.
  const floatx4* src = reinterpret_cast<const floatx4*>(a.input + (live ? row : 0) * (int64_t)a.cols);
  floatx4 xr[kVecIters];
#pragma unroll
  for (int i = 0; i < kVecIters; ++i) {
    const int f = j + 16 * i;
    xr[i] = src[f < nf4 ? f : 0];
  }
#pragma unroll
  for (int i = 0; i < kVecIters; ++i) {
    const int f = j + 16 * i;
    if (f < nf4) *reinterpret_cast<floatx4*>(&lrow[4 * f]) = xr[i];
  }
  // the reference's partial last chunk reads zeros past cols
  if (16 * (nch - 1) + j >= a.cols) lrow[16 * (nch - 1) + j] = 0.0f;
  __syncthreads();

  float v[kMaxChunks];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    if (i < nch) {
      v[i] = lrow[16 * i + j];
      sum += v[i];
    }
  }
  const float mean = reduce_add16(sum) / (float)a.cols;
  float var = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    if (i < nch) {
      const float d = v[i] - mean;
      var = fmaf(d, d, var);
    }
  }
  const float inv_std = 1.0f / sqrtf(reduce_add16(var) / (float)a.cols + a.eps);
  if (!live) return;

  floatx4* dst = reinterpret_cast<floatx4*>(a.output + row * (int64_t)a.cols);
  const int64_t b = a.modulate ? row / a.rows_per_batch : 0;
  const floatx4* sc = a.modulate ? reinterpret_cast<const floatx4*>(a.scale + b * a.mod_batch_stride) : nullptr;
  const floatx4* sh = a.modulate ? reinterpret_cast<const floatx4*>(a.shift + b * a.mod_batch_stride) : nullptr;
  const floatx4* wt = a.affine ? reinterpret_cast<const floatx4*>(a.weight) : nullptr;
  const floatx4* bs = a.affine ? reinterpret_cast<const floatx4*>(a.bias) : nullptr;
  constexpr int kHalf = kVecIters / 2;
#pragma unroll
  for (int h0 = 0; h0 < kVecIters; h0 += kHalf) {
    floatx4 w4[kHalf], b4[kHalf], s4[kHalf], t4[kHalf];
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int f = j + 16 * (h0 + i);
      const int fc = f < nf4 ? f : 0;
      if (a.affine) {
        w4[i] = wt[fc];
        b4[i] = bs[fc];
      }
      if (a.modulate) {
        s4[i] = sc[fc];
        t4[i] = sh[fc];
      }
    }
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int f = j + 16 * (h0 + i);
      if (f >= nf4) continue;
      const floatx4 x = *reinterpret_cast<const floatx4*>(&lrow[4 * f]);
      floatx4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float z = (x[e] - mean) * inv_std;
        if (a.affine) z = fmaf(z, w4[i][e], b4[i][e]);
        if (a.modulate) z = fmaf(z, 1.0f + s4[i][e], t4[i][e]);
        y[e] = z;
      }
      dst[f] = y;
    }
  }
}

// Multi-head RMSNorm of one [dim] vector per 16-lane group
// (native_norm_rope_avx512.c:51-83): y = x * (sqrt(dim) / max(||x||, eps)) * gamma[h].
// Vector (b, l, h) is read at in + (b*L + l) * in_token_stride + h*dim and
// written to [B, L, H, dim] or, with out_bhld, [B, H, L, dim]; with
// normalize = 0 the vector is only moved (the v half of a fused k/v projection).
__global__ __launch_bounds__(kThreads) void head_rmsnorm_kernel(HeadNormParams a) {
  const int tid = threadIdx.x;
  const int j = tid & 15;
  const int64_t vec = (int64_t)blockIdx.x * kRowsPerBlock + (tid >> 4);
  const int64_t nvec = (int64_t)a.B * a.L * a.H;
  if (vec >= nvec) return;  // uniform over the 16-lane group
  const int h = (int)(vec % a.H);
  const int64_t bl = vec / a.H;
  const int64_t b = bl / a.L, l = bl % a.L;
  const float* src = a.input + bl * a.in_token_stride + (int64_t)h * a.dim;
  float* dst = a.output + (a.out_bhld ? ((b * a.H + h) * a.L + l) * a.dim : vec * a.dim);
  const int nch = (a.dim + 15) >> 4;
  if (!a.normalize) {
    for (int i = 0; i < nch; ++i) {
      const int d = 16 * i + j;
      if (d < a.dim) dst[d] = src[d];
    }
    return;
  }
  float ss = 0.0f;
  for (int i = 0; i < nch; ++i) {
    const int d = 16 * i + j;
    const float x = d < a.dim ? src[d] : 0.0f;
    ss = fmaf(x, x, ss);
  }
  const float norm = sqrtf(reduce_add16(ss));
  const float factor = sqrtf((float)a.dim) / fmaxf(norm, a.eps);
  const float* g = a.gamma + (int64_t)h * a.dim;
  for (int i = 0; i < nch; ++i) {
    const int d = 16 * i + j;
    if (d < a.dim) dst[d] = (src[d] * factor) * g[d];
  }
}

// Complex RoPE over interleaved (re, im) pairs (native_norm_rope_avx512.c:85-119):
// y_re = fma(x_re, f_re, -(x_im * f_im)), y_im = fma(x_re, f_im, x_im * f_re).
__global__ __launch_bounds__(kThreads) void rope_complex_kernel(const float* in, const float* f,
                                                               float* out, int64_t pairs) {
  const int64_t p = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (p >= pairs) return;
  const float2 x = reinterpret_cast<const float2*>(in)[p];
  const float2 w = reinterpret_cast<const float2*>(f)[p];
  float2 y;
  y.x = fmaf(x.x, w.x, -(x.y * w.y));
  y.y = fmaf(x.x, w.y, x.y * w.x);
  reinterpret_cast<float2*>(out)[p] = y;
}

// The elementwise updates.  Element i of a [batch, rows, cols] (or [batch,
// per_batch]) array; per-batch operands are rows of length cols (or one
// scalar per batch).
enum EwOp : int { kOpModulate, kOpGated, kOpAdd, kOpGelu, kOpSilu, kOpCfg, kOpEuler, kOpAb2 };

struct EwArgs {
  float* x;         // in/out (modulate h, gated/add base, cfg positive, euler/ab2 sample)
  float* y;         // gated: delta (in/out); gelu/silu: output
  const float* a0;  // modulate scale | gated gate | add delta | gelu/silu input | cfg negative | euler/ab2 prediction
  const float* a1;  // modulate shift | cfg guidance | euler/ab2 dt | ab2 previous prediction
  const float* a2;  // ab2 previous dt
  const float* a3;  // ab2 dt
  int64_t n;        // elements
  int64_t inner;    // elements per batch (modulate/gated: rows * cols)
  int cols;
};

template <int kOp>
__device__ __forceinline__ void ew_one(const EwArgs& a, int64_t i) {
  if constexpr (kOp == kOpModulate) {
    const int64_t b = i / a.inner;
    const int64_t c = b * a.cols + i % a.cols;
    a.x[i] = fmaf(a.x[i], 1.0f + a.a0[c], a.a1[c]);
  } else if constexpr (kOp == kOpGated) {
    const int64_t c = (i / a.inner) * a.cols + i % a.cols;
    const float hv = a.y[i] * a.a0[c];
    a.y[i] = hv;
    a.x[i] = a.x[i] + hv;
  } else if constexpr (kOp == kOpAdd) {
    a.x[i] = a.x[i] + a.a0[i];
  } else if constexpr (kOp == kOpGelu) {
    a.y[i] = gelu_tanh_ref(a.a0[i]);
  } else if constexpr (kOp == kOpSilu) {
    a.y[i] = silu_ref(a.a0[i]);
  } else if constexpr (kOp == kOpCfg) {
    const float g = a.a1[i / a.inner];
    const float gm1 = g - 1.0f;
    a.x[i] = g * a.x[i] - gm1 * a.a0[i];
  } else if constexpr (kOp == kOpEuler) {
    a.x[i] = a.x[i] - a.a1[i / a.inner] * a.a0[i];
  } else {
    const int64_t b = i / a.inner;
    const float dt = a.a3[b];
    const float half_ratio = 0.5f * (dt / fmaxf(a.a2[b], 1.0e-12f));
    const float current_scale = 1.0f + half_ratio;
    const float effective = current_scale * a.a0[i] - half_ratio * a.a1[i];
    a.x[i] = a.x[i] - dt * effective;
  }
}

template <int kOp>
__global__ __launch_bounds__(kThreads) void ew_kernel(EwArgs a) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < a.n; i += stride)
    ew_one<kOp>(a, i);
}

unsigned ew_blocks(int64_t n) {
  // enough waves to cover HBM latency; the grid-stride loop takes the rest
  const int64_t want = (n + kThreads - 1) / kThreads;
  return (unsigned)(want < 65536 ? want : 65536);
}

template <int kOp>
int launch_ew(const EwArgs& a, hipStream_t stream) {
  if (a.n <= 0) return kErrDims;
  hipLaunchKernelGGL((ew_kernel<kOp>), dim3(ew_blocks(a.n)), dim3(kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace

int launch_layernorm(const LayerNormParams& p, hipStream_t stream) {
  if (p.rows <= 0 || p.cols <= 0) return kErrDims;
  const int64_t blocks = (p.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7fffffff) return kErrDims;
  auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool vec = p.cols % 4 == 0 && p.cols <= kVecMaxCols && al16(p.input) && al16(p.output) &&
                   (!p.affine || (al16(p.weight) && al16(p.bias))) &&
                   (!p.modulate || (al16(p.scale) && al16(p.shift) && p.mod_batch_stride % 4 == 0));
  if (vec)
    hipLaunchKernelGGL(layernorm_vec_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(layernorm_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, p);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int launch_head_rmsnorm(const HeadNormParams& p, hipStream_t stream) {
  const int64_t nvec = (int64_t)p.B * p.L * p.H;
  if (nvec <= 0 || p.dim <= 0) return kErrDims;
  const int64_t blocks = (nvec + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7fffffff) return kErrDims;
  hipLaunchKernelGGL(head_rmsnorm_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, p);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int launch_rope_complex(const float* in, const float* f, float* out, int64_t pairs,
                        hipStream_t stream) {
  if (pairs <= 0) return kErrDims;
  const int64_t blocks = (pairs + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return kErrDims;
  hipLaunchKernelGGL(rope_complex_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, in, f,
                     out, pairs);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int launch_modulate(float* h, const float* scale, const float* shift, int batch, int rows, int cols,
                    hipStream_t stream) {
  EwArgs a{h, nullptr, scale, shift, nullptr, nullptr, (int64_t)batch * rows * cols,
           (int64_t)rows * cols, cols};
  return launch_ew<kOpModulate>(a, stream);
}

int launch_gated_residual(float* base, float* delta, const float* gate, int batch, int rows,
                          int cols, hipStream_t stream) {
  EwArgs a{base, delta, gate, nullptr, nullptr, nullptr, (int64_t)batch * rows * cols,
           (int64_t)rows * cols, cols};
  return launch_ew<kOpGated>(a, stream);
}

int launch_add(float* base, const float* delta, int64_t count, hipStream_t stream) {
  EwArgs a{base, nullptr, delta, nullptr, nullptr, nullptr, count, count, 1};
  return launch_ew<kOpAdd>(a, stream);
}

int launch_gelu_tanh(const float* in, float* out, int64_t count, hipStream_t stream) {
  EwArgs a{nullptr, out, in, nullptr, nullptr, nullptr, count, count, 1};
  return launch_ew<kOpGelu>(a, stream);
}

int launch_silu(const float* in, float* out, int64_t count, hipStream_t stream) {
  EwArgs a{nullptr, out, in, nullptr, nullptr, nullptr, count, count, 1};
  return launch_ew<kOpSilu>(a, stream);
}

int launch_cfg_combine(float* positive, const float* negative, const float* guidance, int batch,
                       int64_t per_batch, hipStream_t stream) {
  EwArgs a{positive, nullptr, negative, guidance, nullptr, nullptr, (int64_t)batch * per_batch,
           per_batch, 1};
  return launch_ew<kOpCfg>(a, stream);
}

int launch_euler_update(float* sample, const float* prediction, const float* dt, int batch,
                        int64_t per_batch, hipStream_t stream) {
  EwArgs a{sample, nullptr, prediction, dt, nullptr, nullptr, (int64_t)batch * per_batch,
           per_batch, 1};
  return launch_ew<kOpEuler>(a, stream);
}

int launch_ab2_update(float* sample, const float* prediction, const float* previous_prediction,
                      const float* dt, const float* previous_dt, int batch, int64_t per_batch,
                      hipStream_t stream) {
  EwArgs a{sample, nullptr, prediction, previous_prediction, previous_dt, dt,
           (int64_t)batch * per_batch, per_batch, 1};
  return launch_ew<kOpAb2>(a, stream);
}

}  // namespace tsplat
