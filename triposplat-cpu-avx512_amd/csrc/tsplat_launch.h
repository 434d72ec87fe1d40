// Host-side launch interface between the C-ABI layer (capi.cpp) and the
// kernels (*.hip).  Every launcher assumes its arguments were validated by
// the caller: sizes, alignment and device-pointer extents.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsplat {

// out[m, c] = bias[n0+c] + sum_k x[m, k] * w[k, n0+c],  c in [0, n_count),
// w[k, n] = fp32((int32)code01[k, n] * 256 + q2[k, n]) * scale[n].
struct GemmParams {
  const float* x;
  const int16_t* code01;  // [K, N] row-major (the reference's codes0_t)
  const int8_t* q2;       // [K, N] row-major (the reference's codes1_t)
  const float* scale;     // [N]
  const float* bias;      // [N]
  float* out;             // [M, stride_out]
  int M, K, N;
  int n_start, n_count;
  int stride_x, stride_out;
};
int launch_nf24_gemm(const GemmParams& p, hipStream_t stream);
// Few-row form (1 <= M <= 32), HBM-bound; same result contract.
int launch_nf24_gemv(const GemmParams& p, hipStream_t stream);

// softmax(q k^T / 8 + bias[key]) v over one (b, h) per query row.
struct SdpaParams {
  const float* q;      // [B, H, Lq, 64]
  const float* k;      // [B, H, Lk, 64]  or packed [B, H, 64, Lkp]
  const float* v;      // same layout as k
  const float* bias;   // null, or bias[h * bias_head_stride + key]
  float* out;          // [B, H, Lq, 64] or BLHD [B, Lq, H, 64]
  int B, H, Lq, Lk;
  int kv_packed;       // 1: k/v are [B, H, 64, Lkp] (key-contiguous)
  int Lkp;             // key stride of the packed layout
  int64_t bias_head_stride;  // 0: one [Lk] row shared by all heads
  int out_blhd;        // 1: write [B, Lq, H, 64]
};
int launch_sdpa(const SdpaParams& p, hipStream_t stream);

// qkv [B*L, 3*H*64] -> RoPE then RMSNorm on q and k; q [B, H, L, 64],
// packed k/v [B, H, 64, L_padded] with tokens L..L_padded-1 zero.
struct QkvPostParams {
  const float* qkv;
  const float* freqs;    // [fb, L, H, 64] interleaved (cos, sin)
  const float* q_gamma;  // [H, 64]
  const float* k_gamma;  // [H, 64]
  float* q;
  float* packed_k;
  float* packed_v;
  int B, L, H, L_padded, freq_batches;
};
int launch_qkv_postprocess(const QkvPostParams& p, hipStream_t stream);

// The NF24 projection x [B*L, K] -> [B*L, 3*H*64] with the postprocess
// above applied in the GEMM's epilogue: no [B*L, 3*H*64] intermediate.
// gemm.out is unused; gemm.M = B*L, gemm.N = gemm.n_count = 3*H*64.
struct QkvFusedParams {
  GemmParams gemm;
  const float* freqs;
  const float* q_gamma;
  const float* k_gamma;
  float* q;
  float* packed_k;
  float* packed_v;
  int B, L, H, L_padded, freq_batches;
};
int launch_nf24_gemm_qkv(const QkvFusedParams& p, hipStream_t stream);

// NF24 packer: w [out_f, in_f] fp32 -> code01_t [in_f, out_f], q2_t, scale
// [out_f]; base_tmp [out_f] receives max|w_row| / 127.
int launch_nf24_pack(const float* w, int out_f, int in_f, const float* alphabet, int alphabet_len,
                     float* base_tmp, int16_t* code01_t, int8_t* q2_t, float* scale,
                     hipStream_t stream);

// Grow-only device scratch owned by the library, one buffer per (device,
// stream, slot); null on allocation failure.  Valid until the next call with
// the same key that asks for more bytes.
enum WorkspaceSlot : int { kSlotGemvPartial = 0 };
void* stream_workspace(hipStream_t stream, size_t bytes, int slot);

}  // namespace tsplat
