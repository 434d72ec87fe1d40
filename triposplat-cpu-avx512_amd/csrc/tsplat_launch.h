// Host-side launch interface between the C-ABI layer (capi.cpp) and the
// kernels (*.hip).  Every launcher assumes its arguments were validated by
// the caller: sizes, alignment and device-pointer extents.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsplat {

// out[m, c] = bias[n0+c] + sum_k x[m, k] * w[k, n0+c],  c in [0, n_count),
// w[k, n] = fp32((int32)code01[k, n] * 256 + q2[k, n]) * scale[n].
//
// Product precision (opt-in; kPrecisionFp32 is the strict default):
//   kPrecisionFp32:   fp32 x * fp32 w on fp32 MFMA.
//   kPrecisionBf16:   bf16(x) * bf16(w) on bf16 MFMA, fp32 accumulation;
//                     bf16() rounds to nearest even from the fp32 value.
//   kPrecisionBf16x3: x = xh + xl, w = wh + wl with xh = bf16(x),
//                     xl = bf16(x - xh) (likewise w); the product is
//                     xh*wh + xh*wl + xl*wh on bf16 MFMA, fp32 accumulation.
// Calls with M <= 32 are weight-stream bound and run the fp32 path in every
// precision.
enum GemmPrecision : int { kPrecisionFp32 = 0, kPrecisionBf16 = 1, kPrecisionBf16x3 = 2 };
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
  int precision = kPrecisionFp32;
  // Opt-in bf16 modes: the weights split once into bf16 planes [N, K]
  // (k-contiguous; launch_nf24_bf16_planes), w_hi = bf16(w) and, for bf16x3,
  // w_lo = bf16(w - w_hi) -- the values the kernels otherwise decode and
  // split from the codes in every call.  Null: decode the codes.
  const uint16_t* w_hi = nullptr;
  const uint16_t* w_lo = nullptr;
};
int launch_nf24_gemm(const GemmParams& p, hipStream_t stream);
// The bf16 planes of a packed weight [K, N] (codes, scale): w_hi[n * K + k]
// = bf16(w[k][n]) and, for kPrecisionBf16x3, w_lo likewise (null otherwise).
int launch_nf24_bf16_planes(const int16_t* code01, const int8_t* q2, const float* scale, int K, int N,
                            int precision, uint16_t* w_hi, uint16_t* w_lo, hipStream_t stream);
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
  // Product precision of Q K^T and P V (GemmPrecision): kPrecisionFp32 on
  // fp32 MFMA (default); kPrecisionBf16 / kPrecisionBf16x3 split the
  // operands into bf16 terms as the NF24 GEMM's modes do (q scaled first,
  // p = the unnormalised exponentials); softmax arithmetic stays fp32.
  int precision = kPrecisionFp32;
  // Scratch for the key-split partials of a partial last round of query
  // tiles: null takes the stream's library-owned workspace (which may
  // allocate); non-null uses [scratch, scratch + scratch_bytes) and fails
  // with kErrScratch when the launch plan needs more.
  float* scratch = nullptr;
  size_t scratch_bytes = 0;
};
int launch_sdpa(const SdpaParams& p, hipStream_t stream);
// Queries per workgroup of the most recent SDPA launch (512 before any).
void note_sdpa_query_tile(int queries);
int sdpa_query_tile();
// The bf16-MFMA modes (called by launch_sdpa for precision != fp32).
int launch_sdpa_bf16(const SdpaParams& p, hipStream_t stream);

// qkv [B*L, 3*H*64] -> RoPE then RMSNorm on q and k; q [B, H, L, 64],
// packed k/v [B, H, 64, L_padded] with tokens L..L_padded-1 zero.
// kv_round (every QKV postprocess form): bit 0 stores k, bit 1 stores v
// rounded to the nearest bf16 (kept as fp32); 0 stores them exact.
struct QkvPostParams {
  const float* qkv;
  const float* freqs;    // [fb, L, H, 64] interleaved (cos, sin)
  const float* q_gamma;  // [H, 64]
  const float* k_gamma;  // [H, 64]
  float* q;
  float* packed_k;
  float* packed_v;
  int B, L, H, L_padded, freq_batches;
  int kv_round = 0;
};
int launch_qkv_postprocess(const QkvPostParams& p, hipStream_t stream);

// Selected-rows form: q [B, Lq, H*64] rows take their frequency row from
// selected[t] (in [0, Lk); a row with an index outside is written as zeros),
// kv [B, Lk, 2*H*64] = [k | v] -> packed k/v [B, H, 64, Lk_padded].
struct QkvSelectedParams {
  const float* q;
  const float* kv;
  const float* freqs;       // [fb, Lk, H, 64]
  const int64_t* selected;  // [Lq]
  const float* q_gamma;
  const float* k_gamma;
  float* q_out;             // [B, H, Lq, 64]
  float* packed_k;
  float* packed_v;
  int B, Lq, Lk, H, Lk_padded, freq_batches;
  int kv_round = 0;
};
int launch_qkv_selected_postprocess(const QkvSelectedParams& p, hipStream_t stream);

// The NF24 projection x [B*L, K] -> [B*L, 3*H*64] with the postprocess
// above applied in the GEMM's epilogue: no [B*L, 3*H*64] intermediate.
// gemm.out is unused; gemm.M = B*L, gemm.N = gemm.n_count = 3*H*64.
struct QkvFusedParams {
  GemmParams gemm;
  const float* freqs;
  const float* q_gamma;
  const float* k_gamma;
  float* q;
  float* packed_k;         // [B, H, 64, L_padded], or [B, H, L, 64] with kv_bhld
  float* packed_v;
  int B, L, H, L_padded, freq_batches;
  int kv_bhld = 0;
  int kv_round = 0;
};
int launch_nf24_gemm_qkv(const QkvFusedParams& p, hipStream_t stream);

// NF24 GEMM with an elementwise epilogue on out[m, c] (same GEMM as
// launch_nf24_gemm; bias included before the epilogue):
//   kEpilogueGelu:   out = gelu_tanh(acc)
//   kEpilogueGated:  out = out + acc * gate[(m / rows_per_batch) * gate_stride + n_start + c]
//   kEpilogueAdd:    out = out + acc
// (out is read and written in place for the last two.)
enum GemmEpilogue : int { kEpilogueStore = 0, kEpilogueGelu = 2, kEpilogueGated = 3, kEpilogueAdd = 4 };
struct GemmEpilogueParams {
  int kind;
  const float* gate;
  int64_t gate_stride;
  int rows_per_batch;
};
int launch_nf24_gemm_epilogue(const GemmParams& p, const GemmEpilogueParams& e,
                              hipStream_t stream);

// LayerNorm over rows of `cols` (eps inside the sqrt), optional affine
// (weight, bias [cols]) and modulation y * (1 + scale[b]) + shift[b] with
// b = row / rows_per_batch and scale/shift rows mod_batch_stride apart.
struct LayerNormParams {
  const float* input;
  const float* weight;
  const float* bias;
  float* output;
  int64_t rows;
  int cols;
  float eps;
  int affine;
  int modulate;
  const float* scale;
  const float* shift;
  int64_t mod_batch_stride;
  int64_t rows_per_batch;
};
int launch_layernorm(const LayerNormParams& p, hipStream_t stream);

// Per-head RMSNorm x * sqrt(dim) / max(||x||, eps) * gamma[h] of vectors
// (b, l, h) read at input + (b*L + l) * in_token_stride + h*dim; output
// [B, L, H, dim] or [B, H, L, dim] (out_bhld); normalize = 0 copies.
struct HeadNormParams {
  const float* input;
  const float* gamma;
  float* output;
  int B, L, H, dim;
  int64_t in_token_stride;
  float eps;
  int out_bhld;
  int normalize;
};
int launch_head_rmsnorm(const HeadNormParams& p, hipStream_t stream);

int launch_rope_complex(const float* in, const float* freqs, float* out, int64_t pairs,
                        hipStream_t stream);
int launch_modulate(float* h, const float* scale, const float* shift, int batch, int rows, int cols,
                    hipStream_t stream);
int launch_gated_residual(float* base, float* delta, const float* gate, int batch, int rows,
                          int cols, hipStream_t stream);
int launch_add(float* base, const float* delta, int64_t count, hipStream_t stream);
int launch_gelu_tanh(const float* in, float* out, int64_t count, hipStream_t stream);
int launch_silu(const float* in, float* out, int64_t count, hipStream_t stream);
int launch_cfg_combine(float* positive, const float* negative, const float* guidance, int batch,
                       int64_t per_batch, hipStream_t stream);
int launch_euler_update(float* sample, const float* prediction, const float* dt, int batch,
                        int64_t per_batch, hipStream_t stream);
int launch_ab2_update(float* sample, const float* prediction, const float* previous_prediction,
                      const float* dt, const float* previous_dt, int batch, int64_t per_batch,
                      hipStream_t stream);

// NF24 packer: w [out_f, in_f] fp32 -> code01_t [in_f, out_f], q2_t, scale
// [out_f]; base_tmp [out_f] receives max|w_row| / 127.
int launch_nf24_pack(const float* w, int out_f, int in_f, const float* alphabet, int alphabet_len,
                     float* base_tmp, int16_t* code01_t, int8_t* q2_t, float* scale,
                     hipStream_t stream);

// Exact NF24 decode to fp32: [in_f, out_f] like the codes, or [out_f, in_f]
// (the nn.Linear weight) when transposed.
int launch_nf24_decode(const int16_t* code01_t, const int8_t* q2_t, const float* scale, float* out,
                       int in_f, int out_f, int transposed, hipStream_t stream);

// Device scratch owned by the library, one grow-only buffer per (device,
// stream, slot); null on allocation failure, or when the stream is under
// graph capture and its buffer is too small.  The policy (reuse, free after
// the stream, retire a buffer a capture recorded) is in workspace_pool.h.
enum WorkspaceSlot : int {
  kSlotGemvPartial = 0,
  kSlotSdpaPartial = 1,
  kSlotGemmTail = 2,
  kSlotSdpaPlanes = 3,  // pre-split bf16 K/V tiles of the bf16 SDPA modes
};
void* stream_workspace(hipStream_t stream, size_t bytes, int slot);
// Frees the slot's buffers of the current device that no capture recorded
// (after their streams) and retires the others.
void release_workspace(int slot);
// Buffers allocated for the slot so far, bytes of its current buffers, and
// bytes of superseded buffers kept alive for captured graphs.
void workspace_stats(int slot, uint64_t* allocations, uint64_t* live_bytes,
                     uint64_t* retired_bytes);
// Host time the slot has spent allocating, and waiting for streams + freeing.
void workspace_timing(int slot, uint64_t* alloc_ns, uint64_t* free_ns);

}  // namespace tsplat
