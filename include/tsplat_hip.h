/*
 * tsplat_hip.h -- C ABI of libtsplat_hip.so, the gfx950 (MI355X) kernels for
 * the NF24 packed-weight Linear and the exact SDPA of TripoSplat's flow model.
 *
 * Drop-in boundary.  The first group of each section keeps the exact symbol
 * names, argument lists and status codes of the reference's AVX-512
 * libraries, so an unmodified ctypes binding loads this library instead.
 * Differences, all forced by the device:
 *   - every array argument is a DEVICE pointer (hipMalloc / torch.cuda memory
 *     on the current HIP device).  Host pointers and allocations smaller than
 *     the arguments imply are rejected with status -6 before any launch;
 *   - `threads` is accepted and ignored (there is no OpenMP pool);
 *   - the reference-named calls run on the null stream and return after the
 *     device has finished (blocking, like the CPU call).  The tsplat_*_async
 *     variants only enqueue on the given stream (hipStream_t passed as void*)
 *     and return immediately.
 * Status codes: 0 ok; -1 null pointer; -2 bad sizes / stages / head dim;
 * -3 range, stride or key-bias length mismatch; -4 range not 16-aligned (or a
 * pointer not 16-byte aligned where float4 access is required); -5 device
 * workspace allocation failed; -6 not device memory / allocation too small /
 * other device; -7 HIP launch or runtime error (tsplat_last_hip_error());
 * -8 the no-allocation SDPA entry's static scratch is too small for the call.
 *
 * Weight format NF24 (residual mode 4): w[k][n] = fp32((int32)code01[k][n] *
 * 256 + q2[k][n]) * scale[n], code01 int16 [K][N], q2 int8 [K][N], scale fp32
 * [N] (= max|W_row| / 127 / 1024).  codes2_t, scales1, scales2 and codebook
 * are part of the reference signature; they must be non-null and are unused.
 */
#ifndef TSPLAT_HIP_H
#define TSPLAT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- NF24 GEMM: out = bias + x * W ------------------------ */

/* scripts/gemm_nf24_i16_avx512.c:199-220 (triposplat_gemm_rnf8_avx512).
 * Full GEMM over all N outputs; N must be a multiple of 16 (else -4), as in
 * the reference, which routes other N to the _tail symbol. */
int triposplat_gemm_rnf8_avx512(const float* x, const uint8_t* codes0_t, const uint8_t* codes1_t,
                                const uint8_t* codes2_t, const float* scales0,
                                const float* scales1, const float* scales2, const float* codebook,
                                const float* bias, float* out, int M, int K, int N, int stride_x,
                                int stride_out, int threads, int stages);

/* scripts/gemm_nf24_i16_avx512.c:151-197: outputs [output_start,
 * output_start + output_count) of each row into out[M][stride_out];
 * start and count must be multiples of 16. */
int triposplat_gemm_rnf8_avx512_range(const float* x, const uint8_t* codes0_t,
                                      const uint8_t* codes1_t, const uint8_t* codes2_t,
                                      const float* scales0, const float* scales1,
                                      const float* scales2, const float* codebook,
                                      const float* bias, float* out, int M, int K, int N,
                                      int output_start, int output_count, int stride_x,
                                      int stride_out, int threads, int stages);

/* scripts/gemm_nf24_i16_avx512_tail.c:8-49: any N (e.g. 5 for cam_out_layer). */
int triposplat_gemm_rnf8_avx512_tail(const float* x, const uint8_t* codes0_t,
                                     const uint8_t* codes1_t, const uint8_t* codes2_t,
                                     const float* scales0, const float* scales1,
                                     const float* scales2, const float* codebook,
                                     const float* bias, float* out, int M, int K, int N,
                                     int stride_x, int stride_out, int threads, int stages);

/* scripts/gemm_nf24_i16_avx512.c:222-228: rows per output tile; residual
 * mode id (4 = nf24_i16, checked by the Python patch). */
int triposplat_gemm_rnf8_avx512_row_tile(void);
int triposplat_gemm_rnf8_avx512_residual_mode(void);

/* Asynchronous NF24 GEMM on `stream` (no counterpart in the reference; the
 * range form above without the 16-alignment rule). */
int tsplat_nf24_gemm_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                           const float* scale, const float* bias, float* out, int M, int K, int N,
                           int output_start, int output_count, int stride_x, int stride_out,
                           void* stream);

/* ---------------- exact SDPA (head dim 64, scale 1/8) ------------------ */

/* scripts/native_sdpa_avx512_exact_q8t512.c:137-332.  q [B,H,Lq,64],
 * k/v [B,H,Lk,64], key_bias [Lk] shared by all (b,h) when has_key_bias,
 * out [B,H,Lq,64].  D must be 64; key_bias_len must equal Lk. */
int triposplat_sdpa_f32_avx512_exact_q8t512(const float* q, const float* k, const float* v,
                                            const float* key_bias_or_null, float* out, int B,
                                            int H, int Lq, int Lk, int D, int has_key_bias,
                                            int key_bias_len, int threads);
/* q8t512.c:334-351 alias, and the legacy symbol name that
 * scripts/native_sdpa_ctypes.py:10-11 binds by default (same ABI and math). */
int triposplat_sdpa_f32(const float* q, const float* k, const float* v,
                        const float* key_bias_or_null, float* out, int B, int H, int Lq, int Lk,
                        int D, int has_key_bias, int key_bias_len, int threads);
int triposplat_sdpa_f32_avx512_exact_q8(const float* q, const float* k, const float* v,
                                        const float* key_bias_or_null, float* out, int B, int H,
                                        int Lq, int Lk, int D, int has_key_bias,
                                        int key_bias_len, int threads);

/* scripts/native_sdpa_avx512_exact_q8t512_packed.c:3-158: k/v pre-packed
 * [B,H,64,Lkp] (Lkp >= Lk, multiple of 16, tail keys zero), output BLHD
 * [B,Lq,H,64]. */
int triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd(
    const float* q, const float* packed_k, const float* packed_v, const float* key_bias_or_null,
    float* out_blhd, int B, int H, int Lq, int Lk, int D, int Lkp, int has_key_bias,
    int key_bias_len, int threads);

/* q8t512.c:51-100 and packed.c:160-162 metadata/profile probes.  Key tile
 * and query block report this library's tiles (64 keys, 128 queries).
 * Profile: calls and wall time of the blocking calls (allocate/pack/free
 * report 0: there is no per-call workspace or pack step).
 * Workspace: the SDPA's key-split partials, and the bf16 modes' pre-split
 * K/V image, live in grow-only device buffers, one per (device, stream, use);
 * stats report their allocations and bytes together.
 * Release frees, after its stream, the buffer of every stream on the current
 * device that is idle, and keeps (until the process ends) the buffers a HIP
 * graph captured, those of a stream under capture at that moment (waiting on
 * it would end the capture) and those of streams already destroyed (they
 * cannot be waited on): a stream's buffer is reclaimed only by a release
 * made before the stream is destroyed. */
int triposplat_sdpa_key_tile(void);
int triposplat_sdpa_query_block(void);
int triposplat_sdpa_packed_output_is_blhd(void);
void triposplat_sdpa_q8t512_profile_reset(void);
int triposplat_sdpa_q8t512_profile_get(uint64_t* calls, uint64_t* allocate_ns, uint64_t* pack_ns,
                                       uint64_t* compute_ns, uint64_t* free_ns);
int triposplat_sdpa_q8t512_workspace_stats(uint64_t* allocations, uint64_t* capacity_bytes);
void triposplat_sdpa_q8t512_workspace_release(void);

/* Asynchronous SDPA on `stream` (extension of the two entries above):
 * kv_packed selects k/v [B,H,64,Lkp] instead of [B,H,Lk,64]; out_blhd
 * selects [B,Lq,H,64] output; bias_head_stride = 0 shares one [Lk] bias
 * row, = Lk reads a [H,Lk] per-head bias (the key-bias benchmark variant). */
int tsplat_sdpa_async(const float* q, const float* k, const float* v,
                      const float* key_bias_or_null, float* out, int B, int H, int Lq, int Lk,
                      int D, int has_key_bias, int key_bias_len, int64_t bias_head_stride,
                      int kv_packed, int Lkp, int out_blhd, void* stream);
/* No reference counterpart (an opt-in mode; the reference SDPA is fp32
 * only): tsplat_sdpa_async with the product precision of Q K^T and P V --
 * 0 fp32 (= tsplat_sdpa_async), 1 bf16 (bf16(q') bf16(k), bf16(p) bf16(v)),
 * 2 bf16x3 (three bf16 terms per product: hi*hi + hi*lo + lo*hi, 16
 * significant bits per operand); q' = q * 0.125 * log2(e) in fp32, p the
 * unnormalised exponentials; max, exp2, sums and normalisation in fp32.
 * Other values -> -2.  Modes 1 and 2 on wide grids with at least 12 query
 * tiles of 512 per head (6 with kv_packed) first stage K and V once into a
 * bf16 image in the per-stream workspace (512 bytes per key and head in
 * bf16x3, 256 in bf16, +4 with a key bias; at most 2 GiB); without the
 * workspace (under graph capture with a too small buffer) or above that
 * size they stage in the kernel, with the same result. */
int tsplat_sdpa_precision_async(const float* q, const float* k, const float* v,
                                const float* key_bias_or_null, float* out, int B, int H, int Lq,
                                int Lk, int D, int has_key_bias, int key_bias_len,
                                int64_t bias_head_stride, int kv_packed, int Lkp, int out_blhd,
                                int precision, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  tsplat_sdpa_precision_async, same arguments and
 * result, calling no hipMalloc / hipFree (the bf16 modes stage K and V in
 * the kernel, never in a pre-split image): the key-split partials of a
 * partial last round of query tiles go to a static 66 MiB device array
 * instead of the library's per-stream workspace.  That holds every launch
 * plan of a 256-CU device; a call that would need more returns -8 before any
 * launch.  The array is per GPU and shared by all calls on it, whatever the
 * stream: calls that overlap in time on one GPU race and must be ordered by
 * the caller.  The array is part of the library's code object: every process
 * that loads the library holds 66 MiB of device memory on each GPU it uses,
 * whether or not it calls this entry.  The array's device address is looked
 * up on the first call on each device; that call may itself be under graph
 * capture. */
int tsplat_sdpa_noalloc_async(const float* q, const float* k, const float* v,
                              const float* key_bias_or_null, float* out, int B, int H, int Lq,
                              int Lk, int D, int has_key_bias, int key_bias_len,
                              int64_t bias_head_stride, int kv_packed, int Lkp, int out_blhd,
                              int precision, void* stream);

/* ---------------- QKV RoPE -> RMSNorm -> pack -------------------------- */

/* scripts/native_qkv_postprocess_v2_avx512.c:45-105.  qkv [B*L, 3*H*64]
 * -> q [B,H,L,64], packed k/v [B,H,64,L_padded]; frequencies
 * [frequency_batches, L, H, 64] as (cos, sin) pairs; gammas [H,64]. */
int triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2(const float* qkv, const float* frequencies,
                                                   const float* q_gamma, const float* k_gamma,
                                                   float* q_bhld, float* packed_k,
                                                   float* packed_v, int B, int L, int H, int D,
                                                   int L_padded, int frequency_batches,
                                                   int threads);

/* scripts/native_qkv_postprocess_avx512.c:23-116, the first version: same
 * arguments and result as the _v2 entry (it zeroed all of packed k/v before
 * filling; the bytes left are identical). */
int triposplat_qkv_rope_rmsnorm_pack_f32_avx512(const float* qkv, const float* frequencies,
                                                const float* q_gamma, const float* k_gamma,
                                                float* q_bhld, float* packed_k, float* packed_v,
                                                int B, int L, int H, int D, int L_padded,
                                                int frequency_batches, int threads);
/* native_qkv_postprocess_avx512.c:118-120 probe: tokens per transpose tile
 * (64 here: one workgroup transposes 64 tokens of one (b, h) through LDS). */
int triposplat_qkv_postprocess_token_tile(void);
/* native_qkv_postprocess_v2_avx512.c:193-195 probe: 1, only the padding
 * tokens L..L_padded-1 are cleared. */
int triposplat_qkv_postprocess_v2_tail_only_clear(void);

/* bf16 sensitivity probe of the K/V cache,
 * scripts/native_qkv_postprocess_bf16_probe_avx512.c:34-94 (a build of the
 * postprocess whose packed k and/or v are rounded to bf16 after the exact
 * computation; build_native_qkv_postprocess_bf16_probe_avx512.sh selects
 * k, v or kv at compile time).  Here the selection is the per-call
 * `kv_round` argument of the asynchronous postprocess forms below (the
 * full-sequence, selected-rows and fused NF24 QKV entries): bit 0 rounds
 * the stored k, bit 1 the stored v (nearest bf16, ties to even, kept as
 * fp32; probe file :11-22); 0 stores them exact; outside 0..3 -> -2.  The
 * reference-named entries of this library always store them exact, so the
 * probe-mode query reports 0 (native_qkv_postprocess_bf16_probe_avx512.c:
 * 96-105). */
int triposplat_qkv_postprocess_bf16_probe_mode(void);

/* scripts/native_qkv_postprocess_v2_avx512.c:107-191: selected query rows.
 * q [B, Lq, H*64] (a Q-only projection), kv [B, Lk, 2*H*64] = [k | v];
 * query t is rotated with frequency row selected_indices[t] (int64, device
 * array; any index outside [0, Lk) -> -3 before any work, as the
 * reference); q_bhld [B,H,Lq,64], packed k/v [B,H,64,Lk_padded] with zero
 * tail.  Used for the final block, whose outputs are read only at the
 * latent rows. */
int triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2(
    const float* q, const float* kv, const float* frequencies, const int64_t* selected_indices,
    const float* q_gamma, const float* k_gamma, float* q_bhld, float* packed_k, float* packed_v,
    int B, int Lq, int Lk, int H, int D, int Lk_padded, int frequency_batches, int threads);
/* Asynchronous form; the indices are not read on the host: a query whose
 * index is outside [0, Lk) gets an all-zero q row.  kv_round: see the bf16
 * probe above (0 = exact). */
int tsplat_q_kv_selected_postprocess_async(const float* q, const float* kv,
                                           const float* frequencies,
                                           const int64_t* selected_indices,
                                           const float* q_gamma, const float* k_gamma,
                                           float* q_bhld, float* packed_k, float* packed_v, int B,
                                           int Lq, int Lk, int H, int D, int Lk_padded,
                                           int frequency_batches, int kv_round, void* stream);

/* scripts/gemm_nf24_qkv_direct_avx512.c:87-199: NF24 QKV GEMM (N = 3*H*64)
 * followed by the postprocess above, without returning the [B*L, N]
 * projection to the caller. */
int triposplat_gemm_nf24_qkv_rope_rmsnorm_pack_f32_avx512(
    const float* x, const uint8_t* codes0_t, const uint8_t* codes1_t, const uint8_t* codes2_t,
    const float* scales0, const float* scales1, const float* scales2, const float* codebook,
    const float* bias, const float* frequencies, const float* q_gamma, const float* k_gamma,
    float* q_bhld, float* packed_k, float* packed_v, int B, int L, int K, int N, int H, int D,
    int L_padded, int frequency_batches, int threads, int stages);
/* gemm_nf24_qkv_direct_avx512.c:201-207 probes. */
int triposplat_gemm_nf24_qkv_direct_row_tile(void);
/* gemm_nf24_qkv_direct_tile_avx512.c:149-151: bytes of the tile variant's
 * per-row-tile projection cache; 0 here (the fused epilogue reads the
 * projection from MFMA accumulators, no intermediate buffer). */
int triposplat_gemm_nf24_qkv_direct_tile_bytes(void);
int triposplat_gemm_nf24_qkv_direct_residual_mode(void);

/* Asynchronous forms of the two QKV entries (the postprocess with the
 * probe's per-call kv_round, 0 = exact; the fused entry always exact). */
int tsplat_qkv_postprocess_async(const float* qkv, const float* frequencies, const float* q_gamma,
                                 const float* k_gamma, float* q_bhld, float* packed_k,
                                 float* packed_v, int B, int L, int H, int D, int L_padded,
                                 int frequency_batches, int kv_round, void* stream);
int tsplat_gemm_nf24_qkv_direct_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                      const float* scale, const float* bias,
                                      const float* frequencies, const float* q_gamma,
                                      const float* k_gamma, float* q_bhld, float* packed_k,
                                      float* packed_v, int B, int L, int K, int N, int H, int D,
                                      int L_padded, int frequency_batches, void* stream);

/* ---------------- NF24 packer ------------------------------------------ */

/* scripts/native_linear_rnf8_avx512_patch.py:14-87 (quantize_nf24_i16_per_output_channel),
 * on the device: weight fp32 [out_features, in_features] -> code01_t int16
 * [in, out], q2_t int8 [in, out], scale fp32 [out] (= max|row|/127/1024).
 * alphabet: the sorted NF8-derived integer levels (fp32, 2..256 entries);
 * base_workspace: [out_features] fp32 scratch.  Asynchronous on `stream`. */
int tsplat_nf24_pack_async(const float* weight, int out_features, int in_features,
                           const float* alphabet, int alphabet_len, float* base_workspace,
                           int16_t* code01_t, int8_t* q2_t, float* scale, void* stream);

/* scripts/native_linear_nf24_prepacked.py:17-36 (decode_nf24_i16_weight_t /
 * decode_nf24_i16_weight): exact fp32 weights, out [in, out] like the codes,
 * or [out, in] (the nn.Linear layout) when transposed != 0. */
int tsplat_nf24_decode_async(const int16_t* code01_t, const int8_t* q2_t, const float* scale,
                             float* out, int in_features, int out_features, int transposed,
                             void* stream);

/* ---------------- NF24 GEMM with an elementwise epilogue --------------- */

/* The GEMM of tsplat_nf24_gemm_async with the block's next elementwise step
 * applied to the result before it is stored (no counterpart symbol in the
 * reference, which runs the two steps as separate calls; the elementwise
 * arithmetic is that of the cited reference kernels, bit for bit):
 *   epilogue 0: out = acc
 *   epilogue 2: out = gelu_tanh(acc)            (native_gelu_avx512.c:44-68)
 *   epilogue 3: out += acc * gate[(m / rows_per_batch) * gate_stride + n]
 *                                   (native_block_elementwise_avx512.c:24-35)
 *   epilogue 4: out += acc          (native_block_elementwise_avx512.c:37-46)
 * acc includes the bias.  gate_stride >= N. */
int tsplat_nf24_gemm_epilogue_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                    const float* scale, const float* bias, float* out, int M,
                                    int K, int N, int output_start, int output_count,
                                    int stride_x, int stride_out, int epilogue, const float* gate,
                                    int64_t gate_stride, int rows_per_batch, void* stream);

/* ---------------- opt-in bf16-MFMA precision ----------------------------- */
/* No counterpart in the reference, whose NF24 Linear is fp32 only; its
 * bf16 evidence is a round-trip probe (triposplat_bf16_roundtrip_patch.py:
 * 7-53, torch's round-to-nearest-even float32 -> bfloat16).  `precision`:
 *   0 strict: fp32 products (the result of tsplat_nf24_gemm_epilogue_async)
 *   1 bf16:   bf16(x) * bf16(w) on bf16 MFMA, fp32 accumulation
 *   2 bf16x3: xh*wh + xh*wl + xl*wh, xh = bf16(x), xl = bf16(x - xh), same
 *             for w; about 16 significant bits per product
 * bf16() rounds the fp32 value (w: the exact NF24 decode) to nearest even.
 * Calls with M <= 32 run the strict kernels in every precision (they are
 * bound by the weight stream).  Other arguments and status codes as
 * tsplat_nf24_gemm_epilogue_async; -2 for an unknown precision. */
int tsplat_nf24_gemm_precision_async(const float* x, const int16_t* code01_t,
                                     const int8_t* q2_t, const float* scale, const float* bias,
                                     float* out, int M, int K, int N, int output_start,
                                     int output_count, int stride_x, int stride_out, int epilogue,
                                     const float* gate, int64_t gate_stride, int rows_per_batch,
                                     int precision, void* stream);
/* tsplat_gemm_nf24_qkv_direct_async with the projection in `precision`
 * (the RoPE / RMSNorm epilogue is the same fp32 arithmetic) and a choice of
 * K/V layout: kv_layout 0 packed [B, H, 64, L_padded] (the reference's),
 * 1 [B, H, L, 64] like q (L_padded ignored), the layout the unpacked SDPA
 * reads; kv_round as the bf16 probe above (0 = exact).  No counterpart in
 * the reference. */
int tsplat_gemm_nf24_qkv_direct_ex_async(
    const float* x, const int16_t* code01_t, const int8_t* q2_t, const float* scale,
    const float* bias, const float* frequencies, const float* q_gamma, const float* k_gamma,
    float* q_bhld, float* k_out, float* v_out, int B, int L, int K, int N, int H, int D,
    int L_padded, int frequency_batches, int kv_layout, int precision, int kv_round,
    void* stream);
/* bf16 planes of a packed weight for the opt-in modes (no counterpart in the
 * reference): w_hi = bf16(w) and, for precision 2 (bf16x3), w_lo = bf16 of the
 * exact decode minus w_hi -- the values the bf16 kernels otherwise decode and
 * split from the codes in every call, once.  bf16 bits, k-blocked: element
 * (k, n) at ((k / 32) * N + n) * 32 + k % 32, zeros past K; ceil(K / 32) * 32
 * * N * 2 bytes each; w_lo may be null for precision 1.  -2 for a precision
 * other than 1 or 2. */
int tsplat_nf24_bf16_planes_async(const int16_t* code01_t, const int8_t* q2_t, const float* scale,
                                  int K, int N, int precision, uint16_t* w_hi, uint16_t* w_lo,
                                  void* stream);
/* tsplat_nf24_gemm_precision_async / tsplat_gemm_nf24_qkv_direct_ex_async
 * reading the weights of the bf16 kernels from the planes above (16-byte
 * aligned; otherwise the codes, same result bit for bit).
 * The codes are still read where the strict kernels run (fp32, M <= 32 and
 * row tails).  No counterpart in the reference. */
int tsplat_nf24_gemm_planes_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                  const float* scale, const float* bias, float* out, int M, int K,
                                  int N, int output_start, int output_count, int stride_x,
                                  int stride_out, int epilogue, const float* gate,
                                  int64_t gate_stride, int rows_per_batch, int precision,
                                  const uint16_t* w_hi, const uint16_t* w_lo, void* stream);
int tsplat_gemm_nf24_qkv_direct_planes_async(
    const float* x, const int16_t* code01_t, const int8_t* q2_t, const float* scale,
    const float* bias, const float* frequencies, const float* q_gamma, const float* k_gamma,
    float* q_bhld, float* k_out, float* v_out, int B, int L, int K, int N, int H, int D,
    int L_padded, int frequency_batches, int kv_layout, int precision, int kv_round,
    const uint16_t* w_hi, const uint16_t* w_lo, void* stream);

/* ---------------- flow-block elementwise -------------------------------- */
/* Bit-identical per element to the reference kernels (same operation order,
 * same fused multiply-adds, the reductions in the AVX-512 lane order). */

/* scripts/native_norm_rope_avx512.c:13-49.  rows x cols, eps inside the
 * sqrt; -3 if has_affine and weight/bias is null. */
int triposplat_layernorm_f32_avx512(const float* input, const float* weight, const float* bias,
                                    float* output, int64_t rows, int cols, float eps,
                                    int has_affine, int threads);
/* native_norm_rope_avx512.c:51-83.  [outer, heads, dim] * sqrt(dim) /
 * max(||x||, eps) * gamma[heads, dim]. */
int triposplat_multihead_rmsnorm_f32_avx512(const float* input, const float* gamma, float* output,
                                            int64_t outer, int heads, int dim, float eps,
                                            int threads);
/* native_norm_rope_avx512.c:85-119.  Interleaved complex multiply; dim even;
 * pointers 8-byte aligned (else -4). */
int triposplat_rope_complex_f32_avx512(const float* input, const float* freqs_interleaved,
                                       float* output, int64_t vectors, int dim, int threads);
/* scripts/native_block_elementwise_avx512.c:9-22: h[b] = h[b] * (1 + scale[b]) + shift[b]. */
int triposplat_modulate_inplace_f32_avx512(float* h, const float* scale, const float* shift,
                                           int batch, int rows, int cols, int threads);
/* native_block_elementwise_avx512.c:24-35: delta *= gate[b]; base += delta. */
int triposplat_gated_residual_inplace_f32_avx512(float* base, float* delta, const float* gate,
                                                 int batch, int rows, int cols, int threads);
/* native_block_elementwise_avx512.c:37-46: base += delta. */
int triposplat_add_inplace_f32_avx512(float* base, const float* delta, int64_t count,
                                      int threads);
/* scripts/native_gelu_avx512.c:44-68 (tanh form). */
int triposplat_gelu_tanh_f32_avx512(const float* input, float* output, int64_t count,
                                    int threads);
/* scripts/native_silu_avx512_extra.c: x / (1 + exp(-x)). */
int triposplat_silu_f32_avx512(const float* input, float* output, int64_t count, int threads);

/* Asynchronous forms.  tsplat_layernorm_modulate_async fuses the modulation
 * y * (1 + scale[b]) + shift[b] (b = row / rows_per_batch, scale/shift rows
 * mod_batch_stride floats apart; both null for a plain LayerNorm).
 * tsplat_head_rmsnorm_async normalises vectors (b, l, h) read at input +
 * (b*L + l) * in_token_stride + h*dim into [B, L, H, dim] or, with out_bhld,
 * [B, H, L, dim]; normalize = 0 only moves them. */
int tsplat_layernorm_modulate_async(const float* input, const float* weight, const float* bias,
                                    float* output, int64_t rows, int cols, float eps,
                                    int has_affine, const float* scale, const float* shift,
                                    int64_t mod_batch_stride, int64_t rows_per_batch,
                                    void* stream);
int tsplat_head_rmsnorm_async(const float* input, int64_t in_token_stride, const float* gamma,
                              float* output, int B, int L, int H, int dim, float eps,
                              int out_bhld, int normalize, void* stream);
int tsplat_rope_complex_async(const float* input, const float* freqs_interleaved, float* output,
                              int64_t vectors, int dim, void* stream);
int tsplat_modulate_async(float* h, const float* scale, const float* shift, int batch, int rows,
                          int cols, void* stream);
int tsplat_gated_residual_async(float* base, float* delta, const float* gate, int batch, int rows,
                                int cols, void* stream);
int tsplat_add_async(float* base, const float* delta, int64_t count, void* stream);
int tsplat_gelu_tanh_async(const float* input, float* output, int64_t count, void* stream);
int tsplat_silu_async(const float* input, float* output, int64_t count, void* stream);

/* ---------------- sampler ------------------------------------------------ */

/* scripts/native_sampler_avx512.c:19-54: positive = g*positive - (g-1)*negative
 * per batch (guidance [batch], a device array). */
int triposplat_cfg_combine_inplace_f32_avx512(float* positive, const float* negative,
                                              const float* guidance, int batch,
                                              int64_t elements_per_batch, int threads);
/* native_sampler_avx512.c:56-89: sample -= dt[b] * prediction. */
int triposplat_euler_update_inplace_f32_avx512(float* sample, const float* prediction,
                                               const float* dt, int batch,
                                               int64_t elements_per_batch, int threads);
/* native_sampler_avx512.c:91-134: second-order Adams-Bashforth update. */
int triposplat_ab2_update_inplace_f32_avx512(float* sample, const float* prediction,
                                             const float* previous_prediction, const float* dt,
                                             const float* previous_dt, int batch,
                                             int64_t elements_per_batch, int threads);
int tsplat_cfg_combine_async(float* positive, const float* negative, const float* guidance,
                             int batch, int64_t elements_per_batch, void* stream);
int tsplat_euler_update_async(float* sample, const float* prediction, const float* dt, int batch,
                              int64_t elements_per_batch, void* stream);
int tsplat_ab2_update_async(float* sample, const float* prediction,
                            const float* previous_prediction, const float* dt,
                            const float* previous_dt, int batch, int64_t elements_per_batch,
                            void* stream);

/* ---------------- library ------------------------------------------------ */
int tsplat_abi_version(void);         /* bumped on any ABI change */
int tsplat_last_hip_error(void);      /* last hipError_t seen by this library */
const char* tsplat_build_arch(void);  /* "gfx950" */

#ifdef __cplusplus
}
#endif

#endif /* TSPLAT_HIP_H */
