/*
 * tsplat_oracle.c -- CPU restatement of the reference's two hot paths.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  No product code path calls it, links it or falls back
 * to it.
 *
 * Every function restates, in scalar C, the arithmetic of one reference
 * kernel operation for operation, so that its results are bit-identical to
 * the reference's AVX-512 build on the same inputs.  Build with
 * -ffp-contract=off: each fused multiply-add the reference performs is
 * written here as an explicit fmaf(), and nothing else may be fused.
 *
 * Reference files (paths relative to the reference repository root):
 *   scripts/gemm_nf24_i16_avx512.c            NF24 GEMM + range API
 *   scripts/gemm_nf24_i16_avx512_tail.c       scalar NF24 GEMM
 *   scripts/native_sdpa_avx512_exact_q8t512.c exact SDPA, key tile 512
 *   scripts/native_sdpa_avx512_exact_q8t512_packed.c  packed-K/V, BLHD out
 *   scripts/native_qkv_postprocess_v2_avx512.c RoPE -> RMSNorm -> pack
 *   scripts/gemm_nf24_qkv_direct_avx512.c     fused QKV GEMM + postprocess
 *   scripts/native_norm_rope_avx512.c         LayerNorm, multi-head RMSNorm, RoPE
 *   scripts/native_block_elementwise_avx512.c modulate, gated residual, add
 *   scripts/native_gelu_avx512.c, native_silu_avx512_extra.c  activations
 *   scripts/native_sampler_avx512.c           CFG combine, Euler, AB2
 *
 * The reference builds its elementwise kernels with gcc -O3 -mfma and the
 * default -ffp-contract=fast, under which GCC fuses a multiply whose only
 * use is an add (native_block_elementwise_avx512.c's modulate, the
 * x + 0.044715 x^3 of the GELU); those fusions are written out below and
 * were confirmed against the _ref build.  The sampler is built with
 * -ffp-contract=off and has none.
 *
 * Pinning (how each function is checked, beyond retyping):
 *   - bit-exact against the reference C compiled from its own sources into
 *     oracle/_ref/ (Makefile in this folder), on seeded inputs;
 *   - against the committed fixtures in tests/golden/ that _ref produced;
 *   - against float64 closed forms (GEMM: decoded-weight matmul; SDPA:
 *     textbook softmax(QK^T/8 + b)V; RoPE/RMSNorm: rotation + unit norm)
 *     and invariants (range == slice of full, key permutation, log M bias
 *     == M duplicated keys, Lk == 1 -> V).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { OR_HEAD_DIM = 64, OR_LANES = 16, OR_KEY_TILE = 512, OR_QUERY_BLOCK = 8 };

/* ------------------------------------------------------------------ */
/* NF24 weight decode.  scripts/gemm_nf24_i16_avx512.c:26-33 (decode16):
 * q = (int32)q01 << 8 + (int32)q2, converted to fp32 (exact: |q| < 2^24),
 * times the per-output scale in one fp32 rounding. */
static inline float nf24_decode(int16_t q01, int8_t q2, float scale) {
  const int32_t q = (int32_t)q01 * 256 + (int32_t)q2;
  return (float)q * scale;
}

float oracle_nf24_decode(int q01, int q2, float scale) {
  return nf24_decode((int16_t)q01, (int8_t)q2, scale);
}

/* scripts/gemm_nf24_i16_avx512.c:151-197 (range API) with the per-output
 * arithmetic of kernel_mx16 (:35-123): acc starts at bias[n] and takes one
 * fmaf per k in increasing k -- the same chain as the scalar tail kernel
 * (gemm_nf24_i16_avx512_tail.c:32-47).  Status codes follow :171-175. */
int oracle_nf24_gemm_range(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                           const float* scale, const float* bias, float* out, int M, int K,
                           int N, int output_start, int output_count, int stride_x,
                           int stride_out, int require_aligned) {
  if (!x || !code01_t || !q2_t || !scale || !bias || !out) return -1;
  if (M <= 0 || K <= 0 || N <= 0 || output_start < 0 || output_count <= 0) return -2;
  if (output_start + output_count > N || stride_x < K || stride_out < output_count) return -3;
  if (require_aligned && (((output_start & 15) != 0) || ((output_count & 15) != 0))) return -4;
#pragma omp parallel for schedule(static)
  for (int i = 0; i < M; ++i) {
    const float* xr = x + (int64_t)i * stride_x;
    float* orow = out + (int64_t)i * stride_out;
    for (int local = 0; local < output_count; ++local) {
      const int n = output_start + local;
      const float s = scale[n];
      float acc = bias[n];
      for (int k = 0; k < K; ++k) {
        const int64_t off = (int64_t)k * N + n;
        acc = fmaf(xr[k], nf24_decode(code01_t[off], q2_t[off], s), acc);
      }
      orow[local] = acc;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* Cephes-style exp of scripts/native_sdpa_avx512_exact_q8t512.c:102-131,
 * one lane.  min/max follow the x86 minps/maxps operand rule. */
static inline float exp512_lane(float x) {
  const float exp_hi = 88.3762626647949f;
  const float exp_lo = -88.3762626647949f;
  x = (x < exp_hi) ? x : exp_hi;
  x = (x > exp_lo) ? x : exp_lo;
  float fx = fmaf(x, 1.44269504088896341f, 0.5f);
  fx = floorf(fx);
  x = fmaf(-fx, 0.693359375f, x);
  x = fmaf(-fx, -2.12194440e-4f, x);
  const float z = x * x;
  float y = 1.9875691500e-4f;
  y = fmaf(y, x, 1.3981999507e-3f);
  y = fmaf(y, x, 8.3334519073e-3f);
  y = fmaf(y, x, 4.1665795894e-2f);
  y = fmaf(y, x, 1.6666665459e-1f);
  y = fmaf(y, x, 5.0000001201e-1f);
  y = fmaf(y, z, x);
  y = y + 1.0f;
  int32_t e = (int32_t)fx;
  e = (e + 0x7f) << 23;
  float p;
  memcpy(&p, &e, sizeof p);
  return y * p;
}

float oracle_exp512(float x) { return exp512_lane(x); }

/* 16-lane horizontal sum in the order of GCC's _mm512_reduce_add_ps
 * (halves 8+8, then 4+4, then lanes {0,2}+{1,3}). */
static inline float reduce_add16(const float* a) {
  float t3[8], t6[4];
  for (int i = 0; i < 8; ++i) t3[i] = a[i + 8] + a[i];
  for (int i = 0; i < 4; ++i) t6[i] = t3[i + 4] + t3[i];
  const float t80 = t6[0] + t6[2];
  const float t81 = t6[1] + t6[3];
  return t80 + t81;
}

float oracle_reduce_add16(const float* a) { return reduce_add16(a); }

/* One query row of the exact online-softmax SDPA:
 * scripts/native_sdpa_avx512_exact_q8t512.c:215-319.  kd(j, d) and vd(j, d)
 * address key j / value j at dimension d in whichever layout the caller
 * has.  The key tile is 512, chunks are 16 keys. */
typedef struct {
  const float* base;
  int64_t key_stride; /* elements between consecutive keys */
  int64_t dim_stride; /* elements between consecutive dims */
} kv_view;

static void sdpa_row(const float* qrow, kv_view kv_k, kv_view kv_v, const float* bias, int Lk,
                     float* dst) {
  float global_max = -INFINITY;
  float global_sum = 0.0f;
  float global_acc[OR_HEAD_DIM];
  for (int d = 0; d < OR_HEAD_DIM; ++d) global_acc[d] = 0.0f;
  float scores[OR_KEY_TILE];
  float local_out[OR_HEAD_DIM];

  for (int jb = 0; jb < Lk; jb += OR_KEY_TILE) {
    const int count = (jb + OR_KEY_TILE <= Lk) ? OR_KEY_TILE : (Lk - jb);
    const int chunks = (count + OR_LANES - 1) / OR_LANES;
    float local_max = -INFINITY;
    float local_sum = 0.0f;

    /* scores: q.k as one fmaf chain over d per key, times 0.125, plus bias;
     * keys past Lk inside the last chunk are -inf (q8t512.c:244-268). */
    for (int tc = 0; tc < chunks; ++tc) {
      const int key = jb + tc * OR_LANES;
      const int valid = (Lk - key < OR_LANES) ? (Lk - key) : OR_LANES;
      float lane_s[OR_LANES];
      for (int l = 0; l < OR_LANES; ++l) {
        float s = -INFINITY;
        if (l < valid) {
          const int j = key + l;
          float acc = 0.0f;
          for (int d = 0; d < OR_HEAD_DIM; ++d)
            acc = fmaf(qrow[d], kv_k.base[j * kv_k.key_stride + d * kv_k.dim_stride], acc);
          s = acc * 0.125f;
          if (bias) s = s + bias[j];
        }
        lane_s[l] = s;
        scores[tc * OR_LANES + l] = s;
      }
      float m = lane_s[0];
      for (int l = 1; l < OR_LANES; ++l) m = (lane_s[l] > m) ? lane_s[l] : m;
      if (m > local_max) local_max = m;
    }

    /* weights and local sum (q8t512.c:270-281) */
    for (int tc = 0; tc < chunks; ++tc) {
      const int key = jb + tc * OR_LANES;
      const int valid = (Lk - key < OR_LANES) ? (Lk - key) : OR_LANES;
      float w[OR_LANES];
      for (int l = 0; l < OR_LANES; ++l) {
        float e = exp512_lane(scores[tc * OR_LANES + l] - local_max);
        w[l] = (l < valid) ? e : 0.0f;
        scores[tc * OR_LANES + l] = w[l];
      }
      local_sum += reduce_add16(w);
    }

    /* local output: per d, 16 lane chains over chunks, then the tree sum
     * (q8t512.c:283-296).  Padded keys carry weight 0 and value 0. */
    for (int d = 0; d < OR_HEAD_DIM; ++d) {
      float lanes[OR_LANES];
      for (int l = 0; l < OR_LANES; ++l) lanes[l] = 0.0f;
      for (int tc = 0; tc < chunks; ++tc) {
        const int key = jb + tc * OR_LANES;
        for (int l = 0; l < OR_LANES; ++l) {
          const int j = key + l;
          const float vv = (j < Lk) ? kv_v.base[j * kv_v.key_stride + d * kv_v.dim_stride] : 0.0f;
          lanes[l] = fmaf(scores[tc * OR_LANES + l], vv, lanes[l]);
        }
      }
      local_out[d] = reduce_add16(lanes);
    }

    /* merge into the running state (q8t512.c:298-310).  The running sum
     * update is compiled by GCC -O3 -mfma into one fused multiply-add whose
     * addend is the rounded local product; the reference build in
     * oracle/_ref pins this choice bit for bit. */
    const float new_max = (local_max > global_max) ? local_max : global_max;
    const float old_scale = isinf(global_max) ? 0.0f : expf(global_max - new_max);
    const float local_scale = expf(local_max - new_max);
    for (int d = 0; d < OR_HEAD_DIM; ++d)
      global_acc[d] = fmaf(local_out[d], local_scale, global_acc[d] * old_scale);
#ifndef ORACLE_SUM_UNFUSED
    global_sum = fmaf(global_sum, old_scale, local_sum * local_scale);
#else
    global_sum = global_sum * old_scale + local_sum * local_scale;
#endif
    global_max = new_max;
  }

  const float inv = 1.0f / global_sum;
  for (int d = 0; d < OR_HEAD_DIM; ++d) dst[d] = global_acc[d] * inv;
}

/* scripts/native_sdpa_avx512_exact_q8t512.c:137-153 argument checks and
 * layout: q,k,v [B,H,L,64]; key_bias [Lk] shared by every (b,h); out
 * [B,H,Lq,64].  The K/V pack (:179-198) changes layout only.
 * bias_head_stride extends the ABI: 0 = the reference's shared [Lk] bias,
 * Lk = one bias row per head ([H,Lk], as per-head calls at H=1 would use). */
int oracle_sdpa_q8t512(const float* q, const float* k, const float* v, const float* key_bias,
                       float* out, int B, int H, int Lq, int Lk, int D, int has_key_bias,
                       int key_bias_len, int64_t bias_head_stride) {
  if (!q || !k || !v || !out) return -1;
  if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0 || D != OR_HEAD_DIM) return -2;
  if (has_key_bias && (!key_bias || key_bias_len != Lk)) return -3;
  const int64_t bh_count = (int64_t)B * H;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t bh = 0; bh < bh_count; ++bh) {
    for (int i = 0; i < Lq; ++i) {
      kv_view kk = {k + bh * (int64_t)Lk * OR_HEAD_DIM, OR_HEAD_DIM, 1};
      kv_view vv = {v + bh * (int64_t)Lk * OR_HEAD_DIM, OR_HEAD_DIM, 1};
      const float* b = has_key_bias ? key_bias + (bh % H) * bias_head_stride : NULL;
      sdpa_row(q + (bh * Lq + i) * OR_HEAD_DIM, kk, vv, b, Lk,
               out + (bh * Lq + i) * OR_HEAD_DIM);
    }
  }
  return 0;
}

/* scripts/native_sdpa_avx512_exact_q8t512_packed.c:3-158: q [B,H,Lq,64],
 * K/V pre-packed [B,H,64,Lkp], output BLHD [B,Lq,H,64]. */
int oracle_sdpa_q8t512_packed_blhd(const float* q, const float* packed_k, const float* packed_v,
                                   const float* key_bias, float* out_blhd, int B, int H, int Lq,
                                   int Lk, int D, int Lkp, int has_key_bias, int key_bias_len) {
  if (!q || !packed_k || !packed_v || !out_blhd) return -1;
  if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0 || D != OR_HEAD_DIM || Lkp < Lk || (Lkp & 15) != 0)
    return -2;
  if (has_key_bias && (!key_bias || key_bias_len != Lk)) return -3;
  const int64_t bh_count = (int64_t)B * H;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t bh = 0; bh < bh_count; ++bh) {
    for (int i = 0; i < Lq; ++i) {
      const int64_t b = bh / H, h = bh % H;
      kv_view kk = {packed_k + bh * OR_HEAD_DIM * (int64_t)Lkp, 1, Lkp};
      kv_view vv = {packed_v + bh * OR_HEAD_DIM * (int64_t)Lkp, 1, Lkp};
      sdpa_row(q + (bh * Lq + i) * OR_HEAD_DIM, kk, vv, has_key_bias ? key_bias : NULL, Lk,
               out_blhd + ((b * Lq + i) * H + h) * OR_HEAD_DIM);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* RoPE then RMSNorm of one 64-wide head row:
 * scripts/native_qkv_postprocess_v2_avx512.c:3-24 (transform_q64) with the
 * rope16 of native_qkv_postprocess_avx512.c / gemm_nf24_qkv_direct:11-16.
 * freq holds interleaved (cos, sin) pairs.  Even lane: x_re*c - x_im*s,
 * odd lane: x_re*s + x_im*c, each as one fmaf over a rounded product
 * (vfmaddsub).  Sum of squares: 16 lane chains over 4 chunks, tree sum. */
static void rope_rmsnorm64(const float* src, const float* freq, const float* gamma, float* dst) {
  float rot[OR_HEAD_DIM];
  for (int i = 0; i < OR_HEAD_DIM; i += 2) {
    const float xr = src[i], xi = src[i + 1];
    const float c = freq[i], s = freq[i + 1];
    rot[i] = fmaf(xr, c, -(xi * s));
    rot[i + 1] = fmaf(xr, s, xi * c);
  }
  float lanes[OR_LANES];
  for (int l = 0; l < OR_LANES; ++l) lanes[l] = 0.0f;
  for (int d = 0; d < OR_HEAD_DIM; d += OR_LANES)
    for (int l = 0; l < OR_LANES; ++l) lanes[l] = fmaf(rot[d + l], rot[d + l], lanes[l]);
  const float norm = sqrtf(reduce_add16(lanes));
  const float factor = 8.0f / fmaxf(norm, 1.0e-12f);
  for (int d = 0; d < OR_HEAD_DIM; ++d) dst[d] = (rot[d] * factor) * gamma[d];
}

void oracle_rope_rmsnorm64(const float* src, const float* freq, const float* gamma, float* dst) {
  rope_rmsnorm64(src, freq, gamma, dst);
}

/* scripts/native_qkv_postprocess_v2_avx512.c:45-105: qkv [B*L, 3*H*64]
 * -> Q [B,H,L,64] (RoPE+RMSNorm), packed K [B,H,64,Lpad] (RoPE+RMSNorm),
 * packed V [B,H,64,Lpad] (copy); tokens L..Lpad-1 are zero.
 * frequencies [fb,L,H,64], fb in {1,B}; gammas [H,64]. */
int oracle_qkv_rope_rmsnorm_pack(const float* qkv, const float* freqs, const float* q_gamma,
                                 const float* k_gamma, float* q_bhld, float* packed_k,
                                 float* packed_v, int B, int L, int H, int D, int L_padded,
                                 int frequency_batches) {
  if (!qkv || !freqs || !q_gamma || !k_gamma || !q_bhld || !packed_k || !packed_v) return -1;
  if (B <= 0 || L <= 0 || H <= 0 || D != OR_HEAD_DIM || L_padded < L || (L_padded & 15) != 0 ||
      (frequency_batches != 1 && frequency_batches != B))
    return -2;
  const int64_t bh_count = (int64_t)B * H;
#pragma omp parallel for schedule(static)
  for (int64_t bh = 0; bh < bh_count; ++bh) {
    const int b = (int)(bh / H), h = (int)(bh % H);
    const int fb = frequency_batches == 1 ? 0 : b;
    float* pk = packed_k + bh * D * (int64_t)L_padded;
    float* pv = packed_v + bh * D * (int64_t)L_padded;
    for (int t = 0; t < L; ++t) {
      const float* qs = qkv + (((int64_t)b * L + t) * 3 * H + h) * D;
      const float* ks = qs + (int64_t)H * D;
      const float* vs = ks + (int64_t)H * D;
      const float* f = freqs + (((int64_t)fb * L + t) * H + h) * D;
      float kn[OR_HEAD_DIM];
      rope_rmsnorm64(qs, f, q_gamma + (int64_t)h * D, q_bhld + (bh * L + t) * D);
      rope_rmsnorm64(ks, f, k_gamma + (int64_t)h * D, kn);
      for (int d = 0; d < D; ++d) {
        pk[(int64_t)d * L_padded + t] = kn[d];
        pv[(int64_t)d * L_padded + t] = vs[d];
      }
    }
    for (int d = 0; d < D; ++d)
      for (int t = L; t < L_padded; ++t) {
        pk[(int64_t)d * L_padded + t] = 0.0f;
        pv[(int64_t)d * L_padded + t] = 0.0f;
      }
  }
  return 0;
}

/* scripts/native_qkv_postprocess_v2_avx512.c:107-191: q [B,Lq,H*64] rows
 * rotated with frequency row selected[t], kv [B,Lk,2*H*64] = [k | v] packed
 * with a zero tail; an index outside [0, Lk) is -3 before any work. */
int oracle_q_kv_selected_rope_rmsnorm_pack(const float* q, const float* kv, const float* freqs,
                                           const int64_t* selected, const float* q_gamma,
                                           const float* k_gamma, float* q_bhld, float* packed_k,
                                           float* packed_v, int B, int Lq, int Lk, int H, int D,
                                           int Lk_padded, int frequency_batches) {
  if (!q || !kv || !freqs || !selected || !q_gamma || !k_gamma || !q_bhld || !packed_k || !packed_v)
    return -1;
  if (B <= 0 || Lq <= 0 || Lk <= 0 || H <= 0 || D != OR_HEAD_DIM || Lk_padded < Lk ||
      (Lk_padded & 15) != 0 || (frequency_batches != 1 && frequency_batches != B))
    return -2;
  for (int t = 0; t < Lq; ++t)
    if (selected[t] < 0 || selected[t] >= Lk) return -3;
  for (int64_t bh = 0; bh < (int64_t)B * H; ++bh) {
    const int b = (int)(bh / H), h = (int)(bh % H);
    const int fb = frequency_batches == 1 ? 0 : b;
    for (int t = 0; t < Lq; ++t)
      rope_rmsnorm64(q + (((int64_t)b * Lq + t) * H + h) * D,
                     freqs + (((int64_t)fb * Lk + selected[t]) * H + h) * D,
                     q_gamma + (int64_t)h * D, q_bhld + (bh * Lq + t) * D);
    float* pk = packed_k + bh * D * (int64_t)Lk_padded;
    float* pv = packed_v + bh * D * (int64_t)Lk_padded;
    for (int t = 0; t < Lk; ++t) {
      const float* ks = kv + (((int64_t)b * Lk + t) * 2 * H + h) * D;
      const float* vs = ks + (int64_t)H * D;
      float kn[OR_HEAD_DIM];
      rope_rmsnorm64(ks, freqs + (((int64_t)fb * Lk + t) * H + h) * D, k_gamma + (int64_t)h * D, kn);
      for (int d = 0; d < D; ++d) {
        pk[(int64_t)d * Lk_padded + t] = kn[d];
        pv[(int64_t)d * Lk_padded + t] = vs[d];
      }
    }
    for (int d = 0; d < D; ++d)
      for (int t = Lk; t < Lk_padded; ++t) {
        pk[(int64_t)d * Lk_padded + t] = 0.0f;
        pv[(int64_t)d * Lk_padded + t] = 0.0f;
      }
  }
  return 0;
}

/* scripts/gemm_nf24_qkv_direct_avx512.c:87-199: the NF24 QKV GEMM (same
 * per-output chain as the plain GEMM) immediately followed by the
 * postprocess above; N must be 3*H*64.  Bit-identical to GEMM followed by
 * oracle_qkv_rope_rmsnorm_pack, which is how it is computed here. */
int oracle_gemm_nf24_qkv_direct(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                const float* scale, const float* bias, const float* freqs,
                                const float* q_gamma, const float* k_gamma, float* q_bhld,
                                float* packed_k, float* packed_v, int B, int L, int K, int N,
                                int H, int D, int L_padded, int frequency_batches) {
  if (!x || !code01_t || !q2_t || !scale || !bias || !freqs || !q_gamma || !k_gamma || !q_bhld ||
      !packed_k || !packed_v)
    return -1;
  if (B <= 0 || L <= 0 || K <= 0 || H <= 0 || D != OR_HEAD_DIM || N != 3 * H * D ||
      L_padded < L || (L_padded & 15) != 0 || (frequency_batches != 1 && frequency_batches != B))
    return -2;
  float* qkv = (float*)malloc(sizeof(float) * (size_t)B * L * N);
  if (!qkv) return -5;
  int st = oracle_nf24_gemm_range(x, code01_t, q2_t, scale, bias, qkv, B * L, K, N, 0, N, K, N, 1);
  if (st == 0)
    st = oracle_qkv_rope_rmsnorm_pack(qkv, freqs, q_gamma, k_gamma, q_bhld, packed_k, packed_v, B,
                                      L, H, D, L_padded, frequency_batches);
  free(qkv);
  return st;
}

/* ------------------------------------------------------------------ */
/* Flow-block elementwise kernels.  A row is processed as the reference's
 * 16-lane vectors: lane j accumulates columns j, j+16, ... sequentially and
 * the lanes are combined by reduce_add16; masked lanes read 0. */

/* scripts/native_norm_rope_avx512.c:13-49.  The variance pass subtracts the
 * mean from every lane of every 16-column chunk, so masked lanes of a
 * partial last chunk contribute mean^2 (as the reference does). */
int oracle_layernorm(const float* input, const float* weight, const float* bias, float* output,
                     int64_t rows, int cols, float eps, int has_affine) {
  if (input == 0 || output == 0) return -1;
  if (rows <= 0 || cols <= 0 || eps < 0.0f) return -2;
  if (has_affine && (weight == 0 || bias == 0)) return -3;
  for (int64_t row = 0; row < rows; ++row) {
    const float* src = input + row * (int64_t)cols;
    float* dst = output + row * (int64_t)cols;
    float acc[OR_LANES] = {0};
    for (int col = 0; col < cols; col += OR_LANES)
      for (int j = 0; j < OR_LANES; ++j) acc[j] += (col + j < cols) ? src[col + j] : 0.0f;
    const float mean = reduce_add16(acc) / (float)cols;
    float var[OR_LANES] = {0};
    for (int col = 0; col < cols; col += OR_LANES)
      for (int j = 0; j < OR_LANES; ++j) {
        const float d = ((col + j < cols) ? src[col + j] : 0.0f) - mean;
        var[j] = fmaf(d, d, var[j]);
      }
    const float inv_std = 1.0f / sqrtf(reduce_add16(var) / (float)cols + eps);
    for (int c = 0; c < cols; ++c) {
      float y = (src[c] - mean) * inv_std;
      if (has_affine) y = fmaf(y, weight[c], bias[c]);
      dst[c] = y;
    }
  }
  return 0;
}

/* native_norm_rope_avx512.c:51-83: x * (sqrt(dim) / max(||x||, eps)) * gamma[h]. */
int oracle_multihead_rmsnorm(const float* input, const float* gamma, float* output, int64_t outer,
                             int heads, int dim, float eps) {
  if (input == 0 || gamma == 0 || output == 0) return -1;
  if (outer <= 0 || heads <= 0 || dim <= 0 || eps < 0.0f) return -2;
  for (int64_t vec = 0; vec < outer * heads; ++vec) {
    const float* src = input + vec * dim;
    const float* g = gamma + (int64_t)(vec % heads) * dim;
    float* dst = output + vec * dim;
    float acc[OR_LANES] = {0};
    for (int d = 0; d < dim; d += OR_LANES)
      for (int j = 0; j < OR_LANES; ++j) {
        const float x = (d + j < dim) ? src[d + j] : 0.0f;
        acc[j] = fmaf(x, x, acc[j]);
      }
    const float norm = sqrtf(reduce_add16(acc));
    const float factor = sqrtf((float)dim) / fmaxf(norm, eps);
    for (int d = 0; d < dim; ++d) dst[d] = (src[d] * factor) * g[d];
  }
  return 0;
}

/* native_norm_rope_avx512.c:85-119: fmaddsub(x_re, f, x_im * swap(f)). */
int oracle_rope_complex(const float* input, const float* freqs, float* output, int64_t vectors,
                        int dim) {
  if (input == 0 || freqs == 0 || output == 0) return -1;
  if (vectors <= 0 || dim <= 0 || (dim & 1) != 0) return -2;
  for (int64_t i = 0; i < vectors * dim; i += 2) {
    const float re = input[i], im = input[i + 1], c = freqs[i], s = freqs[i + 1];
    output[i] = fmaf(re, c, -(im * s));
    output[i + 1] = fmaf(re, s, im * c);
  }
  return 0;
}

/* native_block_elementwise_avx512.c:9-22: h * (1 + scale) + shift, one fma. */
int oracle_modulate_inplace(float* h, const float* scale, const float* shift, int batch, int rows,
                            int cols) {
  if (!h || !scale || !shift) return -1;
  if (batch <= 0 || rows <= 0 || cols <= 0) return -2;
  for (int64_t r = 0; r < (int64_t)batch * rows; ++r) {
    const int64_t b = r / rows;
    float* dst = h + r * cols;
    for (int c = 0; c < cols; ++c)
#ifndef ORACLE_EW_UNFUSED
      dst[c] = fmaf(dst[c], 1.0f + scale[b * cols + c], shift[b * cols + c]);
#else /* planted mistake for the tests: the contracted fma written unfused */
      dst[c] = dst[c] * (1.0f + scale[b * cols + c]) + shift[b * cols + c];
#endif
  }
  return 0;
}

/* native_block_elementwise_avx512.c:24-35: delta *= gate; base += delta. */
int oracle_gated_residual_inplace(float* base, float* delta, const float* gate, int batch,
                                  int rows, int cols) {
  if (!base || !delta || !gate) return -1;
  if (batch <= 0 || rows <= 0 || cols <= 0) return -2;
  for (int64_t r = 0; r < (int64_t)batch * rows; ++r) {
    const float* g = gate + (r / rows) * cols;
    for (int c = 0; c < cols; ++c) {
      const float hv = delta[r * cols + c] * g[c];
      delta[r * cols + c] = hv;
      base[r * cols + c] = base[r * cols + c] + hv;
    }
  }
  return 0;
}

/* native_block_elementwise_avx512.c:37-46. */
int oracle_add_inplace(float* base, const float* delta, int64_t count) {
  if (!base || !delta) return -1;
  if (count <= 0) return -2;
  for (int64_t i = 0; i < count; ++i) base[i] = base[i] + delta[i];
  return 0;
}

/* native_gelu_avx512.c:33-68: 0.5x (1 + tanh(0.79788456 (x + 0.044715 x^3)))
 * with tanh(u) = sign(u) (1 - 2 / (exp512(2|u|) + 1)), 0 at u = 0; the
 * x + 0.044715 x^3 is one fma in the reference build. */
static inline float gelu_tanh_lane(float x) {
  const float x2 = x * x;
#ifndef ORACLE_EW_UNFUSED
  const float s = fmaf(0.044715f, x2 * x, x);
#else /* planted mistake for the tests */
  const float s = x + 0.044715f * (x2 * x);
#endif
  const float inner = 0.7978845608028654f * s;
  const float e = exp512_lane(2.0f * fabsf(inner));
  float t = 1.0f - 2.0f / (e + 1.0f);
  t = copysignf(t, inner);
  if (inner == 0.0f) t = 0.0f;
  return (0.5f * x) * (1.0f + t);
}

int oracle_gelu_tanh(const float* input, float* output, int64_t count) {
  if (input == 0 || output == 0) return -1;
  if (count <= 0) return -2;
  for (int64_t i = 0; i < count; ++i) output[i] = gelu_tanh_lane(input[i]);
  return 0;
}

/* native_silu_avx512_extra.c:28-45: x / (1 + exp512(0 - x)). */
int oracle_silu(const float* input, float* output, int64_t count) {
  if (input == 0 || output == 0) return -1;
  if (count <= 0) return -2;
  for (int64_t i = 0; i < count; ++i) output[i] = input[i] / (1.0f + exp512_lane(0.0f - input[i]));
  return 0;
}

/* native_sampler_avx512.c:19-54: positive = g * positive - (g - 1) * negative. */
int oracle_cfg_combine_inplace(float* positive, const float* negative, const float* guidance,
                               int batch, int64_t per_batch) {
  if (!positive || !negative || !guidance) return -1;
  if (batch <= 0 || per_batch <= 0) return -2;
  for (int b = 0; b < batch; ++b) {
    const float g = guidance[b], gm1 = g - 1.0f;
    for (int64_t i = (int64_t)b * per_batch; i < (int64_t)(b + 1) * per_batch; ++i)
      positive[i] = g * positive[i] - gm1 * negative[i];
  }
  return 0;
}

/* native_sampler_avx512.c:56-89: sample -= dt * prediction. */
int oracle_euler_update_inplace(float* sample, const float* prediction, const float* dt, int batch,
                                int64_t per_batch) {
  if (!sample || !prediction || !dt) return -1;
  if (batch <= 0 || per_batch <= 0) return -2;
  for (int b = 0; b < batch; ++b)
    for (int64_t i = (int64_t)b * per_batch; i < (int64_t)(b + 1) * per_batch; ++i)
      sample[i] = sample[i] - dt[b] * prediction[i];
  return 0;
}

/* native_sampler_avx512.c:91-134: with r = 0.5 * dt / max(prev_dt, 1e-12),
 * sample -= dt * ((1 + r) * prediction - r * previous_prediction). */
int oracle_ab2_update_inplace(float* sample, const float* prediction, const float* previous,
                              const float* dt, const float* previous_dt, int batch,
                              int64_t per_batch) {
  if (!sample || !prediction || !previous || !dt || !previous_dt) return -1;
  if (batch <= 0 || per_batch <= 0) return -2;
  for (int b = 0; b < batch; ++b) {
    const float r = 0.5f * (dt[b] / fmaxf(previous_dt[b], 1.0e-12f));
    const float cs = 1.0f + r;
    for (int64_t i = (int64_t)b * per_batch; i < (int64_t)(b + 1) * per_batch; ++i) {
      const float eff = cs * prediction[i] - r * previous[i];
      sample[i] = sample[i] - dt[b] * eff;
    }
  }
  return 0;
}

int oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
