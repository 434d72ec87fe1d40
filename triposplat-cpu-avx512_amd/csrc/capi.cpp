// C-ABI layer of libtsplat_hip.so: argument validation with the reference's
// status codes, device-pointer extent checks, and dispatch to the gfx950
// kernels.  Declarations and the reference interface each symbol replaces
// are in include/tsplat_hip.h.

#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cstdint>
#include <vector>

#include "tsplat_common.h"
#include "tsplat_launch.h"
#include "capi_internal.h"
#include "../../include/tsplat_hip.h"

namespace tsplat {
namespace {
constexpr int kSdpaHeadDim = 64;
std::atomic<int> g_last_hip_error{0};
std::atomic<int> g_sdpa_query_tile{512};
}  // namespace

void note_sdpa_query_tile(int queries) {
  g_sdpa_query_tile.store(queries, std::memory_order_relaxed);
}
int sdpa_query_tile() { return g_sdpa_query_tile.load(std::memory_order_relaxed); }

int note(hipError_t e) {
  if (e != hipSuccess) g_last_hip_error.store((int)e);
  return e == hipSuccess ? kOk : kErrLaunch;
}

int DeviceRanges::check(const void* p, int64_t bytes) {
  if (p == nullptr) return kErrNull;
  if (bytes <= 0) return kOk;
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  if ((uint64_t)bytes > UINTPTR_MAX - lo) return kErrPointer;
  const uintptr_t hi = lo + (uintptr_t)bytes;
  for (int i = 0; i < count_; ++i)
    if (lo >= lo_[i] && hi <= hi_[i]) return kOk;
  if (device_ < 0 && hipGetDevice(&device_) != hipSuccess) {
    device_ = -1;
    return kErrPointer;
  }
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return kErrPointer;
  }
  if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged) return kErrPointer;
  if (attr.device != device_) return kErrPointer;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  e = hipMemGetAddressRange(&base, &size, const_cast<void*>(p));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return kErrPointer;
  }
  const uintptr_t base_lo = reinterpret_cast<uintptr_t>(base);
  if (lo < base_lo || hi - base_lo > (uintptr_t)size) return kErrPointer;
  if (count_ < kMaxRanges) {
    lo_[count_] = base_lo;
    hi_[count_] = base_lo + (uintptr_t)size;
    ++count_;
  }
  return kOk;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int sync_null_stream() { return note(hipStreamSynchronize(nullptr)); }

int sdpa_checked(const float* q, const float* k, const float* v, const float* bias, float* out,
                 int B, int H, int Lq, int Lk, int D, int has_bias, int bias_len,
                 int64_t bias_head_stride, int kv_packed, int Lkp, int out_blhd,
                 hipStream_t stream, int precision, float* scratch, size_t scratch_bytes) {
  if (!q || !k || !v || !out) return kErrNull;
  if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0 || D != kSdpaHeadDim) return kErrDims;
  if (precision != kPrecisionFp32 && precision != kPrecisionBf16 && precision != kPrecisionBf16x3)
    return kErrDims;
  if (kv_packed != 0 && kv_packed != 1) return kErrDims;
  if (kv_packed && (Lkp < Lk || (Lkp & 15) != 0)) return kErrDims;
  if (has_bias && (bias == nullptr || bias_len != Lk)) return kErrRange;
  if (has_bias && bias_head_stride != 0 && bias_head_stride < Lk) return kErrRange;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return kErrAlign;
  const int64_t bh = (int64_t)B * H;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(q, bh * Lq * kSdpaHeadDim * 4));
  const int64_t kv_elems = kv_packed ? bh * kSdpaHeadDim * Lkp : bh * Lk * kSdpaHeadDim;
  TSPLAT_CHECK(ptrs.check(k, kv_elems * 4));
  TSPLAT_CHECK(ptrs.check(v, kv_elems * 4));
  TSPLAT_CHECK(ptrs.check(out, bh * Lq * kSdpaHeadDim * 4));
  if (has_bias) TSPLAT_CHECK(ptrs.check(bias, ((int64_t)(H - 1) * bias_head_stride + Lk) * 4));
  SdpaParams p{q, k, v, has_bias ? bias : nullptr, out, B, H, Lq, Lk, kv_packed, Lkp,
               bias_head_stride, out_blhd, precision, scratch, scratch_bytes};
  const int st = launch_sdpa(p, stream);
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

}  // namespace tsplat

using namespace tsplat;

namespace {

constexpr int kHeadDim = 64;
constexpr int kAbiVersion = 4;

// Profile of the blocking (reference-named) SDPA calls: calls, host time
// spent growing the key-split workspace (allocate), the rest of the call up
// to the device's completion (compute), and workspace release (free).
// There is no pack step: the kernel reads [B, H, L, 64] k/v in place.
std::atomic<uint64_t> g_sdpa_calls{0};
std::atomic<uint64_t> g_sdpa_ns{0};
std::atomic<uint64_t> g_sdpa_alloc_ns{0};
std::atomic<uint64_t> g_sdpa_free_ns{0};

// ---------------------------------------------------------------- GEMM
int gemm_checked(const float* x, const int16_t* code01, const int8_t* q2, const float* scale,
                 const float* bias, float* out, int M, int K, int N, int start, int count,
                 int stride_x, int stride_out, hipStream_t stream) {
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(x, ((int64_t)(M - 1) * stride_x + K) * 4));
  TSPLAT_CHECK(ptrs.check(code01, (int64_t)K * N * 2));
  TSPLAT_CHECK(ptrs.check(q2, (int64_t)K * N));
  TSPLAT_CHECK(ptrs.check(scale, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(bias, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(out, ((int64_t)(M - 1) * stride_out + count) * 4));
  GemmParams p{x, code01, q2, scale, bias, out, M, K, N, start, count, stride_x, stride_out};
  const int st = launch_nf24_gemm(p, stream);
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

bool ref_gemm_ptrs_ok(const void* a, const void* b, const void* c, const void* d, const void* e,
                      const void* f, const void* g, const void* h, const void* i, const void* j) {
  return a && b && c && d && e && f && g && h && i && j;
}

int sdpa_blocking(const float* q, const float* k, const float* v, const float* bias, float* out,
                  int B, int H, int Lq, int Lk, int D, int has_bias, int bias_len, int kv_packed,
                  int Lkp, int out_blhd) {
  const auto t0 = std::chrono::steady_clock::now();
  uint64_t alloc_ns0 = 0, alloc_ns1 = 0;
  workspace_timing(kSlotSdpaPartial, &alloc_ns0, nullptr);
  int st = sdpa_checked(q, k, v, bias, out, B, H, Lq, Lk, D, has_bias, bias_len, 0, kv_packed,
                        Lkp, out_blhd, nullptr, kPrecisionFp32, nullptr, 0);
  if (st == kOk) st = sync_null_stream();
  if (st == kOk) {
    const auto t1 = std::chrono::steady_clock::now();
    workspace_timing(kSlotSdpaPartial, &alloc_ns1, nullptr);
    const uint64_t total =
        (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
    const uint64_t alloc = alloc_ns1 - alloc_ns0;
    g_sdpa_calls.fetch_add(1, std::memory_order_relaxed);
    g_sdpa_alloc_ns.fetch_add(alloc, std::memory_order_relaxed);
    g_sdpa_ns.fetch_add(total > alloc ? total - alloc : 0, std::memory_order_relaxed);
  }
  return st;
}

// ---------------------------------------------------------------- QKV
int post_checked(const float* qkv, const float* freqs, const float* qg, const float* kg,
                 float* q, float* pk, float* pv, int B, int L, int H, int D, int Lp, int fb,
                 hipStream_t stream, int kv_round = 0) {
  if (!qkv || !freqs || !qg || !kg || !q || !pk || !pv) return kErrNull;
  if (kv_round < 0 || kv_round > 3) return kErrDims;
  if (B <= 0 || L <= 0 || H <= 0 || D != kHeadDim || Lp < L || (Lp & 15) != 0 ||
      (fb != 1 && fb != B))
    return kErrDims;
  if (!aligned16(qkv) || !aligned16(freqs) || !aligned16(qg) || !aligned16(kg) ||
      !aligned16(q) || !aligned16(pk) || !aligned16(pv))
    return kErrAlign;
  const int64_t C = (int64_t)H * kHeadDim;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(qkv, (int64_t)B * L * 3 * C * 4));
  TSPLAT_CHECK(ptrs.check(freqs, (int64_t)fb * L * C * 4));
  TSPLAT_CHECK(ptrs.check(qg, C * 4));
  TSPLAT_CHECK(ptrs.check(kg, C * 4));
  TSPLAT_CHECK(ptrs.check(q, (int64_t)B * L * C * 4));
  TSPLAT_CHECK(ptrs.check(pk, (int64_t)B * C * Lp * 4));
  TSPLAT_CHECK(ptrs.check(pv, (int64_t)B * C * Lp * 4));
  QkvPostParams p{qkv, freqs, qg, kg, q, pk, pv, B, L, H, Lp, fb, kv_round};
  const int st = launch_qkv_postprocess(p, stream);
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

int selected_checked(const float* q, const float* kv, const float* freqs, const int64_t* sel,
                     const float* qg, const float* kg, float* q_out, float* pk, float* pv, int B,
                     int Lq, int Lk, int H, int D, int Lkp, int fb, hipStream_t stream,
                     int kv_round = 0) {
  if (!q || !kv || !freqs || !sel || !qg || !kg || !q_out || !pk || !pv) return kErrNull;
  if (kv_round < 0 || kv_round > 3) return kErrDims;
  if (B <= 0 || Lq <= 0 || Lk <= 0 || H <= 0 || D != kHeadDim || Lkp < Lk || (Lkp & 15) != 0 ||
      (fb != 1 && fb != B))
    return kErrDims;
  if (!aligned16(pk) || !aligned16(pv)) return kErrAlign;
  const int64_t C = (int64_t)H * kHeadDim;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(q, (int64_t)B * Lq * C * 4));
  TSPLAT_CHECK(ptrs.check(kv, (int64_t)B * Lk * 2 * C * 4));
  TSPLAT_CHECK(ptrs.check(freqs, (int64_t)fb * Lk * C * 4));
  TSPLAT_CHECK(ptrs.check(sel, (int64_t)Lq * 8));
  TSPLAT_CHECK(ptrs.check(qg, C * 4));
  TSPLAT_CHECK(ptrs.check(kg, C * 4));
  TSPLAT_CHECK(ptrs.check(q_out, (int64_t)B * Lq * C * 4));
  TSPLAT_CHECK(ptrs.check(pk, (int64_t)B * C * Lkp * 4));
  TSPLAT_CHECK(ptrs.check(pv, (int64_t)B * C * Lkp * 4));
  QkvSelectedParams p{q, kv, freqs, sel, qg, kg, q_out, pk, pv, B, Lq, Lk, H, Lkp, fb, kv_round};
  const int st = launch_qkv_selected_postprocess(p, stream);
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

int qkv_direct_checked(const float* x, const int16_t* code01, const int8_t* q2,
                       const float* scale, const float* bias, const float* freqs,
                       const float* qg, const float* kg, float* q, float* pk, float* pv, int B,
                       int L, int K, int N, int H, int D, int Lp, int fb, hipStream_t stream,
                       int precision = kPrecisionFp32, int kv_layout = 0, int kv_round = 0,
                       const uint16_t* w_hi = nullptr, const uint16_t* w_lo = nullptr,
                       bool with_planes = false) {
  if (!x || !code01 || !q2 || !scale || !bias || !freqs || !qg || !kg || !q || !pk || !pv)
    return kErrNull;
  if (with_planes && (!w_hi || (precision == kPrecisionBf16x3 && !w_lo))) return kErrNull;
  if (kv_round < 0 || kv_round > 3) return kErrDims;
  if (precision != kPrecisionFp32 && precision != kPrecisionBf16 && precision != kPrecisionBf16x3)
    return kErrDims;
  if (kv_layout != 0 && kv_layout != 1) return kErrDims;
  if (kv_layout == 1) Lp = ((L + 15) / 16) * 16;  // unused by the [B, H, L, 64] layout
  if (B <= 0 || L <= 0 || K <= 0 || H <= 0 || D != kHeadDim || N != 3 * H * D || Lp < L ||
      (Lp & 15) != 0 || (fb != 1 && fb != B))
    return kErrDims;
  const int64_t M = (int64_t)B * L;
  if (M > 0x7fffffff) return kErrDims;
  if (!aligned16(pk) || !aligned16(pv)) return kErrAlign;
  const int64_t C = (int64_t)H * kHeadDim;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(x, M * K * 4));
  TSPLAT_CHECK(ptrs.check(code01, (int64_t)K * N * 2));
  TSPLAT_CHECK(ptrs.check(q2, (int64_t)K * N));
  TSPLAT_CHECK(ptrs.check(scale, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(bias, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(freqs, (int64_t)fb * L * C * 4));
  TSPLAT_CHECK(ptrs.check(qg, C * 4));
  TSPLAT_CHECK(ptrs.check(kg, C * 4));
  TSPLAT_CHECK(ptrs.check(q, M * C * 4));
  const int64_t kv_keys = kv_layout == 1 ? L : Lp;
  TSPLAT_CHECK(ptrs.check(pk, (int64_t)B * C * kv_keys * 4));
  TSPLAT_CHECK(ptrs.check(pv, (int64_t)B * C * kv_keys * 4));
  if (with_planes) {
    TSPLAT_CHECK(ptrs.check(w_hi, planes_bytes(K, N)));
    if (precision == kPrecisionBf16x3) TSPLAT_CHECK(ptrs.check(w_lo, planes_bytes(K, N)));
  }
  // RoPE, RMSNorm and the q / packed k,v stores run in the GEMM's epilogue.
  QkvFusedParams p{{x, code01, q2, scale, bias, nullptr, (int)M, K, N, 0, N, K, N, precision},
                   freqs, qg, kg, q, pk, pv, B, L, H, Lp, fb, kv_layout, kv_round};
  p.gemm.w_hi = with_planes ? w_hi : nullptr;
  p.gemm.w_lo = with_planes && precision == kPrecisionBf16x3 ? w_lo : nullptr;
  const int st = launch_nf24_gemm_qkv(p, stream);
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

}  // namespace

extern "C" {

// ------------------------------------------------------------------ GEMM
int triposplat_gemm_rnf8_avx512_range(const float* x, const uint8_t* codes0_t,
                                      const uint8_t* codes1_t, const uint8_t* codes2_t,
                                      const float* scales0, const float* scales1,
                                      const float* scales2, const float* codebook,
                                      const float* bias, float* out, int M, int K, int N,
                                      int output_start, int output_count, int stride_x,
                                      int stride_out, int threads, int stages) {
  (void)threads;
  if (!ref_gemm_ptrs_ok(x, codes0_t, codes1_t, codes2_t, scales0, scales1, scales2, codebook,
                        bias, out))
    return kErrNull;
  if (M <= 0 || K <= 0 || N <= 0 || output_start < 0 || output_count <= 0 || stages != 3)
    return kErrDims;
  if (output_start + output_count > N || stride_x < K || stride_out < output_count)
    return kErrRange;
  if ((output_start & 15) != 0 || (output_count & 15) != 0) return kErrAlign;
  int st = gemm_checked(x, reinterpret_cast<const int16_t*>(codes0_t),
                        reinterpret_cast<const int8_t*>(codes1_t), scales0, bias, out, M, K, N,
                        output_start, output_count, stride_x, stride_out, nullptr);
  return st == kOk ? sync_null_stream() : st;
}

int triposplat_gemm_rnf8_avx512(const float* x, const uint8_t* codes0_t, const uint8_t* codes1_t,
                                const uint8_t* codes2_t, const float* scales0,
                                const float* scales1, const float* scales2, const float* codebook,
                                const float* bias, float* out, int M, int K, int N, int stride_x,
                                int stride_out, int threads, int stages) {
  return triposplat_gemm_rnf8_avx512_range(x, codes0_t, codes1_t, codes2_t, scales0, scales1,
                                           scales2, codebook, bias, out, M, K, N, 0, N, stride_x,
                                           stride_out, threads, stages);
}

int triposplat_gemm_rnf8_avx512_tail(const float* x, const uint8_t* codes0_t,
                                     const uint8_t* codes1_t, const uint8_t* codes2_t,
                                     const float* scales0, const float* scales1,
                                     const float* scales2, const float* codebook,
                                     const float* bias, float* out, int M, int K, int N,
                                     int stride_x, int stride_out, int threads, int stages) {
  (void)threads;
  if (!ref_gemm_ptrs_ok(x, codes0_t, codes1_t, codes2_t, scales0, scales1, scales2, codebook,
                        bias, out))
    return kErrNull;
  if (M <= 0 || K <= 0 || N <= 0 || stride_x < K || stride_out < N || stages != 3)
    return kErrDims;
  int st = gemm_checked(x, reinterpret_cast<const int16_t*>(codes0_t),
                        reinterpret_cast<const int8_t*>(codes1_t), scales0, bias, out, M, K, N,
                        0, N, stride_x, stride_out, nullptr);
  return st == kOk ? sync_null_stream() : st;
}

int triposplat_gemm_rnf8_avx512_row_tile(void) { return 128; }
int triposplat_gemm_rnf8_avx512_residual_mode(void) { return 4; }

int tsplat_nf24_gemm_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                           const float* scale, const float* bias, float* out, int M, int K, int N,
                           int output_start, int output_count, int stride_x, int stride_out,
                           void* stream) {
  if (!x || !code01_t || !q2_t || !scale || !bias || !out) return kErrNull;
  if (M <= 0 || K <= 0 || N <= 0 || output_start < 0 || output_count <= 0) return kErrDims;
  if (output_start + output_count > N || stride_x < K || stride_out < output_count)
    return kErrRange;
  return gemm_checked(x, code01_t, q2_t, scale, bias, out, M, K, N, output_start, output_count,
                      stride_x, stride_out, static_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------ SDPA
int triposplat_sdpa_f32_avx512_exact_q8t512(const float* q, const float* k, const float* v,
                                            const float* key_bias_or_null, float* out, int B,
                                            int H, int Lq, int Lk, int D, int has_key_bias,
                                            int key_bias_len, int threads) {
  (void)threads;
  return sdpa_blocking(q, k, v, key_bias_or_null, out, B, H, Lq, Lk, D, has_key_bias,
                       key_bias_len, 0, 0, 0);
}

int triposplat_sdpa_f32(const float* q, const float* k, const float* v,
                        const float* key_bias_or_null, float* out, int B, int H, int Lq, int Lk,
                        int D, int has_key_bias, int key_bias_len, int threads) {
  return triposplat_sdpa_f32_avx512_exact_q8t512(q, k, v, key_bias_or_null, out, B, H, Lq, Lk, D,
                                                 has_key_bias, key_bias_len, threads);
}

int triposplat_sdpa_f32_avx512_exact_q8(const float* q, const float* k, const float* v,
                                        const float* key_bias_or_null, float* out, int B, int H,
                                        int Lq, int Lk, int D, int has_key_bias,
                                        int key_bias_len, int threads) {
  return triposplat_sdpa_f32_avx512_exact_q8t512(q, k, v, key_bias_or_null, out, B, H, Lq, Lk, D,
                                                 has_key_bias, key_bias_len, threads);
}

int triposplat_sdpa_f32_avx512_exact_q8t512_packed_blhd(
    const float* q, const float* packed_k, const float* packed_v, const float* key_bias_or_null,
    float* out_blhd, int B, int H, int Lq, int Lk, int D, int Lkp, int has_key_bias,
    int key_bias_len, int threads) {
  (void)threads;
  return sdpa_blocking(q, packed_k, packed_v, key_bias_or_null, out_blhd, B, H, Lq, Lk, D,
                       has_key_bias, key_bias_len, 1, Lkp, 1);
}

int triposplat_sdpa_key_tile(void) { return 64; }
int triposplat_sdpa_query_block(void) { return sdpa_query_tile(); }
int triposplat_sdpa_packed_output_is_blhd(void) { return 1; }

void triposplat_sdpa_q8t512_profile_reset(void) {
  g_sdpa_calls.store(0);
  g_sdpa_ns.store(0);
  g_sdpa_alloc_ns.store(0);
  g_sdpa_free_ns.store(0);
}

int triposplat_sdpa_q8t512_profile_get(uint64_t* calls, uint64_t* allocate_ns, uint64_t* pack_ns,
                                       uint64_t* compute_ns, uint64_t* free_ns) {
  if (!calls || !allocate_ns || !pack_ns || !compute_ns || !free_ns) return kErrNull;
  *calls = g_sdpa_calls.load();
  *allocate_ns = g_sdpa_alloc_ns.load();
  *pack_ns = 0;
  *compute_ns = g_sdpa_ns.load();
  *free_ns = g_sdpa_free_ns.load();
  return kOk;
}

int triposplat_sdpa_q8t512_workspace_stats(uint64_t* allocations, uint64_t* capacity_bytes) {
  if (!allocations || !capacity_bytes) return kErrNull;
  uint64_t retired = 0, planes_allocations = 0, planes_bytes = 0;
  workspace_stats(kSlotSdpaPartial, allocations, capacity_bytes, &retired);
  workspace_stats(kSlotSdpaPlanes, &planes_allocations, &planes_bytes, &retired);
  *allocations += planes_allocations;
  *capacity_bytes += planes_bytes;
  return kOk;
}

void triposplat_sdpa_q8t512_workspace_release(void) {
  const auto t0 = std::chrono::steady_clock::now();
  release_workspace(kSlotSdpaPartial);
  release_workspace(kSlotSdpaPlanes);
  g_sdpa_free_ns.fetch_add((uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                               std::chrono::steady_clock::now() - t0)
                               .count(),
                           std::memory_order_relaxed);
}

int tsplat_sdpa_async(const float* q, const float* k, const float* v,
                      const float* key_bias_or_null, float* out, int B, int H, int Lq, int Lk,
                      int D, int has_key_bias, int key_bias_len, int64_t bias_head_stride,
                      int kv_packed, int Lkp, int out_blhd, void* stream) {
  return sdpa_checked(q, k, v, key_bias_or_null, out, B, H, Lq, Lk, D, has_key_bias,
                      key_bias_len, bias_head_stride, kv_packed, Lkp, out_blhd,
                      static_cast<hipStream_t>(stream), kPrecisionFp32, nullptr, 0);
}

int tsplat_sdpa_precision_async(const float* q, const float* k, const float* v,
                                const float* key_bias_or_null, float* out, int B, int H, int Lq,
                                int Lk, int D, int has_key_bias, int key_bias_len,
                                int64_t bias_head_stride, int kv_packed, int Lkp, int out_blhd,
                                int precision, void* stream) {
  return sdpa_checked(q, k, v, key_bias_or_null, out, B, H, Lq, Lk, D, has_key_bias,
                      key_bias_len, bias_head_stride, kv_packed, Lkp, out_blhd,
                      static_cast<hipStream_t>(stream), precision, nullptr, 0);
}

// ------------------------------------------------------------------ QKV
int triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2(const float* qkv, const float* frequencies,
                                                   const float* q_gamma, const float* k_gamma,
                                                   float* q_bhld, float* packed_k,
                                                   float* packed_v, int B, int L, int H, int D,
                                                   int L_padded, int frequency_batches,
                                                   int threads) {
  (void)threads;
  int st = post_checked(qkv, frequencies, q_gamma, k_gamma, q_bhld, packed_k, packed_v, B, L, H,
                        D, L_padded, frequency_batches, nullptr);
  return st == kOk ? sync_null_stream() : st;
}

// The first version zeroed the whole packed buffers before filling them; the
// second clears only tokens L..L_padded-1.  Both leave the same bytes, so
// both names run the same kernel.
int triposplat_qkv_rope_rmsnorm_pack_f32_avx512(const float* qkv, const float* frequencies,
                                                const float* q_gamma, const float* k_gamma,
                                                float* q_bhld, float* packed_k, float* packed_v,
                                                int B, int L, int H, int D, int L_padded,
                                                int frequency_batches, int threads) {
  return triposplat_qkv_rope_rmsnorm_pack_f32_avx512_v2(qkv, frequencies, q_gamma, k_gamma,
                                                        q_bhld, packed_k, packed_v, B, L, H, D,
                                                        L_padded, frequency_batches, threads);
}

// The reference-named postprocess entries of this library store k and v
// exactly (the probe's rounding is the per-call kv_round of the async forms).
int triposplat_qkv_postprocess_bf16_probe_mode(void) { return 0; }

// Tokens per workgroup of the postprocess kernel's k/v transpose.
int triposplat_qkv_postprocess_token_tile(void) { return 64; }
// Only the padding tokens of packed k/v are written as zeros.
int triposplat_qkv_postprocess_v2_tail_only_clear(void) { return 1; }

int triposplat_gemm_nf24_qkv_rope_rmsnorm_pack_f32_avx512(
    const float* x, const uint8_t* codes0_t, const uint8_t* codes1_t, const uint8_t* codes2_t,
    const float* scales0, const float* scales1, const float* scales2, const float* codebook,
    const float* bias, const float* frequencies, const float* q_gamma, const float* k_gamma,
    float* q_bhld, float* packed_k, float* packed_v, int B, int L, int K, int N, int H, int D,
    int L_padded, int frequency_batches, int threads, int stages) {
  (void)threads;
  if (!ref_gemm_ptrs_ok(x, codes0_t, codes1_t, codes2_t, scales0, scales1, scales2, codebook,
                        bias, frequencies) ||
      !q_gamma || !k_gamma || !q_bhld || !packed_k || !packed_v)
    return kErrNull;
  if (stages != 3) return kErrDims;
  int st = qkv_direct_checked(x, reinterpret_cast<const int16_t*>(codes0_t),
                              reinterpret_cast<const int8_t*>(codes1_t), scales0, bias,
                              frequencies, q_gamma, k_gamma, q_bhld, packed_k, packed_v, B, L, K,
                              N, H, D, L_padded, frequency_batches, nullptr);
  return st == kOk ? sync_null_stream() : st;
}

int triposplat_q_kv_selected_rope_rmsnorm_pack_f32_avx512_v2(
    const float* q, const float* kv, const float* frequencies, const int64_t* selected_indices,
    const float* q_gamma, const float* k_gamma, float* q_bhld, float* packed_k, float* packed_v,
    int B, int Lq, int Lk, int H, int D, int Lk_padded, int frequency_batches, int threads) {
  (void)threads;
  if (!q || !kv || !frequencies || !selected_indices || !q_gamma || !k_gamma || !q_bhld ||
      !packed_k || !packed_v)
    return kErrNull;
  if (B <= 0 || Lq <= 0 || Lk <= 0 || H <= 0 || D != kHeadDim || Lk_padded < Lk ||
      (Lk_padded & 15) != 0 || (frequency_batches != 1 && frequency_batches != B))
    return kErrDims;
  // The reference rejects an index outside [0, Lk) with -3 before any work;
  // the indices are device data, so they are read back first.
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(selected_indices, (int64_t)Lq * 8));
  std::vector<int64_t> host((size_t)Lq);
  if (note(hipMemcpy(host.data(), selected_indices, (size_t)Lq * 8, hipMemcpyDeviceToHost)) != kOk)
    return kErrLaunch;
  for (int64_t v : host)
    if (v < 0 || v >= Lk) return kErrRange;
  const int st = selected_checked(q, kv, frequencies, selected_indices, q_gamma, k_gamma, q_bhld,
                                  packed_k, packed_v, B, Lq, Lk, H, D, Lk_padded,
                                  frequency_batches, nullptr);
  return st == kOk ? sync_null_stream() : st;
}

int tsplat_q_kv_selected_postprocess_async(const float* q, const float* kv,
                                           const float* frequencies,
                                           const int64_t* selected_indices,
                                           const float* q_gamma, const float* k_gamma,
                                           float* q_bhld, float* packed_k, float* packed_v, int B,
                                           int Lq, int Lk, int H, int D, int Lk_padded,
                                           int frequency_batches, int kv_round, void* stream) {
  return selected_checked(q, kv, frequencies, selected_indices, q_gamma, k_gamma, q_bhld, packed_k,
                          packed_v, B, Lq, Lk, H, D, Lk_padded, frequency_batches,
                          static_cast<hipStream_t>(stream), kv_round);
}

int triposplat_gemm_nf24_qkv_direct_row_tile(void) { return 128; }
// The projection tile stays in MFMA accumulators: no row-tile cache buffer.
int triposplat_gemm_nf24_qkv_direct_tile_bytes(void) { return 0; }
int triposplat_gemm_nf24_qkv_direct_residual_mode(void) { return 4; }

int tsplat_qkv_postprocess_async(const float* qkv, const float* frequencies, const float* q_gamma,
                                 const float* k_gamma, float* q_bhld, float* packed_k,
                                 float* packed_v, int B, int L, int H, int D, int L_padded,
                                 int frequency_batches, int kv_round, void* stream) {
  return post_checked(qkv, frequencies, q_gamma, k_gamma, q_bhld, packed_k, packed_v, B, L, H, D,
                      L_padded, frequency_batches, static_cast<hipStream_t>(stream), kv_round);
}

int tsplat_gemm_nf24_qkv_direct_async(const float* x, const int16_t* code01_t, const int8_t* q2_t,
                                      const float* scale, const float* bias,
                                      const float* frequencies, const float* q_gamma,
                                      const float* k_gamma, float* q_bhld, float* packed_k,
                                      float* packed_v, int B, int L, int K, int N, int H, int D,
                                      int L_padded, int frequency_batches, void* stream) {
  return qkv_direct_checked(x, code01_t, q2_t, scale, bias, frequencies, q_gamma, k_gamma, q_bhld,
                            packed_k, packed_v, B, L, K, N, H, D, L_padded, frequency_batches,
                            static_cast<hipStream_t>(stream));
}

int tsplat_gemm_nf24_qkv_direct_ex_async(
    const float* x, const int16_t* code01_t, const int8_t* q2_t, const float* scale,
    const float* bias, const float* frequencies, const float* q_gamma, const float* k_gamma,
    float* q_bhld, float* k_out, float* v_out, int B, int L, int K, int N, int H, int D,
    int L_padded, int frequency_batches, int kv_layout, int precision, int kv_round,
    void* stream) {
  return qkv_direct_checked(x, code01_t, q2_t, scale, bias, frequencies, q_gamma, k_gamma, q_bhld,
                            k_out, v_out, B, L, K, N, H, D, L_padded, frequency_batches,
                            static_cast<hipStream_t>(stream), precision, kv_layout, kv_round);
}

int tsplat_gemm_nf24_qkv_direct_planes_async(
    const float* x, const int16_t* code01_t, const int8_t* q2_t, const float* scale,
    const float* bias, const float* frequencies, const float* q_gamma, const float* k_gamma,
    float* q_bhld, float* k_out, float* v_out, int B, int L, int K, int N, int H, int D,
    int L_padded, int frequency_batches, int kv_layout, int precision, int kv_round,
    const uint16_t* w_hi, const uint16_t* w_lo, void* stream) {
  return qkv_direct_checked(x, code01_t, q2_t, scale, bias, frequencies, q_gamma, k_gamma, q_bhld,
                            k_out, v_out, B, L, K, N, H, D, L_padded, frequency_batches,
                            static_cast<hipStream_t>(stream), precision, kv_layout, kv_round, w_hi,
                            w_lo, true);
}

int tsplat_nf24_bf16_planes_async(const int16_t* code01_t, const int8_t* q2_t, const float* scale,
                                  int K, int N, int precision, uint16_t* w_hi, uint16_t* w_lo,
                                  void* stream) {
  if (!code01_t || !q2_t || !scale || !w_hi) return kErrNull;
  if (precision != kPrecisionBf16 && precision != kPrecisionBf16x3) return kErrDims;
  if (precision == kPrecisionBf16x3 && !w_lo) return kErrNull;
  if (K <= 0 || N <= 0) return kErrDims;
  const int64_t count = (int64_t)K * N;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(code01_t, count * 2));
  TSPLAT_CHECK(ptrs.check(q2_t, count));
  TSPLAT_CHECK(ptrs.check(scale, (int64_t)N * 4));
  TSPLAT_CHECK(ptrs.check(w_hi, planes_bytes(K, N)));
  if (precision == kPrecisionBf16x3) TSPLAT_CHECK(ptrs.check(w_lo, planes_bytes(K, N)));
  const int st = launch_nf24_bf16_planes(code01_t, q2_t, scale, K, N, precision, w_hi,
                                         precision == kPrecisionBf16x3 ? w_lo : nullptr,
                                         static_cast<hipStream_t>(stream));
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

// ------------------------------------------------------------------ packer
int tsplat_nf24_pack_async(const float* weight, int out_features, int in_features,
                           const float* alphabet, int alphabet_len, float* base_workspace,
                           int16_t* code01_t, int8_t* q2_t, float* scale, void* stream) {
  if (!weight || !alphabet || !base_workspace || !code01_t || !q2_t || !scale) return kErrNull;
  if (out_features <= 0 || in_features <= 0 || alphabet_len < 2 || alphabet_len > 256)
    return kErrDims;
  const int64_t count = (int64_t)out_features * in_features;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(weight, count * 4));
  TSPLAT_CHECK(ptrs.check(alphabet, (int64_t)alphabet_len * 4));
  TSPLAT_CHECK(ptrs.check(base_workspace, (int64_t)out_features * 4));
  TSPLAT_CHECK(ptrs.check(code01_t, count * 2));
  TSPLAT_CHECK(ptrs.check(q2_t, count));
  TSPLAT_CHECK(ptrs.check(scale, (int64_t)out_features * 4));
  const int st = launch_nf24_pack(weight, out_features, in_features, alphabet, alphabet_len,
                                  base_workspace, code01_t, q2_t, scale,
                                  static_cast<hipStream_t>(stream));
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

int tsplat_nf24_decode_async(const int16_t* code01_t, const int8_t* q2_t, const float* scale,
                             float* out, int in_features, int out_features, int transposed,
                             void* stream) {
  if (!code01_t || !q2_t || !scale || !out) return kErrNull;
  if (in_features <= 0 || out_features <= 0) return kErrDims;
  const int64_t count = (int64_t)in_features * out_features;
  DeviceRanges ptrs;
  TSPLAT_CHECK(ptrs.check(code01_t, count * 2));
  TSPLAT_CHECK(ptrs.check(q2_t, count));
  TSPLAT_CHECK(ptrs.check(scale, (int64_t)out_features * 4));
  TSPLAT_CHECK(ptrs.check(out, count * 4));
  const int st = launch_nf24_decode(code01_t, q2_t, scale, out, in_features, out_features,
                                    transposed ? 1 : 0, static_cast<hipStream_t>(stream));
  if (st == kErrLaunch) (void)note(hipErrorLaunchFailure);
  return st;
}

// ------------------------------------------------------------------ library
int tsplat_abi_version(void) { return kAbiVersion; }
int tsplat_last_hip_error(void) { return g_last_hip_error.load(); }
const char* tsplat_build_arch(void) { return "gfx950"; }

}  // extern "C"
