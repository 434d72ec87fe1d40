// Shared definitions for the gfx950 kernels of the NF24 GEMM / exact SDPA path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsplat {

// Status codes.  -1..-5 keep the meaning the reference kernels give them
// (scripts/gemm_nf24_i16_avx512.c:171-175, native_sdpa_avx512_exact_q8t512.c:151-166);
// -6 and -7 are the device-side failures a CPU kernel cannot have; -8 is the
// limit of the no-allocation SDPA entry point.
enum Status : int {
  kOk = 0,
  kErrNull = -1,        // a required pointer is null
  kErrDims = -2,        // bad sizes / stages / head dim
  kErrRange = -3,       // range, stride or key-bias length mismatch
  kErrAlign = -4,       // range not a multiple of 16 (range API)
  kErrWorkspace = -5,   // device workspace could not be allocated
  kErrPointer = -6,     // pointer is not device memory, or its allocation is too small
  kErrLaunch = -7,      // HIP launch / runtime error
  kErrScratch = -8,     // the call needs more scratch than the static no-allocation buffer
};

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// One MFMA step: D(32x32) += A(32x2) * B(2x32), fp32 in, fp32 accumulate.
// Lane l supplies A[l%32][l/32] and B[l/32][l%32]; D register r of lane l
// holds D[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ floatx16 mfma32x32x2(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// fp32 -> bf16 -> fp32 round trip, nearest with ties to even; Inf and NaN
// keep their upper 16 bits (scripts/native_qkv_postprocess_bf16_probe_avx512.c:11-22).
__device__ __forceinline__ float bf16_roundtrip(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) != 0x7f800000u) u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

// Buffer-resource loads.  A raw buffer (stride 0) covers num_records bytes
// from its base; a lane whose byte offset is >= num_records reads 0 and
// touches no memory.  Hot loops address their operands as 32-bit offsets
// from such a base: no 64-bit address arithmetic per load, and bounds that
// would be exec-mask branches become an offset of kBufOob.  Callers keep
// every buffer below 2^31 bytes, so kBufOob plus any in-range step stays out
// of range without wrapping.
constexpr uint32_t kBufOob = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Compute units of the current device, queried once per device (256 on
// MI355X, also the fallback when the query fails; the count only shapes
// launch plans).  Defined in nf24_gemm.hip.
int compute_units();

// Workgroup i of a launch is placed on XCD i % 8.  Renumber so that each XCD
// receives one contiguous run of tile indices (neighbouring tiles share L2).
__device__ __forceinline__ int xcd_tile_index(int id, int count) {
  constexpr int kXcds = 8;
  if (count % kXcds != 0) return id;
  return (id % kXcds) * (count / kXcds) + id / kXcds;
}

}  // namespace tsplat
