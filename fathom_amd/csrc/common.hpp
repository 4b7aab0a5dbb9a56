// Shared device helpers and host error plumbing for the gfx950 key-scan library.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fathom_hip.h"

namespace fathom {

constexpr int kBlk = 64;       // tokens per block: one bit per lane of a wave64 plane word
constexpr int kWave = 64;      // CDNA wavefront width

// ------------------------------------------------------------------ host-side errors
// Records a formatted message for fathom_last_error() and returns `code`.
int fail(int code, const char *fmt, ...);
// Turns a HIP error into FATHOM_ERR_HIP with a message naming `what`.
int hip_fail(hipError_t e, const char *what);

inline int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FATHOM_OK : hip_fail(e, what);
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ conversions
__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// float -> bfloat16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return (uint16_t)((u | 0x400000u) >> 16);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t float_to_f16_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }
__device__ __forceinline__ float f16_bits_to_float(uint16_t b) { return __half2float(__ushort_as_half(b)); }

template <int DT>
__device__ __forceinline__ float load_elem(const void *p, int64_t i);
template <>
__device__ __forceinline__ float load_elem<FATHOM_DT_F32>(const void *p, int64_t i) {
  return static_cast<const float *>(p)[i];
}
template <>
__device__ __forceinline__ float load_elem<FATHOM_DT_F16>(const void *p, int64_t i) {
  return f16_bits_to_float(static_cast<const uint16_t *>(p)[i]);
}
template <>
__device__ __forceinline__ float load_elem<FATHOM_DT_BF16>(const void *p, int64_t i) {
  return bf16_bits_to_float(static_cast<const uint16_t *>(p)[i]);
}

// Orderable key of a score: unsigned order == torch.topk value order
// (NaN above +inf, -0.0 equal to +0.0).
__device__ __forceinline__ uint32_t score_key(float s) {
  const uint32_t u = __float_as_uint(s + 0.0f);  // -0.0 + 0.0 = +0.0
  const uint32_t k = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);  // negative: ~u; else u | sign
  return s != s ? 0xFFFFFFFFu : k;
}
constexpr uint32_t kKeyNegInf = 0x007FFFFFu;  // score_key(-inf)

// Inverse of score_key on non-NaN keys: the float whose key is `key` (keys
// above +inf's key decode to NaN, which compares false).
__device__ __forceinline__ float key_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// ------------------------------------------------------------------ wave primitives
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
// Exclusive prefix sum over the 64 lanes of a wave (lane order).
__device__ __forceinline__ int wave_excl_scan_i(int v, int lane) {
  int incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    int u = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += u;
  }
  return incl - v;
}

// Inclusive prefix sum over the 64 lanes of a wave on DPP: shifts by 1, 2, 4
// and 8 within each row of 16 lanes, then the last lane of row 0 (2) added to
// row 1 (3) and that of row 1 to rows 2 and 3.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0u, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Exact wave sum / exclusive prefix sum of small non-negative integers (below
// 2^BITS): bit-sliced with one ballot per bit, so no lane shuffles.
template <int BITS>
__device__ __forceinline__ int wave_sum_small(int v) {
  int s = 0;
#pragma unroll
  for (int b = 0; b < BITS; ++b) s += __popcll(__ballot((v >> b) & 1)) << b;
  return s;
}
template <int BITS>
__device__ __forceinline__ int wave_excl_scan_small(int v, int lane) {
  const uint64_t lt = (1ull << lane) - 1ull;
  int s = 0;
#pragma unroll
  for (int b = 0; b < BITS; ++b) s += __popcll(__ballot((v >> b) & 1) & lt) << b;
  return s;
}

}  // namespace fathom
