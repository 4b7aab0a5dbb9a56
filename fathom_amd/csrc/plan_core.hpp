// The per-row arithmetic of make_plan (kernels/bitplane.py:83-95), shared by
// the plan kernel and the scan prologue that plans its own row: one wave64
// per row, lane l owning channels CPL l .. CPL l + CPL - 1.
#pragma once

#include "common.hpp"

namespace fathom {
namespace plan {

// float32 log2 shared bit-for-bit with the CPU oracle: x = m 2^e with m folded
// into (1/sqrt2, sqrt2], ln m = 2 atanh(s), s = (m-1)/(m+1), odd series to
// z^11 (z = s^2) in Horner form, log2 x = e + ln m * log2(e), every step a
// separate IEEE float64 operation (no contraction), rounded once to float32.
__device__ inline float flog2(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (isinf(x)) return x;
  const uint32_t bits = __float_as_uint(x);
  int e = (int)((bits >> 23) & 0xFFu) - 127;
  double m = (double)(int)((bits & 0x7FFFFFu) | 0x800000u) / 8388608.0;
  if (m > 1.4142135623730951) {
    m = m * 0.5;
    e += 1;
  }
  const double s = (m - 1.0) / (m + 1.0);
  const double z = s * s;
  double p = 1.0 / 23.0;
  p = p * z; p = p + 1.0 / 21.0;
  p = p * z; p = p + 1.0 / 19.0;
  p = p * z; p = p + 1.0 / 17.0;
  p = p * z; p = p + 1.0 / 15.0;
  p = p * z; p = p + 1.0 / 13.0;
  p = p * z; p = p + 1.0 / 11.0;
  p = p * z; p = p + 1.0 / 9.0;
  p = p * z; p = p + 1.0 / 7.0;
  p = p * z; p = p + 1.0 / 5.0;
  p = p * z; p = p + 1.0 / 3.0;
  p = p * z; p = p + 1.0;
  const double ln_m = (2.0 * s) * p;
  const double r = (double)e + ln_m * 1.4426950408889634;
  return (float)r;
}

// Sum of the 64 lanes' values in every lane, for small integers held as
// floats (every partial sum exact, so the order does not matter): DPP row sums
// (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the four
// rows added by v_permlane32_swap and v_permlane16_swap -- all VALU, so the
// bisection's compare needs no round trip through scalar registers.
__device__ __forceinline__ float wave_total_exact(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, true));
  const uint32_t x = __float_as_uint(v);
  const auto p32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
  const uint32_t y = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(y, y, false, false);
  return __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
}

// The row's water line after `iters` bisection steps over [-60, 60] in
// float32 (kernels/bitplane.py:88-95): lg = log2(max(g, 1e-30)) of the lane's
// channels (-inf past D), Br the row's budget.  Depths are integers in [0,
// bmax]: the row's total (an exact integer below 2^11) equals the float sum
// in any order.  The clamp is v_med3 (lg is never NaN: NaN g takes the 1e-30
// floor).
template <int CPL>
__device__ __forceinline__ float water_line(const float (&lg)[CPL], float Br, float bm, int iters) {
#pragma clang fp contract(off)
  auto over = [&](float mid) {
    float s = __builtin_amdgcn_fmed3f(rintf((lg[0] - mid) * 0.5f), 0.0f, bm);
#pragma unroll
    for (int k = 1; k < CPL; ++k) s += __builtin_amdgcn_fmed3f(rintf((lg[k] - mid) * 0.5f), 0.0f, bm);
    return wave_total_exact(s) > Br;
  };
  float lo = -60.0f, hi = 60.0f;
  for (int it = 0; it < iters; ++it) {
    const float mid = (lo + hi) * 0.5f;
    if (over(mid)) lo = mid; else hi = mid;
  }
  return hi;
}

// lg of channel j of row bh (kernels/bitplane.py:89), -inf past D.
__device__ __forceinline__ float channel_lg(const float *g, int64_t bh, int D, int j) {
  return (j < D) ? flog2(fmaxf(g[bh * D + j], 1e-30f)) : -INFINITY;
}

// The depth of a channel at water line hi (kernels/bitplane.py:95).
__device__ __forceinline__ int depth_at(float lg, float hi, float bm) {
#pragma clang fp contract(off)
  return (int)fminf(fmaxf(rintf((lg - hi) * 0.5f), 0.0f), bm);
}

}  // namespace plan
}  // namespace fathom
