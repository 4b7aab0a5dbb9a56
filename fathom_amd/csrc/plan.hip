// Per-query reverse water-filling plan: one wave64 per (batch, KV head).
//
// Each lane owns CPL consecutive channels.  The 30-step bisection of the water
// line runs in float32 exactly as kernels/bitplane.py:88-95 states it (wave sum
// of the integer depths is exact in any order); the compacted lists are built
// with wave prefix sums so every output array is written in full (zero padded)
// and no separate clear is needed.
#include "common.hpp"

namespace fathom {
namespace {

// float32 log2 shared bit-for-bit with the CPU oracle: x = m 2^e with m folded
// into (1/sqrt2, sqrt2], ln m = 2 atanh(s), s = (m-1)/(m+1), odd series to
// z^11 (z = s^2) in Horner form, log2 x = e + ln m * log2(e), every step a
// separate IEEE float64 operation (no contraction), rounded once to float32.
__device__ float flog2(float x) {
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

template <int CPL>
__global__ __launch_bounds__(64) void plan_kernel(const float *__restrict__ g, const float *__restrict__ budget,
                                                  float budget_value, int D, int bmax, int iters,
                                                  int8_t *__restrict__ t_out,
                                                  int32_t *__restrict__ pairs, int32_t *__restrict__ npairs,
                                                  int32_t *__restrict__ act, int32_t *__restrict__ nact,
                                                  int32_t *__restrict__ cls, int32_t *__restrict__ clsn) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const float bm = (float)bmax;
  float lg[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int j = lane * CPL + k;
    // kernels/bitplane.py:89: lg = log2(max(g, 1e-30)); NaN g takes the 1e-30 floor.
    lg[k] = (j < D) ? flog2(fmaxf(g[bh * D + j], 1e-30f)) : -INFINITY;
  }
  // depths are integers in [0, bmax]: a lane's sum is below 2^6, the row's
  // (an exact integer below 2^11) equals the float sum in any order
  constexpr int kSumBits = CPL <= 1 ? 4 : CPL <= 2 ? 5 : 6;
  const float Br = budget ? budget[bh] : budget_value;
  // the row's depth total at water line mid exceeds the budget; the clamp is
  // v_med3 (lg is never NaN: NaN g takes the 1e-30 floor)
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
  int t[CPL];
  int cnt_act = 0, cnt_pairs = 0;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int j = lane * CPL + k;
    t[k] = (j < D) ? (int)fminf(fmaxf(rintf((lg[k] - hi) * 0.5f), 0.0f), bm) : 0;
    if (j < D) t_out[bh * D + j] = (int8_t)t[k];
    cnt_act += t[k] > 0;
    cnt_pairs += t[k];
  }
  constexpr int kCntBits = CPL <= 1 ? 1 : CPL <= 2 ? 2 : 3;  // per-lane channel counts <= CPL
  // active channels, ascending
  {
    int pos = wave_excl_scan_small<kCntBits>(cnt_act, lane);
    const int total = wave_sum_small<kCntBits>(cnt_act);
#pragma unroll
    for (int k = 0; k < CPL; ++k)
      if (t[k] > 0) act[bh * D + pos++] = lane * CPL + k;
    for (int i = total + lane; i < D; i += kWave) act[bh * D + i] = 0;
    if (lane == 0) nact[bh] = total;
  }
  // (channel, plane) pairs: channel-major, plane ascending
  {
    int pos = wave_excl_scan_small<kSumBits>(cnt_pairs, lane);
    const int total = wave_sum_small<kSumBits>(cnt_pairs);
    const int64_t base = bh * (int64_t)D * bmax;
#pragma unroll
    for (int k = 0; k < CPL; ++k)
      for (int p = 0; p < t[k]; ++p) pairs[base + pos++] = (lane * CPL + k) * bmax + p;
    for (int i = total + lane; i < D * bmax; i += kWave) pairs[base + i] = 0;
    if (lane == 0) npairs[bh] = total;
  }
  // per-depth channel lists
  for (int c = 1; c <= bmax; ++c) {
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < CPL; ++k) cnt += t[k] == c;
    int pos = wave_excl_scan_small<kCntBits>(cnt, lane);
    const int total = wave_sum_small<kCntBits>(cnt);
    const int64_t base = (bh * bmax + (c - 1)) * (int64_t)D;
#pragma unroll
    for (int k = 0; k < CPL; ++k)
      if (t[k] == c) cls[base + pos++] = lane * CPL + k;
    for (int i = total + lane; i < D; i += kWave) cls[base + i] = 0;
    if (lane == 0) clsn[bh * bmax + (c - 1)] = total;
  }
}

// channel_list (kernels/bitplane.py:128-132): the listed channels of a row
// first, ascending, then the others, ascending (a stable sort of ~active); one
// wave per row, 64 channels per step with ballot prefix counts.
__global__ __launch_bounds__(64) void channel_list_kernel(const uint8_t *__restrict__ active, int64_t D,
                                                          int32_t *__restrict__ act, int32_t *__restrict__ nact) {
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const uint8_t *a = active + bh * D;
  int total = 0;
  for (int64_t j0 = 0; j0 < D; j0 += kWave) {
    const bool on = j0 + lane < D && a[j0 + lane] != 0;
    total += __popcll(__ballot(on));
  }
  int on_base = 0, off_base = total;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int64_t j0 = 0; j0 < D; j0 += kWave) {
    const bool in = j0 + lane < D;
    const bool on = in && a[j0 + lane] != 0;
    const uint64_t mon = __ballot(on), moff = __ballot(in && !on);
    if (in) act[bh * D + (on ? on_base + __popcll(mon & below) : off_base + __popcll(moff & below))] = (int32_t)(j0 + lane);
    on_base += __popcll(mon);
    off_base += __popcll(moff);
  }
  if (lane == 0) nact[bh] = total;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

namespace fathom {
namespace {
int make_plan_run(const float *g, const float *budget, float budget_value, int64_t BH, int64_t D, int bmax, int iters,
                  int8_t *t, int32_t *pairs, int32_t *npairs, int32_t *act, int32_t *nact, int32_t *cls, int32_t *clsn,
                  void *stream) {
  if (!g || !t || !pairs || !npairs || !act || !nact || !cls || !clsn)
    return fail(FATHOM_ERR_INVALID, "make_plan: null pointer");
  if (BH < 1 || BH > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "make_plan: BH=%lld unsupported", (long long)BH);
  if (D < 1 || D > 256) return fail(FATHOM_ERR_INVALID, "make_plan: D=%lld outside [1, 256]", (long long)D);
  if (bmax < 1 || bmax > 8) return fail(FATHOM_ERR_INVALID, "make_plan: bmax=%d outside [1, 8]", bmax);
  if (iters < 0 || iters > 200) return fail(FATHOM_ERR_INVALID, "make_plan: iters=%d outside [0, 200]", iters);
  hipStream_t st = (hipStream_t)stream;
  const int d = (int)D;
  const float bv = budget_value;
  if (D <= 64)
    plan_kernel<1><<<(unsigned)BH, 64, 0, st>>>(g, budget, bv, d, bmax, iters, t, pairs, npairs, act, nact, cls, clsn);
  else if (D <= 128)
    plan_kernel<2><<<(unsigned)BH, 64, 0, st>>>(g, budget, bv, d, bmax, iters, t, pairs, npairs, act, nact, cls, clsn);
  else
    plan_kernel<4><<<(unsigned)BH, 64, 0, st>>>(g, budget, bv, d, bmax, iters, t, pairs, npairs, act, nact, cls, clsn);
  return launch_status("plan_kernel");
}
}  // namespace
}  // namespace fathom

extern "C" int fathom_make_plan(const float *g, const float *budget, int64_t BH, int64_t D, int bmax, int iters,
                                int8_t *t, int32_t *pairs, int32_t *npairs, int32_t *act, int32_t *nact, int32_t *cls,
                                int32_t *clsn, void *stream) {
  if (!budget) return fail(FATHOM_ERR_INVALID, "make_plan: null pointer");
  return make_plan_run(g, budget, 0.0f, BH, D, bmax, iters, t, pairs, npairs, act, nact, cls, clsn, stream);
}

extern "C" int fathom_make_plan_uniform(const float *g, float budget, int64_t BH, int64_t D, int bmax, int iters,
                                        int8_t *t, int32_t *pairs, int32_t *npairs, int32_t *act, int32_t *nact,
                                        int32_t *cls, int32_t *clsn, void *stream) {
  return make_plan_run(g, nullptr, budget, BH, D, bmax, iters, t, pairs, npairs, act, nact, cls, clsn, stream);
}

extern "C" int fathom_channel_list(const uint8_t *active, int64_t BH, int64_t D, int32_t *act, int32_t *nact,
                                   void *stream) {
  if (!active || !act || !nact) return fail(FATHOM_ERR_INVALID, "channel_list: null pointer");
  if (BH < 1 || BH > 0x7FFFFFFF || D < 1) return fail(FATHOM_ERR_INVALID, "channel_list: BH=%lld D=%lld", (long long)BH, (long long)D);
  channel_list_kernel<<<(unsigned)BH, kWave, 0, (hipStream_t)stream>>>(active, D, act, nact);
  return launch_status("channel_list_kernel");
}
