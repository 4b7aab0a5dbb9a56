// Per-query reverse water-filling plan: one wave64 per (batch, KV head).
//
// Each lane owns CPL consecutive channels.  The 30-step bisection of the water
// line runs in float32 exactly as kernels/bitplane.py:88-95 states it (wave sum
// of the integer depths is exact in any order); the compacted lists are built
// with wave prefix sums so every output array is written in full (zero padded)
// and no separate clear is needed.
#include "plan_core.hpp"
#include "scan_internal.hpp"

namespace fathom {
namespace {

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
  for (int k = 0; k < CPL; ++k) lg[k] = plan::channel_lg(g, bh, D, lane * CPL + k);
  constexpr int kSumBits = CPL <= 1 ? 4 : CPL <= 2 ? 5 : 6;  // a lane's depth total is below 2^6
  const float Br = budget ? budget[bh] : budget_value;
  const float hi = plan::water_line<CPL>(lg, Br, bm, iters);
  int t[CPL];
  int cnt_act = 0, cnt_pairs = 0;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int j = lane * CPL + k;
    t[k] = (j < D) ? plan::depth_at(lg[k], hi, bm) : 0;
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
