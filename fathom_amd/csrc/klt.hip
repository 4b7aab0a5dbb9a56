// Query side of the KLT-rotated bit-plane store (scripts/R_ruler.py:63-64,
// 82-84, the "planesK" method): the store holds bit planes of (K - mu) @ Vt,
// so each decode step rotates the query the same way, qr = q @ Vt, and plans
// from the gains g_e = sum_g qr_ge^2 * lam_e of the rotated coordinates.
//
// A workgroup owns 16 output coordinates of one (batch, KV head) row, with the
// G query heads staged in LDS: thread (c, p) sums q_g[d] * Vt[d, e0 + c] over
// the p-th of 16 d ranges (fp32 FMAs, ascending d, every load in flight at
// once), and the range sums are added in order; the gain follows in head order.
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kKltThreads = 256;
constexpr int kKltMaxG = 32;                     // query heads per (batch, KV head) row
constexpr int kKltMaxD = 256;
constexpr int kKltCols = 16;                     // output coordinates per workgroup
constexpr int kKltParts = kKltThreads / kKltCols;  // d ranges per coordinate

// MAXG: the heads the workgroup holds (8 for GQA groups of up to 8, else 32).
template <int MAXG>
__global__ __launch_bounds__(kKltThreads) void klt_query_kernel(const float *__restrict__ q,
                                                                 const float *__restrict__ Vt,
                                                                 const float *__restrict__ lam, int G, int D,
                                                                 float *__restrict__ qr, float *__restrict__ gain) {
  __shared__ float qs[MAXG][kKltMaxD];
  __shared__ float part[kKltParts][MAXG][kKltCols];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.y;
  const int e0 = blockIdx.x * kKltCols;
  for (int e = tid; e < G * D; e += kKltThreads) qs[e / D][e % D] = q[bh * G * D + e];
  __syncthreads();
  const float *V = Vt + bh * (int64_t)D * D;
  const int c = tid % kKltCols, pt = tid / kKltCols, e = e0 + c;
  const int per = (D + kKltParts - 1) / kKltParts;
  float acc[MAXG];
#pragma unroll
  for (int g = 0; g < MAXG; ++g) acc[g] = 0.0f;
  if (e < D) {
    for (int i = 0; i < per; ++i) {
      const int d = pt * per + i;
      if (d < D) {
        const float v = V[(int64_t)d * D + e];
#pragma unroll
        for (int g = 0; g < MAXG; ++g)
          if (g < G) acc[g] = fmaf(qs[g][d], v, acc[g]);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < MAXG; ++g) part[pt][g][c] = acc[g];
  __syncthreads();
  if (tid < kKltCols && e0 + tid < D) {
    const int eo = e0 + tid;
    const float l = lam[bh * D + eo];
    float s = 0.0f;
    for (int g = 0; g < G; ++g) {
      float r = 0.0f;
      for (int p = 0; p < kKltParts; ++p) r += part[p][g][tid];  // the d ranges in order
      qr[(bh * G + g) * D + eo] = r;
      s += (r * r) * l;  // ((qr ** 2) * lam).sum over heads, in head order
    }
    gain[bh * D + eo] = s;
  }
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_klt_query(const float *q, const float *Vt, const float *lam, int64_t BH, int64_t G, int64_t D,
                                float *qr, float *gain, void *stream) {
  if (!q || !Vt || !lam || !qr || !gain) return fail(FATHOM_ERR_INVALID, "klt_query: null pointer");
  if (BH < 1 || BH > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "klt_query: BH=%lld", (long long)BH);
  if (G < 1 || G > kKltMaxG) return fail(FATHOM_ERR_INVALID, "klt_query: G=%lld outside [1, %d]", (long long)G, kKltMaxG);
  if (D < 1 || D > kKltMaxD) return fail(FATHOM_ERR_INVALID, "klt_query: D=%lld outside [1, %d]", (long long)D, kKltMaxD);
  const dim3 grid((unsigned)cdiv(D, kKltCols), (unsigned)BH);
  if (BH > 65535) return fail(FATHOM_ERR_INVALID, "klt_query: BH=%lld above 65535", (long long)BH);
  if (G <= 8)
    klt_query_kernel<8><<<grid, kKltThreads, 0, (hipStream_t)stream>>>(q, Vt, lam, (int)G, (int)D, qr, gain);
  else
    klt_query_kernel<kKltMaxG><<<grid, kKltThreads, 0, (hipStream_t)stream>>>(q, Vt, lam, (int)G, (int)D, qr, gain);
  return launch_status("klt_query_kernel");
}
