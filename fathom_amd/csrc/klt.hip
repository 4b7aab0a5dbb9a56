// Query side of the KLT-rotated bit-plane store (scripts/R_ruler.py:63-64,
// 82-84, the "planesK" method): the store holds bit planes of (K - mu) @ Vt,
// so each decode step rotates the query the same way, qr = q @ Vt, and plans
// from the gains g_e = sum_g qr_ge^2 * lam_e of the rotated coordinates.
//
// One workgroup per (batch, KV head) row: the G query heads are staged in LDS;
// thread e owns output coordinate e and walks Vt's column e (row-major Vt, so
// the threads of a wave read consecutive floats of each row d) with one fp32
// FMA per (head, d) in ascending d, then forms the gain in head order.
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kKltThreads = 256;
constexpr int kKltMaxG = 8;
constexpr int kKltMaxD = 256;

__global__ __launch_bounds__(kKltThreads) void klt_query_kernel(const float *__restrict__ q,
                                                                 const float *__restrict__ Vt,
                                                                 const float *__restrict__ lam, int G, int D,
                                                                 float *__restrict__ qr, float *__restrict__ gain) {
  __shared__ float qs[kKltMaxG][kKltMaxD];
  const int64_t bh = blockIdx.x;
  for (int e = threadIdx.x; e < G * D; e += kKltThreads) qs[e / D][e % D] = q[bh * G * D + e];
  __syncthreads();
  const float *V = Vt + bh * (int64_t)D * D;
  for (int e = threadIdx.x; e < D; e += kKltThreads) {
    float acc[kKltMaxG];
#pragma unroll
    for (int g = 0; g < kKltMaxG; ++g) acc[g] = 0.0f;
    for (int d = 0; d < D; ++d) {
      const float v = V[(int64_t)d * D + e];
#pragma unroll
      for (int g = 0; g < kKltMaxG; ++g)
        if (g < G) acc[g] = fmaf(qs[g][d], v, acc[g]);
    }
    const float l = lam[bh * D + e];
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < kKltMaxG; ++g) {
      if (g < G) {
        qr[(bh * G + g) * D + e] = acc[g];
        s += (acc[g] * acc[g]) * l;  // ((qr ** 2) * lam).sum over heads, in head order
      }
    }
    gain[bh * D + e] = s;
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
  klt_query_kernel<<<(unsigned)BH, kKltThreads, 0, (hipStream_t)stream>>>(q, Vt, lam, (int)G, (int)D, qr, gain);
  return launch_status("klt_query_kernel");
}
