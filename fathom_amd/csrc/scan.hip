// Partial-depth bit-plane scan.
//
// One workgroup (4 waves) owns one (batch*KV-head, 16-block tile = 1024
// tokens).  Active channels are processed 32 at a time:
//   1. stage: the tile's plane words of the chunk's (channel, plane) pairs and
//      its block scales are copied to LDS with coalesced 8-byte loads (16
//      consecutive words of one (channel, plane) are 128 contiguous bytes in the
//      superblock layout); planes past a channel's depth are never read, so the
//      bytes moved are exactly sum_j t_j*8 + 2*nact per block;
//   2. weights: per (channel, block, head) w = q * a * 2^(1-t) and the
//      dequantiser's constant q * a * (2^-t - 1) go to LDS / registers;
//   3. accumulate: lane = token of the block; the t-bit code is assembled from
//      the plane words (plane 0 = MSB), converted once and FMA'd into the G
//      head accumulators.
// The staging reads work unchanged on mapped host memory (zero-copy over PCIe).
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kTB = 16;    // blocks per tile
constexpr int kCH = 32;    // active channels per staged chunk
constexpr int kMaxD = 256;

template <int G>
__global__ __launch_bounds__(256) void scan_planes_kernel(const float *__restrict__ q, int D,
                                                          const int8_t *__restrict__ tpl,
                                                          const int32_t *__restrict__ act,
                                                          const int32_t *__restrict__ nact_p,
                                                          const uint64_t *__restrict__ planes,
                                                          const uint16_t *__restrict__ scales, int64_t n, int64_t nsb,
                                                          int64_t sub, int64_t blk0, int64_t blk_end,
                                                          float *__restrict__ out) {
  __shared__ float q_s[G * kMaxD];
  __shared__ int ch_s[kMaxD];
  __shared__ int dep_s[kMaxD];
  __shared__ uint64_t w_s[kCH * 4 * kTB];
  __shared__ float sc_s[kCH * kTB];
  __shared__ float wt_s[kCH * kTB * G];
  __shared__ float cst_s[kTB * G];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = blockIdx.y;
  const int64_t tb0 = blk0 + (int64_t)blockIdx.x * kTB;
  // Plan entries come from device memory: clamp them so a malformed plan can
  // never index outside q, the store or LDS (a channel outside [0, D) or a
  // depth <= 0 contributes nothing; depths above the store's 4 planes read 4).
  const int nact = min(max(nact_p[bh], 0), D);

  for (int i = tid; i < G * D; i += 256) q_s[i] = q[bh * G * D + i];
  for (int a = tid; a < nact; a += 256) {
    const int j = act[bh * D + a];
    const bool ok = j >= 0 && j < D;
    ch_s[a] = ok ? j : 0;
    dep_s[a] = ok ? min(max((int)tpl[bh * D + j], 0), 4) : 0;
  }
  __syncthreads();

  float acc[4][G];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[r][g] = 0.0f;
  float cst_acc = 0.0f;  // thread tid < kTB*G: block tid/G, head tid%G

  for (int a0 = 0; a0 < nact; a0 += kCH) {
    const int na = min(kCH, nact - a0);
    // 1. stage plane words and scales
    for (int idx = tid; idx < na * 4 * kTB; idx += 256) {
      const int bi = idx & (kTB - 1), p = (idx >> 4) & 3, a = idx >> 6;
      if (p < dep_s[a0 + a]) {
        const int64_t b = tb0 + bi;
        uint64_t w = 0;
        if (b < blk_end) {
          const int64_t j = ch_s[a0 + a];
          const int64_t sb = b / sub, bs = b - sb * sub;
          w = planes[((bh * nsb + sb) * D + j) * 4 * sub + p * sub + bs];
        }
        w_s[(a * 4 + p) * kTB + bi] = w;
      }
    }
    for (int idx = tid; idx < na * kTB; idx += 256) {
      const int bi = idx & (kTB - 1), a = idx >> 4;
      const int64_t b = tb0 + bi;
      float sc = 0.0f;
      if (b < blk_end) {
        const int64_t j = ch_s[a0 + a];
        const int64_t sb = b / sub, bs = b - sb * sub;
        sc = f16_bits_to_float(scales[((bh * nsb + sb) * D + j) * sub + bs]);
      }
      sc_s[a * kTB + bi] = sc;
    }
    __syncthreads();
    // 2. per (channel, block, head) weights and the constant term
    for (int idx = tid; idx < na * kTB * G; idx += 256) {
      const int g = idx % G, bi = (idx / G) % kTB, a = idx / (G * kTB);
      const int c = dep_s[a0 + a], j = ch_s[a0 + a];
      wt_s[idx] = q_s[g * D + j] * ldexpf(sc_s[a * kTB + bi], 1 - c);
    }
    if (tid < kTB * G) {
      const int bi = tid / G, g = tid % G;
      for (int a = 0; a < na; ++a) {
        const int c = dep_s[a0 + a], j = ch_s[a0 + a];
        const float cadd = ldexpf(0.5f, 1 - c) - 1.0f;
        cst_acc += q_s[g * D + j] * (sc_s[a * kTB + bi] * cadd);
      }
    }
    __syncthreads();
    // 3. accumulate: lane = token, wave = 4 blocks of the tile
    for (int a = 0; a < na; ++a) {
      const int c = dep_s[a0 + a];
      const uint64_t *wa = &w_s[a * 4 * kTB];
      const float *wt = &wt_s[a * kTB * G];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int bi = wave * 4 + r;
        uint32_t code = 0;
        for (int p = 0; p < c; ++p) code = (code << 1) | (uint32_t)((wa[p * kTB + bi] >> lane) & 1ull);
        const float cf = (float)code;
#pragma unroll
        for (int g = 0; g < G; ++g) acc[r][g] = fmaf(wt[bi * G + g], cf, acc[r][g]);
      }
    }
    __syncthreads();
  }
  if (tid < kTB * G) cst_s[tid] = cst_acc;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int bi = wave * 4 + r;
    const int64_t b = tb0 + bi;
    if (b < blk_end) {
      const int64_t tok = b * kBlk + lane;
      if (tok < n) {
#pragma unroll
        for (int g = 0; g < G; ++g) out[(bh * G + g) * n + tok] = acc[r][g] + cst_s[bi * G + g];
      }
    }
  }
}

template <int G>
void launch_scan(dim3 grid, hipStream_t st, const float *q, int D, const int8_t *t, const int32_t *act,
                 const int32_t *nact, const uint64_t *planes, const uint16_t *scales, int64_t n, int64_t nsb,
                 int64_t sub, int64_t blk0, int64_t blk_end, float *out) {
  scan_planes_kernel<G><<<grid, 256, 0, st>>>(q, D, t, act, nact, planes, scales, n, nsb, sub, blk0, blk_end, out);
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_planes(const float *q, int64_t BH, int64_t G, int64_t D, const int8_t *t,
                                  const int32_t *act, const int32_t *nact, const void *planes_sb,
                                  const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t blk0,
                                  int64_t blk1, float *out, void *stream) {
  if (!q || !t || !act || !nact || !planes_sb || !scales_sb || !out)
    return fail(FATHOM_ERR_INVALID, "scan_planes: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "scan_planes: BH=%lld outside [1, 65535]", (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "scan_planes: G=%lld outside [1, 8]", (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "scan_planes: D=%lld outside [1, %d]", (long long)D, kMaxD);
  if (n < 1 || sub < 1) return fail(FATHOM_ERR_INVALID, "scan_planes: n=%lld sub=%lld", (long long)n, (long long)sub);
  const int64_t nblk = cdiv(n, kBlk);
  if (nsb * sub < nblk)
    return fail(FATHOM_ERR_INVALID, "scan_planes: store holds %lld blocks (nsb=%lld x sub=%lld), n needs %lld",
                (long long)(nsb * sub), (long long)nsb, (long long)sub, (long long)nblk);
  if (blk0 < 0 || blk1 < blk0) return fail(FATHOM_ERR_INVALID, "scan_planes: bad block range [%lld, %lld)", (long long)blk0, (long long)blk1);
  const int64_t blk_end = blk1 < nblk ? blk1 : nblk;
  if (blk_end <= blk0) return FATHOM_OK;
  const int64_t tiles = cdiv(blk_end - blk0, kTB);
  if (tiles > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "scan_planes: too many tiles");
  dim3 grid((unsigned)tiles, (unsigned)BH);
  hipStream_t st = (hipStream_t)stream;
  const uint64_t *pl = static_cast<const uint64_t *>(planes_sb);
  const uint16_t *sc = static_cast<const uint16_t *>(scales_sb);
  const int d = (int)D;
  switch (G) {
    case 1: launch_scan<1>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    case 2: launch_scan<2>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    case 3: launch_scan<3>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    case 4: launch_scan<4>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    case 5: launch_scan<5>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    case 6: launch_scan<6>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    case 7: launch_scan<7>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
    default: launch_scan<8>(grid, st, q, d, t, act, nact, pl, sc, n, nsb, sub, blk0, blk_end, out); break;
  }
  return launch_status("scan_planes_kernel");
}
