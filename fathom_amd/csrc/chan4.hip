// Channel-major 4-bit baseline store scan (Chan4Store.scan).
//
// The store of kernels/bitplane.py:67-74 (pack_chan4) keeps every listed
// channel at full depth: word m of (channel j, block b) holds the 4-bit codes
// of tokens 8m..8m+7, nibble k = token 8m + k, 32 + 2 bytes per (channel,
// block).  A workgroup (4 waves) owns a tile of 32 blocks of one row, wave w
// blocks 8w..8w+7, lane = token.  Chunks of 8 listed channels are staged with
// 16-byte loads into double-buffered LDS; a lane takes its nibble with one
// bit-field extract, forms y = 2a (c - 7.5) = c * 2a - 15a (one FMA of exact
// operands) and the head contraction acc_g += w_g * y (w = q / 16) runs on the
// matrix cores, one v_mfma_f32_4x4x1_16b_f32 per (channel, block) for four
// heads (a second one for heads 4..7), in list order.
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr int kGB = 8;             // blocks per wave
constexpr int kWaves = 4;          // waves per workgroup
constexpr int kTB = kGB * kWaves;  // blocks per tile
constexpr int kMaxD = 128;
constexpr int kThreads = 64 * kWaves;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// w_gj for every channel, QS floats per channel (heads >= G are zero), so the
// MFMA A operand of lane l is w[j][4h + (l & 3)].
template <int G>
struct QShared {
  static constexpr int QS = G <= 4 ? 4 : 8;
  float w[kMaxD * QS];
};

template <int G>
struct QOp {
  static constexpr int NQ = (G + 3) / 4;
  float a[NQ];
};

// Four fp32 accumulators per lane and head quad: component h of v[b][hq] is
// the score of head 4*hq + h for the lane's token of block b.
template <int G>
struct Acc {
  static constexpr int NQ = (G + 3) / 4;
  f32x4 v[kGB][NQ];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int b = 0; b < kGB; ++b)
#pragma unroll
      for (int h = 0; h < NQ; ++h) v[b][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __device__ __forceinline__ float get(int b, int g) const { return v[b][g >> 2][g & 3]; }
};

template <int G>
__device__ __forceinline__ void accum(Acc<G> &acc, int b, const QOp<G> &q, float y) {
#pragma unroll
  for (int h = 0; h < QOp<G>::NQ; ++h) acc.v[b][h] = __builtin_amdgcn_mfma_f32_4x4x1f32(q.a[h], y, acc.v[b][h], 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// Scores of a wave's 8 blocks: out [BH, G, n].
template <int G>
__device__ __forceinline__ void store_scores(float *out, const Acc<G> &acc, int64_t bh, int64_t gb0, int64_t blk0,
                                             int64_t blk_end, int64_t n, int lane) {
#pragma unroll
  for (int r = 0; r < kGB; ++r) {
    const int64_t b = gb0 + r;
    const int64_t tok = b * kBlk + lane;
    if (b >= blk0 && b < blk_end && tok < n) {
#pragma unroll
      for (int g = 0; g < G; ++g) out[(bh * G + g) * n + tok] = acc.get(r, g);
    }
  }
}

constexpr int kC4Chan = 8;                 // channels per staged chunk
constexpr int kC4Row = kTB + 4;            // padded LDS row of one word index over the tile's blocks

struct Chan4Args {
  const float *q;            // [BH, G, D]
  const int32_t *act;        // [BH, D] listed channels first
  const int32_t *nact;       // [BH]
  const uint4 *chan;         // [BH, nsb, D, sub, 8] uint32 words as 16-byte halves
  const uint16_t *scales;    // [BH, nsb, D, sub] fp16 bits
  int64_t n, nsb, sub, blk0, blk_end, tile0;
  int D;
};

template <int G>
struct C4Buf {
  alignas(16) uint32_t w[kC4Chan][8][kC4Row];  // [channel slot][word m][block]
  alignas(16) float P[kC4Chan][kTB];           // 2a
  alignas(16) float Q[kC4Chan][kTB];           // -15a
  alignas(16) float wq[kC4Chan][QShared<G>::QS];
};

template <int G>
struct C4Shared {
  QShared<G> qs;
  uint8_t lst[kMaxD];
  C4Buf<G> buf[2];
};

// A thread stages two 16-byte halves (item e = tid + 256 h: channel slot e / 64,
// block (e / 2) % 32, half e % 2) and the scale of (slot tid / 32, block tid % 32).
struct C4Staged {
  uint4 v[2];
  uint16_t s;
};

__device__ __forceinline__ void c4_load(C4Staged &r, const Chan4Args &a, const uint8_t *lst, int i0, int m, int64_t bh,
                                        int64_t tb0, int tid) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = tid + kThreads * h, ci = e >> 6, b = (e >> 1) & (kTB - 1), half = e & 1;
    const int64_t blk = tb0 + b;
    r.v[h] = make_uint4(0u, 0u, 0u, 0u);
    if (ci < m && blk < a.nsb * a.sub) {
      const int64_t sb = blk / a.sub, off = blk - sb * a.sub;
      r.v[h] = a.chan[(((bh * a.nsb + sb) * a.D + lst[i0 + ci]) * a.sub + off) * 2 + half];
    }
  }
  const int ci = tid >> 5, b = tid & (kTB - 1);
  const int64_t blk = tb0 + b;
  r.s = 0;
  if (ci < m && blk < a.nsb * a.sub) {
    const int64_t sb = blk / a.sub, off = blk - sb * a.sub;
    r.s = a.scales[((bh * a.nsb + sb) * a.D + lst[i0 + ci]) * a.sub + off];
  }
}

template <int G>
__device__ __forceinline__ void c4_store(C4Buf<G> &bf, const C4Staged &r, const QShared<G> &qs, const uint8_t *lst,
                                         int i0, int m, int tid) {
  constexpr int QS = QShared<G>::QS;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = tid + kThreads * h, ci = e >> 6, b = (e >> 1) & (kTB - 1), half = e & 1;
    bf.w[ci][4 * half + 0][b] = r.v[h].x;
    bf.w[ci][4 * half + 1][b] = r.v[h].y;
    bf.w[ci][4 * half + 2][b] = r.v[h].z;
    bf.w[ci][4 * half + 3][b] = r.v[h].w;
  }
  const int ci = tid >> 5, b = tid & (kTB - 1);
  const float a = __half2float(__ushort_as_half(r.s));
  bf.P[ci][b] = 2.0f * a;
  bf.Q[ci][b] = -15.0f * a;
  if (b < QS && ci < m) bf.wq[ci][b] = qs.w[lst[i0 + ci] * QS + b];
}

template <int G>
__device__ __forceinline__ void c4_compute(const C4Buf<G> &bf, int m, int wave, int lane, Acc<G> &acc) {
  const int wm = lane >> 3, sh = 4 * (lane & 7);
  for (int ci = 0; ci < m; ++ci) {
    QOp<G> q;
#pragma unroll
    for (int h = 0; h < QOp<G>::NQ; ++h) q.a[h] = bf.wq[ci][4 * h + (lane & 3)];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint4 w4 = *reinterpret_cast<const uint4 *>(&bf.w[ci][wm][wave * kGB + 4 * hf]);
      const float4 P4 = *reinterpret_cast<const float4 *>(&bf.P[ci][wave * kGB + 4 * hf]);
      const float4 Q4 = *reinterpret_cast<const float4 *>(&bf.Q[ci][wave * kGB + 4 * hf]);
      const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
      const float P[4] = {P4.x, P4.y, P4.z, P4.w}, Q[4] = {Q4.x, Q4.y, Q4.z, Q4.w};
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = fmaf((float)__builtin_amdgcn_ubfe(wd[r], sh, 4), P[r], Q[r]);
#pragma unroll
      for (int r = 0; r < 4; ++r) accum<G>(acc, 4 * hf + r, q, y[r]);
    }
  }
}

template <int G>
__global__ __launch_bounds__(kThreads) void scan_chan4_kernel(Chan4Args a, float *out) {
  constexpr int QS = QShared<G>::QS;
  __shared__ C4Shared<G> sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = blockIdx.y;
  const int64_t tb0 = (a.tile0 + (int64_t)blockIdx.x) * kTB;
  const int na = min(max(ld_uniform(a.nact + bh), 0), a.D);
  for (int i = tid; i < na; i += kThreads) {
    const int j = min(max(a.act[bh * a.D + i], 0), a.D - 1);  // memory-safe
    sh.lst[i] = (uint8_t)j;
#pragma unroll
    for (int g = 0; g < QS; ++g) sh.qs.w[j * QS + g] = g < G ? ldexpf(a.q[(bh * G + g) * a.D + j], -4) : 0.0f;
  }
  Acc<G> acc;
  acc.zero();
  if (tb0 < a.blk_end && tb0 + kTB > a.blk0 && na > 0) {
    __syncthreads();
    C4Staged r;
    const int nk = (na + kC4Chan - 1) / kC4Chan;
    c4_load(r, a, sh.lst, 0, min(kC4Chan, na), bh, tb0, tid);
    c4_store<G>(sh.buf[0], r, sh.qs, sh.lst, 0, min(kC4Chan, na), tid);
    __syncthreads();
    for (int k = 0; k < nk; ++k) {
      const int i0 = k * kC4Chan, m = min(kC4Chan, na - i0);
      const bool more = k + 1 < nk;
      const int i1 = i0 + kC4Chan, m1 = min(kC4Chan, na - i1);
      if (more) c4_load(r, a, sh.lst, i1, m1, bh, tb0, tid);
      c4_compute<G>(sh.buf[k & 1], m, wave, lane, acc);
      if (more) c4_store<G>(sh.buf[(k + 1) & 1], r, sh.qs, sh.lst, i1, m1, tid);
      __syncthreads();
    }
  }
  store_scores<G>(out, acc, bh, tb0 + wave * kGB, a.blk0, a.blk_end, a.n, lane);
}

template <int G>
void launch_chan4_g(const Chan4Args &a, int64_t tiles, int64_t BH, float *out, hipStream_t st) {
  scan_chan4_kernel<G><<<dim3((unsigned)tiles, (unsigned)BH), kThreads, 0, st>>>(a, out);
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_chan4(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *act,
                                 const int32_t *nact, const void *chan_sb, const void *scales_sb, int64_t n,
                                 int64_t nsb, int64_t sub, int64_t blk0, int64_t blk1, float *out, void *stream) {
  if (!q || !act || !nact || !chan_sb || !scales_sb || !out) return fail(FATHOM_ERR_INVALID, "scan_chan4: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "scan_chan4: BH=%lld outside [1, 65535]", (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "scan_chan4: G=%lld outside [1, 8]", (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "scan_chan4: D=%lld outside [1, %d]", (long long)D, kMaxD);
  if (n < 1 || sub < 1 || nsb < 1 || nsb * sub < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "scan_chan4: store of nsb=%lld x sub=%lld blocks does not cover n=%lld",
                (long long)nsb, (long long)sub, (long long)n);
  if ((reinterpret_cast<uintptr_t>(chan_sb) & 15) != 0)
    return fail(FATHOM_ERR_INVALID, "scan_chan4: the nibble store must be 16-byte aligned");
  if (blk0 < 0 || blk1 < blk0)
    return fail(FATHOM_ERR_INVALID, "scan_chan4: bad block range [%lld, %lld)", (long long)blk0, (long long)blk1);
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t blk_end = blk1 < nblk ? blk1 : nblk;
  if (blk_end <= blk0) return FATHOM_OK;
  Chan4Args a{};
  a.q = q;
  a.act = act;
  a.nact = nact;
  a.chan = static_cast<const uint4 *>(chan_sb);
  a.scales = static_cast<const uint16_t *>(scales_sb);
  a.n = n;
  a.nsb = nsb;
  a.sub = sub;
  a.blk0 = blk0;
  a.blk_end = blk_end;
  a.tile0 = blk0 / kTB;
  a.D = (int)D;
  const int64_t tiles = cdiv(blk_end, kTB) - a.tile0;
  hipStream_t st = (hipStream_t)stream;
  switch (G) {
    case 1: launch_chan4_g<1>(a, tiles, BH, out, st); break;
    case 2: launch_chan4_g<2>(a, tiles, BH, out, st); break;
    case 3: launch_chan4_g<3>(a, tiles, BH, out, st); break;
    case 4: launch_chan4_g<4>(a, tiles, BH, out, st); break;
    case 5: launch_chan4_g<5>(a, tiles, BH, out, st); break;
    case 6: launch_chan4_g<6>(a, tiles, BH, out, st); break;
    case 7: launch_chan4_g<7>(a, tiles, BH, out, st); break;
    default: launch_chan4_g<8>(a, tiles, BH, out, st); break;
  }
  return launch_status("scan_chan4_kernel");
}
