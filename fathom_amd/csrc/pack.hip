// Store build: 4-bit quantiser, bit-plane packers and the channel-major
// nibble store of the chan4 baseline (lane = channel layout).
//
// A wave owns 64 consecutive channels of one 64-token block: every key load is
// a coalesced row segment, each lane keeps its channel's 64 values in
// registers, reduces the block absmax serially and assembles the four 64-bit
// plane words in registers (bit i = token 64b+i).  A workgroup of 4 waves
// walks 16 consecutive blocks so each (channel, plane) 128-byte superblock unit
// is written by one workgroup (one XCD's L2).
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kBlocksPerWG = 16;

// Nibble words of one (channel, block) of the chan4 store [.., nsb, D, sub, 8]:
// word m holds tokens 8m..8m+7, nibble k = token 8m + k (kernels/bitplane.py:67-74).
__device__ __forceinline__ void store_chan4_words(uint32_t *chan_sb, const uint32_t (&cw)[8], int64_t bh, int64_t sb,
                                                  int64_t bs, int64_t j, int64_t D, int64_t sub, int64_t nsb) {
  uint4 *dst = reinterpret_cast<uint4 *>(chan_sb + (((bh * nsb + sb) * D + j) * sub + bs) * 8);
  dst[0] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
  dst[1] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
}

// C4: also (or instead of the planes) write the chan4 nibble store chan_sb.
template <int KDT, int SDT, bool C4>
__global__ __launch_bounds__(256) void quantise_pack_kernel(const void *__restrict__ K, int64_t n, int64_t D,
                                                            int64_t nblk, int64_t nblk_cover, int64_t sub,
                                                            int64_t nsb, uint8_t *__restrict__ code,
                                                            void *__restrict__ scales_blk,
                                                            uint64_t *__restrict__ planes_log,
                                                            uint64_t *__restrict__ planes_sb,
                                                            uint16_t *__restrict__ scales_sb,
                                                            uint32_t *__restrict__ chan_sb) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.y * 64 + lane;
  const int64_t bh = blockIdx.z;
  if (j >= D) return;  // no cross-lane traffic below
  for (int r = 0; r < kBlocksPerWG / 4; ++r) {
    const int64_t b = (int64_t)blockIdx.x * kBlocksPerWG + r * 4 + wave;
    if (b >= nblk_cover) return;
    uint32_t wl[4] = {0u, 0u, 0u, 0u}, wh[4] = {0u, 0u, 0u, 0u};
    uint32_t cw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    uint16_t s16 = 0;  // fp16 bits of the superblock-store scale
    if (b < nblk) {
      const int64_t tok0 = b * kBlk;
      const int64_t base = (bh * n + tok0) * D + j;
      float x[kBlk];
      float amax = 0.0f;
      bool has_nan = false;
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        x[i] = (tok0 + i < n) ? load_elem<KDT>(K, base + (int64_t)i * D) : 0.0f;
        const float ax = fabsf(x[i]);
        has_nan |= (ax != ax);
        amax = fmaxf(amax, ax);
      }
      // kernels/bitplane.py:29: amax.clamp_min(1e-8).to(scale_dtype).float(), NaN propagating.
      const float a = has_nan ? __uint_as_float(0x7FC00000u) : fmaxf(amax, 1e-8f);
      float af;
      if (SDT == FATHOM_DT_F16) {
        s16 = float_to_f16_bits(a);
        af = f16_bits_to_float(s16);
        if (scales_blk) static_cast<uint16_t *>(scales_blk)[(bh * nblk + b) * D + j] = s16;
      } else if (SDT == FATHOM_DT_BF16) {
        const uint16_t hb = float_to_bf16_bits(a);
        af = bf16_bits_to_float(hb);
        s16 = float_to_f16_bits(af);
        if (scales_blk) static_cast<uint16_t *>(scales_blk)[(bh * nblk + b) * D + j] = hb;
      } else {
        af = a;
        s16 = float_to_f16_bits(af);
        if (scales_blk) static_cast<float *>(scales_blk)[(bh * nblk + b) * D + j] = af;
      }
      const float s = af / 8.0f;
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        // kernels/bitplane.py:31: clamp(floor(x / s), -8, 7) + 8; NaN -> 0.
        const float v = floorf(x[i] / s);
        const int c = (v != v) ? 0 : (int)fminf(fmaxf(v, -8.0f), 7.0f) + 8;
        const bool real = tok0 + i < n;
        if (code && real) code[base + (int64_t)i * D] = (uint8_t)c;
        const uint32_t cb = real ? (uint32_t)c : 0u;  // pack_planes pads with code 0
        if (C4) cw[i >> 3] |= cb << (4 * (i & 7));
        if (i < 32) {
          wl[0] |= ((cb >> 3) & 1u) << i;
          wl[1] |= ((cb >> 2) & 1u) << i;
          wl[2] |= ((cb >> 1) & 1u) << i;
          wl[3] |= (cb & 1u) << i;
        } else {
          wh[0] |= ((cb >> 3) & 1u) << (i - 32);
          wh[1] |= ((cb >> 2) & 1u) << (i - 32);
          wh[2] |= ((cb >> 1) & 1u) << (i - 32);
          wh[3] |= (cb & 1u) << (i - 32);
        }
      }
      if (planes_log) {
        uint64_t *P = planes_log + ((bh * nblk + b) * D + j) * 4;
#pragma unroll
        for (int p = 0; p < 4; ++p) P[p] = ((uint64_t)wh[p] << 32) | wl[p];
      }
    }
    if (planes_sb || C4) {
      const int64_t sb = b / sub, bs = b - (b / sub) * sub;
      if (planes_sb) {
        uint64_t *P = planes_sb + ((bh * nsb + sb) * D + j) * 4 * sub + bs;
#pragma unroll
        for (int p = 0; p < 4; ++p) P[p * sub] = ((uint64_t)wh[p] << 32) | wl[p];
      }
      if (C4) store_chan4_words(chan_sb, cw, bh, sb, bs, j, D, sub, nsb);
      scales_sb[((bh * nsb + sb) * D + j) * sub + bs] = s16;
    }
  }
}

__global__ __launch_bounds__(256) void pack_planes_kernel(const uint8_t *__restrict__ code, int64_t n, int64_t D,
                                                          int64_t nblk, uint64_t *__restrict__ planes) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.y * 64 + lane;
  const int64_t bh = blockIdx.z;
  if (j >= D) return;
  for (int r = 0; r < kBlocksPerWG / 4; ++r) {
    const int64_t b = (int64_t)blockIdx.x * kBlocksPerWG + r * 4 + wave;
    if (b >= nblk) return;
    const int64_t tok0 = b * kBlk;
    const int64_t base = (bh * n + tok0) * D + j;
    uint32_t wl[4] = {0u, 0u, 0u, 0u}, wh[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      const uint32_t cb = (tok0 + i < n) ? (uint32_t)code[base + (int64_t)i * D] : 0u;
      if (i < 32) {
        wl[0] |= ((cb >> 3) & 1u) << i;
        wl[1] |= ((cb >> 2) & 1u) << i;
        wl[2] |= ((cb >> 1) & 1u) << i;
        wl[3] |= (cb & 1u) << i;
      } else {
        wh[0] |= ((cb >> 3) & 1u) << (i - 32);
        wh[1] |= ((cb >> 2) & 1u) << (i - 32);
        wh[2] |= ((cb >> 1) & 1u) << (i - 32);
        wh[3] |= (cb & 1u) << (i - 32);
      }
    }
    uint64_t *P = planes + ((bh * nblk + b) * D + j) * 4;
#pragma unroll
    for (int p = 0; p < 4; ++p) P[p] = ((uint64_t)wh[p] << 32) | wl[p];
  }
}

__global__ __launch_bounds__(256) void pack_chan4_kernel(const uint8_t *__restrict__ code, int64_t n, int64_t D,
                                                         int64_t nblk_cover, int64_t sub, int64_t nsb,
                                                         uint32_t *__restrict__ chan_sb) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.y * 64 + lane;
  const int64_t bh = blockIdx.z;
  if (j >= D) return;
  for (int r = 0; r < kBlocksPerWG / 4; ++r) {
    const int64_t b = (int64_t)blockIdx.x * kBlocksPerWG + r * 4 + wave;
    if (b >= nblk_cover) return;
    const int64_t tok0 = b * kBlk;
    uint32_t cw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      const uint32_t cb = (tok0 + i < n) ? (uint32_t)(code[(bh * n + tok0 + i) * D + j] & 15u) : 0u;
      cw[i >> 3] |= cb << (4 * (i & 7));
    }
    store_chan4_words(chan_sb, cw, bh, b / sub, b - (b / sub) * sub, j, D, sub, nsb);
  }
}

__global__ __launch_bounds__(256) void unpack_planes_kernel(const uint64_t *__restrict__ planes, int64_t nblk,
                                                            int64_t D, int64_t n, uint8_t *__restrict__ code) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.y * 64 + lane;
  const int64_t bh = blockIdx.z;
  if (j >= D) return;
  for (int r = 0; r < kBlocksPerWG / 4; ++r) {
    const int64_t b = (int64_t)blockIdx.x * kBlocksPerWG + r * 4 + wave;
    if (b >= nblk) return;
    const uint64_t *P = planes + ((bh * nblk + b) * D + j) * 4;
    const uint64_t w0 = P[0], w1 = P[1], w2 = P[2], w3 = P[3];
    const int64_t tok0 = b * kBlk;
    for (int i = 0; i < kBlk && tok0 + i < n; ++i) {
      const uint32_t c = (uint32_t)(((w0 >> i) & 1u) << 3 | ((w1 >> i) & 1u) << 2 | ((w2 >> i) & 1u) << 1 |
                                    ((w3 >> i) & 1u));
      code[(bh * n + tok0 + i) * D + j] = (uint8_t)c;
    }
  }
}

template <typename TS>
__global__ __launch_bounds__(256) void to_superblocks_kernel(const uint64_t *__restrict__ planes,
                                                             const TS *__restrict__ scales, int64_t lead,
                                                             int64_t nblk, int64_t D, int64_t sub, int64_t nsb,
                                                             uint64_t *__restrict__ planes_sb,
                                                             TS *__restrict__ scales_sb) {
  const int64_t total_p = lead * nsb * D * 4 * sub;
  const int64_t total_s = lead * nsb * D * sub;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total_p; o += stride) {
    int64_t rem = o;
    const int64_t bs = rem % sub; rem /= sub;
    const int64_t p = rem % 4; rem /= 4;
    const int64_t j = rem % D; rem /= D;
    const int64_t sb = rem % nsb;
    const int64_t bh = rem / nsb;
    const int64_t b = sb * sub + bs;
    planes_sb[o] = (b < nblk) ? planes[((bh * nblk + b) * D + j) * 4 + p] : 0ull;
  }
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total_s; o += stride) {
    int64_t rem = o;
    const int64_t bs = rem % sub; rem /= sub;
    const int64_t j = rem % D; rem /= D;
    const int64_t sb = rem % nsb;
    const int64_t bh = rem / nsb;
    const int64_t b = sb * sub + bs;
    scales_sb[o] = (b < nblk) ? scales[(bh * nblk + b) * D + j] : (TS)0;
  }
}

template <int SDT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ code, const void *__restrict__ scales,
                                                      const int32_t *__restrict__ t, int64_t lead, int64_t n,
                                                      int64_t D, float *__restrict__ out) {
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t total = lead * n * D;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
    const int64_t j = o % D;
    const int64_t tok = (o / D) % n;
    const int64_t bh = o / (D * n);
    int tj = t[j];
    float val = 0.0f;
    if (tj > 0) {
      tj = tj > 4 ? 4 : tj;
      // kernels/bitplane.py:38-41: ((c >> (4 - t)) + 0.5 - 2^(t-1)) * a / 2^(t-1)
      const float half = ldexpf(1.0f, tj - 1);
      const float ct = (float)((uint32_t)code[o] >> (4 - tj));
      const float a = load_elem<SDT>(scales, (bh * nblk + tok / kBlk) * D + j);
      val = (ct + 0.5f - half) * a / half;
    }
    out[o] = val;
  }
}

template <int KDT, bool C4>
int launch_quantise(const void *K, int64_t lead, int64_t n, int64_t D, int sdt, int64_t nblk, int64_t cover,
                    int64_t sub, int64_t nsb, uint8_t *code, void *scales_blk, uint64_t *planes_log,
                    uint64_t *planes_sb, uint16_t *scales_sb, uint32_t *chan_sb, hipStream_t st) {
  dim3 grid((unsigned)cdiv(cover, kBlocksPerWG), (unsigned)cdiv(D, 64), (unsigned)lead);
  switch (sdt) {
    case FATHOM_DT_F16:
      quantise_pack_kernel<KDT, FATHOM_DT_F16, C4><<<grid, 256, 0, st>>>(
          K, n, D, nblk, cover, sub, nsb, code, scales_blk, planes_log, planes_sb, scales_sb, chan_sb);
      break;
    case FATHOM_DT_BF16:
      quantise_pack_kernel<KDT, FATHOM_DT_BF16, C4><<<grid, 256, 0, st>>>(
          K, n, D, nblk, cover, sub, nsb, code, scales_blk, planes_log, planes_sb, scales_sb, chan_sb);
      break;
    default:
      quantise_pack_kernel<KDT, FATHOM_DT_F32, C4><<<grid, 256, 0, st>>>(
          K, n, D, nblk, cover, sub, nsb, code, scales_blk, planes_log, planes_sb, scales_sb, chan_sb);
      break;
  }
  return launch_status("quantise_pack_kernel");
}

template <bool C4>
int quantise_dispatch(const void *K, int k_dtype, int64_t lead, int64_t n, int64_t D, int sdt, int64_t nblk,
                      int64_t cover, int64_t sub, int64_t nsb, uint8_t *code, void *scales_blk, uint64_t *planes_log,
                      uint64_t *planes_sb, uint16_t *scales_sb, uint32_t *chan_sb, hipStream_t st) {
  switch (k_dtype) {
    case FATHOM_DT_F16:
      return launch_quantise<FATHOM_DT_F16, C4>(K, lead, n, D, sdt, nblk, cover, sub, nsb, code, scales_blk,
                                                planes_log, planes_sb, scales_sb, chan_sb, st);
    case FATHOM_DT_BF16:
      return launch_quantise<FATHOM_DT_BF16, C4>(K, lead, n, D, sdt, nblk, cover, sub, nsb, code, scales_blk,
                                                 planes_log, planes_sb, scales_sb, chan_sb, st);
    default:
      return launch_quantise<FATHOM_DT_F32, C4>(K, lead, n, D, sdt, nblk, cover, sub, nsb, code, scales_blk,
                                                planes_log, planes_sb, scales_sb, chan_sb, st);
  }
}

bool valid_dtype(int dt) { return dt == FATHOM_DT_F32 || dt == FATHOM_DT_F16 || dt == FATHOM_DT_BF16; }

int check_grid(int64_t lead, int64_t D, int64_t nblk_cover, const char *who) {
  if (lead < 1 || lead > 65535) return fail(FATHOM_ERR_INVALID, "%s: lead dimension %lld outside [1, 65535]", who, (long long)lead);
  if (D < 1 || cdiv(D, 64) > 65535) return fail(FATHOM_ERR_INVALID, "%s: D=%lld unsupported", who, (long long)D);
  if (cdiv(nblk_cover, kBlocksPerWG) > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "%s: too many blocks", who);
  return FATHOM_OK;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_quantise_pack(const void *K, int k_dtype, int64_t lead, int64_t n, int64_t D, int scale_dtype,
                                    int64_t sub, uint8_t *code, void *scales_blk, uint64_t *planes_log,
                                    uint64_t *planes_sb, uint16_t *scales_sb, void *stream) {
  if (!K) return fail(FATHOM_ERR_INVALID, "quantise_pack: K is null");
  if (!valid_dtype(k_dtype) || !valid_dtype(scale_dtype)) return fail(FATHOM_ERR_INVALID, "quantise_pack: bad dtype");
  if (n < 1) return fail(FATHOM_ERR_INVALID, "quantise_pack: n=%lld < 1", (long long)n);
  if ((planes_sb == nullptr) != (scales_sb == nullptr))
    return fail(FATHOM_ERR_INVALID, "quantise_pack: planes_sb and scales_sb must both be given or both null");
  if (planes_sb && sub < 1) return fail(FATHOM_ERR_INVALID, "quantise_pack: sub=%lld < 1", (long long)sub);
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t nsb = planes_sb ? cdiv(nblk, sub) : 0;
  const int64_t cover = planes_sb ? nsb * sub : nblk;
  int rc = check_grid(lead, D, cover, "quantise_pack");
  if (rc) return rc;
  if (!code && !scales_blk && !planes_log && !planes_sb) return FATHOM_OK;
  return quantise_dispatch<false>(K, k_dtype, lead, n, D, scale_dtype, nblk, cover, sub, nsb, code, scales_blk,
                                  planes_log, planes_sb, scales_sb, nullptr, (hipStream_t)stream);
}

extern "C" int fathom_quantise_chan4(const void *K, int k_dtype, int64_t lead, int64_t n, int64_t D, int scale_dtype,
                                     int64_t sub, uint8_t *code, void *scales_blk, uint32_t *chan_sb,
                                     uint16_t *scales_sb, void *stream) {
  if (!K || !chan_sb || !scales_sb) return fail(FATHOM_ERR_INVALID, "quantise_chan4: null pointer");
  if (!valid_dtype(k_dtype) || !valid_dtype(scale_dtype)) return fail(FATHOM_ERR_INVALID, "quantise_chan4: bad dtype");
  if (n < 1 || sub < 1) return fail(FATHOM_ERR_INVALID, "quantise_chan4: n=%lld sub=%lld", (long long)n, (long long)sub);
  if (reinterpret_cast<uintptr_t>(chan_sb) & 15) return fail(FATHOM_ERR_INVALID, "quantise_chan4: chan_sb not 16-byte aligned");
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t nsb = cdiv(nblk, sub);
  int rc = check_grid(lead, D, nsb * sub, "quantise_chan4");
  if (rc) return rc;
  return quantise_dispatch<true>(K, k_dtype, lead, n, D, scale_dtype, nblk, nsb * sub, sub, nsb, code, scales_blk,
                                 nullptr, nullptr, scales_sb, chan_sb, (hipStream_t)stream);
}

extern "C" int fathom_pack_chan4(const uint8_t *code, int64_t lead, int64_t n, int64_t D, int64_t sub, uint32_t *chan_sb,
                                 void *stream) {
  if (!code || !chan_sb) return fail(FATHOM_ERR_INVALID, "pack_chan4: null pointer");
  if (n < 1 || sub < 1) return fail(FATHOM_ERR_INVALID, "pack_chan4: n=%lld sub=%lld", (long long)n, (long long)sub);
  if (reinterpret_cast<uintptr_t>(chan_sb) & 15) return fail(FATHOM_ERR_INVALID, "pack_chan4: chan_sb not 16-byte aligned");
  const int64_t nsb = cdiv(cdiv(n, kBlk), sub);
  int rc = check_grid(lead, D, nsb * sub, "pack_chan4");
  if (rc) return rc;
  dim3 grid((unsigned)cdiv(nsb * sub, kBlocksPerWG), (unsigned)cdiv(D, 64), (unsigned)lead);
  pack_chan4_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(code, n, D, nsb * sub, sub, nsb, chan_sb);
  return launch_status("pack_chan4_kernel");
}

extern "C" int fathom_pack_planes(const uint8_t *code, int64_t lead, int64_t n, int64_t D, uint64_t *planes,
                                  void *stream) {
  if (!code || !planes) return fail(FATHOM_ERR_INVALID, "pack_planes: null pointer");
  if (n < 1) return fail(FATHOM_ERR_INVALID, "pack_planes: n=%lld < 1", (long long)n);
  const int64_t nblk = cdiv(n, kBlk);
  int rc = check_grid(lead, D, nblk, "pack_planes");
  if (rc) return rc;
  dim3 grid((unsigned)cdiv(nblk, kBlocksPerWG), (unsigned)cdiv(D, 64), (unsigned)lead);
  pack_planes_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(code, n, D, nblk, planes);
  return launch_status("pack_planes_kernel");
}

extern "C" int fathom_unpack_planes(const uint64_t *planes, int64_t lead, int64_t nblk, int64_t D, int64_t n,
                                    uint8_t *code, void *stream) {
  if (!code || !planes) return fail(FATHOM_ERR_INVALID, "unpack_planes: null pointer");
  if (n < 1 || nblk < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "unpack_planes: n=%lld needs %lld blocks, planes hold %lld", (long long)n,
                (long long)cdiv(n, kBlk), (long long)nblk);
  int rc = check_grid(lead, D, nblk, "unpack_planes");
  if (rc) return rc;
  dim3 grid((unsigned)cdiv(cdiv(n, kBlk), kBlocksPerWG), (unsigned)cdiv(D, 64), (unsigned)lead);
  unpack_planes_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(planes, nblk, D, n, code);
  return launch_status("unpack_planes_kernel");
}

extern "C" int fathom_to_superblocks(const uint64_t *planes, const void *scales, int scale_bytes, int64_t lead,
                                     int64_t nblk, int64_t D, int64_t sub, uint64_t *planes_sb, void *scales_sb,
                                     void *stream) {
  if (!planes || !scales || !planes_sb || !scales_sb) return fail(FATHOM_ERR_INVALID, "to_superblocks: null pointer");
  if (lead < 1 || nblk < 1 || D < 1 || sub < 1)
    return fail(FATHOM_ERR_INVALID, "to_superblocks: bad shape lead=%lld nblk=%lld D=%lld sub=%lld", (long long)lead,
                (long long)nblk, (long long)D, (long long)sub);
  if (scale_bytes != 2 && scale_bytes != 4) return fail(FATHOM_ERR_INVALID, "to_superblocks: scale_bytes must be 2 or 4");
  const int64_t nsb = cdiv(nblk, sub);
  const int64_t total = lead * nsb * D * 4 * sub;
  const unsigned blocks = (unsigned)(cdiv(total, 256) < 65536 ? cdiv(total, 256) : 65536);
  if (scale_bytes == 2)
    to_superblocks_kernel<uint16_t><<<blocks, 256, 0, (hipStream_t)stream>>>(
        planes, (const uint16_t *)scales, lead, nblk, D, sub, nsb, planes_sb, (uint16_t *)scales_sb);
  else
    to_superblocks_kernel<uint32_t><<<blocks, 256, 0, (hipStream_t)stream>>>(
        planes, (const uint32_t *)scales, lead, nblk, D, sub, nsb, planes_sb, (uint32_t *)scales_sb);
  return launch_status("to_superblocks_kernel");
}

extern "C" int fathom_dequant_planes(const uint8_t *code, const void *scales, int scale_dtype, const int32_t *t,
                                     int64_t lead, int64_t n, int64_t D, float *out, void *stream) {
  if (!code || !scales || !t || !out) return fail(FATHOM_ERR_INVALID, "dequant_planes: null pointer");
  if (lead < 1 || n < 1 || D < 1) return fail(FATHOM_ERR_INVALID, "dequant_planes: bad shape");
  if (!valid_dtype(scale_dtype)) return fail(FATHOM_ERR_INVALID, "dequant_planes: bad scale dtype");
  const int64_t total = lead * n * D;
  const unsigned blocks = (unsigned)(cdiv(total, 256) < 65536 ? cdiv(total, 256) : 65536);
  hipStream_t st = (hipStream_t)stream;
  if (scale_dtype == FATHOM_DT_F16)
    dequant_kernel<FATHOM_DT_F16><<<blocks, 256, 0, st>>>(code, scales, t, lead, n, D, out);
  else if (scale_dtype == FATHOM_DT_BF16)
    dequant_kernel<FATHOM_DT_BF16><<<blocks, 256, 0, st>>>(code, scales, t, lead, n, D, out);
  else
    dequant_kernel<FATHOM_DT_F32><<<blocks, 256, 0, st>>>(code, scales, t, lead, n, D, out);
  return launch_status("dequant_kernel");
}
