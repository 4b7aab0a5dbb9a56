// Partial-depth bit-plane scan (PlaneStore.scan) and the fused scan + top-k.
//
// Score of token i of row (bh, g), with depth t_j planes read for channel j:
//   s = sum_j q_gj * a_bj * 2^(1 - t_j) * x_j(i),   x = c_t - (2^t - 1) / 2,
// where c_t is the top-t-bit code and a_bj the block absmax.  This is the
// reference's dequantised value (c_t + 0.5 - 2^(t-1)) * a / 2^(t-1)
// (kernels/bitplane.py:34-42) with the constant term folded into x: x is the
// sum over the t plane bits of +-2^(t-2-p), so it is built from the plane
// words alone by t v_cndmask selections between +-(4, 2, 1, 0.5) -- all inline
// constants -- and t-1 adds, exactly.
//
// Lane = token: a 64-bit plane word holds one bit per lane of a wave64.
// A workgroup owns a tile of 32 blocks (2048 tokens) of one row bh; each of
// its 4 waves owns 8 consecutive blocks ("group") and works alone after the
// workgroup has put q_gj * 2^(1-t_j) for all listed channels in LDS.
// Channels are visited by depth class (the plan's cls lists), so the depth is
// a compile-time constant of the inner loop.  Two kernels reach the planes:
//  * direct (store in HBM, sub % 8 == 0): the group's plane words are 8
//    consecutive words of each (channel, plane) and its 8 fp16 scales 16
//    consecutive bytes, read by scalar loads into SGPRs; each word is the lane
//    mask of a v_cndmask (no per-lane bit extraction) and each scale feeds a
//    v_fma_mix (fp16 operand, no conversion): per (channel, block) the VALU
//    work is 2t + G instructions;
//  * staged (store in mapped host memory, or any other sub): a chunk of
//    channels' words and scales is copied to LDS with coalesced vector loads,
//    so PCIe reads are whole (channel, plane) runs, and lanes extract bits.
// Both build the same exact x, multiply by the same scale and accumulate in
// the same channel order: their scores are bit-identical.
//
// Output modes: scores [BH, G, n] (PlaneStore.scan), sampled keys (every S-th
// tile, for the top-k threshold), or candidate emission (key >= threshold ->
// per-row candidate list, aggregated per workgroup in LDS), the last two
// fusing the scan with the top-k.
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr int kGB = 8;             // blocks per wave
constexpr int kWaves = 4;          // waves per workgroup
constexpr int kTB = kGB * kWaves;  // blocks per tile
constexpr int kMaxD = 256;
constexpr int kCH = 16;            // channels per staged chunk
constexpr uint32_t kRowLocal = 128;  // LDS candidates per (workgroup, row)
static_assert(kTB * kBlk == kTileTok, "scan tile and top-k sample tile must agree");

enum : int { kEmitScores = 0, kEmitSample = 1, kEmitFilter = 2 };

struct Emit {
  float *out;        // scores [BH, G, n]
  uint32_t *samp;    // sampled keys [BH*G, samp_cap]
  int64_t samp_cap;
  TopkSel sel;       // threshold + candidate lists
  int64_t sink, lstart;
};

struct ScanArgs {
  const float *q;          // [BH, G, D]
  const int32_t *cls;      // [BH, bmax, D]
  const int32_t *clsn;     // [BH, bmax]
  const uint64_t *planes;  // [BH, nsb, D, 4, sub]
  const uint16_t *scales;  // [BH, nsb, D, sub] fp16 bits
  int64_t n, nsb, sub;
  int64_t blk0, blk_end;   // blocks [blk0, blk_end) are emitted
  int64_t tile0;           // tile of blockIdx.x == 0 (tile T = blocks [32T, 32T + 32))
  int64_t tile_stride;     // tiles between consecutive workgroups
  int D, bmax, ncls;       // classes 1..ncls are scanned (ncls = min(bmax, 4))
};

typedef unsigned int u32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Wave-uniform loads through the constant address space: scalar loads into
// SGPRs (the store, plan and queries are read-only for the kernel's lifetime).
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

__device__ __forceinline__ int64_t sgpr64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <int G>
struct QShared {
  float qw[kMaxD * G];  // q_gj * 2^(1 - t_j) for listed channels, [channel][head]
};

// Workgroup prologue: the depth-scaled query weights of every listed channel.
// With prefetch, it also touches (one dword each) every plane and scale line
// the tile's four groups will read, so the waves' scalar loads find them in
// L2 instead of waiting on HBM one channel at a time; the returned value is
// only there to keep those loads alive.
template <int G>
__device__ __forceinline__ uint32_t load_qw(QShared<G> &sh, const ScanArgs &a, int64_t bh, int64_t tb0,
                                            bool prefetch) {
  uint32_t pf = 0u;
  const int64_t nblk_store = a.nsb * a.sub;
  for (int c = 1; c <= a.ncls; ++c) {
    const int nc = min(max(a.clsn[bh * a.bmax + c - 1], 0), a.D);
    const int32_t *lst = a.cls + (bh * a.bmax + c - 1) * a.D;
    for (int i = threadIdx.x; i < nc * G; i += 256) {
      const int ci = i / G, g = i - ci * G;
      const int j = lst[ci];
      if (j >= 0 && j < a.D) sh.qw[j * G + g] = ldexpf(a.q[(bh * G + g) * a.D + j], 1 - c);
    }
    if (!prefetch) continue;
    // items: (channel, plane or scale, group) -- c planes + 1 scale line per group
    for (int i = threadIdx.x; i < nc * (c + 1) * kWaves; i += 256) {
      const int w = i % kWaves, p = (i / kWaves) % (c + 1), ci = i / (kWaves * (c + 1));
      const int j = lst[ci];
      const int64_t b = tb0 + w * kGB;
      if (j < 0 || j >= a.D || b >= nblk_store) continue;
      const int64_t sb = (int64_t)((uint64_t)b / (uint64_t)a.sub);
      const int64_t off = b - sb * a.sub;
      if (p < c)
        pf ^= *reinterpret_cast<const uint32_t *>(a.planes + ((bh * a.nsb + sb) * a.D + j) * 4 * a.sub + p * a.sub + off);
      else
        pf ^= *reinterpret_cast<const uint32_t *>(a.scales + ((bh * a.nsb + sb) * a.D + j) * a.sub + (off & ~1));
    }
  }
  return pf;
}

// Exact symmetric code x = c - (2^C - 1)/2 of a lane's token from its C plane
// words (word p is the lane mask of a select between +-2^(C-2-p)).
template <int C>
__device__ __forceinline__ float sym_code(const uint64_t *w) {
#define FATHOM_SEL(p, v) (__builtin_amdgcn_inverse_ballot_w64(w[p]) ? (v) : -(v))
  if (C == 1) return FATHOM_SEL(0, 0.5f);
  if (C == 2) return FATHOM_SEL(0, 1.0f) + FATHOM_SEL(C > 1 ? 1 : 0, 0.5f);
  if (C == 3) return (FATHOM_SEL(0, 2.0f) + FATHOM_SEL(C > 1 ? 1 : 0, 1.0f)) + FATHOM_SEL(C > 2 ? 2 : 0, 0.5f);
  return (FATHOM_SEL(0, 4.0f) + FATHOM_SEL(C > 1 ? 1 : 0, 2.0f)) +
         (FATHOM_SEL(C > 2 ? 2 : 0, 1.0f) + FATHOM_SEL(C > 3 ? 3 : 0, 0.5f));
#undef FATHOM_SEL
}

// Same value from the integer code (staged kernel): exact in fp32.
template <int C>
__device__ __forceinline__ float sym_from_int(uint32_t code) {
  return (float)code - (float)((1 << C) - 1) * 0.5f;
}

// a * x with a given as fp16 bits (v_fma_mix_f32: the fp16 operand needs no
// conversion; + 0 keeps it one rounding, as a product).
__device__ __forceinline__ float scaled(uint16_t a_bits, float x) {
  return fmaf(__half2float(__ushort_as_half(a_bits)), x, 0.0f);
}

// --------------------------------------------------------------------- emission
template <int G>
struct EmitShared {
  uint64_t lbuf[G][kRowLocal];
  uint32_t lcnt[G];
  uint32_t lbase[G];
};

template <int G, int MODE>
__device__ __forceinline__ void emit_group(const Emit &em, EmitShared<G> &es, const float (&acc)[kGB][G],
                                           int64_t bh, int64_t gb0, int64_t blk0, int64_t blk_end, int64_t n,
                                           int wave, int lane, int64_t samp_tile) {
  const int tid = threadIdx.x;
  if (MODE == kEmitFilter) {
    if (tid < G) es.lcnt[tid] = 0u;
    __syncthreads();
  }
  float thr_f[G];
  bool thr_all[G];
  if (MODE == kEmitFilter) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t thr = em.sel.thr[bh * G + g];
      thr_all[g] = thr == 0u;  // fewer samples than kk: every valid token is a candidate
      thr_f[g] = key_value(thr);
    }
  }
#pragma unroll
  for (int r = 0; r < kGB; ++r) {
    const int64_t b = gb0 + r;
    const int64_t tok = b * kBlk + lane;
    const bool valid = b >= blk0 && b < blk_end && tok < n;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = acc[r][g];
      const int64_t row = bh * G + g;
      if (MODE == kEmitScores) {
        if (valid) em.out[row * n + tok] = v;
      } else {
        const bool masked = tok < em.sink || tok >= em.lstart;
        if (MODE == kEmitSample) {
          const uint32_t key = valid ? (masked ? kKeyNegInf : score_key(v)) : 0u;
          em.samp[row * em.samp_cap + samp_tile * kTileTok + (wave * kGB + r) * kBlk + lane] = key;
        } else {
          // key >= thr tested on floats: thr_f is the value whose key is thr
          const float vm = masked ? -INFINITY : v;
          const bool pass = valid && (thr_all[g] || vm >= thr_f[g] || vm != vm);
          wave_append_local(pass, pass ? k64_of(masked ? kKeyNegInf : score_key(v), tok) : 0ull, &es.lcnt[g],
                            es.lbuf[g], kRowLocal, &em.sel.cand_cnt[row], em.sel.cand + row * em.sel.cand_cap,
                            (uint64_t)em.sel.cand_cap, lane);
        }
      }
    }
  }
  if (MODE == kEmitFilter) {
    // one reservation per row, all rows at once, then one copy pass
    __syncthreads();
    if (tid < G) {
      const uint32_t nloc = min(es.lcnt[tid], kRowLocal);
      es.lbase[tid] = nloc ? atomicAdd(&em.sel.cand_cnt[bh * G + tid], nloc) : 0u;
    }
    __syncthreads();
    for (int e = tid; e < G * (int)kRowLocal; e += 256) {
      const int g = e / (int)kRowLocal, i = e % (int)kRowLocal;
      const uint32_t nloc = min(es.lcnt[g], kRowLocal);
      const uint64_t slot = (uint64_t)es.lbase[g] + i;
      if ((uint32_t)i < nloc && slot < (uint64_t)em.sel.cand_cap)
        em.sel.cand[(bh * G + g) * em.sel.cand_cap + slot] = es.lbuf[g][i];
    }
  }
}

// --------------------------------------------------------------------- direct (HBM) kernel
// HB blocks per load group: 8 for depth <= 2, 4 for deeper classes (at most
// 32 SGPRs of plane words live per group).
template <int C>
struct Depth {
  static constexpr int HB = C <= 2 ? 8 : 4;
};

template <int HB>
struct WordVec;
template <>
struct WordVec<8> {
  typedef u32x16 W;
  typedef u32x4 S;
};
template <>
struct WordVec<4> {
  typedef u32x8 W;
  typedef u32x2 S;
};

// One channel of depth C over the wave's 8 blocks: pj = its plane-0 word of the
// group's first block (plane p at + p*sub), sj = its first fp16 scale.
template <int C, int G>
__device__ __forceinline__ void direct_channel(const uint64_t *pj, const uint16_t *sj, int64_t sub, const float *qv,
                                               float (&acc)[kGB][G]) {
  constexpr int HB = Depth<C>::HB;
  typedef typename WordVec<HB>::W WV;
  typedef typename WordVec<HB>::S SV;
#pragma unroll
  for (int h = 0; h < kGB / HB; ++h) {
    // keeps the next half's loads below this half's use (merged loads would
    // need twice the SGPRs)
    if (h > 0) __builtin_amdgcn_sched_barrier(0);
    WV wv[C];
#pragma unroll
    for (int p = 0; p < C; ++p) wv[p] = ld_uniform(reinterpret_cast<const WV *>(pj + p * sub + h * HB));
    const SV sv = ld_uniform(reinterpret_cast<const SV *>(sj + h * HB));
#pragma unroll
    for (int r = 0; r < HB; ++r) {
      uint64_t w[C];
#pragma unroll
      for (int p = 0; p < C; ++p) w[p] = ((uint64_t)wv[p][2 * r + 1] << 32) | wv[p][2 * r];
      const float x = sym_code<C>(w);
      const uint32_t sd = sv[r >> 1];
      const float u = scaled((uint16_t)((r & 1) ? (sd >> 16) : (sd & 0xFFFFu)), x);
#pragma unroll
      for (int g = 0; g < G; ++g) acc[h * HB + r][g] = fmaf(qv[g], u, acc[h * HB + r][g]);
    }
  }
}

template <int C, int G>
__device__ __forceinline__ void direct_class(const ScanArgs &a, const QShared<G> &qs, int64_t bh, const uint64_t *pw,
                                             const uint16_t *ps, float (&acc)[kGB][G]) {
  if (C > a.ncls) return;
  const int nc = min(max(ld_uniform(a.clsn + bh * a.bmax + C - 1), 0), a.D);
  const int32_t *lst = a.cls + (bh * a.bmax + C - 1) * a.D;
  int jn = nc > 0 ? ld_uniform(lst) : 0;
  for (int i = 0; i < nc; ++i) {
    const int j = jn;
    if (i + 1 < nc) jn = ld_uniform(lst + i + 1);
    if ((unsigned)j >= (unsigned)a.D) continue;
    float qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) qv[g] = qs.qw[j * G + g];
    direct_channel<C, G>(pw + (int64_t)j * 4 * a.sub, ps + (int64_t)j * a.sub, a.sub, qv, acc);
  }
}

template <int G, int MODE>
__global__ __launch_bounds__(256) void scan_direct_kernel(ScanArgs a, Emit em) {
  __shared__ QShared<G> qs;
  __shared__ EmitShared<G> es;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t bh = blockIdx.y;
  const int64_t tile = a.tile0 + (int64_t)blockIdx.x * a.tile_stride;
  const int64_t gb0 = tile * kTB + wave * kGB;  // first block of this wave's group
  const uint32_t pf = load_qw<G>(qs, a, bh, tile * kTB, true);
  __syncthreads();
  float acc[kGB][G];
#pragma unroll
  for (int r = 0; r < kGB; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[r][g] = 0.0f;
  // groups outside the emitted range or past the store are not read
  if (gb0 < a.blk_end && gb0 + kGB > a.blk0 && gb0 < a.nsb * a.sub) {
    const int64_t sb = sgpr64(gb0 / a.sub);
    const int64_t off = gb0 - sb * a.sub;
    const uint64_t *pw = a.planes + (bh * a.nsb + sb) * a.D * 4 * a.sub + off;
    const uint16_t *ps = a.scales + (bh * a.nsb + sb) * a.D * a.sub + off;
    direct_class<1, G>(a, qs, bh, pw, ps, acc);
    direct_class<2, G>(a, qs, bh, pw, ps, acc);
    direct_class<3, G>(a, qs, bh, pw, ps, acc);
    direct_class<4, G>(a, qs, bh, pw, ps, acc);
  }
  asm volatile("" ::"v"(pf));  // the prefetch loads retire here
  emit_group<G, MODE>(em, es, acc, bh, gb0, a.blk0, a.blk_end, a.n, wave, lane, blockIdx.x);
}

// --------------------------------------------------------------------- staged kernel
template <int G>
struct StagedShared {
  uint64_t w[kCH * 4 * kTB];   // [channel][plane][block]
  uint16_t s[kCH * kTB];       // [channel][block]
  int ch[kCH];
};

template <int C, int G>
__device__ __forceinline__ void staged_class(const ScanArgs &a, const QShared<G> &qs, StagedShared<G> &st, int64_t bh,
                                             int64_t tb0, int wave, int lane, float (&acc)[kGB][G]) {
  if (C > a.ncls) return;
  const int tid = threadIdx.x;
  const int nc = min(max(a.clsn[bh * a.bmax + C - 1], 0), a.D);
  const int32_t *lst = a.cls + (bh * a.bmax + C - 1) * a.D;
  const int64_t nblk_store = a.nsb * a.sub;
  for (int c0 = 0; c0 < nc; c0 += kCH) {
    const int na = min(kCH, nc - c0);
    __syncthreads();  // the previous chunk is consumed
    if (tid < na) {
      const int j = lst[c0 + tid];
      st.ch[tid] = (j >= 0 && j < a.D) ? j : -1;
    }
    __syncthreads();
    // consecutive threads read consecutive blocks of one (channel, plane):
    // contiguous words within each superblock
    for (int idx = tid; idx < na * C * kTB; idx += 256) {
      const int bi = idx % kTB, p = (idx / kTB) % C, ci = idx / (C * kTB);
      const int j = st.ch[ci];
      const int64_t b = tb0 + bi;
      uint64_t v = 0ull;
      if (j >= 0 && b < nblk_store) {
        const int64_t sb = b / a.sub;
        v = a.planes[((bh * a.nsb + sb) * a.D + j) * 4 * a.sub + p * a.sub + (b - sb * a.sub)];
      }
      st.w[(ci * 4 + p) * kTB + bi] = v;
    }
    for (int idx = tid; idx < na * kTB; idx += 256) {
      const int bi = idx % kTB, ci = idx / kTB;
      const int j = st.ch[ci];
      const int64_t b = tb0 + bi;
      uint16_t v = 0;
      if (j >= 0 && b < nblk_store) {
        const int64_t sb = b / a.sub;
        v = a.scales[((bh * a.nsb + sb) * a.D + j) * a.sub + (b - sb * a.sub)];
      }
      st.s[ci * kTB + bi] = v;
    }
    __syncthreads();
    for (int ci = 0; ci < na; ++ci) {
      const int j = st.ch[ci];
      if (j < 0) continue;
      float qv[G];
#pragma unroll
      for (int g = 0; g < G; ++g) qv[g] = qs.qw[j * G + g];
#pragma unroll
      for (int r = 0; r < kGB; ++r) {
        const int bi = wave * kGB + r;
        uint32_t code = 0;
#pragma unroll
        for (int p = 0; p < C; ++p) code = (code << 1) | (uint32_t)((st.w[(ci * 4 + p) * kTB + bi] >> lane) & 1ull);
        const float u = scaled(st.s[ci * kTB + bi], sym_from_int<C>(code));
#pragma unroll
        for (int g = 0; g < G; ++g) acc[r][g] = fmaf(qv[g], u, acc[r][g]);
      }
    }
  }
}

template <int G, int MODE>
__global__ __launch_bounds__(256) void scan_staged_kernel(ScanArgs a, Emit em) {
  __shared__ QShared<G> qs;
  __shared__ StagedShared<G> st;
  __shared__ EmitShared<G> es;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t bh = blockIdx.y;
  const int64_t tile = a.tile0 + (int64_t)blockIdx.x * a.tile_stride;
  const int64_t tb0 = tile * kTB;
  load_qw<G>(qs, a, bh, tb0, false);
  __syncthreads();
  float acc[kGB][G];
#pragma unroll
  for (int r = 0; r < kGB; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[r][g] = 0.0f;
  // the whole workgroup takes part in staging, so the range test is per tile
  if (tb0 < a.blk_end && tb0 + kTB > a.blk0) {
    staged_class<1, G>(a, qs, st, bh, tb0, wave, lane, acc);
    staged_class<2, G>(a, qs, st, bh, tb0, wave, lane, acc);
    staged_class<3, G>(a, qs, st, bh, tb0, wave, lane, acc);
    staged_class<4, G>(a, qs, st, bh, tb0, wave, lane, acc);
  }
  emit_group<G, MODE>(em, es, acc, bh, tb0 + wave * kGB, a.blk0, a.blk_end, a.n, wave, lane, blockIdx.x);
}

// --------------------------------------------------------------------- launch
template <int G, int MODE>
void launch_g(const ScanArgs &a, int64_t tiles, int64_t BH, bool staged, const Emit &em, hipStream_t st) {
  dim3 grid((unsigned)tiles, (unsigned)BH);
  if (staged)
    scan_staged_kernel<G, MODE><<<grid, 256, 0, st>>>(a, em);
  else
    scan_direct_kernel<G, MODE><<<grid, 256, 0, st>>>(a, em);
}

template <int MODE>
int launch_scan(const ScanArgs &a, int64_t G, int64_t tiles, int64_t BH, bool staged, const Emit &em,
                hipStream_t st) {
  if (tiles <= 0) return FATHOM_OK;
  switch (G) {
    case 1: launch_g<1, MODE>(a, tiles, BH, staged, em, st); break;
    case 2: launch_g<2, MODE>(a, tiles, BH, staged, em, st); break;
    case 3: launch_g<3, MODE>(a, tiles, BH, staged, em, st); break;
    case 4: launch_g<4, MODE>(a, tiles, BH, staged, em, st); break;
    case 5: launch_g<5, MODE>(a, tiles, BH, staged, em, st); break;
    case 6: launch_g<6, MODE>(a, tiles, BH, staged, em, st); break;
    case 7: launch_g<7, MODE>(a, tiles, BH, staged, em, st); break;
    default: launch_g<8, MODE>(a, tiles, BH, staged, em, st); break;
  }
  return launch_status(staged ? "scan_staged_kernel" : "scan_direct_kernel");
}

// Stores in pinned host memory take the staged kernel (whole-run PCIe reads),
// as do superblock sizes that do not hold whole 8-block groups.
bool use_staged(const void *planes, int64_t sub) {
  if (sub % kGB != 0) return true;
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, planes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return attr.type == hipMemoryTypeHost;
}

int check_scan(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax,
               const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, const char *who) {
  if (!q || !cls || !clsn || !planes_sb || !scales_sb) return fail(FATHOM_ERR_INVALID, "%s: null pointer", who);
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "%s: BH=%lld outside [1, 65535]", who, (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "%s: G=%lld outside [1, 8]", who, (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "%s: D=%lld outside [1, %d]", who, (long long)D, kMaxD);
  if (bmax < 1 || bmax > 8) return fail(FATHOM_ERR_INVALID, "%s: bmax=%d outside [1, 8]", who, bmax);
  if (n < 1 || n > (1LL << 31) || sub < 1)
    return fail(FATHOM_ERR_INVALID, "%s: n=%lld sub=%lld unsupported", who, (long long)n, (long long)sub);
  if (nsb < 1 || nsb * sub < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "%s: store holds %lld blocks (nsb=%lld x sub=%lld), n needs %lld", who,
                (long long)(nsb * sub), (long long)nsb, (long long)sub, (long long)cdiv(n, kBlk));
  return FATHOM_OK;
}

ScanArgs make_args(const float *q, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax, const void *planes_sb,
                   const void *scales_sb, int64_t n, int64_t nsb, int64_t sub) {
  ScanArgs a{};
  a.q = q;
  a.cls = cls;
  a.clsn = clsn;
  a.planes = static_cast<const uint64_t *>(planes_sb);
  a.scales = static_cast<const uint16_t *>(scales_sb);
  a.n = n;
  a.nsb = nsb;
  a.sub = sub;
  a.D = (int)D;
  a.bmax = bmax;
  a.ncls = bmax < 4 ? bmax : 4;
  a.tile_stride = 1;
  return a;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_planes(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                  const int32_t *clsn, int bmax, const void *planes_sb, const void *scales_sb,
                                  int64_t n, int64_t nsb, int64_t sub, int64_t blk0, int64_t blk1, float *out,
                                  void *stream) {
  int rc = check_scan(q, BH, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub, "scan_planes");
  if (rc) return rc;
  if (!out) return fail(FATHOM_ERR_INVALID, "scan_planes: null output");
  if (blk0 < 0 || blk1 < blk0)
    return fail(FATHOM_ERR_INVALID, "scan_planes: bad block range [%lld, %lld)", (long long)blk0, (long long)blk1);
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t blk_end = blk1 < nblk ? blk1 : nblk;
  if (blk_end <= blk0) return FATHOM_OK;
  ScanArgs a = make_args(q, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = blk0;
  a.blk_end = blk_end;
  a.tile0 = blk0 / kTB;
  const int64_t tiles = cdiv(blk_end, kTB) - a.tile0;
  Emit em{};
  em.out = out;
  return launch_scan<kEmitScores>(a, G, tiles, BH, use_staged(planes_sb, sub), em, (hipStream_t)stream);
}

extern "C" size_t fathom_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t n, int64_t k, int64_t sink,
                                                   int64_t local) {
  const int64_t kk = k - sink - local;
  if (BH < 1 || G < 1 || n < 1 || kk < 0) return 0;
  return topk_layout(BH * G, n, k, nullptr, nullptr, nullptr, nullptr, nullptr);
}

extern "C" int fathom_scan_topk(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                const int32_t *clsn, int bmax, const void *planes_sb, const void *scales_sb,
                                int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink,
                                int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_scan(q, BH, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub, "scan_topk");
  if (rc) return rc;
  if (!idx) return fail(FATHOM_ERR_INVALID, "scan_topk: null output");
  const int64_t rows = BH * G;
  rc = check_topk_args(rows, n, m, k, sink, local, "scan_topk");
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int64_t kk = k - sink - local;
  if (kk == 0) return launch_fixed_only(rows, m, k, sink, local, idx, st);
  const size_t need = topk_layout(rows, n, k, nullptr, nullptr, nullptr, nullptr, nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "scan_topk: workspace %zu bytes, need %zu", workspace_bytes, need);
  Emit em{};
  int64_t S = 1;
  topk_layout(rows, n, k, static_cast<char *>(workspace), &em.samp, &em.samp_cap, &em.sel, &S);
  em.sink = sink;
  em.lstart = (m - local) > 0 ? (m - local) : 0;
  const int64_t nblk = cdiv(n, kBlk);
  const bool staged = use_staged(planes_sb, sub);
  ScanArgs a = make_args(q, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = 0;
  a.blk_end = nblk;
  a.tile0 = 0;
  a.tile_stride = S;
  rc = launch_scan<kEmitSample>(a, G, topk_sample_tiles(n, S), BH, staged, em, st);
  if (rc) return rc;
  rc = launch_select_keys(em.samp, rows, em.samp_cap, kk, em.sel, st);
  if (rc) return rc;
  a.tile_stride = 1;
  rc = launch_scan<kEmitFilter>(a, G, cdiv(nblk, kTB), BH, staged, em, st);
  if (rc) return rc;
  return launch_finalize(rows, m, k, sink, local, em.sel, idx, st);
}
