// Partial-depth bit-plane scan (PlaneStore.scan) and the fused scan + top-k.
//
// A workgroup (4 waves) owns one (batch*KV head, tile of 32 blocks = 2048
// tokens); wave w owns blocks 8w..8w+7 of the tile and lane = token of a block.
// Active channels are processed 32 at a time.  For each chunk the workgroup
// writes to LDS the per (channel, block, head) weight q_gj * a_bj * 2^(1-t_j)
// (the dequantiser's step) and accumulates the constant q_gj a_bj (2^-t_j - 1);
// then every wave adds weight * code for its tokens.
//
// Two ways of reaching the plane words (chosen per call from the store's memory
// type):
//  * direct (store in HBM): the words of a (channel, plane) for the wave's 8
//    blocks are wave-uniform, so they arrive by scalar loads (two 32-byte loads
//    when the 8 blocks are consecutive words) into SGPRs, and each word is used
//    as the lane mask of v_cndmask (inverse ballot): the t-bit code of the
//    lane's token is a sum of t masked power-of-two constants -- 2t-1 VALU ops,
//    no per-lane bit extraction and no LDS traffic for the planes;
//  * staged (store in mapped host memory): the chunk's words and scales are
//    copied to LDS with coalesced 8-byte vector loads, so the PCIe reads are
//    whole (channel, plane) runs, and lanes extract bits from LDS.
// Both produce bit-identical scores (same products, same summation order).
//
// Output modes: scores [BH, G, n] (PlaneStore.scan), sampled keys (every S-th
// tile, for the top-k threshold), or candidate emission (key >= threshold ->
// per-row candidate list, aggregated per workgroup in LDS), the last two
// fusing the scan with the top-k.
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr int kTB = 32;     // blocks per tile
constexpr int kBPW = 8;     // blocks per wave
constexpr int kCH = 32;     // active channels per chunk
constexpr int kMaxD = 256;
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

typedef unsigned int u32x8 __attribute__((ext_vector_type(8)));  // four 64-bit plane words

// Wave-uniform loads through the constant address space: always scalar loads
// into SGPRs (the store and plan are read-only for the kernel's lifetime).
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// Weight exponent: codes of depth 4 are formed as code/2 (the inline constants
// 4, 2, 1, 0.5), so their weight carries one more factor of two.
__device__ __forceinline__ int wexp(int c) { return c >= 4 ? -2 : 1 - c; }

__device__ __forceinline__ int64_t word_base(int64_t bh, int64_t b, int64_t nsb, int64_t sub, int D) {
  const int64_t sb = b / sub;
  return (bh * nsb + sb) * D * 4 * sub + (b - sb * sub);
}

__device__ __forceinline__ int64_t scale_index(int64_t bh, int64_t b, int64_t nsb, int64_t sub, int D, int j) {
  const int64_t sb = b / sub;
  return ((bh * nsb + sb) * D + j) * sub + (b - sb * sub);
}

template <int G>
struct ScanShared {
  float q[G * kMaxD];
  int ch[kCH];
  int dep[kCH];
  float sc[kCH * kTB];
  float wt[kCH * kTB * G];  // [channel][block][head]
  float cst[kTB * G];
  uint64_t lbuf[G][kRowLocal];
  uint32_t lcnt[G];
  uint32_t lbase[G];
};

// Chunk prologue: channel list, block scales, weights, constant term.
template <int G>
__device__ __forceinline__ void chunk_prepare(ScanShared<G> &sh, const int8_t *tpl, const int32_t *act,
                                              const uint16_t *scales, int64_t bh, int64_t tb0, int64_t blk_end,
                                              int64_t nsb, int64_t sub, int D, int a0, int na, float &cst_acc) {
  const int tid = threadIdx.x;
  if (tid < na) {
    const int j = act[bh * D + a0 + tid];
    const bool ok = j >= 0 && j < D;
    sh.ch[tid] = ok ? j : 0;
    sh.dep[tid] = ok ? min(max((int)tpl[bh * D + j], 0), 4) : 0;
  }
  __syncthreads();
  for (int idx = tid; idx < na * kTB; idx += 256) {
    const int bi = idx % kTB, a = idx / kTB;
    const int64_t b = tb0 + bi;
    sh.sc[idx] = (b < blk_end && sh.dep[a] > 0) ? f16_bits_to_float(scales[scale_index(bh, b, nsb, sub, D, sh.ch[a])])
                                                : 0.0f;
  }
  __syncthreads();
  for (int idx = tid; idx < na * kTB * G; idx += 256) {
    const int g = idx % G, bi = (idx / G) % kTB, a = idx / (G * kTB);
    sh.wt[idx] = sh.q[g * D + sh.ch[a]] * ldexpf(sh.sc[a * kTB + bi], wexp(sh.dep[a]));
  }
  if (tid < kTB * G) {
    const int bi = tid / G, g = tid % G;
    for (int a = 0; a < na; ++a) {
      const float cadd = ldexpf(0.5f, 1 - sh.dep[a]) - 1.0f;  // 2^-t - 1
      cst_acc += sh.q[g * D + sh.ch[a]] * (sh.sc[a * kTB + bi] * cadd);
    }
  }
  __syncthreads();
}

template <int G, int MODE>
__device__ __forceinline__ void emit_tile(const Emit &em, ScanShared<G> &sh, float (&acc)[kBPW][G],
                                          float cst_acc, int64_t bh, int64_t tb0, int64_t blk_end, int64_t n,
                                          int wave, int lane, int64_t tile_idx) {
  const int tid = threadIdx.x;
  if (tid < kTB * G) sh.cst[tid] = cst_acc;
  if (MODE == kEmitFilter && tid < G) sh.lcnt[tid] = 0u;
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
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kBPW; ++r) {
    const int bi = wave * kBPW + r;
    const int64_t b = tb0 + bi;
    const int64_t tok = b * kBlk + lane;
    const bool valid = b < blk_end && tok < n;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = acc[r][g] + sh.cst[bi * G + g];
      const int64_t row = bh * G + g;
      if (MODE == kEmitScores) {
        if (valid) em.out[row * n + tok] = v;
      } else {
        const bool masked = tok < em.sink || tok >= em.lstart;
        if (MODE == kEmitSample) {
          const uint32_t key = valid ? (masked ? kKeyNegInf : score_key(v)) : 0u;
          em.samp[row * em.samp_cap + tile_idx * kTileTok + bi * kBlk + lane] = key;
        } else {
          // key >= thr tested on floats: thr_f is the value whose key is thr
          const float vm = masked ? -INFINITY : v;
          const bool pass = valid && (thr_all[g] || vm >= thr_f[g] || vm != vm);
          wave_append_local(pass, pass ? k64_of(masked ? kKeyNegInf : score_key(v), tok) : 0ull, &sh.lcnt[g],
                            sh.lbuf[g], kRowLocal, &em.sel.cand_cnt[row], em.sel.cand + row * em.sel.cand_cap,
                            (uint64_t)em.sel.cand_cap, lane);
        }
      }
    }
  }
  if (MODE == kEmitFilter) {
    // one reservation per row, all rows at once, then one copy pass
    __syncthreads();
    if (tid < G) {
      const uint32_t nloc = min(sh.lcnt[tid], kRowLocal);
      sh.lbase[tid] = nloc ? atomicAdd(&em.sel.cand_cnt[bh * G + tid], nloc) : 0u;
    }
    __syncthreads();
    for (int e = tid; e < G * (int)kRowLocal; e += 256) {
      const int g = e / (int)kRowLocal, i = e % (int)kRowLocal;
      const uint32_t nloc = min(sh.lcnt[g], kRowLocal);
      const uint64_t slot = (uint64_t)sh.lbase[g] + i;
      if ((uint32_t)i < nloc && slot < (uint64_t)em.sel.cand_cap)
        em.sel.cand[(bh * G + g) * em.sel.cand_cap + slot] = sh.lbuf[g][i];
    }
  }
}

// --------------------------------------------------------------------- direct (HBM) kernel
// Value of a depth-C code of block r from its C plane words held in SGPRs: each
// word is the lane mask of a v_cndmask between 0 and a power of two (inline
// constants; depth 4 yields code / 2).
template <int C>
__device__ __forceinline__ float code_value(const uint64_t (&w)[C][4], int r) {
  if (C == 1) return __builtin_amdgcn_inverse_ballot_w64(w[0][r]) ? 1.0f : 0.0f;
  if (C == 2)
    return (__builtin_amdgcn_inverse_ballot_w64(w[0][r]) ? 2.0f : 0.0f) +
           (__builtin_amdgcn_inverse_ballot_w64(w[C > 1 ? 1 : 0][r]) ? 1.0f : 0.0f);
  if (C == 3)
    return ((__builtin_amdgcn_inverse_ballot_w64(w[0][r]) ? 4.0f : 0.0f) +
            (__builtin_amdgcn_inverse_ballot_w64(w[C > 1 ? 1 : 0][r]) ? 2.0f : 0.0f)) +
           (__builtin_amdgcn_inverse_ballot_w64(w[C > 2 ? 2 : 0][r]) ? 1.0f : 0.0f);
  return ((__builtin_amdgcn_inverse_ballot_w64(w[0][r]) ? 4.0f : 0.0f) +
          (__builtin_amdgcn_inverse_ballot_w64(w[C > 1 ? 1 : 0][r]) ? 2.0f : 0.0f)) +
         ((__builtin_amdgcn_inverse_ballot_w64(w[C > 2 ? 2 : 0][r]) ? 1.0f : 0.0f) +
          (__builtin_amdgcn_inverse_ballot_w64(w[C > 3 ? 3 : 0][r]) ? 0.5f : 0.0f));
}

__device__ __forceinline__ uint64_t word_of(const u32x8 &v, int r) {
  return ((uint64_t)v[2 * r + 1] << 32) | v[2 * r];
}

__device__ __forceinline__ int64_t sgpr64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// One active channel of depth C for the wave's 8 blocks, in two halves of 4
// blocks (at most 32 SGPRs of plane words live): every plane word of a half is
// requested before the first is used, then weight * code.  CONTIG: the 8 blocks
// are 8 consecutive words of each (channel, plane) starting at wb0, one 32-byte
// scalar load per plane and half; otherwise one scalar load per block from the
// per-block word offsets in LDS (negative: block past the scanned range).
template <int C, int G, bool CONTIG>
__device__ __forceinline__ void accum_channel(const uint64_t *planes, int64_t wb0, const int64_t *wbs, int64_t coff,
                                              int64_t sub, const float *wt, float (&acc)[kBPW][G]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // keeps the second half's loads below the first half's use (merged into
    // one 64-byte load per plane they would need up to 64 SGPRs and spill)
    if (h == 1 && C >= 3) __builtin_amdgcn_sched_barrier(0);
    uint64_t w[C][4];
#pragma unroll
    for (int p = 0; p < C; ++p) {
      if (CONTIG) {
        const u32x8 v = ld_uniform(reinterpret_cast<const u32x8 *>(planes + wb0 + coff + p * sub + 4 * h));
#pragma unroll
        for (int r = 0; r < 4; ++r) w[p][r] = word_of(v, r);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t b = sgpr64(wbs[4 * h + r]);
          w[p][r] = b >= 0 ? ld_uniform(planes + b + coff + p * sub) : 0ull;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cf = code_value<C>(w, r);
#pragma unroll
      for (int g = 0; g < G; ++g) acc[4 * h + r][g] = fmaf(wt[(4 * h + r) * G + g], cf, acc[4 * h + r][g]);
    }
  }
}

template <int G, bool CONTIG>
__device__ __forceinline__ void accum_switch(int c, const uint64_t *planes, int64_t wb0, const int64_t *wbs,
                                             int64_t coff, int64_t sub, const float *wt, float (&acc)[kBPW][G]) {
  switch (c) {
    case 1: accum_channel<1, G, CONTIG>(planes, wb0, wbs, coff, sub, wt, acc); break;
    case 2: accum_channel<2, G, CONTIG>(planes, wb0, wbs, coff, sub, wt, acc); break;
    case 3: accum_channel<3, G, CONTIG>(planes, wb0, wbs, coff, sub, wt, acc); break;
    case 4: accum_channel<4, G, CONTIG>(planes, wb0, wbs, coff, sub, wt, acc); break;
    default: break;
  }
}

template <int G, int MODE>
__global__ __launch_bounds__(256) void scan_direct_kernel(
    const float *__restrict__ q, int D, const int8_t *__restrict__ tpl, const int32_t *__restrict__ act,
    const int32_t *__restrict__ nact_p, const uint64_t *__restrict__ planes, const uint16_t *__restrict__ scales,
    int64_t n, int64_t nsb, int64_t sub, int64_t blk0, int64_t blk_end, int64_t tile_stride, Emit em) {
  __shared__ ScanShared<G> sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = blockIdx.y;
  const int64_t tb0 = blk0 + (int64_t)blockIdx.x * tile_stride * kTB;
  // Plan entries come from device memory: a channel outside [0, D) or a depth
  // <= 0 contributes nothing, depths above the store's 4 planes read 4.
  const int nact = min(max(nact_p[bh], 0), D);

  for (int i = tid; i < G * D; i += 256) sh.q[i] = q[bh * G * D + i];
  // word offsets of the tile's blocks (-1 past the scanned range)
  __shared__ int64_t wbs[kTB];
  if (tid < kTB) {
    const int64_t b = tb0 + tid;
    wbs[tid] = b < blk_end ? word_base(bh, b, nsb, sub, D) : -1;
  }
  __syncthreads();
  const int64_t *wbw = &wbs[wave * kBPW];
  const int64_t wb0 = sgpr64(wbw[0]);
  const bool contig = wb0 >= 0 && sgpr64(wbw[kBPW - 1]) == wb0 + (kBPW - 1);
  float acc[kBPW][G];
#pragma unroll
  for (int r = 0; r < kBPW; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[r][g] = 0.0f;
  float cst_acc = 0.0f;

  for (int a0 = 0; a0 < nact; a0 += kCH) {
    const int na = min(kCH, nact - a0);
    __syncthreads();  // LDS of the previous chunk is consumed
    // L2 prefetch: one dword per (channel, plane, half tile) pulls the chunk's
    // 128-byte plane lines into L2 while the prologue runs, so the scalar
    // loads below hit L2 instead of waiting on HBM one channel at a time.
    uint32_t pf = 0u;
    {
      const int a = tid >> 3, p = (tid >> 1) & 3, hb = (tid & 1) * (kTB / 2);
      if (a < na) {
        const int j = act[bh * D + a0 + a];
        if (j >= 0 && j < D && p < (int)tpl[bh * D + j]) {
          const int64_t b = tb0 + hb;
          if (b < blk_end)
            pf = *reinterpret_cast<const uint32_t *>(planes + word_base(bh, b, nsb, sub, D) + ((int64_t)j * 4 + p) * sub);
        }
      }
    }
    chunk_prepare<G>(sh, tpl, act, scales, bh, tb0, blk_end, nsb, sub, D, a0, na, cst_acc);
    for (int a = 0; a < na; ++a) {
      // readfirstlane: the compiler cannot prove the loop index wave-uniform
      // across the barriers above; channel and depth stay in SGPRs
      const int ai = __builtin_amdgcn_readfirstlane(a0 + a);
      const int j0 = __builtin_amdgcn_readfirstlane(ld_uniform(act + bh * D + ai));
      const bool ok = j0 >= 0 && j0 < D;
      const int j = ok ? j0 : 0;
      const int c = __builtin_amdgcn_readfirstlane(ok ? min(max((int)ld_uniform(tpl + bh * D + j), 0), 4) : 0);
      const int64_t coff = (int64_t)j * 4 * sub;
      const float *wt = &sh.wt[(a * kTB + wave * kBPW) * G];
      if (contig)
        accum_switch<G, true>(c, planes, wb0, wbw, coff, sub, wt, acc);
      else
        accum_switch<G, false>(c, planes, wb0, wbw, coff, sub, wt, acc);
    }
    asm volatile("" ::"v"(pf));  // the prefetched dword is retired here, after the chunk's work
  }
  __syncthreads();
  emit_tile<G, MODE>(em, sh, acc, cst_acc, bh, tb0, blk_end, n, wave, lane, blockIdx.x);
}

// --------------------------------------------------------------------- staged (host-resident) kernel
template <int G>
struct StagedShared {
  ScanShared<G> s;
  uint64_t w[kCH * 4 * kTB];  // [channel][plane][block]
};

template <int G, int MODE>
__global__ __launch_bounds__(256) void scan_staged_kernel(
    const float *__restrict__ q, int D, const int8_t *__restrict__ tpl, const int32_t *__restrict__ act,
    const int32_t *__restrict__ nact_p, const uint64_t *__restrict__ planes, const uint16_t *__restrict__ scales,
    int64_t n, int64_t nsb, int64_t sub, int64_t blk0, int64_t blk_end, int64_t tile_stride, Emit em) {
  __shared__ StagedShared<G> st;
  ScanShared<G> &sh = st.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = blockIdx.y;
  const int64_t tb0 = blk0 + (int64_t)blockIdx.x * tile_stride * kTB;
  const int nact = min(max(nact_p[bh], 0), D);

  for (int i = tid; i < G * D; i += 256) sh.q[i] = q[bh * G * D + i];
  float acc[kBPW][G];
#pragma unroll
  for (int r = 0; r < kBPW; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[r][g] = 0.0f;
  float cst_acc = 0.0f;

  for (int a0 = 0; a0 < nact; a0 += kCH) {
    const int na = min(kCH, nact - a0);
    __syncthreads();
    chunk_prepare<G>(sh, tpl, act, scales, bh, tb0, blk_end, nsb, sub, D, a0, na, cst_acc);
    // stage the tile's plane words of the chunk: consecutive threads read
    // consecutive blocks of one (channel, plane), i.e. contiguous 8-byte words
    for (int idx = tid; idx < na * 4 * kTB; idx += 256) {
      const int bi = idx % kTB, p = (idx / kTB) % 4, a = idx / (4 * kTB);
      if (p < sh.dep[a]) {
        const int64_t b = tb0 + bi;
        st.w[idx] = (b < blk_end) ? planes[word_base(bh, b, nsb, sub, D) + ((int64_t)sh.ch[a] * 4 + p) * sub] : 0ull;
      }
    }
    __syncthreads();
    for (int a = 0; a < na; ++a) {
      const int c = sh.dep[a];
      const uint64_t *wa = &st.w[a * 4 * kTB];
#pragma unroll
      for (int r = 0; r < kBPW; ++r) {
        const int bi = wave * kBPW + r;
        uint32_t code = 0;
        for (int p = 0; p < c; ++p) code = (code << 1) | (uint32_t)((wa[p * kTB + bi] >> lane) & 1ull);
        // same encoding as the direct kernel: depth-4 codes enter as code/2
        const float cf = (c >= 4) ? 0.5f * (float)code : (float)code;
        const float *wt = &sh.wt[(a * kTB + bi) * G];
#pragma unroll
        for (int g = 0; g < G; ++g) acc[r][g] = fmaf(wt[g], cf, acc[r][g]);
      }
    }
  }
  __syncthreads();
  emit_tile<G, MODE>(em, sh, acc, cst_acc, bh, tb0, blk_end, n, wave, lane, blockIdx.x);
}

struct ScanCall {
  const float *q;
  int64_t BH, G;
  int D;
  const int8_t *t;
  const int32_t *act, *nact;
  const uint64_t *planes;
  const uint16_t *scales;
  int64_t n, nsb, sub, blk0, blk_end;
  bool host_store;
};

// The sampling pass runs few workgroups, too few to hide the direct kernel's
// per-channel scalar-load latency: it takes the staged kernel, which issues a
// chunk's loads together (same scores bit for bit).
template <int G, int MODE>
void launch_g(const ScanCall &c, int64_t tiles, int64_t stride, const Emit &em, hipStream_t st) {
  dim3 grid((unsigned)tiles, (unsigned)c.BH);
  if (c.host_store || MODE == kEmitSample)
    scan_staged_kernel<G, MODE><<<grid, 256, 0, st>>>(c.q, c.D, c.t, c.act, c.nact, c.planes, c.scales, c.n, c.nsb,
                                                      c.sub, c.blk0, c.blk_end, stride, em);
  else
    scan_direct_kernel<G, MODE><<<grid, 256, 0, st>>>(c.q, c.D, c.t, c.act, c.nact, c.planes, c.scales, c.n, c.nsb,
                                                      c.sub, c.blk0, c.blk_end, stride, em);
}

template <int MODE>
int launch_scan(const ScanCall &c, int64_t tiles, int64_t stride, const Emit &em, hipStream_t st) {
  if (tiles <= 0) return FATHOM_OK;
  switch (c.G) {
    case 1: launch_g<1, MODE>(c, tiles, stride, em, st); break;
    case 2: launch_g<2, MODE>(c, tiles, stride, em, st); break;
    case 3: launch_g<3, MODE>(c, tiles, stride, em, st); break;
    case 4: launch_g<4, MODE>(c, tiles, stride, em, st); break;
    case 5: launch_g<5, MODE>(c, tiles, stride, em, st); break;
    case 6: launch_g<6, MODE>(c, tiles, stride, em, st); break;
    case 7: launch_g<7, MODE>(c, tiles, stride, em, st); break;
    default: launch_g<8, MODE>(c, tiles, stride, em, st); break;
  }
  return launch_status((c.host_store || MODE == kEmitSample) ? "scan_staged_kernel" : "scan_direct_kernel");
}

// Stores in pinned host memory take the staged kernel (whole-run PCIe reads);
// device memory takes the direct kernel.
bool is_host_memory(const void *p) {
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return attr.type == hipMemoryTypeHost;
}

int check_scan(const float *q, int64_t BH, int64_t G, int64_t D, const int8_t *t, const int32_t *act,
               const int32_t *nact, const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub,
               const char *who) {
  if (!q || !t || !act || !nact || !planes_sb || !scales_sb) return fail(FATHOM_ERR_INVALID, "%s: null pointer", who);
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "%s: BH=%lld outside [1, 65535]", who, (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "%s: G=%lld outside [1, 8]", who, (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "%s: D=%lld outside [1, %d]", who, (long long)D, kMaxD);
  if (n < 1 || sub < 1) return fail(FATHOM_ERR_INVALID, "%s: n=%lld sub=%lld", who, (long long)n, (long long)sub);
  if (nsb * sub < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "%s: store holds %lld blocks (nsb=%lld x sub=%lld), n needs %lld", who,
                (long long)(nsb * sub), (long long)nsb, (long long)sub, (long long)cdiv(n, kBlk));
  return FATHOM_OK;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_planes(const float *q, int64_t BH, int64_t G, int64_t D, const int8_t *t,
                                  const int32_t *act, const int32_t *nact, const void *planes_sb,
                                  const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t blk0,
                                  int64_t blk1, float *out, void *stream) {
  int rc = check_scan(q, BH, G, D, t, act, nact, planes_sb, scales_sb, n, nsb, sub, "scan_planes");
  if (rc) return rc;
  if (!out) return fail(FATHOM_ERR_INVALID, "scan_planes: null output");
  if (blk0 < 0 || blk1 < blk0)
    return fail(FATHOM_ERR_INVALID, "scan_planes: bad block range [%lld, %lld)", (long long)blk0, (long long)blk1);
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t blk_end = blk1 < nblk ? blk1 : nblk;
  if (blk_end <= blk0) return FATHOM_OK;
  const int64_t tiles = cdiv(blk_end - blk0, kTB);
  if (tiles > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "scan_planes: too many tiles");
  ScanCall c{q, BH, G, (int)D, t, act, nact, static_cast<const uint64_t *>(planes_sb),
             static_cast<const uint16_t *>(scales_sb), n, nsb, sub, blk0, blk_end, is_host_memory(planes_sb)};
  Emit em{};
  em.out = out;
  return launch_scan<kEmitScores>(c, tiles, 1, em, (hipStream_t)stream);
}

extern "C" size_t fathom_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t n, int64_t k, int64_t sink,
                                                   int64_t local) {
  const int64_t kk = k - sink - local;
  if (BH < 1 || G < 1 || n < 1 || kk < 0) return 0;
  return topk_layout(BH * G, n, k, nullptr, nullptr, nullptr, nullptr, nullptr);
}

extern "C" int fathom_scan_topk(const float *q, int64_t BH, int64_t G, int64_t D, const int8_t *t, const int32_t *act,
                                const int32_t *nact, const void *planes_sb, const void *scales_sb, int64_t n,
                                int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink, int64_t local,
                                int64_t *idx, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_scan(q, BH, G, D, t, act, nact, planes_sb, scales_sb, n, nsb, sub, "scan_topk");
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
  const int64_t tiles = cdiv(nblk, kTB);
  ScanCall c{q, BH, G, (int)D, t, act, nact, static_cast<const uint64_t *>(planes_sb),
             static_cast<const uint16_t *>(scales_sb), n, nsb, sub, 0, nblk, is_host_memory(planes_sb)};
  rc = launch_scan<kEmitSample>(c, topk_sample_tiles(n, S), S, em, st);
  if (rc) return rc;
  rc = launch_select_keys(em.samp, rows, em.samp_cap, kk, em.sel, st);
  if (rc) return rc;
  rc = launch_scan<kEmitFilter>(c, tiles, 1, em, st);
  if (rc) return rc;
  return launch_finalize(rows, m, k, sink, local, em.sel, idx, st);
}
