// The wave-tile machinery of the bit-plane scan (PlaneStore.scan): plan tables,
// the (channel, plane) contraction on the matrix cores, and the emission modes.
// Shared by the scan kernels and the fused top-k's finalize (its fallback rescan).
//
// Score of token i of row (bh, h), with depth t_j planes read for channel j
// (the dequantised value of kernels/bitplane.py:34-42; code bits b_jp, p = 0
// the most significant; a_bj the absmax scale of token block b):
//   s = sum_(j, p < t_j) q_hj a_bj 2^-p b_jp(i)  +  C_hb,
//   C_hb = sum_j q_hj a_bj (2^-t_j - 1).
//
// Matrix-core mapping (v_mfma_f32_16x16x32_f16, D[16 x 16] += A[16 x 32] B[32 x 16]).
// A wave owns a wave-tile of 16 consecutive token blocks (1024 tokens); MFMA
// column c is block c of the tile.  The contraction index k runs over the plan's
// (channel, plane) units, 32 per instruction:
//   A  row 2h + part: head h's weights Q_hu = q_hj 2^-(p + sigma_h) as an f16
//      hi part (truncated) or lo part (the remainder): 21 significant bits;
//      constant over the row, so loaded once per workgroup;
//   B  unit u's bit of one token of block c, as the f16 number bit * 2^e times
//      the block's rescaled scale a'_cj = a_cj 2^-s_c (one AND and one packed
//      f16 multiply per two units);
//   D  row 2h + part, column c: that token's partial sums, hi and lo.
// Rows 2G .. 15 are zero.  A token step r (0..15) of quarter qs (0..3) takes
// token 16 qs + r of every block of the tile: 64 steps cover the tile.  Each
// lane's 16-bit quarter of a plane word is half of a dword (two units per
// dword); shifting each half once per four steps puts the bits of tokens
// 4v..4v+3 on f16 exponent bits 11..14, so masking one leaves 0 or 2^e_w
// (e_w = -13, -11, -7, 1 for w = r mod 4).  Every product is exact and the
// accumulation is fp32; the score is
//   s = (D_hi + D_lo) * 2^(sigma_h + s_c - e_w) + C_hc,
// one fused multiply-add of an exact power-of-two product.  C comes from the
// same matrix instruction with B = the block's raw scales and A = the split of
// q_hj 2^-sigma_h (2^-t_j - 1) on each channel's first unit.
//
// A token's score is one chain of instructions over the plan's units in a fixed
// order: 32-unit slice pairs from zero (an odd last slice of 16 units with a
// zero upper half).  How the units are grouped in registers does not
// change the chain, so every emission mode, both register layouts (plans of at
// most 64 units held whole, larger ones in groups) and stores in HBM or in
// mapped host memory give the same scores bit for bit.
#pragma once
#include "topk_internal.hpp"
#include "plan_core.hpp"

namespace fathom {
namespace sc {

constexpr int kWB = 16;                // token blocks per wave-tile: one MFMA column each
constexpr int kWTok = kWB * kBlk;      // tokens per wave-tile
constexpr int kQS = 4;                 // quarters of a block (16 tokens each)
constexpr int kR = 16;                 // token steps per quarter
constexpr int kWaves = 4;              // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxD = 128;             // the reference's head dimension (kernels/bitplane.py:313)
constexpr int kMaxUnits = 4 * kMaxD;   // (channel, plane) units of a plan
constexpr int kSlice = 16;             // units per slice: four per lane group
constexpr int kGS = 4;                 // slices per register group
constexpr int kGU = kGS * kSlice;      // units per register group
constexpr int kMaxG = 8;               // query heads per matrix row tile (rows: head x {hi, lo})
constexpr int kRows = 16;
static_assert(kWTok == kRegTok, "a candidate region is one wave-tile");
static_assert(kR == kGroupTok, "a lane's quarter is one group of the group maxima");

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum : int { kEmitScores = 0, kEmitSample = 1, kEmitFilter = 2, kEmitScoresMax = 3 };

struct ScanArgs {
  const float *q;          // [BH, G, D]
  const int32_t *cls;      // [BH, bmax, D]
  const int32_t *clsn;     // [BH, bmax]
  const uint32_t *planes;  // [BH, nsb, D, 4, sub] 64-bit words, read as dwords
  const uint16_t *scales;  // [BH, nsb, D, sub] fp16 bits
  int64_t n, nsb, sub;
  int64_t blk0, blk_end;   // blocks [blk0, blk_end) are emitted
  int64_t wt0;             // wave-tile of list entry 0 (wave-tile T = blocks [16T, 16T + 16))
  int64_t wt_stride;       // wave-tiles between consecutive list entries
  int64_t nwt;             // list entries per row
  int D, G, bmax, ncls;    // classes 1..ncls are scanned (ncls = min(bmax, 4))
  // g non-null: the prologue plans its row itself (make_plan of g [BH, D] and
  // the row's budget, budget[bh] or budget_value, `iters` bisection steps;
  // cls and clsn unused) and the first workgroup of a row writes the plan's
  // depths to t_out [BH, D] (if non-null)
  const float *g, *budget;
  float budget_value;
  int iters;
  int8_t *t_out;
};

struct PlanTab;

struct Emit {
  float *out;        // scores [BH, G, n]
  uint32_t *gmax;    // kEmitScoresMax: [BH * G, ceil(n / 16)] each 16-token group's largest masked key
  uint32_t *samp;    // sampled keys [BH * G, samp_cap]: list entry L at L * kWTok
  int64_t samp_cap;
  TopkSel sel;       // thresholds + candidate regions
  int64_t sink, lstart;
  PlanTab *tab;      // [BH] plan tables: the sample pass writes them, the candidate pass reads them (null: none)
};

// Wave-uniform loads through the constant address space (scalar loads).
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// e_w: the f16 number 2^e_w that step class w's bit stands for once masked
// (exponent bit 11 + w of a half).
__host__ __device__ constexpr int bit_exp(int w) { return w == 0 ? -13 : w == 1 ? -11 : w == 2 ? -7 : 1; }

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The dword x with each 16-bit half shifted so that bits 4v..4v+3 land on
// bits 11..14 (higher bits of the half are dropped, lower ones stay below).
template <int V>
__device__ __forceinline__ uint32_t half_shift(uint32_t x) {
  const u16x2 h = __builtin_bit_cast(u16x2, x);
  constexpr int L = 11 - 4 * V;
  u16x2 r;
  if constexpr (L >= 0) r = h << (unsigned short)L;
  else r = h >> (unsigned short)(-L);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t pk_mul(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b));
}

// Plan tables of a row, built once per workgroup.  Units are in class order
// (the class 1 channel list, then 2, 3, 4; a channel's planes consecutive),
// padded to whole slices with units of zero weight and zero scale.
struct Shared {
  union {
    struct {
      uint32_t uoff[kMaxUnits];          // unit -> plane word byte offset in a superblock ((4 j + p) sub 8)
      uint32_t soff[kMaxUnits];          // unit -> scale byte offset in a superblock (j sub 2)
    };
    float qs[kMaxG][kMaxD];              // the queries (prologue, before the offsets are written)
  };
  _Float16 qa[kRows][kMaxUnits];         // score A rows: 2h = hi(q_hj 2^-(p + sigma_h)), 2h + 1 = lo
  _Float16 ca[kRows][kMaxUnits];         // C A rows: the split of q_hj 2^-sigma_h (2^-t_j - 1), first units only
  uint16_t schan[kMaxD];                 // channel slot -> channel (prologue)
  int pnc[4];                            // class sizes of a plan made in the prologue
  int sig[kMaxG];                        // sigma_h: the exponent of the head's largest |q|
  int U;                                 // units, padded to whole slices
  int ureal;                             // units of the plan
};

// The plan tables of one row, as the fused scan + top-k's sample pass leaves
// them for its candidate pass (plans of at most kTabUnits units): the
// candidate pass then starts from one copy instead of rebuilding them from the
// queries and class lists.
constexpr int kMaxNS = 6;              // slices a kernel holds in registers (96 units)
constexpr int kTabUnits = kMaxNS * kSlice;
struct PlanTab {
  int32_t U, ureal, pad[2];
  int32_t sig[kMaxG];
  uint32_t uoff[kTabUnits], soff[kTabUnits];
  _Float16 qa[kRows][kTabUnits], ca[kRows][kTabUnits];
};
static_assert(sizeof(PlanTab) % 16 == 0, "tables copy as 16-byte vectors");

// Orders a wave's LDS accesses: every lane's writes before any lane's reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A CU's waves of equal priority issue oldest first, so the workgroups placed
// first on a CU race ahead and the last ones run the kernel's tail at low
// occupancy.  Waves with more tiles left take a higher priority instead.
__device__ __forceinline__ void set_priority_by_tiles_left(int64_t left) {
  if (left >= 3) __builtin_amdgcn_s_setprio(3);
  else if (left == 2) __builtin_amdgcn_s_setprio(2);
  else if (left == 1) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// f16 truncation (round toward zero) of x.
__device__ __forceinline__ _Float16 f16_rtz(float x) { return __builtin_amdgcn_cvt_pkrtz(x, 0.0f)[0]; }

// The row's plan made by one wave (a.g set): make_plan's depths of the row's
// channels (2 per lane, the plan kernel's arithmetic), written to a.t_out by
// the row's first workgroup, and its class lists -- channels of depth c + 1,
// ascending, as make_plan's cls -- into sh.schan with their sizes in sh.pnc.
__device__ __forceinline__ void plan_row(Shared &sh, const ScanArgs &a, int64_t bh, int lane) {
  static_assert(kMaxD == 2 * kWave, "two channels per lane");
  const float bm = (float)a.bmax;
  float lg[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) lg[k] = plan::channel_lg(a.g, bh, a.D, 2 * lane + k);
  const float Br = a.budget ? a.budget[bh] : a.budget_value;
  const float hi = plan::water_line<2>(lg, Br, bm, a.iters);
  int t[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int j = 2 * lane + k;
    t[k] = j < a.D ? plan::depth_at(lg[k], hi, bm) : 0;
    if (a.t_out && blockIdx.x == 0 && j < a.D) a.t_out[bh * a.D + j] = (int8_t)t[k];
  }
  int s = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int cnt = c < a.ncls ? (t[0] == c + 1) + (t[1] == c + 1) : 0;
    int pos = s + wave_excl_scan_small<2>(cnt, lane);
    const int total = wave_sum_small<2>(cnt);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (c < a.ncls && t[k] == c + 1) sh.schan[pos++] = (uint16_t)(2 * lane + k);
    if (lane == 0) sh.pnc[c] = total;
    s += total;
  }
}

// Workgroup prologue: the plan tables in LDS, with zero units from the plan's
// last up to upad units (at least to a whole slice).  Returns the padded unit
// count.
__device__ __forceinline__ int plan_tables(Shared &sh, const ScanArgs &a, int64_t bh, int upad) {
  const int tid = threadIdx.x;
  const bool own = a.g != nullptr;  // the row planned here
  int nc[4], SF[4], UE[4];
  int s = 0, u = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    nc[c] = !own && c < a.ncls ? min(max(ld_uniform(a.clsn + bh * a.bmax + c), 0), a.D) : 0;
    nc[c] = min(nc[c], a.D - s);  // at most D slots in all
    s += nc[c];
    u += nc[c] * (c + 1);
    SF[c] = s;
    UE[c] = u;
  }
  // the prologue's global loads are issued together: the class lists (every
  // in-range entry of the bmax x D table) and the queries; or wave 0 plans the
  // row while the other waves load the queries
  {
    static_assert(kMaxD == 2 * kWave, "two channels per lane");
    static_assert(kThreads >= 2 * kWave, "a wave besides the planning one");
    const int nthr = (int)blockDim.x;
    const int w = tid >> 6, l = tid & 63;
    if (own && w == 0) plan_row(sh, a, bh, l);
    const int qw = own ? w - 1 : w, nw = own ? (nthr >> 6) - 1 : nthr >> 6;  // query waves: all but the planner
    for (int i0 = tid; !own && i0 < 4 * kMaxD; i0 += 2 * nthr) {
      int jr[2];
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        const int i = i0 + u2 * nthr, c = i / kMaxD, e = i % kMaxD;
        jr[u2] = (i < 4 * kMaxD && c < a.ncls && e < a.D) ? a.cls[(bh * a.bmax + c) * a.D + e] : 0;  // no wait on nc
      }
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        const int i = i0 + u2 * nthr, c = i / kMaxD, e = i % kMaxD;
        if (i < 4 * kMaxD && c < a.ncls && e < nc[c])  // slot SF[c - 1] + e (make_plan lists only valid channels)
          sh.schan[(c == 0 ? 0 : SF[c - 1]) + e] = (uint16_t)min(max(jr[u2], 0), a.D - 1);
      }
    }
    // a wave per head (heads qw, qw + nw, ...): its largest |q| gives sigma_h
    for (int h0 = qw; qw >= 0 && h0 < kMaxG; h0 += 2 * nw) {
      float qv[2][2];
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        const int h = h0 + u2 * nw;
        const bool on = h < kMaxG && h < a.G;
        qv[u2][0] = (on && l < a.D) ? a.q[(bh * a.G + h) * a.D + l] : 0.0f;
        qv[u2][1] = (on && l + 64 < a.D) ? a.q[(bh * a.G + h) * a.D + l + 64] : 0.0f;
      }
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        const int h = h0 + u2 * nw;
        if (h >= kMaxG) continue;  // uniform
        sh.qs[h][l] = qv[u2][0];
        sh.qs[h][l + 64] = qv[u2][1];
        float m = fmaxf(fabsf(qv[u2][0]), fabsf(qv[u2][1]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (l == 0) sh.sig[h] = __builtin_amdgcn_frexp_expf(m);
      }
    }
  }
  if (own) {  // uniform: the class sizes of the plan made above
    __syncthreads();
    s = u = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      nc[c] = sh.pnc[c];
      s += nc[c];
      u += nc[c] * (c + 1);
      SF[c] = s;
      UE[c] = u;
    }
  }
  const int nact = s, ureal = u;
  const int U = (ureal + kSlice - 1) / kSlice * kSlice;
  const int UP = min(max(U, upad), kMaxUnits);
  if (tid == 0) {
    sh.U = U;
    sh.ureal = ureal;
  }
  __syncthreads();
  // the A rows: a unit per thread (consecutive threads, consecutive units of
  // every row: no bank conflicts), its channel read once, then the heads;
  // zero rows past G and zero-weight, zero-scale padding units past ureal
  // (they read plane word 0 of the superblock)
  const int G = a.G;
  for (int v = tid; v < UP; v += (int)blockDim.x) {
    int c = 0, p = 0, j = 0;
    if (v < ureal) {
      c = (v >= UE[0]) + (v >= UE[1]) + (v >= UE[2]);  // the unit's class: c + 1 planes
      const int r = v - (c == 0 ? 0 : UE[c - 1]);
      const int q = c == 0 ? r : c == 1 ? r >> 1 : c == 3 ? r >> 2 : (int)(((uint32_t)r * 0xAAABu) >> 17);  // r / (c + 1)
      p = r - q * (c + 1);
      j = sh.schan[(c == 0 ? 0 : SF[c - 1]) + q];
    }
    const float cf = ldexpf(1.0f, -(c + 1)) - 1.0f;
#pragma unroll
    for (int h = 0; h < kMaxG; ++h) {
      if (h >= G) {  // uniform: a zero row (-0 C weights where a real unit starts a channel, as 0 * (2^-(c+1) - 1))
        const _Float16 z = (_Float16)0.0f, cz = p == 0 && v < ureal ? (_Float16)-0.0f : z;
        sh.qa[2 * h][v] = sh.qa[2 * h + 1][v] = z;
        sh.ca[2 * h][v] = cz;
        sh.ca[2 * h + 1][v] = z;
        continue;
      }
      const bool on = v < ureal;
      const float qv = on ? sh.qs[h][j] : 0.0f;
      const int sg = on ? sh.sig[h] : 0;
      const float Q = ldexpf(qv, -(p + sg));
      const _Float16 qh = f16_rtz(Q);
      sh.qa[2 * h][v] = qh;
      sh.qa[2 * h + 1][v] = f16_rtz(Q - (float)qh);
      const float cq = p == 0 && on ? ldexpf(qv * cf, -sg) : 0.0f;  // padding: +0
      const _Float16 ch = f16_rtz(cq);
      sh.ca[2 * h][v] = ch;
      sh.ca[2 * h + 1][v] = f16_rtz(cq - (float)ch);
    }
  }
  __syncthreads();  // the queries are read: the offsets take their place
  const uint32_t sub = (uint32_t)a.sub;
  for (int e = tid; e < nact; e += (int)blockDim.x) {
    const int c = (e >= SF[0]) + (e >= SF[1]) + (e >= SF[2]);
    const int lo = c == 0 ? 0 : SF[c - 1];
    const int ub = (c == 0 ? 0 : UE[c - 1]) + (e - lo) * (c + 1);
    const uint32_t j = sh.schan[e];
    for (int p = 0; p <= c; ++p) {
      sh.uoff[ub + p] = (j * 4u + (uint32_t)p) * sub * 8u;
      sh.soff[ub + p] = j * sub * 2u;
    }
  }
  for (int v = ureal + tid; v < UP; v += (int)blockDim.x) sh.uoff[v] = sh.soff[v] = 0u;
  __syncthreads();
  return U;
}

// Writes the workgroup's plan tables (built by plan_tables, padded to nu
// units) to t.  A plan of more units writes only its header: the candidate
// pass then builds its own tables.
__device__ __forceinline__ void save_tables(const Shared &sh, PlanTab *t, int nu) {
  const int tid = threadIdx.x, nthr = (int)blockDim.x;
  const int U = sh.U;
  if (tid == 0) {
    t->U = U;
    t->ureal = sh.ureal;
  }
  if (U > nu) return;  // uniform
  if (tid < kMaxG) t->sig[tid] = sh.sig[tid];
  for (int i = tid; i < nu; i += nthr) {
    t->uoff[i] = sh.uoff[i];
    t->soff[i] = sh.soff[i];
  }
  const int per = nu / 8;  // 8 halves per 16-byte vector
  for (int i = tid; i < kRows * per; i += nthr) {
    const int r = i / per, v = (i - r * per) * 8;
    *reinterpret_cast<uint4 *>(&t->qa[r][v]) = *reinterpret_cast<const uint4 *>(&sh.qa[r][v]);
    *reinterpret_cast<uint4 *>(&t->ca[r][v]) = *reinterpret_cast<const uint4 *>(&sh.ca[r][v]);
  }
}

// Loads the plan tables of t (nu units, as save_tables wrote them) into the
// workgroup's LDS.  False (nothing loaded) when t holds no tables for nu
// units.  The offsets are range-checked against the superblock, so tables
// that no sample pass wrote give wrong scores but no access outside the store.
__device__ __forceinline__ bool load_tables(Shared &sh, const ScanArgs &a, const PlanTab *t, int nu) {
  const int tid = threadIdx.x, nthr = (int)blockDim.x;
  const int U = ld_uniform(&t->U), ureal = ld_uniform(&t->ureal);
  if (U < 0 || U > nu || U % kSlice != 0 || ureal < 0 || ureal > U) return false;  // uniform
  const uint32_t lim_u = (uint32_t)a.D * 4u * (uint32_t)a.sub * 8u, lim_s = (uint32_t)a.D * (uint32_t)a.sub * 2u;
  for (int i = tid; i < nu; i += nthr) {
    const uint32_t u = t->uoff[i], v = t->soff[i];
    sh.uoff[i] = u < lim_u ? u : 0u;
    sh.soff[i] = v < lim_s ? v : 0u;
  }
  if (tid < kMaxG) sh.sig[tid] = t->sig[tid];
  const int per = nu / 8;
  for (int i = tid; i < kRows * per; i += nthr) {
    const int r = i / per, v = (i - r * per) * 8;
    *reinterpret_cast<uint4 *>(&sh.qa[r][v]) = *reinterpret_cast<const uint4 *>(&t->qa[r][v]);
    *reinterpret_cast<uint4 *>(&sh.ca[r][v]) = *reinterpret_cast<const uint4 *>(&t->ca[r][v]);
  }
  if (tid == 0) {
    sh.U = U;
    sh.ureal = ureal;
  }
  __syncthreads();
  return true;
}

// --------------------------------------------------------------------- a tile
// A lane's addressing of one wave-tile: buffer resources based at the row's
// superblock sb0 (the tile's first), and the byte offsets of the lane's block
// (column c) from there.  Lanes whose block lies past the store read the tile's
// first block instead: columns are independent, and tokens past n are never
// emitted.
struct TileAddr {
  __amdgpu_buffer_rsrc_t pr, sr;
  uint32_t pl, sl;
  const struct HostStage *hs;  // staged tiles (host stores): the workgroup's stage, hb its first block
  int hb;
};

// ------------------------------------------------------------- host staging
// A store in mapped host memory is read over PCIe, where the request size
// sets the rate.  In superblocks of a multiple of 64 blocks the four
// wave-tiles of a workgroup step are 64 consecutive blocks of one superblock:
// each (channel, plane) unit of the plan is one 512-byte run and each active
// channel's scales one 128-byte run.  The workgroup copies them into LDS with
// 16-byte loads (plans of at most kHostUnits units), then each wave scans its
// tile from there.
constexpr int kHostUnits = 64;
constexpr int kHostBlk = 4 * kWB;     // blocks per workgroup step (four wave-tiles)
constexpr int kHostRow = 2 * kHostBlk + 4;  // a unit's plane dwords, padded (16-byte rows)
struct HostStage {
  uint32_t pw[kHostUnits][kHostRow];   // unit -> plane dwords of the 64 blocks (two per block)
  uint16_t sc[kHostUnits][kHostBlk];   // channel slot -> scales of the 64 blocks
  uint32_t soff1[kHostUnits];          // channel slot -> scale byte offset in the superblock
  uint8_t uslot[kHostUnits];           // unit -> channel slot
  int nch;                             // channel slots
};

constexpr int kBufFlags = 0x00020000;  // raw 32-bit buffer (gfx9 resource word 3)

__device__ __forceinline__ TileAddr tile_addr(const ScanArgs &a, int64_t bh, int64_t beta0, int c) {
  TileAddr ta;
  // block indices fit 32 bits (n <= 2^31); the lane's block is beta0 + c
  const uint32_t sub = (uint32_t)a.sub, D = (uint32_t)a.D;
  // the division runs on the vector unit: readfirstlane keeps the buffer
  // resources in scalar registers (a vector-register resource costs a loop
  // per load)
  const uint32_t sb0 = __builtin_amdgcn_readfirstlane((uint32_t)beta0 / sub), off0 = (uint32_t)beta0 - sb0 * sub;
  const uint32_t x = off0 + (uint32_t)c;
  const uint32_t dq = sub >= (uint32_t)kWB ? (x >= sub ? 1u : 0u) : x / sub;
  const uint32_t off = x - dq * sub;
  const uint32_t *pb = a.planes + ((bh * a.nsb + sb0) * a.D * 4) * a.sub * 2;
  const uint16_t *sbp = a.scales + ((bh * a.nsb + sb0) * a.D) * a.sub;
  ta.pr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(pb), (short)0, 0x7FFFFFFF, kBufFlags);
  ta.sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(sbp), (short)0, 0x7FFFFFFF, kBufFlags);
  ta.pl = ta.sl = 0u;
  ta.hs = nullptr;
  ta.hb = 0;
  if ((int64_t)sb0 + dq < a.nsb) {
    ta.pl = ((dq * D * 4u) * sub + off) * 8u;
    ta.sl = ((dq * D) * sub + off) * 2u;
  }
  return ta;
}

// Per-lane state of a tile: the emission constants of the lane's two heads
// (rows 4 g' .. 4 g' + 3 of the accumulators: heads 2 g' and 2 g' + 1) for its
// block, and the block's scale exponent.
struct TileK {
  int sx;          // s_c: the block's scales are rescaled by 2^-s_c
  float C[2];      // C of heads 2g', 2g' + 1
  int fe[2];       // sigma_h + s_c
};

// Quarter-pair planes of NS slices from slice s0: dwords of units 4g + m
// (m < 4), quarters 2 qp, 2 qp + 1 of the lane's block.
template <int NS, bool HOST = false>
__device__ __forceinline__ void load_planes(uint32_t (&d)[NS][4], const Shared &sh, const TileAddr &ta, int s0, int g,
                                            int qp) {
  if constexpr (HOST) {
    const int col = (ta.hb + (int)(threadIdx.x & 15)) * 2 + qp;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int m = 0; m < 4; ++m) d[s][m] = ta.hs->pw[(s0 + s) * kSlice + 4 * g + m][col];
    return;
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint4 uo = *reinterpret_cast<const uint4 *>(&sh.uoff[(s0 + s) * kSlice + 4 * g]);
    d[s][0] = __builtin_amdgcn_raw_buffer_load_b32(ta.pr, ta.pl + uo.x, 4 * qp, 0);
    d[s][1] = __builtin_amdgcn_raw_buffer_load_b32(ta.pr, ta.pl + uo.y, 4 * qp, 0);
    d[s][2] = __builtin_amdgcn_raw_buffer_load_b32(ta.pr, ta.pl + uo.z, 4 * qp, 0);
    d[s][3] = __builtin_amdgcn_raw_buffer_load_b32(ta.pr, ta.pl + uo.w, 4 * qp, 0);
  }
}

// Raw scales of NS slices from slice s0: pairs (units 4g, 4g + 1),
// (4g + 2, 4g + 3) per slice.
template <int NS, bool HOST = false>
__device__ __forceinline__ void load_scales(uint32_t (&ap)[NS][2], const Shared &sh, const TileAddr &ta, int s0, int g) {
  if constexpr (HOST) {
    const int col = ta.hb + (int)(threadIdx.x & 15);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint32_t v[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) v[m] = ta.hs->sc[ta.hs->uslot[(s0 + s) * kSlice + 4 * g + m]][col];
      ap[s][0] = v[0] | (v[1] << 16);
      ap[s][1] = v[2] | (v[3] << 16);
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint4 so = *reinterpret_cast<const uint4 *>(&sh.soff[(s0 + s) * kSlice + 4 * g]);
    const uint32_t a0 = __builtin_amdgcn_raw_buffer_load_b16(ta.sr, ta.sl + so.x, 0, 0);
    const uint32_t a1 = __builtin_amdgcn_raw_buffer_load_b16(ta.sr, ta.sl + so.y, 0, 0);
    const uint32_t a2 = __builtin_amdgcn_raw_buffer_load_b16(ta.sr, ta.sl + so.z, 0, 0);
    const uint32_t a3 = __builtin_amdgcn_raw_buffer_load_b16(ta.sr, ta.sl + so.w, 0, 0);
    ap[s][0] = a0 | (a1 << 16);
    ap[s][1] = a2 | (a3 << 16);
  }
}

// Zeroes the scales of padding units (units >= ureal).
template <int NS>
__device__ __forceinline__ void mask_pad_scales(uint32_t (&ap)[NS][2], int s0, int g, int ureal) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if ((s0 + s + 1) * kSlice > ureal) {  // uniform
      const int u = (s0 + s) * kSlice + 4 * g;
      const uint32_t m0 = (u < ureal ? 0xFFFFu : 0u) | (u + 1 < ureal ? 0xFFFF0000u : 0u);
      const uint32_t m1 = (u + 2 < ureal ? 0xFFFFu : 0u) | (u + 3 < ureal ? 0xFFFF0000u : 0u);
      ap[s][0] &= m0;
      ap[s][1] &= m1;
    }
  }
}

// A operand pieces of NS slices from slice s0 (four halves per slice) from an
// LDS table.
template <int NS>
__device__ __forceinline__ void load_arows(uint32_t (&qa)[NS][2], const _Float16 (*tab)[kMaxUnits], int s0, int row,
                                           int g) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint2 v = *reinterpret_cast<const uint2 *>(&tab[row][(s0 + s) * kSlice + 4 * g]);
    qa[s][0] = v.x;
    qa[s][1] = v.y;
  }
}

// One step of the chain over NS slices: acc (+)= sum over the slices of
// A(qa) B(b), 32 units per instruction; an odd last slice of 16 units is one
// 32-unit instruction whose upper half is zero (one instruction shape
// throughout: a 16x16x16 instruction reading a 16x16x32 result as its
// accumulator a few instructions later gave wrong sums).
// FIRST: the first instruction starts from zero (the chain's first group).
template <int NS, bool FIRST>
__device__ __forceinline__ f4 chain(f4 acc, const uint32_t (&qa)[NS][2], const uint32_t (&b)[NS][2]) {
#pragma unroll
  for (int s = 0; s < NS; s += 2) {
    const f4 cin = (FIRST && s == 0) ? f4{0.0f, 0.0f, 0.0f, 0.0f} : acc;
    const bool two = s + 1 < NS;
    uint32_t av[4] = {qa[s][0], qa[s][1], two ? qa[s + 1 < NS ? s + 1 : s][0] : 0u, two ? qa[s + 1 < NS ? s + 1 : s][1] : 0u};
    uint32_t bv[4] = {b[s][0], b[s][1], two ? b[s + 1 < NS ? s + 1 : s][0] : 0u, two ? b[s + 1 < NS ? s + 1 : s][1] : 0u};
    h8 A, B;
    __builtin_memcpy(&A, av, sizeof(A));
    __builtin_memcpy(&B, bv, sizeof(B));
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, cin, 0, 0, 0);
  }
  return acc;
}

// The quarter's plane halves: X[s][k] = [unit 4g + 2k | unit 4g + 2k + 1], the
// 16-bit quarter (Q odd: the high halves of the quarter-pair dwords).
template <int NS, int Q>
__device__ __forceinline__ void quarter_halves(uint32_t (&X)[NS][2], const uint32_t (&d)[NS][4]) {
  constexpr uint32_t sel = Q ? 0x07060302u : 0x05040100u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    X[s][0] = __builtin_amdgcn_perm(d[s][1], d[s][0], sel);
    X[s][1] = __builtin_amdgcn_perm(d[s][3], d[s][2], sel);
  }
}

// B operands of step class w from the shifted halves Y and the scale pairs.
template <int NS, int W>
__device__ __forceinline__ void b_operands(uint32_t (&b)[NS][2], const uint32_t (&Y)[NS][2],
                                           const uint32_t (&ap)[NS][2]) {
  constexpr uint32_t m = 0x08000800u << W;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    b[s][0] = pk_mul(Y[s][0] & m, ap[s][0]);
    b[s][1] = pk_mul(Y[s][1] & m, ap[s][1]);
  }
}

template <int NS, int V>
__device__ __forceinline__ void shifted(uint32_t (&Y)[NS][2], const uint32_t (&X)[NS][2]) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    Y[s][0] = half_shift<V>(X[s][0]);
    Y[s][1] = half_shift<V>(X[s][1]);
  }
}

// Cross-row maximum of a lane's value over the four lane groups (lanes c,
// c + 16, c + 32, c + 48): every lane of a column gets the same value.
__device__ __forceinline__ float rows_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

// Rescales the scale pairs of a group by 2^-sx: a' = a 2^-sx rounded to f16
// (exact where a' is a normal f16; a subnormal a' rounds to nearest even).
// When 2^-sx is itself a normal f16 this is one packed multiply per pair;
// otherwise the same value comes through fp32 (an exact ldexp, one rounding).
template <int NS>
__device__ __forceinline__ void rescale(uint32_t (&ap)[NS][2], int sx) {
  if (sx >= -15 && sx <= 14) {
    const uint32_t f = (uint32_t)(15 - sx) << 10;
    const uint32_t f2 = f | (f << 16);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      ap[s][0] = pk_mul(ap[s][0], f2);
      ap[s][1] = pk_mul(ap[s][1], f2);
    }
  } else {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint32_t v = ap[s][k];
        const float lo = ldexpf(f16_bits_to_float((uint16_t)(v & 0xFFFFu)), -sx);
        const float hi = ldexpf(f16_bits_to_float((uint16_t)(v >> 16)), -sx);
        ap[s][k] = (uint32_t)float_to_f16_bits(lo) | ((uint32_t)float_to_f16_bits(hi) << 16);
      }
    }
  }
}

// ------------------------------------------------------------------ scale pass
// The tile's scales for the lane's block (column c): the block's largest
// listed scale gives s_c (a' < 2^13); C of every head comes from the matrix
// instruction (B = raw scale pairs, A = the C rows), chained over the plan's
// slices like the scores.
// STK (stacked step classes): rows 8..15 repeat the C rows of rows 0..7.
// HOST: the scales come from the workgroup's stage.
template <int NS, bool FIRST, bool STK = false, bool HOST = false>
__device__ __forceinline__ void scale_group(uint32_t (&raw)[NS][2], float &amax, f4 &dc, const Shared &sh,
                                            const TileAddr &ta, int s0, int lane, int ureal) {
  const int c = lane & 15, g = lane >> 4;
  uint32_t cr[NS][2];
  load_scales<NS, HOST>(raw, sh, ta, s0, g);
  load_arows<NS>(cr, sh.ca, s0, STK ? (c & 7) : c, g);
  mask_pad_scales<NS>(raw, s0, g, ureal);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const h2 m = __builtin_elementwise_max(__builtin_bit_cast(h2, raw[s][0]), __builtin_bit_cast(h2, raw[s][1]));
    amax = fmaxf(amax, fmaxf((float)m[0], (float)m[1]));
  }
  dc = chain<NS, FIRST>(dc, cr, raw);
}

// s_c and the lane's C and exponents from the block maximum and the C sums
// (STK: lanes 32..63 hold the heads of lanes 0..31).
template <bool STK = false>
__device__ __forceinline__ TileK scale_finish(float amax, const f4 &dc, const Shared &sh, const ScanArgs &a, int lane) {
  const int g = STK ? (lane >> 4) & 1 : lane >> 4;
  amax = rows_max(amax);
  TileK k;
  k.sx = amax > 0.0f ? __builtin_amdgcn_frexp_expf(amax) - 13 : 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * g + i;
    const float cs = i == 0 ? dc[0] + dc[1] : dc[2] + dc[3];
    const int sg = h < a.G ? sh.sig[h] : 0;
    k.C[i] = ldexpf(cs, sg);
    k.fe[i] = sg + k.sx;
  }
  return k;
}

// The scale pairs of NS slices from s0 (plans of several groups), rescaled.
template <int NS>
__device__ __forceinline__ void group_scales(uint32_t (&ap)[NS][2], const Shared &sh, const TileAddr &ta, int s0,
                                             int g, int sx, int ureal) {
  load_scales<NS>(ap, sh, ta, s0, g);
  mask_pad_scales<NS>(ap, s0, g, ureal);
  rescale<NS>(ap, sx);
}

// -------------------------------------------------------------------- emission
// Threshold of a row as a float for "key >= thr".
__device__ __forceinline__ float threshold_value(uint32_t thr) {
  if (thr <= kKeyNegInf) return -INFINITY;
  if (thr > 0xFF800000u) return INFINITY;  // above +inf's key: NaN and +inf pass
  return key_value(thr);
}

// Accumulator-domain threshold numerator of a head for a tile with no masked
// token: T_w = ((thr - C) - margin) / 2^(fe0 - e_w) = X 2^(e_w - fe0).  The
// score is RN(x 2^(fe0 - e_w) + C) with the product exact, so a score >= thr
// needs x >= T_w; the margin covers the rounding of that sum and of thr - C
// (NaN passes both).  When a factor 2^(fe0 - e_w) is not a normal float, X is
// NaN and every token of the tile takes the exact path.
__device__ __forceinline__ float acc_threshold(float thr, float C, int fe0) {
  const float margin = (fabsf(thr) + fabsf(C)) * 0x1p-20f + 0x1p-126f;
  const bool ok = fabsf(C) < INFINITY && fe0 - bit_exp(3) >= -126 && fe0 - bit_exp(0) <= 127;
  return ok ? (thr - C) - margin : __int_as_float(0x7FC00000);
}

// Prefilter threshold of step class w for the high accumulator row alone: a
// token can score >= thr only if hi + lo >= X_w = X 2^(e_w - fe), and the low
// row's accumulator is at most M 2^e_w in magnitude (M = sum_u |lo_u| a'_u;
// zero where the caller compares hi + lo itself).  The slack covers the
// rounding of this arithmetic and of the matrix sums; NaN and infinities
// propagate to NaN or the right sign (a NaN threshold passes every token).
__device__ __forceinline__ float hi_threshold(float X, int fe, int w, float M) {
  if (!(fabsf(X) < INFINITY)) return X;  // +inf: no token; -inf, NaN: every token
  const float t = ldexpf(X, bit_exp(w) - fe);
  const float mw = ldexpf(M, bit_exp(w)) * (1.0f + 0x1p-16f);
  return ((t - mw) - fabsf(t) * 0x1p-20f) - 0x1p-120f;
}

// Emission state of a lane over a tile: its two heads (slots) 2 g' + i.
struct EmitState {
  float T[2][4];       // candidate prefilter thresholds per slot and step class, accumulator
                       // units (NaN: every token takes the exact path; +inf: none does)
  float Ts[2][2];      // stacked step classes: the lane's T of pair p (class p + 2 (lane >= 32))
  float thr[2];        // row thresholds as floats
  uint32_t off[2];     // candidates written so far into the tile's region (per head)
  float gm[2];         // group maxima: running max of the quarter's masked scores
  bool gnan[2];
  uint32_t gk[2];      // sample pass: running max of the quarter's masked keys
  bool head[2];        // the slot's head is in the row and not skipped
  bool plain;          // no masking anywhere in the tile
  // tile-relative token intervals (wave-uniform): tokens of the scanned range
  // [vlo, vlo + vlen) and unmasked tokens [mlo, mlo + mlen)
  uint32_t vlo, vlen, mlo, mlen;
};

// The candidates of one step class whose prefilter some lane passed: the
// exact scores of both slots, their keys, ranked within each head's 16 lanes
// by ballots and written into the tile's region.  In a tile with no masked
// token a head outside the row or skipped has T = +inf and never passes the
// prefilter; other tiles (T = NaN: every lane passes) check each token.
template <int W>
__device__ __forceinline__ void filter_hit(const Emit &em, const ScanArgs &a, float xa, float xb, bool pa, bool pb,
                                           const TileK &k, EmitState &es, int64_t bh, int64_t beta0, int qs, int V,
                                           int lane) {
  const int c = lane & 15, gp = lane >> 4;
  // the token within the tile and in the row (n <= 2^31); in a tile with no
  // masked token both intervals hold the whole tile (one branch-free path:
  // a uniform branch on the tile kind measured slower)
  const uint32_t tt = (uint32_t)(c * kBlk) + (uint32_t)(16 * qs + 4 * V + W);
  const uint32_t tok = (uint32_t)(beta0 * kBlk) + tt;
  const bool inr = tt - es.vlo < es.vlen, um = tt - es.mlo < es.mlen;
  const uint32_t sh = 8u * (uint32_t)gp;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float v = fmaf(i == 0 ? xa : xb, ldexpf(1.0f, k.fe[i] - bit_exp(W)), k.C[i]);
    const float vm = um ? v : -INFINITY;  // score_key(-inf) is kKeyNegInf
    const bool pass = es.head[i] && inr && (i == 0 ? pa : pb) && !(vm < es.thr[i]);
    const uint64_t m = __builtin_amdgcn_ballot_w64(pass);
    if (m == 0ull) continue;  // uniform
    // per row group (16 lanes, one head): the passing lanes below each group
    // and in it, one byte per group (wave-uniform)
    const uint32_t n0 = (uint32_t)__builtin_popcountll(m & 0xFFFFull);
    const uint32_t n1 = (uint32_t)__builtin_popcountll(m & 0xFFFF0000ull);
    const uint32_t n2 = (uint32_t)__builtin_popcountll(m & 0xFFFF00000000ull);
    const uint32_t n3 = (uint32_t)__builtin_popcountll(m >> 48);
    const uint32_t below = (n0 << 8) | ((n0 + n1) << 16) | ((n0 + n1 + n2) << 24);
    const uint32_t in = n0 | (n1 << 8) | (n2 << 16) | (n3 << 24);
    if (pass) {
      const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      const uint32_t at = es.off[i] + before - ((below >> sh) & 0xFFu);
      uint64_t *dst = em.sel.cand + (bh * a.G + i) * em.sel.cand_cap + beta0 * kBlk +
                      (uint64_t)(uint32_t)(2 * gp) * (uint64_t)em.sel.cand_cap;
      dst[at] = k64_of(score_key(vm), tok);
    }
    es.off[i] += (in >> sh) & 0xFFu;
  }
}

// Candidate emission of step class w of step group V of quarter qs (token
// 16 qs + 4V + w of every block): a compare per slot against T in the
// accumulator domain (HI: the high row alone, T allowing for the low row;
// else the sum of both rows); only steps where some lane passes compute
// exact scores and keys (filter_hit).  Heads in skipm emit nothing.
template <int W, bool HI>
__device__ __forceinline__ void emit_filter_w(const Emit &em, const ScanArgs &a, const f4 &acc, const TileK &k,
                                              EmitState &es, int64_t bh, int64_t beta0, int qs, int V, int lane) {
  bool pa, pb;
  if constexpr (HI) {
    pa = !(acc[0] < es.T[0][W]);
    pb = !(acc[2] < es.T[1][W]);
  } else {
    pa = !(acc[0] + acc[1] < es.T[0][W]);
    pb = !(acc[2] + acc[3] < es.T[1][W]);
  }
  if (__builtin_amdgcn_ballot_w64(pa || pb) == 0ull) return;  // uniform
  filter_hit<W>(em, a, acc[0] + acc[1], acc[2] + acc[3], pa, pb, k, es, bh, beta0, qs, V, lane);
}

// Scores of step group V of quarter qs, from the four step classes' scores
// s4[slot][w]: each lane stores its block's four consecutive tokens per head
// (and, GMAX, folds them into the quarter's group maximum, written once the
// quarter ends).
template <bool GMAX>
__device__ __forceinline__ void store_scores(const Emit &em, const ScanArgs &a, const float (&s4)[2][4], EmitState &es,
                                             int64_t bh, int64_t beta0, int qs, int V, int lane) {
  const int c = lane & 15, gp = lane >> 4;
  const int64_t blk = beta0 + c;
  const bool inr = blk >= a.blk0 && blk < a.blk_end;
  const int64_t tq = blk * kBlk + 16 * qs;  // the quarter's first token
  const int64_t t4 = tq + 4 * V;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * gp + i;
    if (h >= a.G || !inr || tq >= a.n) continue;
    const float *s = s4[i];
    float *dst = em.out + (bh * a.G + h) * a.n + t4;
    if (t4 + 4 <= a.n && (a.n & 3) == 0) {
      *reinterpret_cast<f4 *>(dst) = f4{s[0], s[1], s[2], s[3]};
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        if (t4 + w < a.n) dst[w] = s[w];
    }
    if constexpr (GMAX) {  // a quarter's step groups come V = 3 first, V = 0 last
      if (V == 3) {
        es.gm[i] = -INFINITY;
        es.gnan[i] = false;
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int64_t tok = t4 + w;
        const float v = (es.plain || (tok < a.n && tok >= em.sink && tok < em.lstart)) ? s[w] : -INFINITY;
        es.gm[i] = fmaxf(es.gm[i], v);
        es.gnan[i] = es.gnan[i] || (v != v);
      }
      if (V == 0) {
        const int64_t ngrp = (a.n + kR - 1) / kR;
        em.gmax[(bh * a.G + h) * ngrp + blk * 4 + qs] = es.gnan[i] ? 0xFFFFFFFFu : score_key(es.gm[i]);
      }
    }
  }
}

// Sampled keys of step group V of quarter qs of list entry L: each lane keeps
// the largest key of its 16 tokens of the quarter (sink/local masked to -inf,
// 0 beyond the row) and writes it once the quarter ends -- 64 group maxima per
// tile and head, [L][block][quarter].
__device__ __forceinline__ void store_sample(const Emit &em, const ScanArgs &a, const float (&s4)[2][4], EmitState &es,
                                             int64_t bh, int64_t beta0, int64_t L, int qs, int V, int lane) {
  const int c = lane & 15, gp = lane >> 4;
  const int64_t t4 = (beta0 + c) * kBlk + 16 * qs + 4 * V;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * gp + i;
    if (h >= a.G) continue;
    if (V == 3) es.gk[i] = 0u;  // a quarter's step groups come V = 3 first, V = 0 last
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int64_t tok = t4 + w;
      const bool masked = tok < em.sink || tok >= em.lstart;
      const uint32_t key = tok < a.n ? (masked ? kKeyNegInf : score_key(s4[i][w])) : 0u;
      es.gk[i] = max(es.gk[i], key);
    }
    if (V == 0)
      em.samp[(bh * a.G + h) * em.samp_cap + L * (kWTok / kGroupTok) + c * kQS + qs] = es.gk[i];
  }
}

// Per-step-class emission state of a step group: the two slots' scores of the
// four classes (score modes).
struct StepOut {
  float s4[2][4];
};

// Emission of step class W of step group V: the candidate compare at once, or
// the scores kept for the group's stores.
template <int MODE, int W, bool HI>
__device__ __forceinline__ void emit_w(const Emit &em, const ScanArgs &a, const f4 &acc, const TileK &k, EmitState &es,
                                       StepOut &o, int64_t bh, int64_t beta0, int qs, int V, int lane) {
  if constexpr (MODE == kEmitFilter) {
    emit_filter_w<W, HI>(em, a, acc, k, es, bh, beta0, qs, V, lane);
  } else {
    const float f0 = ldexpf(1.0f, k.fe[0] - bit_exp(W)), f1 = ldexpf(1.0f, k.fe[1] - bit_exp(W));
    o.s4[0][W] = fmaf(acc[0] + acc[1], f0, k.C[0]);
    o.s4[1][W] = fmaf(acc[2] + acc[3], f1, k.C[1]);
  }
}

// The stores of a step group's scores (score modes).
template <int MODE>
__device__ __forceinline__ void emit_flush(const Emit &em, const ScanArgs &a, EmitState &es, const StepOut &o,
                                           int64_t bh, int64_t beta0, int64_t L, int qs, int V, int lane) {
  if constexpr (MODE == kEmitScores) store_scores<false>(em, a, o.s4, es, bh, beta0, qs, V, lane);
  if constexpr (MODE == kEmitScoresMax) store_scores<true>(em, a, o.s4, es, bh, beta0, qs, V, lane);
  if constexpr (MODE == kEmitSample) store_sample(em, a, o.s4, es, bh, beta0, L, qs, V, lane);
}

// ------------------------------------------------------------------ tile loop
// A candidate wave's constants of its row (every tile of a wave is in one
// row): the lane's two heads' thresholds and whether they emit (in the row
// and not skipped).
struct RowK {
  float thr[2];
  bool head[2];
};

__device__ __forceinline__ RowK row_consts(const Emit &em, const ScanArgs &a, int64_t bh, int lane, bool fb,
                                           uint32_t skipm, bool stk) {
  RowK r;
  const uint32_t *thr = fb ? em.sel.thr_lo : em.sel.thr;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * (stk ? (lane >> 4) & 1 : lane >> 4) + i;
    r.head[i] = h < a.G && !((skipm >> h) & 1u);
    r.thr[i] = r.head[i] ? threshold_value(thr[bh * a.G + h]) : INFINITY;
  }
  return r;
}

// Per-mode state set up once a tile's scale pass is done; M: the bound of
// the low rows' accumulators per unit 2^e_w (zero where the prefilter
// compares both rows).
template <int MODE, bool STK = false>
__device__ __forceinline__ void tile_setup(EmitState &es, const Emit &em, const ScanArgs &a, const TileK &k,
                                           int64_t beta0, const RowK &rk, const float (&M)[2], int lane) {
  const int64_t t0 = beta0 * kBlk, t1 = t0 + kWTok;
  es.plain = beta0 >= a.blk0 && beta0 + kWB <= a.blk_end && t1 <= a.n && t0 >= em.sink && t1 <= em.lstart;
  es.off[0] = es.off[1] = 0u;
  if constexpr (MODE == kEmitFilter) {
    if (es.plain) {  // uniform
      es.vlo = es.mlo = 0u;
      es.vlen = es.mlen = (uint32_t)kWTok;
    } else {
      // [lo, hi) of the row clipped to the tile, relative to its first token
      auto rel = [&](int64_t lo, int64_t hi, uint32_t &rlo, uint32_t &rlen) {
        const int64_t l = min(max(lo - t0, (int64_t)0), (int64_t)kWTok);
        const int64_t h = min(max(hi - t0, (int64_t)0), (int64_t)kWTok);
        rlo = (uint32_t)l;
        rlen = (uint32_t)max(h - l, (int64_t)0);
      };
      rel(max(a.blk0 * kBlk, (int64_t)0), min(a.blk_end * kBlk, a.n), es.vlo, es.vlen);
      rel(em.sink, em.lstart, es.mlo, es.mlen);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      es.head[i] = rk.head[i];
      es.thr[i] = rk.thr[i];
      // masked tiles too: a masked token scores -inf in the exact check, so
      // only thr = -inf (X = -inf: every token) lets one through
      const float X = es.head[i] ? acc_threshold(es.thr[i], k.C[i], k.fe[i]) : INFINITY;
      // T_w = T_0 2^(e_w - e_0) exactly (a threshold past the float range
      // becomes +inf, which no finite accumulator reaches)
      es.T[i][0] = hi_threshold(X, k.fe[i], 0, M[i]);
#pragma unroll
      for (int w = 1; w < 4; ++w) es.T[i][w] = es.T[i][0] * (float)(1 << (bit_exp(w) - bit_exp(0)));
      if constexpr (STK) {
        es.Ts[i][0] = lane >= 32 ? es.T[i][2] : es.T[i][0];
        es.Ts[i][1] = lane >= 32 ? es.T[i][3] : es.T[i][1];
      }
    }
  }
}

// The region counts of a candidate tile (lane c = 0 of each row group).
__device__ __forceinline__ void tile_counts(const Emit &em, const ScanArgs &a, const EmitState &es, int64_t bh,
                                            int64_t beta0, int lane, bool fb, uint32_t skipm) {
  const int c = lane & 15, gp = lane >> 4;
  if (c != 0) return;
  // the row's base is wave-uniform; a head's offset in it fits 32 bits
  // (nreg <= 2^21 regions)
  uint32_t *rc = (fb ? em.sel.rc2 : em.sel.rc1) + bh * a.G * em.sel.nreg;
  const uint32_t region = (uint32_t)(beta0 / kWB);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * gp + i;
    if (h < a.G && !((skipm >> h) & 1u)) rc[(uint32_t)h * (uint32_t)em.sel.nreg + region] = es.off[i];
  }
}

// The quarter halves X shifted for step group V (bits 4V..4V+3 of each half on
// bits 11..14); V is wave-uniform.
template <int NS>
__device__ __forceinline__ void shifted_v(uint32_t (&Y)[NS][2], const uint32_t (&X)[NS][2], int V) {
  if (V == 3) {
    shifted<NS, 3>(Y, X);
  } else {
    const unsigned short L = (unsigned short)(11 - 4 * V);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      Y[s][0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, X[s][0]) << L);
      Y[s][1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, X[s][1]) << L);
    }
  }
}

// One step group (four step classes w of shift variant V) over NS slices:
// acc[w] (+)= their contributions to token 16 qs + 4V + w of every block.
template <int NS, bool FIRST>
__device__ __forceinline__ void step_group(f4 (&acc)[4], const uint32_t (&qa)[NS][2], const uint32_t (&ap)[NS][2],
                                           const uint32_t (&X)[NS][2], int V) {
  uint32_t Y[NS][2];
  shifted_v<NS>(Y, X, V);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t b[NS][2];
    if (w == 0) b_operands<NS, 0>(b, Y, ap);
    if (w == 1) b_operands<NS, 1>(b, Y, ap);
    if (w == 2) b_operands<NS, 2>(b, Y, ap);
    if (w == 3) b_operands<NS, 3>(b, Y, ap);
    acc[w] = chain<NS, FIRST>(acc[w], qa, b);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Emission of step group V of quarter qs from its four accumulators (the
// grouped path), whichever the mode.
template <int MODE>
__device__ __forceinline__ void emit_group(const Emit &em, const ScanArgs &a, const f4 (&acc)[4], const TileK &k,
                                           EmitState &es, int64_t bh, int64_t beta0, int64_t L, int qs, int V,
                                           int lane) {
  StepOut o;
  emit_w<MODE, 0, false>(em, a, acc[0], k, es, o, bh, beta0, qs, V, lane);
  emit_w<MODE, 1, false>(em, a, acc[1], k, es, o, bh, beta0, qs, V, lane);
  emit_w<MODE, 2, false>(em, a, acc[2], k, es, o, bh, beta0, qs, V, lane);
  emit_w<MODE, 3, false>(em, a, acc[3], k, es, o, bh, beta0, qs, V, lane);
  emit_flush<MODE>(em, a, es, o, bh, beta0, L, qs, V, lane);
}

// One step group of a plan of NS slices held in registers (Y: the quarter's
// halves shifted for step group V), each step class emitted as soon as its
// chain is done (one accumulator live at a time).
template <int MODE, int NS>
__device__ __forceinline__ void step_group_emit(const uint32_t (&qa)[NS][2], const uint32_t (&ap)[NS][2],
                                                const uint32_t (&Y)[NS][2], const Emit &em, const ScanArgs &a,
                                                const TileK &k, EmitState &es, int64_t bh, int64_t beta0, int64_t L,
                                                int qs, int V, int lane) {
  StepOut o;
  // each step class's chain is issued before the previous class is emitted,
  // so the emission does not wait on the matrix pipe
  f4 prev;
  {
    uint32_t b[NS][2];
    b_operands<NS, 0>(b, Y, ap);
    prev = chain<NS, true>(f4{}, qa, b);
  }
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    uint32_t b[NS][2];
    if (w == 1) b_operands<NS, 1>(b, Y, ap);
    if (w == 2) b_operands<NS, 2>(b, Y, ap);
    if (w == 3) b_operands<NS, 3>(b, Y, ap);
    const f4 acc = chain<NS, true>(f4{}, qa, b);
    if (w == 1) emit_w<MODE, 0, true>(em, a, prev, k, es, o, bh, beta0, qs, V, lane);
    if (w == 2) emit_w<MODE, 1, true>(em, a, prev, k, es, o, bh, beta0, qs, V, lane);
    if (w == 3) emit_w<MODE, 2, true>(em, a, prev, k, es, o, bh, beta0, qs, V, lane);
    prev = acc;
    __builtin_amdgcn_sched_barrier(0);
  }
  emit_w<MODE, 3, true>(em, a, prev, k, es, o, bh, beta0, qs, V, lane);
  emit_flush<MODE>(em, a, es, o, bh, beta0, L, qs, V, lane);
}

// ------------------------------------------------------ stacked step classes
// Rows of at most four heads (G <= 4) leave rows 8..15 of the matrix tile
// free.  A step group then runs as two pairs of step classes, (0, 2) and
// (1, 3), each pair in one accumulator: the first class in rows 0..7, the
// second in rows 8..15.  A slice pair of the first class is one instruction
// with the A rows in rows 0..7 (zero below), the same slice pair of the second
// class one with the A rows moved to rows 8..15 (zero above); each adds exact
// zeros to the other half.  An odd last slice takes both classes in one
// instruction: the first class's units in the lower four of each lane's eight
// k values, the second's in the upper four.  Each class's rows see the same
// nonzero products in the same order as the unstacked chain, so the scores
// are the same bit for bit; a pair costs one instruction fewer for an odd
// slice count, and one compare per head covers two classes.  Lane l of a pair
// accumulator holds rows 4 (l / 16) .. + 3: heads 2 ((l / 16) & 1) + i of class
// p (lanes 0..31) or p + 2 (lanes 32..63).

// The A rows of rows 0..7 moved to rows 8..15 (zero in rows 0..7).
template <int NS>
__device__ __forceinline__ void load_arows_hi(uint32_t (&qhi)[NS][2], const _Float16 (*tab)[kMaxUnits], int s0,
                                              int lane) {
  const int r = lane & 15;
  load_arows<NS>(qhi, tab, s0, r & 7, lane >> 4);
  const uint32_t keep = r >= 8 ? 0xFFFFFFFFu : 0u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qhi[s][0] &= keep;
    qhi[s][1] &= keep;
  }
}

__device__ __forceinline__ f4 mfma4(const uint32_t (&av)[4], const uint32_t (&bv)[4], f4 c) {
  h8 A, B;
  __builtin_memcpy(&A, av, sizeof(A));
  __builtin_memcpy(&B, bv, sizeof(B));
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, c, 0, 0, 0);
}

// The chain of one pair of step classes from zero: ba the first class's B
// operands (rows 0..7), bb the second's (rows 8..15).
template <int NS>
__device__ __forceinline__ f4 chain_stk(const uint32_t (&qlo)[NS][2], const uint32_t (&qhi)[NS][2],
                                        const uint32_t (&ba)[NS][2], const uint32_t (&bb)[NS][2]) {
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < NS; s += 2) {
    if (s + 1 < NS) {
      const int t = s + 1 < NS ? s + 1 : s;
      const uint32_t a0[4] = {qlo[s][0], qlo[s][1], qlo[t][0], qlo[t][1]};
      const uint32_t b0[4] = {ba[s][0], ba[s][1], ba[t][0], ba[t][1]};
      const uint32_t a1[4] = {qhi[s][0], qhi[s][1], qhi[t][0], qhi[t][1]};
      const uint32_t b1[4] = {bb[s][0], bb[s][1], bb[t][0], bb[t][1]};
      acc = mfma4(a0, b0, s == 0 ? f4{0.0f, 0.0f, 0.0f, 0.0f} : acc);
      acc = mfma4(a1, b1, acc);
    } else {
      const uint32_t a0[4] = {qlo[s][0], qlo[s][1], qhi[s][0], qhi[s][1]};
      const uint32_t b0[4] = {ba[s][0], ba[s][1], bb[s][0], bb[s][1]};
      acc = mfma4(a0, b0, s == 0 ? f4{0.0f, 0.0f, 0.0f, 0.0f} : acc);
    }
  }
  return acc;
}

// The candidates of pair P whose prefilter some lane passed (filter_hit for
// stacked classes): a head's candidates come from lane groups (g & 1) and
// (g & 1) + 2, ranked over both by one ballot.
template <int P>
__device__ __forceinline__ void filter_hit_stk(const Emit &em, const ScanArgs &a, float xa, float xb, bool pa, bool pb,
                                               const TileK &k, EmitState &es, int64_t bh, int64_t beta0, int qs, int V,
                                               int lane) {
  const int c = lane & 15, gh = (lane >> 4) & 1, up = lane >> 5;
  const int ew = up ? bit_exp(P + 2) : bit_exp(P);
  const uint32_t tt = (uint32_t)(c * kBlk) + (uint32_t)(16 * qs + 4 * V + P + 2 * up);
  const uint32_t tok = (uint32_t)(beta0 * kBlk) + tt;
  const bool inr = tt - es.vlo < es.vlen, um = tt - es.mlo < es.mlen;
  constexpr uint64_t kH0 = 0x0000FFFF0000FFFFull;  // lane groups 0 and 2
  const uint64_t hm = gh ? ~kH0 : kH0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float v = fmaf(i == 0 ? xa : xb, ldexpf(1.0f, k.fe[i] - ew), k.C[i]);
    const float vm = um ? v : -INFINITY;  // score_key(-inf) is kKeyNegInf
    const bool pass = es.head[i] && inr && (i == 0 ? pa : pb) && !(vm < es.thr[i]);
    const uint64_t m = __builtin_amdgcn_ballot_w64(pass);
    if (m == 0ull) continue;  // uniform
    const uint32_t n0 = (uint32_t)__builtin_popcountll(m & kH0), n1 = (uint32_t)__builtin_popcountll(m & ~kH0);
    if (pass) {
      const uint64_t mh = m & hm;
      const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(mh >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mh, 0u));
      uint64_t *dst = em.sel.cand + (bh * a.G + 2 * gh + i) * em.sel.cand_cap + beta0 * kBlk;
      dst[es.off[i] + before] = k64_of(score_key(vm), tok);
    }
    es.off[i] += gh ? n1 : n0;
  }
}

// Scores of a step group's two pairs (score modes): s[slot][p].
struct StepOut2 {
  float s[2][2];
};

template <int MODE, int P>
__device__ __forceinline__ void emit_pair(const Emit &em, const ScanArgs &a, const f4 &acc, const TileK &k,
                                          EmitState &es, StepOut2 &o, int64_t bh, int64_t beta0, int qs, int V,
                                          int lane) {
  if constexpr (MODE == kEmitFilter) {
    const bool pa = !(acc[0] < es.Ts[0][P]);
    const bool pb = !(acc[2] < es.Ts[1][P]);
    if (__builtin_amdgcn_ballot_w64(pa || pb) == 0ull) return;  // uniform
    filter_hit_stk<P>(em, a, acc[0] + acc[1], acc[2] + acc[3], pa, pb, k, es, bh, beta0, qs, V, lane);
  } else {
    const int up = lane >> 5;
    const int ew = up ? bit_exp(P + 2) : bit_exp(P);
    o.s[0][P] = fmaf(acc[0] + acc[1], ldexpf(1.0f, k.fe[0] - ew), k.C[0]);
    o.s[1][P] = fmaf(acc[2] + acc[3], ldexpf(1.0f, k.fe[1] - ew), k.C[1]);
  }
}

// store_scores for stacked classes: each lane stores its block's two
// consecutive tokens 4V + 2 (lane >= 32) + {0, 1} per head; a quarter's group
// maximum joins the halves of lanes l and l ^ 32.
template <bool GMAX>
__device__ __forceinline__ void store_scores_stk(const Emit &em, const ScanArgs &a, const float (&s2)[2][2],
                                                 EmitState &es, int64_t bh, int64_t beta0, int qs, int V, int lane) {
  const int c = lane & 15, gh = (lane >> 4) & 1, up = lane >> 5;
  const int64_t blk = beta0 + c;
  const bool inr = blk >= a.blk0 && blk < a.blk_end;
  const int64_t tq = blk * kBlk + 16 * qs;  // the quarter's first token
  const int64_t t2 = tq + 4 * V + 2 * up;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * gh + i;
    const bool on = h < a.G && inr && tq < a.n;
    if (on) {
      float *dst = em.out + (bh * a.G + h) * a.n + t2;
      if (t2 + 2 <= a.n && (a.n & 1) == 0) {
        *reinterpret_cast<f2 *>(dst) = f2{s2[i][0], s2[i][1]};
      } else {
        if (t2 < a.n) dst[0] = s2[i][0];
        if (t2 + 1 < a.n) dst[1] = s2[i][1];
      }
    }
    if constexpr (GMAX) {  // a quarter's step groups come V = 3 first, V = 0 last
      if (V == 3) {
        es.gm[i] = -INFINITY;
        es.gnan[i] = false;
      }
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const int64_t tok = t2 + w;
        const float v = (es.plain || (tok < a.n && tok >= em.sink && tok < em.lstart)) ? s2[i][w] : -INFINITY;
        es.gm[i] = fmaxf(es.gm[i], v);
        es.gnan[i] = es.gnan[i] || (v != v);
      }
      if (V == 0) {
        const float og = __shfl_xor(es.gm[i], 32, 64);
        const int on2 = __shfl_xor((int)es.gnan[i], 32, 64);
        const bool gnan = es.gnan[i] || on2 != 0;
        const float gm = fmaxf(es.gm[i], og);
        if (on && up == 0) {
          const int64_t ngrp = (a.n + kR - 1) / kR;
          em.gmax[(bh * a.G + h) * ngrp + blk * 4 + qs] = gnan ? 0xFFFFFFFFu : score_key(gm);
        }
      }
    }
  }
}

// store_sample for stacked classes.
__device__ __forceinline__ void store_sample_stk(const Emit &em, const ScanArgs &a, const float (&s2)[2][2],
                                                 EmitState &es, int64_t bh, int64_t beta0, int64_t L, int qs, int V,
                                                 int lane) {
  const int c = lane & 15, gh = (lane >> 4) & 1, up = lane >> 5;
  const int64_t t2 = (beta0 + c) * kBlk + 16 * qs + 4 * V + 2 * up;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int h = 2 * gh + i;
    if (V == 3) es.gk[i] = 0u;  // a quarter's step groups come V = 3 first, V = 0 last
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int64_t tok = t2 + w;
      const bool masked = tok < em.sink || tok >= em.lstart;
      const uint32_t key = tok < a.n ? (masked ? kKeyNegInf : score_key(s2[i][w])) : 0u;
      es.gk[i] = max(es.gk[i], key);
    }
    if (V == 0) {
      const uint32_t gk = max(es.gk[i], (uint32_t)__shfl_xor((int)es.gk[i], 32, 64));
      if (h < a.G && up == 0)
        em.samp[(bh * a.G + h) * em.samp_cap + L * (kWTok / kGroupTok) + c * kQS + qs] = gk;
    }
  }
}

// One step group of stacked classes (step_group_emit for G <= 4).
template <int MODE, int NS>
__device__ __forceinline__ void step_group_stk(const uint32_t (&qlo)[NS][2], const uint32_t (&qhi)[NS][2],
                                               const uint32_t (&ap)[NS][2], const uint32_t (&Y)[NS][2],
                                               const Emit &em, const ScanArgs &a, const TileK &k, EmitState &es,
                                               int64_t bh, int64_t beta0, int64_t L, int qs, int V, int lane) {
  StepOut2 o;
  f4 p0, p1;
  {
    uint32_t ba[NS][2], bb[NS][2];
    b_operands<NS, 0>(ba, Y, ap);
    b_operands<NS, 2>(bb, Y, ap);
    p0 = chain_stk<NS>(qlo, qhi, ba, bb);
  }
  {
    uint32_t ba[NS][2], bb[NS][2];
    b_operands<NS, 1>(ba, Y, ap);
    b_operands<NS, 3>(bb, Y, ap);
    p1 = chain_stk<NS>(qlo, qhi, ba, bb);
  }
  emit_pair<MODE, 0>(em, a, p0, k, es, o, bh, beta0, qs, V, lane);
  __builtin_amdgcn_sched_barrier(0);
  emit_pair<MODE, 1>(em, a, p1, k, es, o, bh, beta0, qs, V, lane);
  if constexpr (MODE == kEmitScores) store_scores_stk<false>(em, a, o.s, es, bh, beta0, qs, V, lane);
  if constexpr (MODE == kEmitScoresMax) store_scores_stk<true>(em, a, o.s, es, bh, beta0, qs, V, lane);
  if constexpr (MODE == kEmitSample) store_sample_stk(em, a, o.s, es, bh, beta0, L, qs, V, lane);
}

// The work of one wave on one tile: wave-tile beta0 (blocks beta0 .. beta0 +
// 15 of row bh), quarters [qa0, qa1) (all four but in the sample pass), list
// entry L; fb / skipm: the candidate pass's fallback rescan and the heads it
// leaves alone.
struct TileJob {
  int64_t bh, beta0, L;
  int qa0, qa1, lane, ureal;
  bool fb;
  uint32_t skipm;
  RowK rk;
  const HostStage *hs = nullptr;  // staged tiles: the workgroup's stage and the tile's first block in it
  int hb = 0;
};

// The bound M of the low rows' accumulators of the lane's heads per unit
// 2^e_w: sum_u |lo_u| |a'_u|, by the matrix instruction (rows 4g' + 1 and
// 4g' + 3 of |A| |B| are the low rows of heads 2g' and 2g' + 1).
template <int NS>
__device__ __forceinline__ void lo_bound(float (&M)[2], const uint32_t (&qreg)[NS][2], const uint32_t (&ap)[NS][2]) {
  uint32_t aq[NS][2], ab[NS][2];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    aq[s][0] = qreg[s][0] & 0x7FFF7FFFu;
    aq[s][1] = qreg[s][1] & 0x7FFF7FFFu;
    ab[s][0] = ap[s][0] & 0x7FFF7FFFu;
    ab[s][1] = ap[s][1] & 0x7FFF7FFFu;
  }
  const f4 d = chain<NS, true>(f4{}, aq, ab);
  M[0] = d[1];
  M[1] = d[3];
}

// lo_bound for stacked classes: rows 8..15 of |A| repeat rows 0..7.
template <int NS>
__device__ __forceinline__ void lo_bound_stk(float (&M)[2], const uint32_t (&qlo)[NS][2], const uint32_t (&qhi)[NS][2],
                                             const uint32_t (&ap)[NS][2]) {
  uint32_t aq[NS][2];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    aq[s][0] = qlo[s][0] | qhi[s][0];
    aq[s][1] = qlo[s][1] | qhi[s][1];
  }
  lo_bound<NS>(M, aq, ap);
}

// The four step groups of quarter qs, V = 3 down to 0, on the quarter's halves
// Y (consumed).  Each dword turns as a whole: right by one for V = 3, then left
// by four per step group, so the half bits 4V..4V+3 sit on bits 11..14 of each
// half at step group V.  No bit is lost; the bits that wrap from one half into
// the other land on bits 0..10 or 15 of a half, which no mask selects.
// The chain of pair P of stacked step classes (P, P + 2) of the halves Y.
template <int NS, int P>
__device__ __forceinline__ f4 pair_chain(const uint32_t (&qlo)[NS][2], const uint32_t (&qhi)[NS][2],
                                         const uint32_t (&ap)[NS][2], const uint32_t (&Y)[NS][2]) {
  uint32_t ba[NS][2], bb[NS][2];
  b_operands<NS, P>(ba, Y, ap);
  b_operands<NS, P + 2>(bb, Y, ap);
  return chain_stk<NS>(qlo, qhi, ba, bb);
}

// STK: stacked step classes (qhi: the A rows in rows 8..15).  The candidate
// pass compares pair 1 of a step group after pair 0 of the next one is
// issued, so no compare waits on the chain just issued.
template <int MODE, int NS, bool STK>
__device__ __forceinline__ void quarter_fast(const uint32_t (&qreg)[NS][2], const uint32_t (&qhi)[NS][2],
                                             const uint32_t (&ap)[NS][2], uint32_t (&Y)[NS][2], const Emit &em,
                                             const ScanArgs &a, const TileK &k, EmitState &es, const TileJob &j,
                                             int qs) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    Y[s][0] = __builtin_rotateright32(Y[s][0], 1);
    Y[s][1] = __builtin_rotateright32(Y[s][1], 1);
  }
  if constexpr (STK && MODE == kEmitFilter) {
    StepOut2 o;  // unused by the candidate emission
    f4 p0 = pair_chain<NS, 0>(qreg, qhi, ap, Y);
    f4 p1 = pair_chain<NS, 1>(qreg, qhi, ap, Y);
    emit_pair<MODE, 0>(em, a, p0, k, es, o, j.bh, j.beta0, qs, 3, j.lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
    for (int V = 2; V >= 0; --V) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        Y[s][0] = __builtin_rotateleft32(Y[s][0], 4);
        Y[s][1] = __builtin_rotateleft32(Y[s][1], 4);
      }
      p0 = pair_chain<NS, 0>(qreg, qhi, ap, Y);
      emit_pair<MODE, 1>(em, a, p1, k, es, o, j.bh, j.beta0, qs, V + 1, j.lane);
      __builtin_amdgcn_sched_barrier(0);
      p1 = pair_chain<NS, 1>(qreg, qhi, ap, Y);
      emit_pair<MODE, 0>(em, a, p0, k, es, o, j.bh, j.beta0, qs, V, j.lane);
      __builtin_amdgcn_sched_barrier(0);
    }
    emit_pair<MODE, 1>(em, a, p1, k, es, o, j.bh, j.beta0, qs, 0, j.lane);
    return;
  }
  if constexpr (STK) step_group_stk<MODE, NS>(qreg, qhi, ap, Y, em, a, k, es, j.bh, j.beta0, j.L, qs, 3, j.lane);
  else step_group_emit<MODE, NS>(qreg, ap, Y, em, a, k, es, j.bh, j.beta0, j.L, qs, 3, j.lane);
#pragma unroll 1
  for (int V = 2; V >= 0; --V) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      Y[s][0] = __builtin_rotateleft32(Y[s][0], 4);
      Y[s][1] = __builtin_rotateleft32(Y[s][1], 4);
    }
    if constexpr (STK) step_group_stk<MODE, NS>(qreg, qhi, ap, Y, em, a, k, es, j.bh, j.beta0, j.L, qs, V, j.lane);
    else step_group_emit<MODE, NS>(qreg, ap, Y, em, a, k, es, j.bh, j.beta0, j.L, qs, V, j.lane);
  }
}

// A plan of NS (1..4) slices: the scales stay in registers for the whole tile
// and the A rows (qreg) for every tile.  Both quarters' halves are taken from a
// quarter pair's plane dwords at once; the next pair's dwords load while the
// second quarter computes.
template <int MODE, int NS, bool STK, bool HOST = false>
__device__ __forceinline__ void tile_fast(const ScanArgs &a, const Emit &em, const Shared &sh,
                                          const uint32_t (&qreg)[NS][2], const uint32_t (&qhi)[NS][2],
                                          const TileJob &j) {
  const int c = j.lane & 15, g = j.lane >> 4;
  TileAddr ta;
  if constexpr (HOST) {
    ta.hs = j.hs;
    ta.hb = j.hb;
  } else {
    ta = tile_addr(a, j.bh, j.beta0, c);
  }
  const int qp0 = j.qa0 >> 1, qp1 = (j.qa1 + 1) >> 1;
  uint32_t d[NS][4];
  load_planes<NS, HOST>(d, sh, ta, 0, g, qp0);
  uint32_t ap[NS][2];
  float amax = 0.0f;
  f4 dc;
  scale_group<NS, true, STK, HOST>(ap, amax, dc, sh, ta, 0, j.lane, j.ureal);
  const TileK k = scale_finish<STK>(amax, dc, sh, a, j.lane);
  rescale<NS>(ap, k.sx);
  float M[2] = {0.0f, 0.0f};
  if constexpr (MODE == kEmitFilter) {
    if constexpr (STK) lo_bound_stk<NS>(M, qreg, qhi, ap);
    else lo_bound<NS>(M, qreg, ap);
  }
  EmitState es;
  tile_setup<MODE, STK>(es, em, a, k, j.beta0, j.rk, M, j.lane);
#pragma unroll 1
  for (int qp = qp0; qp < qp1; ++qp) {
    uint32_t X0[NS][2], X1[NS][2];
    quarter_halves<NS, 0>(X0, d);
    quarter_halves<NS, 1>(X1, d);
    if (2 * qp >= j.qa0) quarter_fast<MODE, NS, STK>(qreg, qhi, ap, X0, em, a, k, es, j, 2 * qp);
    if (qp + 1 < qp1) load_planes<NS, HOST>(d, sh, ta, 0, g, qp + 1);  // in flight during the second quarter
    if (2 * qp + 1 < j.qa1) quarter_fast<MODE, NS, STK>(qreg, qhi, ap, X1, em, a, k, es, j, 2 * qp + 1);
  }
  if constexpr (MODE == kEmitFilter) tile_counts(em, a, es, j.bh, j.beta0, j.lane, j.fb, j.skipm);
}

// One register group of a larger plan: its planes (quarter qs), A rows and
// rescaled scales, then ACC step groups from V0 chained onto acc.
template <int NS, bool FIRST, int ACC>
__device__ __forceinline__ void run_group(f4 (&acc)[ACC][4], const Shared &sh, const TileAddr &ta, int s0, int lane,
                                          int sx, int ureal, int qs, int V0) {
  const int c = lane & 15, g = lane >> 4;
  uint32_t d[NS][4], ap[NS][2], qa[NS][2], X[NS][2];
  load_planes<NS>(d, sh, ta, s0, g, qs >> 1);
  load_arows<NS>(qa, sh.qa, s0, c, g);
  group_scales<NS>(ap, sh, ta, s0, g, sx, ureal);
  if (qs & 1) quarter_halves<NS, 1>(X, d);
  else quarter_halves<NS, 0>(X, d);
#pragma unroll
  for (int v = 0; v < ACC; ++v) step_group<NS, FIRST>(acc[v], qa, ap, X, V0 + v);
}

// A plan of more slices than the kernel holds in registers: every step
// group's chain runs over register groups of GS slices in order (GS even, so
// the slices pair as in one chain), each group's planes, A rows and scales
// reloaded per pass of ACC step groups.
template <int MODE, int ACC, int GS>
__device__ __forceinline__ void tile_grouped(const ScanArgs &a, const Emit &em, const Shared &sh, int nsl,
                                             const TileJob &j) {
  static_assert(GS % 2 == 0, "register groups of whole slice pairs");
  const int c = j.lane & 15;
  const TileAddr ta = tile_addr(a, j.bh, j.beta0, c);
  const int nfull = nsl / GS, tail = nsl - nfull * GS;
  float amax = 0.0f;
  f4 dc;
  {
    uint32_t raw[GS][2];
    scale_group<GS, true>(raw, amax, dc, sh, ta, 0, j.lane, j.ureal);
#pragma unroll 1
    for (int gi = 1; gi < nfull; ++gi) scale_group<GS, false>(raw, amax, dc, sh, ta, gi * GS, j.lane, j.ureal);
    uint32_t r1[1][2], r2[2][2], r3[3][2];
    if (tail == 1) scale_group<1, false>(r1, amax, dc, sh, ta, nfull * GS, j.lane, j.ureal);
    if (GS > 2 && tail == 2) scale_group<2, false>(r2, amax, dc, sh, ta, nfull * GS, j.lane, j.ureal);
    if (GS > 3 && tail == 3) scale_group<3, false>(r3, amax, dc, sh, ta, nfull * GS, j.lane, j.ureal);
  }
  const TileK k = scale_finish(amax, dc, sh, a, j.lane);
  const float M[2] = {0.0f, 0.0f};  // the grouped path compares both rows
  EmitState es;
  tile_setup<MODE>(es, em, a, k, j.beta0, j.rk, M, j.lane);
#pragma unroll 1
  for (int qs = j.qa0; qs < j.qa1; ++qs) {
#pragma unroll 1
    for (int V0 = 4 - ACC; V0 >= 0; V0 -= ACC) {
      f4 acc[ACC][4];
      run_group<GS, true, ACC>(acc, sh, ta, 0, j.lane, k.sx, j.ureal, qs, V0);
#pragma unroll 1
      for (int gi = 1; gi < nfull; ++gi) run_group<GS, false, ACC>(acc, sh, ta, gi * GS, j.lane, k.sx, j.ureal, qs, V0);
      if (tail == 1) run_group<1, false, ACC>(acc, sh, ta, nfull * GS, j.lane, k.sx, j.ureal, qs, V0);
      if (GS > 2 && tail == 2) run_group<2, false, ACC>(acc, sh, ta, nfull * GS, j.lane, k.sx, j.ureal, qs, V0);
      if (GS > 3 && tail == 3) run_group<3, false, ACC>(acc, sh, ta, nfull * GS, j.lane, k.sx, j.ureal, qs, V0);
#pragma unroll
      for (int v = ACC - 1; v >= 0; --v) emit_group<MODE>(em, a, acc[v], k, es, j.bh, j.beta0, j.L, qs, V0 + v, j.lane);
    }
  }
  if constexpr (MODE == kEmitFilter) tile_counts(em, a, es, j.bh, j.beta0, j.lane, j.fb, j.skipm);
}

// The tile loop of one plan kind (NSK slices 1..4, the plan padded with zero
// units; -1: more than the kernel holds): list entries L0, L0 + Ls, ... <
// nlist, quarters [qa0, qa1).  FB: the candidate pass's fallback rescan (T_lo,
// second count array; heads in skipm emit nothing).  The candidate pass's
// entries past the row's tiles (padding regions) get zero counts.
template <int MODE, int NSK, int ACC, bool FB, int GS, bool STK = false>
__device__ __forceinline__ void tile_loop(const ScanArgs &a, const Emit &em, const Shared &sh, int64_t bh, int lane,
                                          int64_t L0, int64_t Ls, int64_t nlist, int qa0, int qa1, uint32_t skipm,
                                          int nsl, int ureal) {
  constexpr bool kCand = MODE == kEmitFilter;
  constexpr int NQ = NSK > 0 ? NSK : 1;
  static_assert(!STK || NSK > 0, "stacked step classes on the register-held path");
  uint32_t *rcp = FB ? em.sel.rc2 : em.sel.rc1;
  uint32_t qreg[NQ][2], qhi[NQ][2];
  if constexpr (NSK > 0) load_arows<NQ>(qreg, sh.qa, 0, lane & 15, lane >> 4);
  if constexpr (STK) load_arows_hi<NQ>(qhi, sh.qa, 0, lane);
  RowK rk{};
  if constexpr (kCand) rk = row_consts(em, a, bh, lane, FB, skipm, STK);
  int64_t left = L0 < nlist ? (nlist - 1 - L0) / Ls : 0;  // the wave's entries after the current one
#pragma unroll 1
  for (int64_t L = L0; L < nlist; L += Ls, --left) {
    if (kCand && L >= a.nwt) {
      if (lane < a.G && !((skipm >> lane) & 1u)) rcp[(bh * a.G + lane) * em.sel.nreg + L] = 0u;
      continue;
    }
    const int64_t beta0 = (a.wt0 + L * a.wt_stride) * kWB;
    if (beta0 >= a.blk_end || beta0 + kWB <= a.blk0) continue;  // uniform per wave
    set_priority_by_tiles_left(left);
    const TileJob j{bh, beta0, L, qa0, qa1, lane, ureal, FB, skipm, rk};
    if constexpr (NSK > 0) tile_fast<MODE, NQ, STK>(a, em, sh, qreg, qhi, j);
    else tile_grouped<MODE, ACC, GS>(a, em, sh, nsl, j);
  }
}

// The workgroup's unit -> channel slot map of the stage (units of one channel
// are consecutive and share a scale offset) and the slots' scale offsets.
__device__ __forceinline__ void host_slots(HostStage &hs, const Shared &sh, int ureal) {
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const int u = tid;
    const bool first = u < ureal && (u == 0 || sh.soff[u] != sh.soff[u - 1]);
    const uint64_t m = __builtin_amdgcn_ballot_w64(first);
    const uint64_t le = u == kWave - 1 ? ~0ull : (2ull << u) - 1ull;  // lanes <= u
    const int slot = (int)__builtin_popcountll(m & le) - 1;
    hs.uslot[u] = (uint8_t)(u < ureal && slot >= 0 ? slot : 0);
    if (first) hs.soff1[slot] = sh.soff[u];
    if (u == 0) hs.nch = (int)__builtin_popcountll(m);
  }
}

// Copies the plan's plane runs (U units) and scale runs (nch channels) of
// blocks 16 L4 .. 16 L4 + 63 of row bh into the stage: 16-byte loads, all
// issued before the first LDS write.
__device__ __forceinline__ void host_stage(HostStage &hs, const ScanArgs &a, const Shared &sh, int64_t bh, int64_t L4,
                                           int U, int nch) {
  const int tid = threadIdx.x, nthr = (int)blockDim.x;
  const uint32_t sub = (uint32_t)a.sub, b0 = (uint32_t)(L4 * kWB);
  const uint32_t sb = b0 / sub, off0 = b0 - sb * sub;
  const char *pb = reinterpret_cast<const char *>(a.planes + ((bh * a.nsb + sb) * a.D * 4) * a.sub * 2) + off0 * 8u;
  const char *sbp = reinterpret_cast<const char *>(a.scales + ((bh * a.nsb + sb) * a.D) * a.sub) + off0 * 2u;
  constexpr int kRunQ = kHostBlk * 8 / 16;  // 16-byte pieces of a unit's run
  constexpr int kScQ = kHostBlk * 2 / 16;   // 16-byte pieces of a channel's scales
  constexpr int kPer = kHostUnits * kRunQ / kThreads, kPerS = kHostUnits * kScQ / kThreads;
  // every load is issued (pieces past the plan re-read piece 0), so the
  // pieces stay in registers
  uint4 v[kPer], w[kPerS];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int i0 = tid + r * nthr, i = i0 < U * kRunQ ? i0 : 0;
    v[r] = *reinterpret_cast<const uint4 *>(pb + sh.uoff[i / kRunQ] + (i % kRunQ) * 16);
  }
#pragma unroll
  for (int r = 0; r < kPerS; ++r) {
    const int i0 = tid + r * nthr, i = i0 < nch * kScQ ? i0 : 0;
    w[r] = *reinterpret_cast<const uint4 *>(sbp + hs.soff1[i / kScQ] + (i % kScQ) * 16);
  }
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int i = tid + r * nthr;
    if (i < U * kRunQ) *reinterpret_cast<uint4 *>(&hs.pw[i / kRunQ][(i % kRunQ) * 4]) = v[r];
  }
#pragma unroll
  for (int r = 0; r < kPerS; ++r) {
    const int i = tid + r * nthr;
    if (i < nch * kScQ) *reinterpret_cast<uint4 *>(&hs.sc[i / kScQ][(i % kScQ) * 8]) = w[r];
  }
}

// tile_loop for stores in mapped host memory (the candidate pass, plans held
// in registers): the workgroup steps through groups of four consecutive
// wave-tiles in lockstep, stages each group, then each wave scans its tile
// from the stage.
template <int MODE, int NSK, bool FB, bool STK>
__device__ __forceinline__ void host_tile_loop(const ScanArgs &a, const Emit &em, const Shared &sh, HostStage &hs,
                                               int64_t bh, int lane, int wave, int64_t nlist, uint32_t skipm, int nsl,
                                               int ureal) {
  static_assert(MODE == kEmitFilter && NSK > 0 && NSK * kSlice <= kHostUnits, "staged candidate pass");
  uint32_t *rcp = FB ? em.sel.rc2 : em.sel.rc1;
  host_slots(hs, sh, ureal);
  __syncthreads();
  const int nch = __builtin_amdgcn_readfirstlane(hs.nch);
  uint32_t qreg[NSK][2], qhi[NSK][2];
  load_arows<NSK>(qreg, sh.qa, 0, lane & 15, lane >> 4);
  if constexpr (STK) load_arows_hi<NSK>(qhi, sh.qa, 0, lane);
  const RowK rk = row_consts(em, a, bh, lane, FB, skipm, STK);
  const int64_t step = (int64_t)gridDim.x * kWaves;
#pragma unroll 1
  for (int64_t L4 = (int64_t)blockIdx.x * kWaves; L4 < nlist; L4 += step) {
    const int64_t L = L4 + wave;
    if (L4 < a.nwt) host_stage(hs, a, sh, bh, L4, nsl * kSlice, nch);  // uniform
    __syncthreads();
    if (L < nlist && L >= a.nwt) {
      if (lane < a.G && !((skipm >> lane) & 1u)) rcp[(bh * a.G + lane) * em.sel.nreg + L] = 0u;
    } else if (L < nlist) {
      TileJob j{bh, L * kWB, L, 0, kQS, lane, ureal, FB, skipm, rk};
      j.hs = &hs;
      j.hb = wave * kWB;
      tile_fast<MODE, NSK, STK, true>(a, em, sh, qreg, qhi, j);
    }
    __syncthreads();
  }
}

// Every tile of a wave.  A plan of up to NSMAX slices (the workgroup's tables
// padded to NSMAX slices by plan_tables) runs with everything in registers,
// rows of at most four heads with stacked step classes; a larger plan in
// register groups (a kernel picked for small plans still scans any plan
// correctly, only slower).  Zero units add exact zeros to every chain (a
// chain from zero is never -0), so the scores do not depend on the padding.
template <int MODE, int ACC, bool FB, int NSMAX>
__device__ __forceinline__ void tile_pass(const ScanArgs &a, const Emit &em, const Shared &sh, int64_t bh, int lane,
                                          int64_t L0, int64_t Ls, int64_t nlist, int qa0, int qa1, uint32_t skipm) {
  static_assert(NSMAX >= 1 && NSMAX <= kMaxNS, "one to six slices held in registers");
  constexpr int GS = ACC == 4 ? kGS : 2;  // the register groups of a kernel tuned for small plans stay small
  const int nsl = __builtin_amdgcn_readfirstlane(sh.U) / kSlice;
  const int ureal = __builtin_amdgcn_readfirstlane(sh.ureal);
  if (nsl <= NSMAX && a.G <= kMaxG / 2)
    tile_loop<MODE, NSMAX, ACC, FB, GS, true>(a, em, sh, bh, lane, L0, Ls, nlist, qa0, qa1, skipm, nsl, ureal);
  else if (nsl <= NSMAX)
    tile_loop<MODE, NSMAX, ACC, FB, GS>(a, em, sh, bh, lane, L0, Ls, nlist, qa0, qa1, skipm, nsl, ureal);
  else
    tile_loop<MODE, -1, ACC, FB, GS>(a, em, sh, bh, lane, L0, Ls, nlist, qa0, qa1, skipm, nsl, ureal);
}

}  // namespace sc

// Exact top kk of every row of the fused scan + top-k from its candidate
// regions; a row whose first pass holds fewer than kk candidates (a sample that
// misled T_hi) is first rescanned with T_lo by its finalize workgroup.
int launch_finalize_fused(const sc::ScanArgs &a, const sc::Emit &em, int64_t rows, int64_t m, int64_t k, int64_t sink,
                          int64_t local, int64_t *idx, hipStream_t st);

}  // namespace fathom
