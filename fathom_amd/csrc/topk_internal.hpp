// Selection machinery shared by the standalone top-k and the fused scan+top-k.
//
// Exact top-kk of a row in four steps:
//   select    from a sample of the row (tiles of 2048 tokens, every S-th
//             tile): T_lo, a lower bound of the sample's kk-th largest key,
//             and T_hi, a lower bound of its r-th largest, r = about
//             kAlphaX2 / 2 * kk * (sample size / n).  A sample is a subset of the
//             row, so T_lo never exceeds the row's kk-th largest key; T_hi is
//             a guess that about kAlphaX2 / 2 * kk elements of the row reach;
//   filter    elements with key >= T_hi become the row's candidates.  If there
//             are at least kk, T_hi <= the row's kk-th largest key and they
//             hold the whole top kk;
//   fallback  rows with fewer than kk candidates (a sample that was not
//             representative) are filtered again with T_lo, into the same
//             buffer under a second count; other rows skip the pass (the
//             fused scan's finalize workgroup rescans such a row itself);
//   finalize  one workgroup per row selects the exact kk largest candidates by
//             K64 = key << 32 | (0xFFFFFFFF - index) and writes them sorted.
// Exactness never depends on the sample: a poor sample only costs a fallback
// pass or more candidates (the buffer holds a whole row, so it cannot overflow).
//
// Candidates are kept in one of two layouts:
//   list      (score-row filter) appended at a row counter: cand[0, count);
//   regions   (fused scan) region r of a row holds the candidates of tokens
//             [r * kRegTok, (r + 1) * kRegTok) -- one wave's blocks -- at
//             cand[r * kRegTok, r * kRegTok + rc[r]), written with the count
//             rc[r] by that wave alone: no atomics.  A pass writes every
//             region of a row it does not skip.
#pragma once
#include "common.hpp"

namespace fathom {

constexpr int64_t kTileTok = 2048;  // tokens per sample tile of the score-row top-k
constexpr int64_t kRegTok = 1024;   // tokens per candidate region and sample tile of the fused scan (one wave-tile)
constexpr int64_t kMaxSample = 65536; // sampled keys per row (held in registers by select)

// expected first-pass candidates per row, in units of kk: kAlphaX2 / 2
constexpr int64_t kAlphaX2 = 5;

// Score rows up to this length (their 32-bit keys fit in one workgroup's LDS)
// select their top kk in one kernel, one workgroup per row, instead of
// sample -> select -> filter -> finalize: fewer launches for short rows.  The
// fused scan + top-k keeps the chain (its first pass writes no scores).
constexpr int64_t kRowSelectMax = 32768;

// Tokens per group of the group maxima that the fused scan's short-row pass
// writes beside its scores (one lane's 16 tokens of a block).
constexpr int64_t kGroupTok = 16;

// Candidate counters of a row, one per 256 bytes: every workgroup of a pass
// adds to its row's counter, and atomics to one cache line serialise.
constexpr int64_t kCntStride = 64;

struct TopkSel {
  uint32_t *thr;        // [rows] first-pass threshold key T_hi
  uint32_t *thr_lo;     // [rows] safe threshold key T_lo
  uint32_t *cand_cnt;   // [rows * kCntStride] candidates of the first pass
  uint32_t *cand2_cnt;  // [rows * kCntStride] candidates of the fallback pass
  uint64_t *cand;       // [rows, cand_cap] K64 candidates (of the pass in effect)
  int64_t cand_cap;
  uint32_t *rc1;        // region layout: [rows, nreg] counts of the first pass (null: list layout)
  uint32_t *rc2;        // region layout: [rows, nreg] counts of the fallback pass
  int64_t nreg;         // regions per row (cand_cap / kRegTok)
  uint32_t kk;
  __host__ __device__ uint32_t *cnt1(int64_t row) const { return cand_cnt + row * kCntStride; }
  __host__ __device__ uint32_t *cnt2(int64_t row) const { return cand2_cnt + row * kCntStride; }
};

// Sample stride in tiles of `tile` tokens: about 16384 sampled tokens per row
// (32768 for the fused scan's wave-tiles, whose first-pass threshold then sits
// at about 40 sampled keys for 1M-token rows: a fallback rescan of a row, the
// price of a threshold above the row's kk-th key, stays below 1e-6 per row),
// more where the sample must hold 2 kk keys or where about 16 sampled keys must
// reach the first-pass threshold (kAlphaX2 / 2 * kk * sample / n >= 16), at
// most kMaxSample keys.  The stride rounds up, so the sample never exceeds
// that many tiles.
inline int64_t topk_tile_stride(int64_t n, int64_t kk, int64_t tile) {
  const int64_t ntiles = cdiv(n, tile);
  int64_t want = tile == kRegTok ? 32 : cdiv(8 * kTileTok, tile);
  // the fused scan's sample keeps 64 group maxima per tile: at least 2 kk of them
  if (tile == kRegTok && kk > 0) {
    const int64_t g = cdiv(2 * kk, kRegTok / kGroupTok);
    want = g > want ? g : want;
  }
  if (kk > 0) {
    const int64_t a = cdiv(2 * kk, tile), b = cdiv(32 * n, kAlphaX2 * kk * tile);
    want = a > want ? a : want;
    want = b > want ? b : want;
  }
  const int64_t cap = kMaxSample / tile;
  if (want > cap) want = cap;
  const int64_t S = cdiv(ntiles, want);
  return S < 1 ? 1 : S;
}

inline int64_t topk_sample_tiles(int64_t n, int64_t S, int64_t tile) { return cdiv(cdiv(n, tile), S); }

// Rank in the sample of the first-pass threshold: about kAlphaX2 / 2 * kk of the row's
// n elements are expected at or above it (kk when the sample is the row).
inline int64_t topk_hi_rank(int64_t n, int64_t S, int64_t kk, int64_t tile) {
  int64_t sampled = 0;
  for (int64_t t = 0, nt = topk_sample_tiles(n, S, tile); t < nt; ++t) {
    const int64_t left = n - t * S * tile;
    sampled += left < tile ? (left > 0 ? left : 0) : tile;
  }
  const int64_t r = (kAlphaX2 * kk * sampled + 2 * n - 1) / (2 * n);
  return r < 1 ? 1 : (r > kk ? kk : r);
}

// 256-byte section alignment inside workspaces
inline size_t ws_align(size_t x) { return (x + 255) & ~(size_t)255; }

// Layout of the selection state inside a workspace; returns bytes used.
// nreg > 0: region layout with nreg regions per row (cand_cap = nreg * kRegTok).
size_t topk_sel_layout(int64_t rows, int64_t cand_cap, int64_t nreg, char *base, TopkSel *s);

// Whole top-k workspace: sampled keys [rows, samp_cap] + selection state with
// candidate room for a full row (regions: whole groups of four regions, the
// list layout otherwise).  Samples are tiles of kRegTok tokens with regions,
// kTileTok otherwise.  S is sized for kk = k (an upper bound on k - sink - local; a
// larger kk only means a denser sample).
size_t topk_layout(int64_t rows, int64_t n, int64_t k, bool regions, char *base, uint32_t **samp, int64_t *samp_cap,
                   TopkSel *sel, int64_t *S_out);

// T_lo (rank kk) and T_hi (rank r_hi <= kk) of every row's sample; clears the counters.
int launch_select_keys(const uint32_t *samp, int64_t rows, int64_t samp_cap, int64_t kk, int64_t r_hi, TopkSel s,
                       hipStream_t st);
// Thresholds of the fused scan's rows from their sample's group maxima
// (ng <= 4096 per row).
int launch_select_groups(const uint32_t *gmax, int64_t rows, int64_t ng, int64_t kk, int64_t r_hi, TopkSel s,
                         hipStream_t st);
int launch_sample_scores(const float *scores, int64_t rows, int64_t n, int64_t S, int64_t sink, int64_t lstart,
                         uint32_t *samp, int64_t samp_cap, hipStream_t st);
// First pass (fallback = false) or fallback pass (rows whose first pass found fewer than kk).
int launch_filter_scores(const float *scores, int64_t rows, int64_t n, int64_t sink, int64_t lstart, TopkSel s,
                         bool fallback, hipStream_t st);
// Either layout (s.rc1 set: regions).
int launch_finalize(int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, TopkSel s, int64_t *idx,
                    hipStream_t st);
// Exact top kk of whole score rows [rows, n] (n <= kRowSelectMax).
int launch_rowselect(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local,
                     int64_t *idx, hipStream_t st);
// The same from the rows' 16-token group maxima (gmax [rows, ceil(n / 16)]
// largest masked keys): only the groups that can hold a top-kk key are read.
int launch_rowselect_gmax(const float *scores, const uint32_t *gmax, int64_t rows, int64_t n, int64_t m, int64_t k,
                          int64_t sink, int64_t local, int64_t *idx, hipStream_t st);
// launch_rowselect_gmax, then in the same workgroup the attention of each row's
// query head (row = bh * G + g) over its k <= 512 selected positions: K, V
// bf16 rows [BH, cap, D = 128] in device memory, out [rows, D] fp32, equal to
// gather_attention's output for those indices.
int launch_rowselect_gmax_attn(const float *scores, const uint32_t *gmax, int64_t rows, int64_t n, int64_t m, int64_t k,
                               int64_t sink, int64_t local, int64_t *idx, const float *q, int64_t G, const void *K,
                               const void *V, int64_t cap, float scale, float *out, hipStream_t st);
// kk == 0: only the sink and local positions are written.
int launch_fixed_only(int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, int64_t *idx, hipStream_t st);
// Largest kk of the LDS-resident selections (sample -> select -> filter ->
// finalize, row-select, the fused scan's chains); larger kk take the wide path.
constexpr int64_t kSelMaxK = 2048;
// State of the wide selection (exact top kk of candidate lists for any kk by a
// 64-bit radix select, then a counting or bitonic sort; launches of
// data-independent shape).
size_t wide_select_bytes(int64_t rows, int64_t kk);
// Ranks of the kk <= kRankListMax distinct values of each row of sel [rows, P]
// by one counting sort, written as idx [rows, k] (then the fixed positions).
constexpr int64_t kRankListMax = 8192;
int launch_rank_list(const uint64_t *sel, int64_t P, int64_t rows, int64_t kk, int64_t m, int64_t k, int64_t sink,
                     int64_t local, int64_t *idx, hipStream_t st);
// The wide selection over the candidate lists (list layout) of the chain's filter passes.
int wide_select_list(const TopkSel &s, int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, int64_t *idx,
                     void *workspace, size_t workspace_bytes, hipStream_t st);
// Top-k of score rows with kk above kSelMaxK: sample -> select -> filter (and
// the fallback pass), then the wide selection over each row's candidate list;
// workspace of wide_topk_bytes(rows, n, k) (k bounds kk from above).
size_t wide_topk_bytes(int64_t rows, int64_t n, int64_t k);
int wide_topk_run(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local,
                  int64_t *idx, void *workspace, size_t workspace_bytes, hipStream_t st);
// Shape checks shared by the top-k entry points (FATHOM_OK or an error status).
int check_topk_args(int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local, const char *who);

// Wave-aggregated append of K64 values whose predicate holds to a row's list.
__device__ __forceinline__ void wave_append(bool pred, uint64_t val, uint32_t *counter, uint64_t *buf, uint64_t cap,
                                            int lane) {
  const uint64_t m = __ballot(pred);
  if (m == 0) return;
  const int leader = __ffsll((unsigned long long)m) - 1;
  uint32_t base = 0;
  if (lane == leader) base = atomicAdd(counter, (uint32_t)__popcll(m));
  base = __builtin_amdgcn_readlane(base, leader);
  const uint64_t slot = (uint64_t)base + __popcll(m & ((1ull << lane) - 1ull));
  if (pred && slot < cap) buf[slot] = val;
}

// Wave-aggregated append into a workgroup-local LDS list; entries past lcap go
// straight to the global list (one atomic each: only hit by adversarial rows).
__device__ __forceinline__ void wave_append_local(bool pred, uint64_t val, uint32_t *lcnt, uint64_t *lbuf,
                                                  uint32_t lcap, uint32_t *gcnt, uint64_t *gbuf, uint64_t gcap,
                                                  int lane) {
  const uint64_t m = __ballot(pred);
  if (m == 0) return;
  const int leader = __ffsll((unsigned long long)m) - 1;
  uint32_t base = 0;
  if (lane == leader) base = atomicAdd(lcnt, (uint32_t)__popcll(m));
  base = __builtin_amdgcn_readlane(base, leader);
  const uint32_t slot = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
  if (pred) {
    if (slot < lcap) {
      lbuf[slot] = val;
    } else {
      const uint32_t p = atomicAdd(gcnt, 1u);
      if ((uint64_t)p < gcap) gbuf[p] = val;
    }
  }
}

// Copies a workgroup's LDS list to the global list with one reservation.
// Call from all threads after a barrier that completes the appends.
__device__ __forceinline__ void flush_local(const uint32_t *lcnt, const uint64_t *lbuf, uint32_t lcap,
                                            uint32_t *gcnt, uint64_t *gbuf, uint64_t gcap, uint32_t *s_base) {
  const uint32_t nloc = min(*lcnt, lcap);
  if (threadIdx.x == 0) *s_base = nloc ? atomicAdd(gcnt, nloc) : 0u;
  __syncthreads();
  const uint32_t base = *s_base;
  for (uint32_t i = threadIdx.x; i < nloc; i += blockDim.x)
    if ((uint64_t)base + i < gcap) gbuf[base + i] = lbuf[i];
}

__device__ __forceinline__ uint64_t k64_of(uint32_t key, int64_t i) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

}  // namespace fathom
