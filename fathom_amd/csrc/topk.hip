// Sink/local-masked exact top-k over score rows.
//
// Orderable keys: score_key maps a float to a uint32 whose unsigned order is
// torch.topk's value order; K64 = key << 32 | (0xFFFFFFFF - index) makes every
// element of a row distinct and orders equal scores by ascending index.
// The selection runs select -> filter -> finalize (topk_internal.hpp); the
// fused scan+top-k path replaces `filter` by the scan kernel's own emission.
//
// Selection of the need-th largest value of a set (range_select): the active
// values lie in [lo, hi]; a 2048-bin LDS histogram of (v - lo) >> s, with s
// chosen so the bins span exactly that range, locates the bin holding the
// need-th largest; the range shrinks to that bin (by >= 11 bits) and the
// search repeats until the bin holds exactly the values still needed.  Bins
// follow the values' actual spread, so a row's candidates -- all packed just
// above a threshold -- still spread over many bins (few atomic collisions),
// and a 64-bit K64 needs at most six rounds.
#include "topk_internal.hpp"
#include "scan_core.hpp"
#include "attn_core.hpp"

namespace fathom {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelPer = (int)(kMaxSample / kSelThreads);  // keys per thread in select
constexpr int kFinThreads = 1024;
constexpr int kFilterThreads = 256;
constexpr int64_t kFilterChunk = 16384;
constexpr uint32_t kFilterLocal = 2048;  // LDS candidates per filter workgroup
constexpr int kCandLds = 16384;          // candidates selected in LDS (128 KB)
constexpr int kMaxK = (int)kSelMaxK;      // largest kk of these selections
constexpr int kBins = 2048;
constexpr int kMaxWaves = 16;            // waves of a 1024-thread workgroup

struct RangeShared {
  uint32_t hist[kBins];
  uint64_t wmin[kMaxWaves], wmax[kMaxWaves];
  uint32_t wsum[kMaxWaves];
  uint64_t fin[kWave];  // the last few values of a range, selected by one wave
  uint64_t lo, hi, thr;
  uint32_t need, done, hsel, fcnt, hcnt;
};

// The two values of lane pair {i & ~J, i | J} (in some order) for a compare-
// exchange at distance J, on the VALU: DPP quad permutes (J = 1, 2), a quad
// reversal then a half-row mirror (J = 4: i ^ 3 ^ 7), a row rotation by 8
// (J = 8), and the gfx950 row swaps v_permlane16/32_swap (J = 16, 32: the
// values of lanes i & ~J and i | J).
template <int J>
__device__ __forceinline__ void lane_pair(uint64_t v, uint64_t &x, uint64_t &y) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  uint32_t l0, l1, h0, h1;
  if constexpr (J == 16 || J == 32) {
    const auto pl = J == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                            : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto ph = J == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                            : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    l0 = pl[0];
    l1 = pl[1];
    h0 = ph[0];
    h1 = ph[1];
  } else {
    l0 = lo;
    h0 = hi;
    if constexpr (J == 1) {
      l1 = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
      h1 = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false);
    } else if constexpr (J == 2) {
      l1 = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
      h1 = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, false);
    } else if constexpr (J == 4) {  // quad_perm [3,2,1,0], then row_half_mirror
      l1 = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(lo, 0x1B, 0xF, 0xF, false), 0x141, 0xF, 0xF, false);
      h1 = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(hi, 0x1B, 0xF, 0xF, false), 0x141, 0xF, 0xF, false);
    } else {
      static_assert(J == 8, "compare-exchange distance");
      l1 = __builtin_amdgcn_mov_dpp(lo, 0x128, 0xF, 0xF, false);  // row_ror:8
      h1 = __builtin_amdgcn_mov_dpp(hi, 0x128, 0xF, 0xF, false);
    }
  }
  x = ((uint64_t)h0 << 32) | l0;
  y = ((uint64_t)h1 << 32) | l1;
}

template <int KB, int J>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t v, int lane) {
  uint64_t x, y;
  lane_pair<J>(v, x, y);
  const bool keep_max = ((lane & J) == 0) == ((lane & KB) == 0);
  const uint64_t mx = x > y ? x : y, mn = x > y ? y : x;
  v = keep_max ? mx : mn;
  if constexpr (J > 1) v = bitonic_merge<KB, J / 2>(v, lane);
  return v;
}

// Descending bitonic sort of the 64 values of a wave (one per lane), in
// registers: 21 compare-exchange stages of a few VALU instructions each.
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t v, int lane) {
  v = bitonic_merge<2, 1>(v, lane);
  v = bitonic_merge<4, 2>(v, lane);
  v = bitonic_merge<8, 4>(v, lane);
  v = bitonic_merge<16, 8>(v, lane);
  v = bitonic_merge<32, 16>(v, lane);
  v = bitonic_merge<64, 32>(v, lane);
  return v;
}

// Wave-wide minimum and maximum of 64-bit values (every lane gets both):
// butterfly over the same lane pairs as the sort.
template <int J>
__device__ __forceinline__ void minmax_step(uint64_t &mn, uint64_t &mx) {
  uint64_t a, b, c, d;
  lane_pair<J>(mn, a, b);
  lane_pair<J>(mx, c, d);
  mn = a < b ? a : b;
  mx = c > d ? c : d;
}
__device__ __forceinline__ void wave_minmax_u64(uint64_t &mn, uint64_t &mx) {
  minmax_step<1>(mn, mx);
  minmax_step<2>(mn, mx);
  minmax_step<4>(mn, mx);
  minmax_step<8>(mn, mx);
  minmax_step<16>(mn, mx);
  minmax_step<32>(mn, mx);
}

// Descending ranks of the first nlim slots (a power of two, 64 <= nlim <= E *
// 1024) of E * 1024 values, thread t holding slots t + 1024 e (the whole
// workgroup calls it; slots from nlim on take no part).  Each wave sorts its
// 64-value runs in registers; merge levels in LDS double the runs until at
// most 8 remain; then a value's rank is the number of greater values over all
// runs (binary searches), and put(rank, value) is called for every slot below
// nlim.  Distinct values get distinct ranks; equal values share one.  a and b:
// LDS buffers of nlim values.
template <int E, typename Put>
__device__ __forceinline__ void block_rank_desc(const uint64_t (&v)[E], uint64_t *a, uint64_t *b, int nlim, Put put) {
  const int t = threadIdx.x, lane = t & 63;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (t + 1024 * e < nlim) a[t + 1024 * e] = wave_sort_desc(v[e], lane);  // uniform per wave
  __syncthreads();
  int w = kWave;
  for (; nlim > 8 * w; w <<= 1) {
    // merge: an element's new place is its index in its own run plus the
    // partner run's elements ahead of it (strictly greater for the left run,
    // greater or equal for the right one: equal values keep run order)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = t + 1024 * e;
      if (i >= nlim) continue;
      const uint64_t x = a[i];
      const int r = i / w, p = i - r * w;
      const bool left = (r & 1) == 0;
      const uint64_t *part = a + (r ^ 1) * w;
      int c = 0;
      for (int step = w; step > 0; step >>= 1) {
        if (c + step <= w) {
          const uint64_t y = part[c + step - 1];
          if (left ? (y > x) : (y >= x)) c += step;
        }
      }
      b[(r >> 1) * 2 * w + p + c] = x;
    }
    __syncthreads();
    uint64_t *tmp = a;
    a = b;
    b = tmp;
  }
  const int nr = nlim / w;  // at most 8 runs
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = t + 1024 * e;
    if (i >= nlim) continue;
    const uint64_t x = a[i];
    // greater values per run, by binary searches in all runs at once (eight
    // independent LDS reads per step); x's own run counts the values before it
    int c[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) c[q] = 0;
    for (int step = w; step > 0; step >>= 1) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int j = min(c[q] + step, w) - 1;
        const uint64_t y = a[(q < nr ? q * w : 0) + j];  // in bounds for every q
        if (q < nr && c[q] + step <= w && y > x) c[q] += step;
      }
    }
    int rank = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) rank += c[q];
    put(rank, x);
  }
}

// Descending ranks of the cnt valid values of E * 1024 (thread t holding slots
// t + 1024 e; the valid ones are the slots below cnt, all distinct) by a
// counting sort: 2048 bins of (v - min) >> s over the values' range, each
// value's place in its bin from a returning LDS atomic, the bins' offsets by a
// prefix sum from the top bin down, then every value's rank = the values in
// higher bins + the greater values of its own bin (a few, read from the
// values placed in bin order).  Values crowd a bin only where their range is
// dominated by a few outliers: then (more than kCrowd in one bin) the ranks
// come from block_rank_desc over the first nlim slots instead.  put(rank, v)
// is called for every valid value.  scratch: LDS of max(E * 1024 + 2048,
// 2 * nlim) values.
constexpr uint32_t kCrowd = 48;
template <int E, typename Put>
__device__ __forceinline__ void bin_rank_desc(const uint64_t (&v)[E], int cnt, uint64_t *scratch, RangeShared &sh,
                                              int nlim, Put put) {
  static_assert(kBins == 2 * kFinThreads, "two bins per thread");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nw = kFinThreads >> 6;
  uint64_t *placed = scratch;                                           // [E * 1024] values in bin order
  uint32_t *hist = reinterpret_cast<uint32_t *>(scratch + E * 1024);    // [2048] values per bin
  uint32_t *above = hist + kBins;                                       // [2048] values in higher bins
  uint64_t mn = ~0ull, mx = 0ull;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (t + 1024 * e < cnt) {
      mn = v[e] < mn ? v[e] : mn;
      mx = v[e] > mx ? v[e] : mx;
    }
  wave_minmax_u64(mn, mx);
  if (lane == 0) {
    sh.wmin[wave] = mn;
    sh.wmax[wave] = mx;
  }
  hist[t] = hist[t + kFinThreads] = 0u;
  if (t == 0) sh.fcnt = 0u;
  __syncthreads();
  uint64_t lo = ~0ull, hi = 0ull;
  for (int w = 0; w < nw; ++w) {
    lo = sh.wmin[w] < lo ? sh.wmin[w] : lo;
    hi = sh.wmax[w] > hi ? sh.wmax[w] : hi;
  }
  const uint64_t R = cnt > 0 ? hi - lo : 0ull;
  const int bl = R ? 64 - __clzll((long long)R) : 0;
  const int sft = bl > 11 ? bl - 11 : 0;  // (v - lo) >> sft < 2048
  uint32_t bin[E], slot[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (t + 1024 * e < cnt) {
      bin[e] = (uint32_t)((v[e] - lo) >> sft);
      slot[e] = atomicAdd(&hist[bin[e]], 1u);
    }
  __syncthreads();
  // values in higher bins: thread t holds bins 2047 - 2t, 2046 - 2t
  const uint32_t c0 = hist[kBins - 1 - 2 * t], c1 = hist[kBins - 2 - 2 * t], c = c0 + c1;
  const uint32_t wi = wave_incl_scan_u32(c);
  if (lane == kWave - 1) sh.wsum[wave] = wi;
  if (c0 > kCrowd || c1 > kCrowd) sh.fcnt = 1u;  // any thread: the same value
  __syncthreads();
  if (sh.fcnt) {  // uniform
    block_rank_desc<E>(v, scratch, scratch + nlim, nlim, [&](int rank, uint64_t x) {
      if (rank < cnt) put(rank, x);
    });
    return;
  }
  uint32_t ab = wi - c;
  for (int w = 0; w < wave; ++w) ab += sh.wsum[w];
  above[kBins - 1 - 2 * t] = ab;
  above[kBins - 2 - 2 * t] = ab + c0;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (t + 1024 * e < cnt) placed[above[bin[e]] + slot[e]] = v[e];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (t + 1024 * e < cnt) {
      const uint32_t base = above[bin[e]], n = hist[bin[e]];
      uint32_t rank = base;
      for (uint32_t j = 0; j < n; ++j) rank += placed[base + j] > v[e] ? 1u : 0u;
      put((int)rank, v[e]);
    }
}

// Value sources of the selections.  for_each(f) calls f(ok, v) for every value
// v of the set, each thread of the workgroup for its share, in loops that are
// uniform over the workgroup (all threads call it; f runs with every lane
// active, v meaningful where ok).  The selections never depend on the order.
struct ArraySrc {  // values p[0, cnt) (LDS or global memory)
  const uint64_t *p;
  int64_t cnt;
  template <typename F>
  __device__ __forceinline__ void for_each(F f) const {
    for (int64_t i0 = 0; i0 < cnt; i0 += blockDim.x) {
      const int64_t i = i0 + threadIdx.x;
      const bool ok = i < cnt;
      f(ok, ok ? p[i] : 0ull);
    }
  }
};

template <typename Get>
struct IndexSrc {  // values get(0), ..., get(cnt - 1)
  Get get;
  int64_t cnt;
  template <typename F>
  __device__ __forceinline__ void for_each(F f) const {
    for (int64_t i0 = 0; i0 < cnt; i0 += blockDim.x) {
      const int64_t i = i0 + threadIdx.x;
      const bool ok = i < cnt;
      f(ok, ok ? get(i) : 0ull);
    }
  }
};
template <typename Get>
__device__ __forceinline__ IndexSrc<Get> index_src(Get get, int64_t cnt) {
  return IndexSrc<Get>{get, cnt};
}

// A row's candidates in the region layout: region r holds rc[r] values at
// cand[r * kRegTok, ...).  Each wave takes batches of 64 regions (the next
// batch's counts load while the current one is read); lane e of a step reads
// the batch's e-th value, found by a binary search over the lanes' exclusive
// prefix sums of the counts.
static_assert(kRegTok < (1 << 11), "region counts fit the 11-bit wave sums of RegionSrc");
struct RegionSrc {
  const uint32_t *rc;
  const uint64_t *cand;
  int64_t nreg;
  template <typename F>
  __device__ __forceinline__ void for_each(F f) const {
    const int lane = threadIdx.x & 63;
    const int64_t step = (int64_t)(blockDim.x >> 6) * kWave;
    int64_t r0 = (int64_t)(threadIdx.x >> 6) * kWave;
    uint32_t c = r0 + lane < nreg ? min(rc[r0 + lane], (uint32_t)kRegTok) : 0u;
    while (r0 < nreg) {  // uniform per wave
      const int64_t r1 = r0 + step;
      const uint32_t cn = r1 + lane < nreg ? min(rc[r1 + lane], (uint32_t)kRegTok) : 0u;
      const uint32_t pre = (uint32_t)wave_excl_scan_small<11>((int)c, lane);  // counts <= kRegTok = 1024
      const uint32_t tot = (uint32_t)wave_sum_small<11>((int)c);
      for (uint32_t e0 = 0; e0 < tot; e0 += kWave) {
        const uint32_t e = e0 + lane;
        int j = 0;  // the last lane whose prefix is <= e: its region holds value e
#pragma unroll
        for (int sft = 32; sft > 0; sft >>= 1)
          if (__shfl(pre, j + sft, kWave) <= e) j += sft;
        const uint32_t pj = __shfl(pre, j, kWave);
        const bool ok = e < tot;
        f(ok, ok ? cand[(r0 + j) * kRegTok + (e - pj)] : 0ull);
      }
      r0 = r1;
      c = cn;
    }
  }
};

// Wave-aggregated append of the values whose ok holds to an LDS list (one LDS
// atomic per wave); the counter keeps counting past cap, values past it are
// dropped.  Call with every lane of the wave active.
__device__ __forceinline__ void lds_append(bool ok, uint64_t v, uint32_t *cnt, uint64_t *buf, uint32_t cap, int lane) {
  const uint64_t m = __ballot(ok);
  if (m == 0ull) return;
  const int leader = __ffsll((unsigned long long)m) - 1;
  uint32_t base = 0u;
  if (lane == leader) base = atomicAdd(cnt, (uint32_t)__popcll(m));
  base = __builtin_amdgcn_readlane(base, leader);
  const uint32_t slot = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
  if (ok && slot < cap) buf[slot] = v;
}

// Copies a source's values to LDS (at most cap of them); returns how many the
// source holds.  All threads call it; s_cnt is free again on return.
template <typename Src>
__device__ __forceinline__ uint32_t stage_lds(const Src &src, uint64_t *buf, uint32_t cap, uint32_t &s_cnt) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x == 0) s_cnt = 0u;
  __syncthreads();
  src.for_each([&](bool ok, uint64_t v) { lds_append(ok, v, &s_cnt, buf, cap, lane); });
  __syncthreads();
  const uint32_t tot = s_cnt;
  __syncthreads();
  return tot;
}

// Copies a row's candidates in the region layout to LDS (at most cap of them)
// and returns how many it holds.  Per chunk of up to 4 * kFinThreads regions:
// each thread loads 4 counts at once, a workgroup prefix sum turns them into
// the regions' first slots (in pre: 4 * kFinThreads words of LDS), then value
// e of the chunk is read by thread e mod kFinThreads after a binary search in
// pre -- every load of a chunk is in flight at once, however unevenly the
// candidates spread.  nreg: a multiple of 4.  All threads call it.
__device__ __forceinline__ uint32_t stage_regions(const uint32_t *rc, const uint64_t *cand, int64_t nreg, uint64_t *buf, uint32_t cap,
                                  uint32_t *pre, RangeShared &sh) {
  constexpr int kR = 4 * kFinThreads;  // regions per chunk
  constexpr int kU = 4;                // values per thread read together
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  uint32_t base = 0u;
  for (int64_t c0 = 0; c0 < nreg; c0 += kR) {
    const int nr = (int)min((int64_t)kR, nreg - c0);
    uint4 c = make_uint4(0u, 0u, 0u, 0u);
    if (4 * tid < nr) c = *reinterpret_cast<const uint4 *>(rc + c0 + 4 * tid);
    c.x = min(c.x, (uint32_t)kRegTok);
    c.y = min(c.y, (uint32_t)kRegTok);
    c.z = min(c.z, (uint32_t)kRegTok);
    c.w = min(c.w, (uint32_t)kRegTok);
    const uint32_t t = c.x + c.y + c.z + c.w;
    const uint32_t wi = wave_incl_scan_u32(t), wx = wi - t;
    if (lane == kWave - 1) sh.wsum[wave] = wi;
    __syncthreads();
    uint32_t off = wx, tot = 0u;
    for (int w = 0; w < nw; ++w) {
      const uint32_t ws = sh.wsum[w];
      off += w < wave ? ws : 0u;
      tot += ws;
    }
    if (4 * tid < nr) {
      pre[4 * tid] = off;
      pre[4 * tid + 1] = off + c.x;
      pre[4 * tid + 2] = off + c.x + c.y;
      pre[4 * tid + 3] = off + c.x + c.y + c.z;
    }
    __syncthreads();
    for (uint32_t e0 = 0; e0 < tot; e0 += kU * kFinThreads) {
      uint64_t v[kU];
      uint32_t slot[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const uint32_t e = e0 + u * kFinThreads + tid;
        slot[u] = ~0u;
        v[u] = 0ull;
        if (e < tot) {
          int lo = 0, hi = nr - 1;  // the last region whose first slot is <= e
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pre[mid] <= e) lo = mid;
            else hi = mid - 1;
          }
          v[u] = cand[(c0 + lo) * kRegTok + (e - pre[lo])];
          slot[u] = base + e;
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (slot[u] < cap) buf[slot[u]] = v[u];
    }
    base += tot;
    __syncthreads();  // pre and wsum are rewritten by the next chunk
  }
  return base;
}

// Smallest value >= lo of the need-th largest element among the cnt values of
// src (all threads of the workgroup call it).  Returns thr with #{v >= thr} >=
// need, equality when the values are distinct; thr = 0 when there are fewer
// than need values.
template <typename Src>
__device__ __forceinline__ uint64_t range_select(const Src &src, int64_t cnt, uint32_t need, RangeShared &sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  if (cnt < (int64_t)need || need == 0) return 0ull;
  // value range
  uint64_t mn = ~0ull, mx = 0ull;
  src.for_each([&](bool ok, uint64_t v) {
    if (ok) {
      mn = v < mn ? v : mn;
      mx = v > mx ? v : mx;
    }
  });
  wave_minmax_u64(mn, mx);
  if (lane == 0) {
    sh.wmin[wave] = mn;
    sh.wmax[wave] = mx;
  }
  __syncthreads();
  if (tid == 0) {
    uint64_t a = ~0ull, b = 0ull;
    for (int w = 0; w < nw; ++w) {
      a = sh.wmin[w] < a ? sh.wmin[w] : a;
      b = sh.wmax[w] > b ? sh.wmax[w] : b;
    }
    sh.lo = a;
    sh.hi = b;
    sh.need = need;
    sh.done = 0u;
    sh.hsel = ~0u;
    sh.thr = a;
  }
  __syncthreads();
  // each round narrows the range of distinct 64-bit values by at least 11
  // bits, so six rounds end it; the bound keeps a source that yields fewer
  // values than cnt from looping
  for (int round = 0; round < 8; ++round) {
    const uint64_t lo = sh.lo, hi = sh.hi;
    const uint32_t nd = sh.need;
    const uint64_t R = hi - lo;
    const int bl = R ? 64 - __clzll((long long)R) : 0;
    const int s = bl > 11 ? bl - 11 : 0;
    const int nb = (int)(R >> s) + 1;
    for (int b = tid; b < nb; b += blockDim.x) sh.hist[b] = 0u;
    __syncthreads();
    src.for_each([&](bool ok, uint64_t v) {
      if (ok && v >= lo && v <= hi) atomicAdd(&sh.hist[(v - lo) >> s], 1u);
    });
    __syncthreads();
    // values in the bins above each thread's pair (thread t owns bins 2t, 2t + 1)
    const int b0 = 2 * tid;
    const uint32_t h0 = b0 < nb ? sh.hist[b0] : 0u, h1 = b0 + 1 < nb ? sh.hist[b0 + 1] : 0u;
    const uint32_t x = h0 + h1;
    const uint32_t incl = wave_incl_scan_u32(x);
    const uint32_t wtot = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (lane == 0) sh.wsum[wave] = wtot;
    __syncthreads();
    uint32_t later = 0u;
    for (int w = wave + 1; w < nw; ++w) later += sh.wsum[w];
    const uint32_t above = wtot - incl + later;  // values in bins above b0 + 1
    int bsel = -1;
    uint32_t nsel = 0u, hsel = 0u;
    if (above < nd && above + h1 >= nd) {
      bsel = b0 + 1;
      nsel = nd - above;
      hsel = h1;
    } else if (above + h1 < nd && above + h1 + h0 >= nd) {
      bsel = b0;
      nsel = nd - above - h1;
      hsel = h0;
    }
    __syncthreads();  // every thread has read lo/hi/need
    if (bsel >= 0) {
      const uint64_t nlo = lo + ((uint64_t)bsel << s);
      const uint64_t width = s ? (((uint64_t)1 << s) - 1ull) : 0ull;
      sh.lo = nlo;
      sh.hi = (hi - nlo) > width ? nlo + width : hi;
      sh.need = nsel;
      sh.thr = nlo;
      sh.hsel = hsel;
      sh.done = (hsel == nsel || s == 0) ? 1u : 0u;
    }
    __syncthreads();
    if (sh.done) break;
    if (sh.hsel <= (uint32_t)kWave) {
      // at most 64 values left in the range: gather them, one wave sorts them
      // and the need-th largest is the threshold
      const uint64_t flo = sh.lo, fhi = sh.hi;
      const uint32_t fneed = sh.need;
      if (tid == 0) sh.fcnt = 0u;
      __syncthreads();
      src.for_each([&](bool ok, uint64_t v) {
        lds_append(ok && v >= flo && v <= fhi, v, &sh.fcnt, sh.fin, (uint32_t)kWave, lane);
      });
      __syncthreads();
      if (wave == 0) {
        const uint32_t fc = min(sh.fcnt, (uint32_t)kWave);
        const uint64_t y = wave_sort_desc((uint32_t)lane < fc ? sh.fin[lane] : 0ull, lane);
        if ((uint32_t)lane == fneed - 1u) sh.thr = y;
      }
      __syncthreads();
      break;
    }
  }
  return sh.thr;
}

__device__ __forceinline__ uint32_t masked_key(const float *row, int64_t i, int64_t sink, int64_t lstart) {
  return (i < sink || i >= lstart) ? kKeyNegInf : score_key(row[i]);
}

__global__ __launch_bounds__(256) void sample_scores_kernel(const float *__restrict__ scores, int64_t n, int64_t S,
                                                            int64_t sink, int64_t lstart, uint32_t *__restrict__ samp,
                                                            int64_t samp_cap) {
  const int64_t row = blockIdx.y;
  const float *rs = scores + row * n;
  const int64_t ti = blockIdx.x;
  for (int o = threadIdx.x; o < kTileTok; o += 256) {
    const int64_t pos = ti * S * kTileTok + o;
    samp[row * samp_cap + ti * kTileTok + o] = pos < n ? masked_key(rs, pos, sink, lstart) : 0u;
  }
}

// Candidates of score rows (keys >= the row's threshold), 4 scores per thread
// and step when rows are 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(kFilterThreads) void filter_scores_kernel(const float *__restrict__ scores, int64_t n,
                                                                       int64_t sink, int64_t lstart, TopkSel s,
                                                                       bool fallback) {
  __shared__ uint64_t lbuf[kFilterLocal];
  __shared__ uint32_t lcnt, lbase;
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t row = blockIdx.y;
  if (fallback && *s.cnt1(row) >= s.kk) return;  // the first pass holds the row's top kk
  const float *rs = scores + row * n;
  const uint32_t thr = fallback ? s.thr_lo[row] : s.thr[row];
  uint32_t *cnt = fallback ? s.cnt2(row) : s.cnt1(row);
  uint64_t *cand = s.cand + row * s.cand_cap;
  if (tid == 0) lcnt = 0u;
  __syncthreads();
  const int64_t start = (int64_t)blockIdx.x * kFilterChunk;
  const int64_t end = min(start + kFilterChunk, n);
  if (VEC) {
    for (int64_t i0 = start; i0 < end; i0 += 4 * kFilterThreads) {
      const int64_t i = i0 + 4 * tid;
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < end) f = *reinterpret_cast<const float4 *>(rs + i);
      const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t iu = i + u;
        const bool in = iu < end;
        const uint32_t key = in ? ((iu < sink || iu >= lstart) ? kKeyNegInf : score_key(fv[u])) : 0u;
        wave_append_local(in && key >= thr, k64_of(key, iu), &lcnt, lbuf, kFilterLocal, cnt, cand,
                          (uint64_t)s.cand_cap, lane);
      }
    }
  } else {
    for (int64_t i0 = start; i0 < end; i0 += kFilterThreads) {
      const int64_t i = i0 + tid;
      const bool in = i < end;
      const uint32_t key = in ? masked_key(rs, i, sink, lstart) : 0u;
      wave_append_local(in && key >= thr, k64_of(key, i), &lcnt, lbuf, kFilterLocal, cnt, cand,
                        (uint64_t)s.cand_cap, lane);
    }
  }
  __syncthreads();
  flush_local(&lcnt, lbuf, kFilterLocal, cnt, cand, (uint64_t)s.cand_cap, &lbase);
}

// Writes the tail of a row's output: zeros after the got selected positions
// (fewer candidates than kk), then the sink and local positions.
__device__ __forceinline__ void write_fixed(int64_t *out, int got, int64_t kk, int64_t m, int64_t sink, int64_t local) {
  for (int i = got + (int)threadIdx.x; i < (int)kk; i += kFinThreads) out[i] = 0;
  for (int i = threadIdx.x; i < (int)(sink + local); i += kFinThreads)
    out[kk + i] = (i < sink) ? (int64_t)i : (int64_t)(m - local + (i - sink));
}

// Exact top kk of the cnt distinct K64 values of src, sorted descending (score
// descending, index ascending), written to out, followed by the sink and local
// positions (the whole workgroup calls it).  cl: LDS scratch of kCandLds
// values; with stage set and cnt <= kCandLds the values are copied there first
// (src must not read cl then).
template <typename Src>
__device__ __forceinline__ void select_sorted(const Src &src, int64_t cnt, int64_t kk, int64_t m, int64_t sink,
                                              int64_t local, int64_t *out, uint64_t *cl, uint64_t *ss,
                                              RangeShared &sh, uint32_t &s_cnt, bool stage) {
  const int tid = threadIdx.x, lane = tid & 63;
  // the exact kk largest first (range selection), then sorted
  auto survivors = [&](const auto &sr) {
    const uint64_t thr = range_select(sr, cnt, (uint32_t)kk, sh);
    if (tid == 0) s_cnt = 0u;
    __syncthreads();
    sr.for_each([&](bool ok, uint64_t v) { lds_append(ok && v >= thr, v, &s_cnt, ss, (uint32_t)kMaxK, lane); });
  };
  if (stage && cnt <= kCandLds) {
    stage_lds(src, cl, (uint32_t)kCandLds, s_cnt);
    survivors(ArraySrc{cl, cnt});
  } else {
    survivors(src);
  }
  __syncthreads();
  const int nv = (int)min(min(s_cnt, (uint32_t)kMaxK), (uint32_t)kk);
  uint64_t v2[2];  // zero: padding (below every K64)
  v2[0] = tid < nv ? ss[tid] : 0ull;
  v2[1] = tid + kFinThreads < nv ? ss[tid + kFinThreads] : 0ull;
  __syncthreads();  // cl is the sort scratch from here
  int nlim = kWave;
  while (nlim < nv) nlim <<= 1;  // the survivors fill the first nv <= 2048 slots
  const int got = nv < (int)kk ? nv : (int)kk;
  // only the survivors are ranked and written
  bin_rank_desc<2>(v2, nv, cl, sh, nlim, [&](int rank, uint64_t x) {
    if (rank < got) out[rank] = (int64_t)(0xFFFFFFFFu - (uint32_t)x);
  });
  write_fixed(out, got, kk, m, sink, local);
}

// Exact top kk of a row's candidates (list layout): those of the first pass,
// or, where it found fewer than kk, those of the fallback pass (which ran for
// exactly such rows); counts in the row counters.
__global__ __launch_bounds__(kFinThreads) void finalize_kernel(int64_t m, int64_t k, int64_t sink, int64_t local,
                                                               TopkSel s, int64_t *__restrict__ idx) {
  __shared__ uint64_t cl[kCandLds];
  __shared__ uint64_t ss[kMaxK];
  __shared__ RangeShared sh;
  __shared__ uint32_t s_cnt;
  const int64_t row = blockIdx.x;
  const int64_t kk = k - sink - local;
  const uint64_t *gc = s.cand + row * s.cand_cap;
  int64_t *out = idx + row * k;
  const uint32_t c1 = *s.cnt1(row);
  const int64_t cnt = min((int64_t)(c1 >= s.kk ? c1 : *s.cnt2(row)), s.cand_cap);
  select_sorted(ArraySrc{gc, cnt}, cnt, kk, m, sink, local, out, cl, ss, sh, s_cnt, true);
}

// The fallback of the fused scan + top-k, run by the finalize workgroup of a
// row whose candidate pass found fewer than kk candidates: the row (head h of
// bh) is rescanned with T_lo into the regions under the second count array by
// the workgroup's first waves, with the scan's plan tables in tsh (LDS that the
// caller frees for it).  The rescan computes the scores of the candidate pass
// bit for bit (the same chain of matrix instructions per token).
__device__ __forceinline__ void rescan_row(const sc::ScanArgs &a, const sc::Emit &em, int64_t bh, int h,
                                           sc::Shared &tsh) {
  sc::plan_tables(tsh, a, bh, sc::kGS * sc::kSlice);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (wave < sc::kWaves) {
    const int64_t nlist = em.sel.nreg > a.nwt ? em.sel.nreg : a.nwt;
    const uint32_t skipm = ((1u << a.G) - 1u) & ~(1u << h);
    sc::tile_pass<sc::kEmitFilter, 1, true, sc::kGS>(a, em, tsh, bh, lane, wave, sc::kWaves, nlist, 0, sc::kQS, skipm);
    __builtin_amdgcn_s_setprio(0);
  }
  // the rescan's region counts and candidates are read back by other waves of
  // the workgroup, and their old values may sit in the CU's L1: write back and
  // invalidate before the barrier
  __threadfence();
  __syncthreads();
}

// Exact top kk of a row of the fused scan + top-k from its candidate regions
// (row = bh * G + h), copied to LDS while they are counted; a row with more
// than kCandLds candidates is selected from its regions in place.  A row with
// fewer than kk first-pass candidates is rescanned first (rescan_row).
__global__ __launch_bounds__(kFinThreads) void finalize_fused_kernel(int64_t m, int64_t k, int64_t sink, int64_t local,
                                                                     sc::ScanArgs a, sc::Emit em,
                                                                     int64_t *__restrict__ idx) {
  __shared__ uint64_t cl[kCandLds];
  __shared__ uint64_t ss[kMaxK];
  __shared__ RangeShared sh;
  __shared__ uint32_t s_cnt;
  static_assert(sizeof(sc::Shared) <= sizeof(cl), "the rescan's plan tables fit the candidate buffer");
  const TopkSel &s = em.sel;
  const int64_t row = blockIdx.x;
  const int64_t kk = k - sink - local;
  const uint64_t *gc = s.cand + row * s.cand_cap;
  int64_t *out = idx + row * k;
  uint32_t *pre = reinterpret_cast<uint32_t *>(ss);  // free until the survivors are collected
  RegionSrc src{s.rc1 + row * s.nreg, gc, s.nreg};
  uint32_t cnt = stage_regions(src.rc, gc, s.nreg, cl, (uint32_t)kCandLds, pre, sh);
  if (cnt < s.kk) {  // uniform
    __syncthreads();  // cl holds the plan tables from here
    rescan_row(a, em, row / a.G, (int)(row % a.G), *reinterpret_cast<sc::Shared *>(cl));
    src.rc = s.rc2 + row * s.nreg;
    cnt = stage_regions(src.rc, gc, s.nreg, cl, (uint32_t)kCandLds, pre, sh);
  }
  if (cnt <= (uint32_t)(4 * kFinThreads)) {  // uniform
    // every candidate ranked at once (a few times kk of them): the top kk by
    // rank, written in order
    uint64_t v4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t i = threadIdx.x + (uint32_t)e * kFinThreads;
      v4[e] = i < cnt ? cl[i] : 0ull;
    }
    __syncthreads();  // cl is the ranking scratch from here
    int nlim = kWave;
    while (nlim < (int)cnt) nlim <<= 1;
    const int got = (int64_t)cnt < kk ? (int)cnt : (int)kk;
    bin_rank_desc<4>(v4, (int)cnt, cl, sh, nlim, [&](int rank, uint64_t x) {
      if (rank < got) out[rank] = (int64_t)(0xFFFFFFFFu - (uint32_t)x);
    });
    write_fixed(out, got, kk, m, sink, local);
  } else if (cnt <= (uint32_t)kCandLds) {
    select_sorted(ArraySrc{cl, (int64_t)cnt}, cnt, kk, m, sink, local, out, cl, ss, sh, s_cnt, false);
  } else {
    select_sorted(src, cnt, kk, m, sink, local, out, cl, ss, sh, s_cnt, false);
  }
}

// Exact top kk of a whole score row (rows up to kRowSelectMax): every element
// is a candidate.  Rows up to 2 * kCandLds keep their 32-bit keys in LDS (all
// of a thread's loads in flight together; the K64 of element i is rebuilt from
// its key and index).  For kk <= 1024 a prefilter keeps the selection small:
// the maxima of P >= kk interleaved groups of keys are ranked, the kk-th of
// them, T, bounds the row's kk-th largest key from below (kk elements reach
// it), and only the keys >= T (a few per cent of a row) are selected from --
// unless more than kMaxK reach it (ties, clustered rows), when the whole row
// is.  Longer rows are read from global memory.
__global__ __launch_bounds__(kFinThreads) void rowselect_kernel(const float *__restrict__ scores, int64_t n, int64_t m,
                                                                int64_t k, int64_t sink, int64_t local,
                                                                int64_t *__restrict__ idx) {
  constexpr int kLoad = 2 * kCandLds / kFinThreads;  // keys per thread
  __shared__ uint64_t cl[kCandLds];
  __shared__ uint64_t ss[kMaxK];
  __shared__ RangeShared sh;
  __shared__ uint32_t s_cnt;
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t row = blockIdx.x;
  const float *rs = scores + row * n;
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  const int64_t kk = k - sink - local;
  int64_t *out = idx + row * k;
  if (n > 2 * kCandLds) {
    const auto src = index_src([&](int64_t i) { return k64_of(masked_key(rs, i, sink, lstart), i); }, n);
    select_sorted(src, n, kk, m, sink, local, out, cl, ss, sh, s_cnt, true);
    return;
  }
  uint32_t *kl = reinterpret_cast<uint32_t *>(cl);
  uint32_t key[kLoad];  // the thread's keys t + 1024 u stay in registers
  {
    float v[kLoad];
#pragma unroll
    for (int u = 0; u < kLoad; ++u) {
      const int64_t i = tid + (int64_t)u * kFinThreads;
      v[u] = i < n ? rs[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kLoad; ++u) {
      const int64_t i = tid + (int64_t)u * kFinThreads;
      key[u] = i < n ? ((i < sink || i >= lstart) ? kKeyNegInf : score_key(v[u])) : 0u;
      if (i < n) kl[i] = key[u];
    }
  }
  __syncthreads();
  auto whole = [&]() {
    const auto src = index_src([&](int64_t i) { return ((uint64_t)kl[i] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i); }, n);
    select_sorted(src, n, kk, m, sink, local, out, cl, ss, sh, s_cnt, false);
  };
  if (kk > kFinThreads || n <= kMaxK) {
    whole();
    return;
  }
  // group maxima: thread t covers keys t + 1024 u; group s < P combines the
  // threads s, s + P, ... (keys i with i mod P == s); padding keys are 0
  int P = kWave;
  while (P < (int)kk) P <<= 1;
  uint32_t mk = 0u;
#pragma unroll
  for (int u = 0; u < kLoad; ++u) mk = max(mk, key[u]);
  sh.hist[tid] = mk;
  __syncthreads();
  uint32_t gm = 0u;
  if (tid < P)
    for (int j = tid; j < kFinThreads; j += P) gm = max(gm, sh.hist[j]);
  const uint64_t wg[1] = {((uint64_t)gm << 32) | (uint32_t)(tid + 1)};
  block_rank_desc<1>(wg, ss, ss + kFinThreads, P, [&](int rank, uint64_t x) {
    if (rank == (int)kk - 1) sh.lo = x;
  });
  __syncthreads();
  const uint32_t T = (uint32_t)(sh.lo >> 32);
  // the keys >= T: counted per thread, a workgroup prefix sum places them
  uint32_t c = 0u;
#pragma unroll
  for (int u = 0; u < kLoad; ++u) c += (tid + (int64_t)u * kFinThreads < n && key[u] >= T) ? 1u : 0u;
  const int wave = tid >> 6, nw = kFinThreads >> 6;
  const uint32_t wi = wave_incl_scan_u32(c);
  if (lane == kWave - 1) sh.wsum[wave] = wi;
  __syncthreads();
  uint32_t off = wi - c, cnt = 0u;
  for (int w = 0; w < nw; ++w) {
    const uint32_t ws = sh.wsum[w];
    off += w < wave ? ws : 0u;
    cnt += ws;
  }
  if (cnt > (uint32_t)kMaxK) {  // uniform
    whole();
    return;
  }
#pragma unroll
  for (int u = 0; u < kLoad; ++u) {
    const int64_t i = tid + (int64_t)u * kFinThreads;
    if (i < n && key[u] >= T) ss[off++] = ((uint64_t)key[u] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
  }
  __syncthreads();
  // the candidates are in ss and the keys are no longer needed: survivors go to
  // cl, the sort works in cl + 2 * kMaxK
  select_sorted(ArraySrc{ss, (int64_t)cnt}, cnt, kk, m, sink, local, out, cl + 2 * kMaxK, cl, sh, s_cnt, false);
}

// Wave-wide minimum and maximum of 32-bit values (in every lane): DPP row
// reductions, then the four rows' results read out.
template <int CTL>
__device__ __forceinline__ void minmax_dpp(uint32_t &mn, uint32_t &mx) {
  mn = min(mn, (uint32_t)__builtin_amdgcn_mov_dpp((int)mn, CTL, 0xF, 0xF, false));
  mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, CTL, 0xF, 0xF, false));
}
__device__ __forceinline__ void wave_minmax_u32(uint32_t &mn, uint32_t &mx) {
  minmax_dpp<0xB1>(mn, mx);   // quad_perm [1,0,3,2]
  minmax_dpp<0x4E>(mn, mx);   // quad_perm [2,3,0,1]
  minmax_dpp<0x141>(mn, mx);  // row_half_mirror
  minmax_dpp<0x140>(mn, mx);  // row_mirror
  mn = min(min((uint32_t)__builtin_amdgcn_readlane((int)mn, 0), (uint32_t)__builtin_amdgcn_readlane((int)mn, 16)),
           min((uint32_t)__builtin_amdgcn_readlane((int)mn, 32), (uint32_t)__builtin_amdgcn_readlane((int)mn, 48)));
  mx = max(max((uint32_t)__builtin_amdgcn_readlane((int)mx, 0), (uint32_t)__builtin_amdgcn_readlane((int)mx, 16)),
           max((uint32_t)__builtin_amdgcn_readlane((int)mx, 32), (uint32_t)__builtin_amdgcn_readlane((int)mx, 48)));
}

// Histogram round of kth_bound: the values v with (v - base) >> sh_in == bin_in
// (all when sh_in < 0) counted into 2048 bins of (v - base) >> sft; sets
// sh.hsel to the bin holding the need-th largest of them and sh.need to the
// count of those above it.
template <int PER>
__device__ __forceinline__ void bound_round(const uint32_t (&v)[PER], int cnt, uint32_t need, uint32_t base, int sft,
                                            int sh_in, uint32_t bin_in, RangeShared &sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (tid + u * kFinThreads < cnt && v[u] >= base && (sh_in < 0 || ((v[u] - base) >> sh_in) == bin_in))
      atomicAdd(&sh.hist[(v[u] - base) >> sft], 1u);
  __syncthreads();
  // running counts from the top bin down: thread t holds bins 2047 - 2t, 2046 - 2t
  const uint32_t c0 = sh.hist[kBins - 1 - 2 * tid], c1 = sh.hist[kBins - 2 - 2 * tid], c = c0 + c1;
  const uint32_t wi = wave_incl_scan_u32(c);
  if (lane == kWave - 1) sh.wsum[wave] = wi;
  __syncthreads();
  uint32_t above = wi - c;
  for (int w = 0; w < wave; ++w) above += sh.wsum[w];
  if (above < need && above + c0 >= need) {
    sh.hsel = (uint32_t)(kBins - 1 - 2 * tid);
    sh.need = above;
    sh.hcnt = c0;
  }
  if (above + c0 < need && above + c >= need) {
    sh.hsel = (uint32_t)(kBins - 2 - 2 * tid);
    sh.need = above + c0;
    sh.hcnt = c1;
  }
  sh.hist[tid] = 0u;  // for the next round
  sh.hist[tid + kFinThreads] = 0u;
  __syncthreads();
}

// A lower bound of the need-th largest of the cnt values v (thread t holds
// values t + 1024 u; need <= cnt).  The values at or below kKeyNegInf (group
// maxima of masked positions) are left out of the range: with fewer than need
// values above it the bound is 0.  A 2048-bin histogram over [min, max] of the
// others gives the bin that holds the need-th largest; its lower edge is the
// bound when at most kBoundFine values share the bin (a few extra candidates),
// else one more round over that bin refines it to within (max - min) / 2^22.
constexpr uint32_t kBoundFine = 32;
template <int PER>
__device__ __forceinline__ uint32_t kth_bound(const uint32_t (&v)[PER], int cnt, uint32_t need, RangeShared &sh) {
  static_assert(kBins == 2 * kFinThreads, "two bins per thread");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = kFinThreads >> 6;
  uint32_t mn = ~0u, mx = 0u, nv = 0u;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const bool on = tid + u * kFinThreads < cnt && v[u] > kKeyNegInf;
    if (on) {
      mn = min(mn, v[u]);
      mx = max(mx, v[u]);
    }
    nv += (uint32_t)__popcll(__ballot(on));
  }
  wave_minmax_u32(mn, mx);
  if (lane == 0) {
    sh.wmin[wave] = mn;
    sh.wmax[wave] = ((uint64_t)nv << 32) | mx;  // the wave's count beside its maximum
  }
  sh.hist[tid] = 0u;
  sh.hist[tid + kFinThreads] = 0u;
  __syncthreads();
  uint32_t lo = ~0u, hi = 0u, nvalid = 0u;
  for (int w = 0; w < nw; ++w) {
    lo = min(lo, (uint32_t)sh.wmin[w]);
    hi = max(hi, (uint32_t)sh.wmax[w]);
    nvalid += (uint32_t)(sh.wmax[w] >> 32);
  }
  if (nvalid < need) return 0u;  // uniform
  const uint32_t R = hi - lo;
  const int bl = R ? 32 - __clz((int)R) : 0;
  const int sft = bl > 11 ? bl - 11 : 0;  // (v - lo) >> sft < 2048
  bound_round<PER>(v, cnt, need, lo, sft, -1, 0u, sh);
  const uint32_t b = sh.hsel, base = lo + (b << sft);
  if (sft == 0 || sh.hcnt <= kBoundFine) return base;  // uniform
  const int sft2 = sft > 11 ? sft - 11 : 0;
  const uint32_t need2 = need - sh.need;
  __syncthreads();  // every thread has read sh.hsel, sh.need and sh.hcnt
  bound_round<PER>(v, cnt, need2, base, sft2, sft, 0u, sh);
  return base + (sh.hsel << sft2);
}

// Histogram scan of a round of two_bounds: bins counted from the top; for
// each of the two ranks, the bin that holds it and the count above that bin.
__device__ __forceinline__ void two_bins(const uint32_t *hist, uint32_t na, uint32_t nb, RangeShared &sh,
                                         uint32_t (&sel)[2], uint32_t (&above_sel)[2], uint32_t *s_sel) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t c0 = hist[kBins - 1 - 2 * tid], c1 = hist[kBins - 2 - 2 * tid], c = c0 + c1;
  const uint32_t wi = wave_incl_scan_u32(c);
  if (lane == kWave - 1) sh.wsum[wave] = wi;
  __syncthreads();
  uint32_t above = wi - c;
  for (int w = 0; w < wave; ++w) above += sh.wsum[w];
  const uint32_t need[2] = {na, nb};
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (above < need[r] && above + c0 >= need[r]) {
      s_sel[2 * r] = (uint32_t)(kBins - 1 - 2 * tid);
      s_sel[2 * r + 1] = above;
    }
    if (above + c0 < need[r] && above + c >= need[r]) {
      s_sel[2 * r] = (uint32_t)(kBins - 2 - 2 * tid);
      s_sel[2 * r + 1] = above + c0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    sel[r] = s_sel[2 * r];
    above_sel[r] = s_sel[2 * r + 1];
  }
}

// Lower bounds of the na-th and the nb-th largest of the cnt values v (thread
// t holds values t + 1024 u; nb, na <= cnt) in two histogram rounds shared by
// both ranks: 2048 bins over [min, max], then 2048 bins over each rank's bin
// (the second histogram in hist2).  Each bound is the lower edge of the final
// bin that holds its rank: at least that many values reach it, and it lies
// within (max - min) / 2^22 of the value of that rank.  Only values >= floor
// take part (floor must not exceed the na-th largest value: the ranks are the
// same among them), so a floor near the ranks keeps the bins narrow and the
// histogram atomics few.
template <int PER>
__device__ __forceinline__ void two_bounds(const uint32_t (&v)[PER], int cnt, uint32_t na, uint32_t nb,
                                           RangeShared &sh, uint32_t *hist2, uint32_t *s_sel, uint32_t &ta,
                                           uint32_t &tb, uint32_t floor = 0u, bool coarse_ok = false) {
  static_assert(kBins == 2 * kFinThreads, "two bins per thread");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = kFinThreads >> 6;
  uint32_t mn = ~0u, mx = 0u, nv = 0u;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const bool on = tid + u * kFinThreads < cnt && v[u] >= floor;
    if (on) {
      mn = min(mn, v[u]);
      mx = max(mx, v[u]);
    }
    nv += (uint32_t)__popcll(__ballot(on));
  }
  wave_minmax_u32(mn, mx);
  if (lane == 0) {
    sh.wmin[wave] = mn;
    sh.wmax[wave] = ((uint64_t)nv << 32) | mx;  // the wave's count beside its maximum
  }
  sh.hist[tid] = sh.hist[tid + kFinThreads] = 0u;
  hist2[tid] = hist2[tid + kFinThreads] = 0u;
  __syncthreads();
  uint32_t lo = ~0u, hi = 0u, nvalid = 0u;
  for (int w = 0; w < nw; ++w) {
    lo = min(lo, (uint32_t)sh.wmin[w]);
    hi = max(hi, (uint32_t)sh.wmax[w]);
    nvalid += (uint32_t)(sh.wmax[w] >> 32);
  }
  if (nvalid < na || nvalid < nb) {  // uniform: fewer values at or above floor than a rank
    ta = tb = 0u;
    return;
  }
  const uint32_t R = hi - lo;
  const int bl = R ? 32 - __clz((int)R) : 0;
  const int sft = bl > 11 ? bl - 11 : 0;  // (v - lo) >> sft < 2048
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (tid + u * kFinThreads < cnt && v[u] >= floor) atomicAdd(&sh.hist[(v[u] - lo) >> sft], 1u);
  __syncthreads();
  uint32_t sel[2], above[2];
  two_bins(sh.hist, na, nb, sh, sel, above, s_sel);
  const uint32_t base_a = lo + (sel[0] << sft), base_b = lo + (sel[1] << sft);
  bool coarse = false;
  if (coarse_ok) {  // uniform: both bins hold at most kBoundFine values
    coarse = sh.hist[sel[0]] <= kBoundFine && sh.hist[sel[1]] <= kBoundFine;
    __syncthreads();  // every thread has read the counts before the clear below
  }
  // one value per bin: the bins' values are the ranks' values; coarse: the
  // bins' lower edges
  if (sft == 0 || coarse) {  // uniform
    ta = base_a;
    tb = base_b;
    return;
  }
  const int sft2 = sft > 11 ? sft - 11 : 0;
  sh.hist[tid] = sh.hist[tid + kFinThreads] = 0u;  // every thread has read both histograms (two_bins' barriers)
  __syncthreads();
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (tid + u * kFinThreads < cnt && v[u] >= floor) {
      const uint32_t b = (v[u] - lo) >> sft;
      if (b == sel[0]) atomicAdd(&sh.hist[(v[u] - base_a) >> sft2], 1u);
      if (b == sel[1]) atomicAdd(&hist2[(v[u] - base_b) >> sft2], 1u);
    }
  __syncthreads();
  uint32_t sa[2], aa[2], sb[2], ab[2];
  two_bins(sh.hist, na - above[0], na - above[0], sh, sa, aa, s_sel);
  two_bins(hist2, nb - above[1], nb - above[1], sh, sb, ab, s_sel);
  ta = base_a + (sa[0] << sft2);
  tb = base_b + (sb[0] << sft2);
}

// Thresholds of a row from its sampled keys (the row's samp_cap keys, PER per
// thread): T_lo a lower bound of the sample's kk-th largest key, T_hi one of
// its r_hi-th largest (r_hi <= kk, so T_hi >= T_lo up to the bounds' bins).
// The sample is a subset of the row, so T_lo never exceeds the row's kk-th
// largest: every element of the row's top kk has key >= T_lo.  Also clears
// the row's candidate counters (list layout; the region layout has none).
template <int PER>
__global__ __launch_bounds__(kSelThreads) void select_keys_kernel(const uint32_t *__restrict__ samp,
                                                                  int64_t samp_cap, uint32_t kk, uint32_t r_hi,
                                                                  TopkSel s) {
  static_assert(kSelThreads == kFinThreads, "the bounds use the finalize block size");
  __shared__ RangeShared sh;
  __shared__ uint32_t hist2[kBins];
  __shared__ uint32_t s_sel[4];
  const int64_t row = blockIdx.x;
  const uint32_t *src = samp + row * samp_cap;
  uint32_t v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t i = threadIdx.x + (int64_t)u * kSelThreads;
    v[u] = i < samp_cap ? src[i] : 0u;
  }
  uint32_t t_lo = 0u, t_hi = 0u;  // fewer samples than kk: every element is a candidate
  if (samp_cap >= (int64_t)kk) two_bounds<PER>(v, (int)samp_cap, kk, r_hi < kk ? r_hi : kk, sh, hist2, s_sel, t_lo, t_hi);
  if (threadIdx.x == 0) {
    s.thr[row] = r_hi < kk ? t_hi : t_lo;
    s.thr_lo[row] = t_lo;
    if (!s.rc1) {  // the list layout's filter passes append at these counters
      *s.cnt1(row) = 0u;
      *s.cnt2(row) = 0u;
    }
  }
}

// The same thresholds from the maxima of the sample's 16-key groups (thread t
// holds groups t + 1024 u): each maximum is a sampled key, so the kk-th
// largest maximum bounds the sample's kk-th largest key from below (T_lo stays
// safe), and T_hi only falls (more candidates) where a group holds several of
// the top r_hi keys -- rare when kk is at most a quarter of the groups, the
// launch's condition.  Ranks 16 times fewer values than select_keys_kernel.
// DIRECT: samp already holds group maxima (the fused scan's sample, samp_cap
// of them per row), ranked as they are.
template <int PER, bool DIRECT>
__global__ __launch_bounds__(kSelThreads) void select_groups_kernel(const uint32_t *__restrict__ samp,
                                                                    int64_t samp_cap, uint32_t kk, uint32_t r_hi,
                                                                    TopkSel s) {
  __shared__ RangeShared sh;
  __shared__ uint32_t hist2[kBins];
  __shared__ uint32_t s_sel[4];
  const int64_t row = blockIdx.x;
  const int ng = (int)(DIRECT ? samp_cap : samp_cap / 16);
  uint32_t g[PER];
  if constexpr (DIRECT) {
    const uint32_t *src = samp + row * samp_cap;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = (int)threadIdx.x + u * kSelThreads;
      g[u] = i < ng ? src[i] : 0u;
    }
  } else {
    const uint4 *src = reinterpret_cast<const uint4 *>(samp + row * samp_cap);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = (int)threadIdx.x + u * kSelThreads;
      uint4 q[4] = {};
      if (i < ng) {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = src[4 * i + j];
      }
      uint32_t m = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) m = max(m, max(max(q[j].x, q[j].y), max(q[j].z, q[j].w)));
      g[u] = m;
    }
  }
  uint32_t t_lo = 0u, t_hi = 0u;  // fewer values than kk: every element is a candidate
  // the range leaves out the groups of masked positions (keys at or below
  // -inf); lower bounds from one round where the ranks' bins are sparse
  if (ng >= (int)kk && kk > 0)
    two_bounds<PER>(g, ng, kk, r_hi < kk ? r_hi : kk, sh, hist2, s_sel, t_lo, t_hi, kKeyNegInf + 1u, true);
  if (threadIdx.x == 0) {
    s.thr[row] = r_hi < kk ? t_hi : t_lo;
    s.thr_lo[row] = t_lo;
    if (!s.rc1) {
      *s.cnt1(row) = 0u;
      *s.cnt2(row) = 0u;
    }
  }
}

// Exact top kk of short score rows whose 16-token group maxima the scan
// wrote beside them (gmax [rows, ceil(n / 16)]: the largest masked key of each
// group).  T, a lower bound of the kk-th largest group maximum, bounds the
// row's kk-th largest key from below (kk groups each hold a key >= T), and
// every key >= T lies in a group whose maximum is >= T: only those groups'
// scores are read, and their keys >= T are the candidates (a little over kk
// for spread scores).  Up to 2048 candidates are ranked by one sort; more are
// selected first; rows whose candidates outgrow the LDS list (ties around T)
// are selected from the whole row.
constexpr int kGmaxGroups = (int)(kRowSelectMax / kGroupTok);
// ranked (LDS of k int32, past the sort's scratch in cl; null: none): rows of
// at most 2048 candidates also leave their k output tokens there, and the
// call returns true.
__device__ __forceinline__ bool rowselect_gmax_row(const float *__restrict__ scores, const uint32_t *__restrict__ gmax,
                                                   int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local,
                                                   int64_t *__restrict__ idx, uint64_t *cl, uint64_t *ss,
                                                   RangeShared &sh, uint16_t *glist, uint32_t &s_cnt,
                                                   int32_t *ranked = nullptr) {
  constexpr int kPer = kGmaxGroups / kFinThreads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = kFinThreads >> 6;
  const int64_t row = blockIdx.x;
  const float *rs = scores + row * n;
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  const int64_t kk = k - sink - local;
  const int ngrp = (int)cdiv(n, kGroupTok);
  int64_t *out = idx + row * k;
  uint32_t gm[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int g = tid + u * kFinThreads;
    gm[u] = g < ngrp ? gmax[row * ngrp + g] : 0u;
  }
  const uint32_t T = ngrp > kk ? kth_bound<kPer>(gm, ngrp, (uint32_t)kk, sh) : 0u;
  // the groups reaching T, listed in order
  uint32_t ngr = 0u;
  {
    uint32_t c = 0u;
#pragma unroll
    for (int u = 0; u < kPer; ++u) c += (tid + u * kFinThreads < ngrp && gm[u] >= T) ? 1u : 0u;
    const uint32_t wi = wave_incl_scan_u32(c);
    if (lane == kWave - 1) sh.wsum[wave] = wi;
    __syncthreads();
    uint32_t off = wi - c;
    for (int w = 0; w < nw; ++w) {
      const uint32_t ws = sh.wsum[w];
      off += w < wave ? ws : 0u;
      ngr += ws;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int g = tid + u * kFinThreads;
      if (g < ngrp && gm[u] >= T) glist[off++] = (uint16_t)g;
    }
    __syncthreads();
  }
  // their keys >= T, one group per thread, placed by a workgroup prefix sum
  uint32_t cnt = 0u;
  for (uint32_t e0 = 0; e0 < ngr; e0 += kFinThreads) {  // uniform
    const uint32_t e = e0 + tid;
    const int64_t t0 = e < ngr ? (int64_t)glist[e] * kGroupTok : n;
    float v[kGroupTok];
    if (t0 + kGroupTok <= n && (n & 3) == 0) {
#pragma unroll
      for (int r = 0; r < kGroupTok; r += 4) {
        const float4 f = *reinterpret_cast<const float4 *>(rs + t0 + r);
        v[r] = f.x;
        v[r + 1] = f.y;
        v[r + 2] = f.z;
        v[r + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int r = 0; r < kGroupTok; ++r) v[r] = t0 + r < n ? rs[t0 + r] : 0.0f;
    }
    uint32_t key[kGroupTok], c = 0u;
#pragma unroll
    for (int r = 0; r < kGroupTok; ++r) {
      const int64_t i = t0 + r;
      key[r] = (i < sink || i >= lstart) ? kKeyNegInf : score_key(v[r]);
      c += (i < n && key[r] >= T) ? 1u : 0u;
    }
    const uint32_t wi = wave_incl_scan_u32(c);
    if (lane == kWave - 1) sh.wsum[wave] = wi;
    __syncthreads();
    uint32_t off = cnt + wi - c;
    for (int w = 0; w < nw; ++w) {
      const uint32_t ws = sh.wsum[w];
      off += w < wave ? ws : 0u;
      cnt += ws;
    }
#pragma unroll
    for (int r = 0; r < kGroupTok; ++r) {
      const int64_t i = t0 + r;
      if (i < n && key[r] >= T) {
        if (off < (uint32_t)kCandLds) cl[off] = k64_of(key[r], i);
        ++off;
      }
    }
    __syncthreads();  // sh.wsum is rewritten by the next step
  }
  if (cnt > (uint32_t)kCandLds) {  // uniform: ties around T
    const auto src = index_src([&](int64_t i) { return k64_of(masked_key(rs, i, sink, lstart), i); }, n);
    select_sorted(src, n, kk, m, sink, local, out, cl, ss, sh, s_cnt, true);
    return false;
  }
  if (cnt > (uint32_t)(2 * kFinThreads)) {
    select_sorted(ArraySrc{cl, (int64_t)cnt}, cnt, kk, m, sink, local, out, cl, ss, sh, s_cnt, false);
    return false;
  }
  // at most 2048 candidates: one sort ranks them, the first kk are written
  uint64_t v2[2];
  v2[0] = (uint32_t)tid < cnt ? cl[tid] : 0ull;  // zero: padding (below every K64)
  v2[1] = (uint32_t)(tid + kFinThreads) < cnt ? cl[tid + kFinThreads] : 0ull;
  __syncthreads();  // cl is the sort scratch from here
  int nlim = kWave;
  while (nlim < (int)cnt) nlim <<= 1;
  const int got = (int64_t)cnt < kk ? (int)cnt : (int)kk;
  bin_rank_desc<2>(v2, (int)cnt, cl, sh, nlim, [&](int rank, uint64_t x) {
    if (rank < got) {
      const uint32_t tok = 0xFFFFFFFFu - (uint32_t)x;
      out[rank] = (int64_t)tok;
      if (ranked) ranked[rank] = (int32_t)tok;
    }
  });
  write_fixed(out, got, kk, m, sink, local);
  if (ranked) {  // the same tokens as write_fixed's
    for (int i = got + tid; i < (int)kk; i += kFinThreads) ranked[i] = 0;
    for (int i = tid; i < (int)(sink + local); i += kFinThreads)
      ranked[kk + i] = (int32_t)((i < sink) ? (int64_t)i : (m - local + (i - sink)));
  }
  return ranked != nullptr;
}

// The selection of rowselect_gmax_row, one workgroup per row.  ATTN (the
// decode step's selection + attention, k <= 512, rows in device memory): the
// workgroup then runs the attention of its query head over the k indices it
// wrote, exactly as gather_attention's attn_stream_kernel does for one split
// (16 waves of 32 positions), so out equals gather_attention's output.
struct RowAttn {
  const float *q;  // [rows, D] fp32 query heads (row = bh * G + g)
  int64_t G;
  attn::RowSrc rs;
  float scale;
  float *out;      // [rows, D] fp32
};
template <bool ATTN>
__global__ __launch_bounds__(kFinThreads) void rowselect_gmax_kernel(const float *__restrict__ scores,
                                                                     const uint32_t *__restrict__ gmax, int64_t n,
                                                                     int64_t m, int64_t k, int64_t sink, int64_t local,
                                                                     int64_t *__restrict__ idx, RowAttn ra) {
  __shared__ uint64_t cl[kCandLds];
  __shared__ uint64_t ss[kMaxK];
  __shared__ RangeShared sh;
  __shared__ uint16_t glist[kGmaxGroups];
  __shared__ uint32_t s_cnt;
  // ATTN: the ranked tokens also in LDS, in cl's upper half (past the sort's
  // scratch and the attention's triples)
  int32_t *ranked = ATTN ? reinterpret_cast<int32_t *>(cl + kCandLds / 2) : nullptr;
  static_assert(kCandLds / 2 >= 2 * 2 * kFinThreads + kBins && 2 * (kCandLds / 2) >= kMaxK + kFinThreads,
                "the ranked tokens lie past the sort's scratch and hold k of them");
  const bool in_lds = rowselect_gmax_row(scores, gmax, n, m, k, sink, local, idx, cl, ss, sh, glist, s_cnt, ranked);
  if constexpr (ATTN) {
    constexpr int NW = kFinThreads / kWave;
    static_assert(NW == 16, "one attention split of 16 waves");
    static_assert(sizeof(float) * (2 * NW + NW * attn::kAttnD) <= sizeof(uint64_t) * (kCandLds / 2),
                  "the attention's LDS in cl's lower half");
    __syncthreads();  // the row's indices are written (and cl's lower half is free)
    const int64_t row = blockIdx.x, bh = row / ra.G;
    const int64_t *ig = idx + row * k;
    float *wm = reinterpret_cast<float *>(cl), *wl = wm + NW;
    auto wo = reinterpret_cast<float(*)[attn::kAttnD]>(wl + NW);
    const float *qr = ra.q + row * attn::kAttnD;
    float *orow = ra.out + row * attn::kAttnD;
    if (in_lds)  // uniform: the tokens from LDS, else from the index list just written
      attn::attn_stream_block<NW, false>(qr, [&](int64_t j) { return (int64_t)ranked[j]; }, k, 0, bh, ra.rs, ra.scale,
                                         wm, wl, wo, orow, nullptr, true);
    else
      attn::attn_stream_block<NW, false>(qr, [&](int64_t j) { return ig[j]; }, k, 0, bh, ra.rs, ra.scale, wm, wl, wo,
                                         orow, nullptr, true);
  }
}

// The wide selection's kk <= 8192 values of a row (sel [rows, P], all
// distinct) ranked by one counting sort and written as the row's indices, then
// the sink and local positions.
template <int E>
__global__ __launch_bounds__(kFinThreads) void rank_list_kernel(const uint64_t *__restrict__ sel, int64_t P, int64_t kk,
                                                               int64_t m, int64_t k, int64_t sink, int64_t local,
                                                               int64_t *__restrict__ idx) {
  __shared__ uint64_t cl[kCandLds];
  __shared__ RangeShared sh;
  static_assert(E * kFinThreads + kBins <= kCandLds, "the sort's scratch");
  const int64_t row = blockIdx.x;
  const uint64_t *src = sel + row * P;
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int64_t i = threadIdx.x + e * kFinThreads;
    v[e] = i < kk ? src[i] : 0ull;
  }
  int nlim = kWave;
  while (nlim < (int)kk) nlim <<= 1;
  int64_t *out = idx + row * k;
  bin_rank_desc<E>(v, (int)kk, cl, sh, nlim,
                   [&](int rank, uint64_t x) { out[rank] = (int64_t)(0xFFFFFFFFu - (uint32_t)x); });
  write_fixed(out, (int)kk, kk, m, sink, local);
}

__global__ __launch_bounds__(256) void fixed_only_kernel(int64_t rows, int64_t m, int64_t k, int64_t sink,
                                                         int64_t local, int64_t *__restrict__ idx) {
  const int64_t total = rows * k;
  for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
    const int64_t i = o % k;
    idx[o] = (i < sink) ? i : (m - local + (i - sink));
  }
}

}  // namespace

size_t topk_sel_layout(int64_t rows, int64_t cand_cap, int64_t nreg, char *base, TopkSel *s) {
  const size_t row_b = ws_align((size_t)rows * 4);                // thr, thr_lo
  const size_t cnt_b = ws_align((size_t)rows * 4 * kCntStride);  // cand_cnt, cand2_cnt
  const size_t reg_b = nreg > 0 ? ws_align((size_t)rows * (size_t)nreg * 4) : 0;  // rc1, rc2
  const size_t cand_b = ws_align((size_t)rows * (size_t)cand_cap * 8);
  if (s) {
    char *p = base;
    s->thr = reinterpret_cast<uint32_t *>(p);
    s->thr_lo = reinterpret_cast<uint32_t *>(p += row_b);
    s->cand_cnt = reinterpret_cast<uint32_t *>(p += row_b);
    s->cand2_cnt = reinterpret_cast<uint32_t *>(p += cnt_b);
    s->rc1 = nreg > 0 ? reinterpret_cast<uint32_t *>(p + cnt_b) : nullptr;
    s->rc2 = nreg > 0 ? reinterpret_cast<uint32_t *>(p + cnt_b + reg_b) : nullptr;
    s->nreg = nreg > 0 ? nreg : 0;
    s->cand = reinterpret_cast<uint64_t *>(p + cnt_b + 2 * reg_b);
    s->cand_cap = cand_cap;
    s->kk = 0u;
  }
  return 2 * row_b + 2 * cnt_b + 2 * reg_b + cand_b;
}

size_t topk_layout(int64_t rows, int64_t n, int64_t k, bool regions, char *base, uint32_t **samp, int64_t *samp_cap,
                   TopkSel *sel, int64_t *S_out) {
  const int64_t kk = k > 0 ? k : 0;
  const int64_t tile = regions ? kRegTok : kTileTok;
  const int64_t S = topk_tile_stride(n, kk, tile);
  // the fused scan's sample holds each tile's 64 group maxima, the score-row
  // top-k's every sampled key
  const int64_t cap = topk_sample_tiles(n, S, tile) * (regions ? kRegTok / kGroupTok : tile);
  const size_t samp_b = ws_align((size_t)rows * (size_t)cap * 4);
  if (samp) *samp = reinterpret_cast<uint32_t *>(base);
  if (samp_cap) *samp_cap = cap;
  if (S_out) *S_out = S;
  const int64_t cand_cap = regions ? cdiv(n, 4 * kRegTok) * 4 * kRegTok : n;
  return samp_b + topk_sel_layout(rows, cand_cap, regions ? cand_cap / kRegTok : 0, base ? base + samp_b : nullptr, sel);
}

int launch_select_keys(const uint32_t *samp, int64_t rows, int64_t samp_cap, int64_t kk, int64_t r_hi, TopkSel s,
                       hipStream_t st) {
  if (samp_cap > kMaxSample) return fail(FATHOM_ERR_INVALID, "select: %lld sampled keys exceed %lld", (long long)samp_cap, (long long)kMaxSample);
  const unsigned g = (unsigned)rows;
  const uint32_t ukk = (uint32_t)kk, urh = (uint32_t)r_hi;
  const int64_t ng = samp_cap / 16;
  if (samp_cap % 16 == 0 && ng >= 4 * kk && kk > 0) {  // 16-key group maxima (see select_groups_kernel)
    if (ng <= kSelThreads)
      select_groups_kernel<1, false><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
    else if (ng <= 2 * kSelThreads)
      select_groups_kernel<2, false><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
    else
      select_groups_kernel<4, false><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
    return launch_status("select_groups_kernel");
  }
  if (samp_cap <= 8 * kSelThreads)
    select_keys_kernel<8><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
  else if (samp_cap <= 16 * kSelThreads)
    select_keys_kernel<16><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
  else if (samp_cap <= 32 * kSelThreads)
    select_keys_kernel<32><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
  else
    select_keys_kernel<kSelPer><<<g, kSelThreads, 0, st>>>(samp, samp_cap, ukk, urh, s);
  return launch_status("select_keys_kernel");
}

int launch_select_groups(const uint32_t *gmax, int64_t rows, int64_t ng, int64_t kk, int64_t r_hi, TopkSel s,
                         hipStream_t st) {
  if (ng > 4 * kSelThreads) return fail(FATHOM_ERR_INVALID, "select: %lld group maxima exceed %d", (long long)ng, 4 * kSelThreads);
  const unsigned g = (unsigned)rows;
  const uint32_t ukk = (uint32_t)kk, urh = (uint32_t)r_hi;
  if (ng <= kSelThreads)
    select_groups_kernel<1, true><<<g, kSelThreads, 0, st>>>(gmax, ng, ukk, urh, s);
  else if (ng <= 2 * kSelThreads)
    select_groups_kernel<2, true><<<g, kSelThreads, 0, st>>>(gmax, ng, ukk, urh, s);
  else
    select_groups_kernel<4, true><<<g, kSelThreads, 0, st>>>(gmax, ng, ukk, urh, s);
  return launch_status("select_groups_kernel");
}

int launch_sample_scores(const float *scores, int64_t rows, int64_t n, int64_t S, int64_t sink, int64_t lstart,
                         uint32_t *samp, int64_t samp_cap, hipStream_t st) {
  sample_scores_kernel<<<dim3((unsigned)(samp_cap / kTileTok), (unsigned)rows), 256, 0, st>>>(scores, n, S, sink,
                                                                                            lstart, samp, samp_cap);
  return launch_status("sample_scores_kernel");
}

int launch_filter_scores(const float *scores, int64_t rows, int64_t n, int64_t sink, int64_t lstart, TopkSel s,
                         bool fallback, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(n, kFilterChunk), (unsigned)rows);
  if (n % 4 == 0 && reinterpret_cast<uintptr_t>(scores) % 16 == 0)
    filter_scores_kernel<true><<<grid, kFilterThreads, 0, st>>>(scores, n, sink, lstart, s, fallback);
  else
    filter_scores_kernel<false><<<grid, kFilterThreads, 0, st>>>(scores, n, sink, lstart, s, fallback);
  return launch_status("filter_scores_kernel");
}

int launch_finalize(int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, TopkSel s, int64_t *idx,
                    hipStream_t st) {
  finalize_kernel<<<(unsigned)rows, kFinThreads, 0, st>>>(m, k, sink, local, s, idx);
  return launch_status("finalize_kernel");
}

int launch_finalize_fused(const sc::ScanArgs &a, const sc::Emit &em, int64_t rows, int64_t m, int64_t k, int64_t sink,
                          int64_t local, int64_t *idx, hipStream_t st) {
  finalize_fused_kernel<<<(unsigned)rows, kFinThreads, 0, st>>>(m, k, sink, local, a, em, idx);
  return launch_status("finalize_fused_kernel");
}

int launch_rowselect(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local,
                     int64_t *idx, hipStream_t st) {
  rowselect_kernel<<<(unsigned)rows, kFinThreads, 0, st>>>(scores, n, m, k, sink, local, idx);
  return launch_status("rowselect_kernel");
}

int launch_rowselect_gmax(const float *scores, const uint32_t *gmax, int64_t rows, int64_t n, int64_t m, int64_t k,
                          int64_t sink, int64_t local, int64_t *idx, hipStream_t st) {
  rowselect_gmax_kernel<false><<<(unsigned)rows, kFinThreads, 0, st>>>(scores, gmax, n, m, k, sink, local, idx, RowAttn{});
  return launch_status("rowselect_gmax_kernel");
}

int launch_rowselect_gmax_attn(const float *scores, const uint32_t *gmax, int64_t rows, int64_t n, int64_t m, int64_t k,
                               int64_t sink, int64_t local, int64_t *idx, const float *q, int64_t G, const void *K,
                               const void *V, int64_t cap, float scale, float *out, hipStream_t st) {
  if (k > kFinThreads / 2) return fail(FATHOM_ERR_INVALID, "rowselect_gmax_attn: k=%lld exceeds 512", (long long)k);
  RowAttn ra{q, G, attn::RowSrc{(const char *)K, (const char *)V, nullptr, nullptr, cap, 0, n, 2 * attn::kAttnD}, scale,
             out};
  rowselect_gmax_kernel<true><<<(unsigned)rows, kFinThreads, 0, st>>>(scores, gmax, n, m, k, sink, local, idx, ra);
  return launch_status("rowselect_gmax_kernel");
}

int launch_rank_list(const uint64_t *sel, int64_t P, int64_t rows, int64_t kk, int64_t m, int64_t k, int64_t sink,
                     int64_t local, int64_t *idx, hipStream_t st) {
  if (kk > kRankListMax) return fail(FATHOM_ERR_INVALID, "rank_list: kk=%lld exceeds %lld", (long long)kk, (long long)kRankListMax);
  if (kk <= 4 * kFinThreads)
    rank_list_kernel<4><<<(unsigned)rows, kFinThreads, 0, st>>>(sel, P, kk, m, k, sink, local, idx);
  else
    rank_list_kernel<8><<<(unsigned)rows, kFinThreads, 0, st>>>(sel, P, kk, m, k, sink, local, idx);
  return launch_status("rank_list_kernel");
}

int launch_fixed_only(int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, int64_t *idx, hipStream_t st) {
  if (k == 0) return FATHOM_OK;
  fixed_only_kernel<<<(unsigned)min(cdiv(rows * k, 256), (int64_t)65535), 256, 0, st>>>(rows, m, k, sink, local, idx);
  return launch_status("fixed_only_kernel");
}

size_t wide_topk_bytes(int64_t rows, int64_t n, int64_t k) {
  return topk_layout(rows, n, k, false, nullptr, nullptr, nullptr, nullptr, nullptr) +
         wide_select_bytes(rows, k < n ? k : n);
}

int wide_topk_run(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local,
                  int64_t *idx, void *workspace, size_t workspace_bytes, hipStream_t st) {
  const int64_t kk = k - sink - local;
  const size_t chain = topk_layout(rows, n, k, false, nullptr, nullptr, nullptr, nullptr, nullptr);
  const size_t need = chain + wide_select_bytes(rows, kk);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "top-k (kk=%lld): workspace %zu bytes, need %zu", (long long)kk, workspace_bytes,
                need);
  TopkSel s;
  uint32_t *samp = nullptr;
  int64_t samp_cap = 0, S = 1;
  topk_layout(rows, n, k, false, static_cast<char *>(workspace), &samp, &samp_cap, &s, &S);
  s.kk = (uint32_t)kk;
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  const int64_t r_hi = topk_hi_rank(n, S, kk, kTileTok);
  int rc = launch_sample_scores(scores, rows, n, S, sink, lstart, samp, samp_cap, st);
  if (rc) return rc;
  rc = launch_select_keys(samp, rows, samp_cap, kk, r_hi, s, st);
  if (rc) return rc;
  rc = launch_filter_scores(scores, rows, n, sink, lstart, s, false, st);
  if (rc) return rc;
  if (r_hi < kk) {  // rows whose first pass found fewer than kk take T_lo
    rc = launch_filter_scores(scores, rows, n, sink, lstart, s, true, st);
    if (rc) return rc;
  }
  return wide_select_list(s, rows, m, k, sink, local, idx, static_cast<char *>(workspace) + chain,
                          workspace_bytes - chain, st);
}

int check_topk_args(int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local, const char *who) {
  if (rows < 1 || rows > 65535) return fail(FATHOM_ERR_INVALID, "%s: rows=%lld outside [1, 65535]", who, (long long)rows);
  if (n < 1 || n > 0x7FFFFFFFLL) return fail(FATHOM_ERR_INVALID, "%s: n=%lld unsupported", who, (long long)n);
  if (sink < 0 || local < 0 || k < 0) return fail(FATHOM_ERR_INVALID, "%s: negative k/sink/local", who);
  const int64_t kk = k - sink - local;
  if (kk < 0) return fail(FATHOM_ERR_INVALID, "%s: k=%lld < sink+local=%lld", who, (long long)k, (long long)(sink + local));
  if (kk > n) return fail(FATHOM_ERR_INVALID, "%s: k - sink - local = %lld exceeds n=%lld", who, (long long)kk, (long long)n);
  if (sink > n || m < n || local > m)
    return fail(FATHOM_ERR_INVALID, "%s: need sink <= n <= m and local <= m (sink=%lld n=%lld m=%lld local=%lld)", who,
                (long long)sink, (long long)n, (long long)m, (long long)local);
  return FATHOM_OK;
}

}  // namespace fathom

using namespace fathom;

namespace fathom {
namespace {
// k bounds kk = k - sink - local from above: where kk may exceed kSelMaxK the
// chain's layout is followed by the wide selection's state.
size_t topk_ws(int64_t rows, int64_t n, int64_t k) {
  return k <= kSelMaxK ? topk_layout(rows, n, k, false, nullptr, nullptr, nullptr, nullptr, nullptr)
                       : wide_topk_bytes(rows, n, k);
}
}  // namespace
}  // namespace fathom

extern "C" size_t fathom_topk_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows < 1 || n < 1 || k < 0) return 0;
  return topk_ws(rows, n, k);
}

extern "C" int fathom_sink_local_topk(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k,
                                      int64_t sink, int64_t local, int64_t *idx, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  if (!scores || !idx) return fail(FATHOM_ERR_INVALID, "sink_local_topk: null pointer");
  int rc = check_topk_args(rows, n, m, k, sink, local, "sink_local_topk");
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int64_t kk = k - sink - local;
  if (kk == 0) return launch_fixed_only(rows, m, k, sink, local, idx, st);
  if (kk > kSelMaxK) return wide_topk_run(scores, rows, n, m, k, sink, local, idx, workspace, workspace_bytes, st);
  const size_t need = topk_layout(rows, n, k, false, nullptr, nullptr, nullptr, nullptr, nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "sink_local_topk: workspace %zu bytes, need %zu", workspace_bytes, need);
  TopkSel s;
  uint32_t *samp = nullptr;
  int64_t samp_cap = 0, S = 1;
  topk_layout(rows, n, k, false, static_cast<char *>(workspace), &samp, &samp_cap, &s, &S);
  s.kk = (uint32_t)kk;
  if (n <= kRowSelectMax) return launch_rowselect(scores, rows, n, m, k, sink, local, idx, st);
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  const int64_t r_hi = topk_hi_rank(n, S, kk, kTileTok);
  rc = launch_sample_scores(scores, rows, n, S, sink, lstart, samp, samp_cap, st);
  if (rc) return rc;
  rc = launch_select_keys(samp, rows, samp_cap, kk, r_hi, s, st);
  if (rc) return rc;
  rc = launch_filter_scores(scores, rows, n, sink, lstart, s, false, st);
  if (rc) return rc;
  if (r_hi < kk) {  // T_hi may exceed a row's kk-th largest key
    rc = launch_filter_scores(scores, rows, n, sink, lstart, s, true, st);
    if (rc) return rc;
  }
  return launch_finalize(rows, m, k, sink, local, s, idx, st);
}
