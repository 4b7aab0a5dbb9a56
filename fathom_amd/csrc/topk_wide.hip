// Top-kk of score rows for any kk up to n: the path of k - sink - local above
// the LDS-resident selections' limit (torch.topk has no limit,
// kernels/bitplane.py:372-378).  It runs over a row's candidate list from the
// sample -> select -> filter chain (which holds the row's top kk; about 2.5 kk
// values for spread scores).
//
// Every element of a row is the 64-bit value K64 = key << 32 | (2^32 - 1 - i)
// (distinct within a row; unsigned order = score descending, index ascending).
//   radix select  the exact kk-th largest K64 of each row, 11 + 11 + 10 bits of
//                 the key, then of the inverted index, one digit per round: a
//                 grid-wide histogram of the digit over the elements that match
//                 the bits fixed so far (LDS counts added to the row's global
//                 counts), then one workgroup per row picks the digit.  A round
//                 whose chosen bin holds exactly the remaining rank ends the
//                 row's search (the later rounds return at once): with float
//                 scores the key's three rounds usually suffice;
//   compaction    the kk elements with K64 >= the threshold, appended at a row
//                 counter (one atomic per wave);
//   sort          up to 8192 values: one counting sort per row (the LDS-resident
//                 selections' ranking); more: bitonic, descending, over the kk
//                 values padded with zeros to a power of two P: chunks of up to
//                 16384 values sorted in LDS, then for each merge size above
//                 that the steps of strides of at least a chunk in global
//                 memory and the rest in LDS;
//   output        indices of the sorted values, then the sink and local
//                 positions.
// Every launch is data-independent in shape, so the whole path can be captured
// in a graph.
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr int kWideThreads = 256;    // histogram / compaction workgroup
constexpr int kWidePer = 64;         // elements per thread of those passes
constexpr int64_t kWideChunk = (int64_t)kWideThreads * kWidePer;
constexpr int kWideBins = 2048;      // 11-bit digits
constexpr int kSortThreads = 1024;
constexpr int64_t kSortLds = 16384;  // values per LDS sort chunk (128 KiB)
constexpr int kRounds = 6;
// (shift, width) of the radix rounds, most significant first
constexpr int kShift[kRounds] = {53, 42, 32, 21, 10, 0};
constexpr int kWidth[kRounds] = {11, 11, 10, 11, 11, 10};

struct WideState {
  uint64_t *thr;   // [rows] bits fixed so far; the threshold once done
  uint32_t *rem;   // [rows] rank still to find among the matching elements
  uint32_t *done;  // [rows] 1: thr is the row's kk-th largest K64
  uint32_t *cnt;   // [rows * kCntStride] compaction counters
  uint32_t *hist;  // [rows, kWideBins] digit counts of the current round
  uint64_t *sel;   // [rows, P] selected values, then sorted
  int64_t P;
};

// The values a row's selection runs over: the K64 candidates of the sample ->
// select -> filter chain (list layout: the first pass's if it found kk, else
// the fallback pass's), which hold the row's top kk.
struct WideSrc {
  const uint64_t *cand;  // [rows, cand_cap]
  int64_t cand_cap;
  const uint32_t *cnt1, *cnt2;  // per row, kCntStride apart
  uint32_t kk;
  __device__ __forceinline__ int64_t count(int64_t row) const {
    const uint32_t c1 = cnt1[row * kCntStride];
    const int64_t c = c1 >= kk ? c1 : cnt2[row * kCntStride];
    return c < cand_cap ? c : cand_cap;
  }
  __device__ __forceinline__ uint64_t at(int64_t row, int64_t i) const { return cand[row * cand_cap + i]; }
};

__global__ __launch_bounds__(kWideThreads) void wide_init_kernel(WideState w, uint32_t kk) {
  const int64_t row = blockIdx.x;
  for (int b = threadIdx.x; b < kWideBins; b += kWideThreads) w.hist[row * kWideBins + b] = 0u;
  if (threadIdx.x == 0) {
    w.thr[row] = 0ull;
    w.rem[row] = kk;
    w.done[row] = 0u;
    w.cnt[row * kCntStride] = 0u;
  }
}

// Digit counts of the elements of one chunk of a row that match the fixed bits.
__global__ __launch_bounds__(kWideThreads) void wide_hist_kernel(WideSrc src, WideState w, int shift, int width) {
  const int64_t row = blockIdx.y;
  const int64_t n = src.count(row);
  const int64_t per = cdiv(n, (int64_t)gridDim.x);  // the row's values spread over the grid's workgroups
  const int64_t start = (int64_t)blockIdx.x * per;
  if (w.done[row] || start >= n) return;  // uniform
  __shared__ uint32_t h[kWideBins];
  const int tid = threadIdx.x;
  for (int b = tid; b < kWideBins; b += kWideThreads) h[b] = 0u;
  __syncthreads();
  const int top = shift + width;  // bits [top, 64) are fixed
  const uint64_t fixed = top < 64 ? (w.thr[row] >> top) : 0ull;
  const uint32_t dmask = (1u << width) - 1u;
  const int64_t end = start + per < n ? start + per : n;
  const int lane = tid & (kWave - 1), wave = tid >> 6;
  for (int64_t i0 = start + wave * kWave; i0 < end; i0 += kWideThreads) {  // wave-uniform trip count
    const int64_t i = i0 + lane;
    const uint64_t v = i < end ? src.at(row, i) : 0ull;
    const bool on = i < end && (top >= 64 || (v >> top) == fixed);
    const uint32_t dg = (uint32_t)(v >> shift) & dmask;
    // the lanes sharing the first counted lane's digit add with one atomic
    // (a row's values crowd into few bins), the others one by one
    const uint64_t mm = __ballot(on);
    if (mm == 0ull) continue;
    const int first = __ffsll((long long)mm) - 1;
    const uint32_t df = (uint32_t)__shfl((int)dg, first);
    const bool same = on && dg == df;
    const uint64_t ms = __ballot(same);
    if (lane == first) atomicAdd(&h[df], (uint32_t)__popcll(ms));
    if (on && !same) atomicAdd(&h[dg], 1u);
  }
  __syncthreads();
  uint32_t *gh = w.hist + row * kWideBins;
  for (int b = tid; b < kWideBins; b += kWideThreads)
    if (h[b]) atomicAdd(&gh[b], h[b]);
}

// One workgroup per row: the bin holding the remaining rank (counted from the
// top), its digit fixed; the row's counts are cleared for the next round.
__global__ __launch_bounds__(kWideThreads) void wide_pick_kernel(WideState w, int shift, int last) {
  const int64_t row = blockIdx.x;
  if (w.done[row]) return;  // uniform
  constexpr int kPer = kWideBins / kWideThreads;  // 8 bins per thread, thread t: bins [8t, 8t + 8)
  __shared__ uint32_t part[kWideThreads];
  __shared__ uint32_t s_bin, s_rem, s_exact;
  const int tid = threadIdx.x;
  uint32_t *gh = w.hist + row * kWideBins;
  uint32_t c[kPer];
  uint32_t tot = 0u;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    c[e] = gh[tid * kPer + e];
    tot += c[e];
  }
  part[tid] = tot;
  if (tid == 0) {  // kept if no bin holds the rank (never: rem <= the matching count)
    s_bin = 0u;
    s_rem = 1u;
    s_exact = 1u;
  }
  __syncthreads();
  // counts strictly above the thread's bins: a suffix sum over the threads
  for (int off = 1; off < kWideThreads; off <<= 1) {
    const uint32_t add = tid + off < kWideThreads ? part[tid + off] : 0u;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  const uint32_t rem = w.rem[row];
  uint32_t above = part[tid] - tot;  // bins of higher threads
  if (above < rem && rem <= above + tot) {  // exactly one thread
    for (int e = kPer - 1; e >= 0; --e) {
      if (above + c[e] >= rem) {
        s_bin = (uint32_t)(tid * kPer + e);
        s_rem = rem - above;
        s_exact = c[e] == rem - above;
        break;
      }
      above += c[e];
    }
  }
#pragma unroll
  for (int e = 0; e < kPer; ++e) gh[tid * kPer + e] = 0u;
  __syncthreads();
  if (tid == 0) {
    w.thr[row] |= (uint64_t)s_bin << shift;
    w.rem[row] = s_rem;
    if (s_exact || last) w.done[row] = 1u;
  }
}

// The kk values >= the threshold, appended at the row's counter: each wave
// counts its elements of the chunk, the workgroup reserves its range with one
// atomic, then each wave writes at its own running offset (no atomics).
__global__ __launch_bounds__(kWideThreads) void wide_compact_kernel(WideSrc src, WideState w, uint32_t kk) {
  constexpr int kW = kWideThreads / kWave;
  __shared__ uint32_t s_wc[kW];
  __shared__ uint32_t s_base;
  const int64_t row = blockIdx.y;
  const int64_t n = src.count(row);
  const int64_t per = cdiv(n, (int64_t)gridDim.x);
  const int64_t start = (int64_t)blockIdx.x * per;
  if (start >= n) return;  // uniform
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const uint64_t thr = w.thr[row];
  const int64_t end = start + per < n ? start + per : n;
  uint32_t c = 0u;
  for (int64_t i = start + threadIdx.x; i < end; i += kWideThreads) c += src.at(row, i) >= thr ? 1u : 0u;
  c = (uint32_t)wave_sum_i((int)c);
  if (lane == 0) s_wc[wave] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0u;
#pragma unroll
    for (int v = 0; v < kW; ++v) t += s_wc[v];
    s_base = t ? atomicAdd(w.cnt + row * kCntStride, t) : 0u;
  }
  __syncthreads();
  uint32_t off = s_base;
  for (int v = 0; v < wave; ++v) off += s_wc[v];
  uint64_t *sel = w.sel + row * w.P;
  for (int64_t i0 = start + wave * kWave; i0 < end; i0 += kWideThreads) {  // wave-uniform trip count
    const int64_t i = i0 + lane;
    const uint64_t v = i < end ? src.at(row, i) : 0ull;
    const bool take = i < end && v >= thr;
    const uint64_t mask = __ballot(take);
    const uint32_t pos = off + (uint32_t)__popcll(mask & ((1ull << lane) - 1ull));
    if (take && pos < kk) sel[pos] = v;
    off += (uint32_t)__popcll(mask);
  }
}

// Bitonic compare-exchange of a[i] and a[i + j]: descending where
// (i & size) == 0, ascending otherwise (all descending at size = P).
__device__ __forceinline__ void bitonic_cx(uint64_t &x, uint64_t &y, bool desc) {
  if ((x < y) == desc) {
    const uint64_t t = x;
    x = y;
    y = t;
  }
}

// One chunk of L values of a row in LDS (blockIdx.x: chunk).  first: load the
// compacted values (zeros past kk) and run every step of sizes 2..L; else the
// steps of strides L/2..1 of merge size `size`.
__global__ __launch_bounds__(kSortThreads) void wide_sort_local_kernel(WideState w, int64_t L, int64_t size,
                                                                       uint32_t kk, int first) {
  __shared__ uint64_t a[kSortLds];
  const int64_t row = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * L;
  uint64_t *sel = w.sel + row * w.P;
  const int tid = threadIdx.x;
  for (int64_t t = tid; t < L; t += kSortThreads) {
    const int64_t i = base + t;
    a[t] = (!first || i < (int64_t)kk) ? sel[i] : 0ull;
  }
  __syncthreads();
  const int64_t half = L >> 1;
  auto steps = [&](int64_t sz, int64_t j0) {
    for (int64_t j = j0; j > 0; j >>= 1) {
      for (int64_t p = tid; p < half; p += kSortThreads) {
        const int64_t i = p + (p & ~(j - 1));  // local index (j a power of two), partner i + j
        bitonic_cx(a[i], a[i + j], ((base + i) & sz) == 0);
      }
      __syncthreads();
    }
  };
  if (first) {
    for (int64_t sz = 2; sz <= L; sz <<= 1) steps(sz, sz >> 1);
  } else {
    steps(size, half);
  }
  for (int64_t t = tid; t < L; t += kSortThreads) sel[base + t] = a[t];
}

// One step of stride j >= L of merge size `size` in global memory.
__global__ __launch_bounds__(256) void wide_sort_global_kernel(WideState w, int64_t size, int64_t j) {
  const int64_t row = blockIdx.y;
  uint64_t *sel = w.sel + row * w.P;
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= (w.P >> 1)) return;
  const int64_t i = p + (p & ~(j - 1));
  uint64_t x = sel[i], y = sel[i + j];
  bitonic_cx(x, y, (i & size) == 0);
  sel[i] = x;
  sel[i + j] = y;
}

__global__ __launch_bounds__(256) void wide_output_kernel(WideState w, int64_t m, int64_t k, int64_t kk, int64_t sink,
                                                          int64_t local, int64_t *__restrict__ idx) {
  const int64_t row = blockIdx.y;
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= k) return;
  int64_t v;
  if (r < kk)
    v = (int64_t)(0xFFFFFFFFu - (uint32_t)w.sel[row * w.P + r]);
  else if (r < kk + sink)
    v = r - kk;
  else
    v = m - local + (r - kk - sink);
  idx[row * k + r] = v;
}

int64_t pow2_at_least(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

}  // namespace

size_t wide_select_bytes(int64_t rows, int64_t kk) {
  if (kk < 1) kk = 1;
  const int64_t P = pow2_at_least(kk);
  return ws_align((size_t)rows * 8) + 2 * ws_align((size_t)rows * 4) + ws_align((size_t)rows * 4 * kCntStride) +
         ws_align((size_t)rows * kWideBins * 4) + ws_align((size_t)rows * (size_t)P * 8);
}

namespace {
// The selection over src (span: an upper bound of every row's count, for the
// grids of the passes over the values).
int wide_select_src(const WideSrc &src, int64_t span, int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local,
                    int64_t *idx, void *workspace, size_t workspace_bytes, hipStream_t st) {
  const int64_t kk = k - sink - local;
  const size_t need = wide_select_bytes(rows, kk);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "top-k (kk=%lld): workspace %zu bytes, need %zu", (long long)kk, workspace_bytes,
                need);
  WideState w{};
  w.P = pow2_at_least(kk);
  char *p = static_cast<char *>(workspace);
  w.thr = reinterpret_cast<uint64_t *>(p);
  p += ws_align((size_t)rows * 8);
  w.rem = reinterpret_cast<uint32_t *>(p);
  p += ws_align((size_t)rows * 4);
  w.done = reinterpret_cast<uint32_t *>(p);
  p += ws_align((size_t)rows * 4);
  w.cnt = reinterpret_cast<uint32_t *>(p);
  p += ws_align((size_t)rows * 4 * kCntStride);
  w.hist = reinterpret_cast<uint32_t *>(p);
  p += ws_align((size_t)rows * kWideBins * 4);
  w.sel = reinterpret_cast<uint64_t *>(p);
  const uint32_t ukk = (uint32_t)kk;
  // about kWideChunk values per workgroup of a full row; a row's actual values
  // (a candidate list's count) are spread evenly over these workgroups
  const dim3 pass((unsigned)cdiv(span, kWideChunk), (unsigned)rows);
  wide_init_kernel<<<(unsigned)rows, kWideThreads, 0, st>>>(w, ukk);
  int rc = launch_status("wide_init_kernel");
  for (int r = 0; r < kRounds && !rc; ++r) {
    wide_hist_kernel<<<pass, kWideThreads, 0, st>>>(src, w, kShift[r], kWidth[r]);
    rc = launch_status("wide_hist_kernel");
    if (rc) break;
    wide_pick_kernel<<<(unsigned)rows, kWideThreads, 0, st>>>(w, kShift[r], r == kRounds - 1);
    rc = launch_status("wide_pick_kernel");
  }
  if (rc) return rc;
  wide_compact_kernel<<<pass, kWideThreads, 0, st>>>(src, w, ukk);
  rc = launch_status("wide_compact_kernel");
  if (rc) return rc;
  // up to 8192 values: one counting sort per row ranks them and writes the indices
  if (kk <= kRankListMax) return launch_rank_list(w.sel, w.P, rows, kk, m, k, sink, local, idx, st);
  const int64_t L = w.P < kSortLds ? w.P : kSortLds;
  const dim3 chunks((unsigned)(w.P / L), (unsigned)rows);
  wide_sort_local_kernel<<<chunks, kSortThreads, 0, st>>>(w, L, 0, ukk, 1);
  rc = launch_status("wide_sort_local_kernel");
  const dim3 gpairs((unsigned)cdiv(w.P / 2, 256), (unsigned)rows);
  for (int64_t size = 2 * L; size <= w.P && !rc; size <<= 1) {
    for (int64_t j = size >> 1; j >= L && !rc; j >>= 1) {
      wide_sort_global_kernel<<<gpairs, 256, 0, st>>>(w, size, j);
      rc = launch_status("wide_sort_global_kernel");
    }
    if (rc) break;
    wide_sort_local_kernel<<<chunks, kSortThreads, 0, st>>>(w, L, size, ukk, 0);
    rc = launch_status("wide_sort_local_kernel");
  }
  if (rc) return rc;
  wide_output_kernel<<<dim3((unsigned)cdiv(k, 256), (unsigned)rows), 256, 0, st>>>(w, m, k, kk, sink, local, idx);
  return launch_status("wide_output_kernel");
}
}  // namespace

int wide_select_list(const TopkSel &s, int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, int64_t *idx,
                     void *workspace, size_t workspace_bytes, hipStream_t st) {
  WideSrc src{};
  src.cand = s.cand;
  src.cand_cap = s.cand_cap;
  src.cnt1 = s.cand_cnt;
  src.cnt2 = s.cand2_cnt;
  src.kk = s.kk;
  return wide_select_src(src, s.cand_cap, rows, m, k, sink, local, idx, workspace, workspace_bytes, st);
}

}  // namespace fathom
