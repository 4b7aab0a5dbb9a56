// Top-kk of score rows for any kk up to n: the path of k - sink - local above
// the LDS-resident selections' limit (torch.topk has no limit,
// kernels/bitplane.py:372-378).
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
//   sort          bitonic, descending, over the kk values padded with zeros to
//                 a power of two P: chunks of up to 16384 values sorted in LDS,
//                 then for each merge size above that the steps of strides of
//                 at least a chunk in global memory and the rest in LDS;
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

__device__ __forceinline__ uint64_t wide_k64(const float *row, int64_t i, int64_t sink, int64_t lstart) {
  const uint32_t key = (i < sink || i >= lstart) ? kKeyNegInf : score_key(row[i]);
  return k64_of(key, i);
}

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
__global__ __launch_bounds__(kWideThreads) void wide_hist_kernel(const float *__restrict__ scores, int64_t n,
                                                                 int64_t sink, int64_t lstart, WideState w, int shift,
                                                                 int width) {
  const int64_t row = blockIdx.y;
  if (w.done[row]) return;  // uniform
  __shared__ uint32_t h[kWideBins];
  const int tid = threadIdx.x;
  for (int b = tid; b < kWideBins; b += kWideThreads) h[b] = 0u;
  __syncthreads();
  const int top = shift + width;  // bits [top, 64) are fixed
  const uint64_t fixed = top < 64 ? (w.thr[row] >> top) : 0ull;
  const uint32_t dmask = (1u << width) - 1u;
  const float *rs = scores + row * n;
  const int64_t start = (int64_t)blockIdx.x * kWideChunk;
  const int64_t end = start + kWideChunk < n ? start + kWideChunk : n;
  for (int64_t i = start + tid; i < end; i += kWideThreads) {
    const uint64_t v = wide_k64(rs, i, sink, lstart);
    if (top >= 64 || (v >> top) == fixed) atomicAdd(&h[(uint32_t)(v >> shift) & dmask], 1u);
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

// The kk values >= the threshold, appended at the row's counter.
__global__ __launch_bounds__(kWideThreads) void wide_compact_kernel(const float *__restrict__ scores, int64_t n,
                                                                    int64_t sink, int64_t lstart, WideState w,
                                                                    uint32_t kk) {
  const int64_t row = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t thr = w.thr[row];
  const float *rs = scores + row * n;
  uint64_t *sel = w.sel + row * w.P;
  uint32_t *cnt = w.cnt + row * kCntStride;
  const int64_t start = (int64_t)blockIdx.x * kWideChunk;
  const int64_t end = start + kWideChunk < n ? start + kWideChunk : n;
  for (int64_t i0 = start; i0 < end; i0 += kWideThreads) {  // uniform trip count
    const int64_t i = i0 + threadIdx.x;
    const uint64_t v = i < end ? wide_k64(rs, i, sink, lstart) : 0ull;
    const bool take = i < end && v >= thr;
    const uint64_t mask = __ballot(take);
    if (mask == 0ull) continue;
    uint32_t base = 0u;
    if (lane == 0) base = atomicAdd(cnt, (uint32_t)__popcll(mask));
    base = __shfl(base, 0);
    const uint32_t pos = base + (uint32_t)__popcll(mask & ((1ull << lane) - 1ull));
    if (take && pos < kk) sel[pos] = v;
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

int wide_select_run(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local,
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
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  const uint32_t ukk = (uint32_t)kk;
  const dim3 pass((unsigned)cdiv(n, kWideChunk), (unsigned)rows);
  wide_init_kernel<<<(unsigned)rows, kWideThreads, 0, st>>>(w, ukk);
  int rc = launch_status("wide_init_kernel");
  for (int r = 0; r < kRounds && !rc; ++r) {
    wide_hist_kernel<<<pass, kWideThreads, 0, st>>>(scores, n, sink, lstart, w, kShift[r], kWidth[r]);
    rc = launch_status("wide_hist_kernel");
    if (rc) break;
    wide_pick_kernel<<<(unsigned)rows, kWideThreads, 0, st>>>(w, kShift[r], r == kRounds - 1);
    rc = launch_status("wide_pick_kernel");
  }
  if (rc) return rc;
  wide_compact_kernel<<<pass, kWideThreads, 0, st>>>(scores, n, sink, lstart, w, ukk);
  rc = launch_status("wide_compact_kernel");
  if (rc) return rc;
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

}  // namespace fathom
