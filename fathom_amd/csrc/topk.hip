// Sink/local-masked exact top-k over score rows.
//
// Orderable keys: score_key maps a float to a uint32 whose unsigned order is
// torch.topk's value order; K64 = key << 32 | (0xFFFFFFFF - index) makes every
// element of a row distinct and orders equal scores by ascending index.
// The selection runs select -> filter -> finalize (topk_internal.hpp); the
// fused scan+top-k path replaces `filter` by the scan kernel's own emission.
//
// Radix rounds (8-bit digits, most significant first) build LDS histograms
// with wave-aggregated updates -- the leader lane of each distinct digit in a
// wave adds the popcount of its ballot -- so the few hot exponent buckets of a
// score row cost one atomic per wave and digit.  A round ends the search as
// soon as the chosen bucket holds exactly the elements still needed.
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelPer = (int)(kMaxSample / kSelThreads);  // keys per thread in select
constexpr int kFinThreads = 1024;
constexpr int kFilterThreads = 256;
constexpr int64_t kFilterChunk = 16384;
constexpr uint32_t kFilterLocal = 2048;  // LDS candidates per filter workgroup
constexpr int kCandLds = 16384;          // candidates selected in LDS (128 KB)
constexpr int kMaxK = 2048;              // largest kk

__device__ __forceinline__ void wave_hist_add(uint32_t *hist, uint32_t dg, bool act, int lane) {
  uint64_t rem = __ballot(act);
  while (rem) {
    const int leader = __ffsll((unsigned long long)rem) - 1;
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)dg, leader);
    const uint64_t m = __ballot(act && dg == d) & rem;
    if (lane == leader) atomicAdd(&hist[d], (uint32_t)__popcll(m));
    rem &= ~m;
  }
}

template <typename K>
struct SelShared {
  uint32_t hist[256];
  K prefix;
  uint32_t need;
  uint32_t done;
};

template <typename K>
__device__ __forceinline__ void sel_begin(SelShared<K> &sh, uint32_t need) {
  if (threadIdx.x == 0) {
    sh.prefix = 0;
    sh.need = need;
    sh.done = 0u;
  }
  for (int d = threadIdx.x; d < 256; d += blockDim.x) sh.hist[d] = 0u;
  __syncthreads();
}

// After the histogram of a round: wave 0 picks the digit holding the need-th
// largest element, then the histogram is cleared for the next round.
template <typename K>
__device__ __forceinline__ void sel_pick(SelShared<K> &sh, int shift) {
  const int tid = threadIdx.x;
  __syncthreads();
  if (tid < 64) {
    uint32_t h[4];
    uint32_t s = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      h[u] = sh.hist[4 * tid + u];
      s += h[u];
    }
    uint32_t incl = s;  // inclusive suffix sum over lanes (digits above)
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t v = __shfl_down(incl, o, kWave);
      if (tid + o < 64) incl += v;
    }
    uint32_t above = incl - s;
    const uint32_t nd = sh.need;
    const K pre = sh.prefix;
#pragma unroll
    for (int u = 3; u >= 0; --u) {
      if (above < nd && above + h[u] >= nd) {
        sh.prefix = pre | ((K)(4 * tid + u) << shift);
        sh.need = nd - above;
        if (h[u] == nd - above) sh.done = 1u;
      }
      above += h[u];
    }
  }
  __syncthreads();
  for (int d = tid; d < 256; d += blockDim.x) sh.hist[d] = 0u;
  __syncthreads();
}

// Exact need-th largest of the values held M per thread (count = M * blockDim
// values, all taking part): radix rounds over registers.
template <int M>
__device__ uint32_t select_small(const uint32_t (&v)[M], uint32_t need, SelShared<uint32_t> &sh) {
  const int lane = threadIdx.x & 63;
  sel_begin(sh, need);
  for (int shift = 24; shift >= 0; shift -= 8) {
    const uint32_t pre = sh.prefix;
    const uint32_t hmask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
#pragma unroll
    for (int u = 0; u < M; ++u) wave_hist_add(sh.hist, (v[u] >> shift) & 255u, (v[u] & hmask) == (pre & hmask), lane);
    sel_pick(sh, shift);
    if (sh.done) break;
  }
  return sh.prefix;
}

// Lower bound T on the need-th largest of the kSelPer keys per thread (zeros
// for slots past the sample): each thread keeps its M largest keys and T is the
// need-th largest of those M * blockDim values.  Those are need distinct
// sample elements >= T, so T <= the sample's need-th largest <= the row's.
// With M * blockDim >= 2 need, T lands near the sample's (1-2) * need-th
// largest, at a fraction of the cost of an exact selection over the sample.
template <int M>
__device__ uint32_t select_bound(const uint32_t (&v)[kSelPer], uint32_t need, SelShared<uint32_t> &sh) {
  uint32_t top[M];
#pragma unroll
  for (int i = 0; i < M; ++i) top[i] = 0u;
#pragma unroll
  for (int u = 0; u < kSelPer; ++u) {
    uint32_t x = v[u];
#pragma unroll
    for (int i = 0; i < M; ++i) {
      const uint32_t hi = max(top[i], x);
      x = min(top[i], x);
      top[i] = hi;
    }
  }
  return select_small<M>(top, need, sh);
}

__device__ __forceinline__ uint32_t masked_key(const float *row, int64_t i, int64_t sink, int64_t lstart) {
  return (i < sink || i >= lstart) ? kKeyNegInf : score_key(row[i]);
}

__global__ __launch_bounds__(kSelThreads) void select_keys_kernel(const uint32_t *__restrict__ samp,
                                                                  int64_t samp_cap, uint32_t kk, TopkSel s) {
  __shared__ SelShared<uint32_t> sh;
  const int64_t row = blockIdx.x;
  const uint32_t *src = samp + row * samp_cap;
  uint32_t v[kSelPer];
#pragma unroll
  for (int u = 0; u < kSelPer; ++u) {
    const int64_t i = threadIdx.x + (int64_t)u * kSelThreads;
    v[u] = i < samp_cap ? src[i] : 0u;
  }
  uint32_t thr = 0u;  // fewer samples than kk: every element is a candidate
  if (samp_cap >= (int64_t)kk) {
    if (2 * kk <= kSelThreads)
      thr = select_bound<1>(v, kk, sh);
    else if (kk <= kSelThreads)
      thr = select_bound<2>(v, kk, sh);
    else
      thr = select_bound<4>(v, kk, sh);
  }
  if (threadIdx.x == 0) {
    s.thr[row] = thr;
    s.cand_cnt[row] = 0u;
  }
}

// Sampled keys of score rows: tile ti of the sample is tile ti * S of the row.
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

__global__ __launch_bounds__(kFilterThreads) void filter_scores_kernel(const float *__restrict__ scores, int64_t n,
                                                                       int64_t sink, int64_t lstart, TopkSel s) {
  __shared__ uint64_t lbuf[kFilterLocal];
  __shared__ uint32_t lcnt, lbase;
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t row = blockIdx.y;
  const float *rs = scores + row * n;
  const uint32_t thr = s.thr[row];
  uint64_t *cand = s.cand + row * s.cand_cap;
  if (tid == 0) lcnt = 0u;
  __syncthreads();
  const int64_t start = (int64_t)blockIdx.x * kFilterChunk;
  const int64_t end = min(start + kFilterChunk, n);
  for (int64_t i0 = start; i0 < end; i0 += kFilterThreads) {
    const int64_t i = i0 + tid;
    const bool in = i < end;
    const uint32_t key = in ? masked_key(rs, i, sink, lstart) : 0u;
    wave_append_local(in && key >= thr, k64_of(key, i), &lcnt, lbuf, kFilterLocal, &s.cand_cnt[row], cand,
                      (uint64_t)s.cand_cap, lane);
  }
  __syncthreads();
  flush_local(&lcnt, lbuf, kFilterLocal, &s.cand_cnt[row], cand, (uint64_t)s.cand_cap, &lbase);
}

// Exact kk-th largest K64 among cnt candidates read through get(i).
template <typename Get>
__device__ uint64_t select_k64(Get get, int64_t cnt, uint32_t need, SelShared<uint64_t> &sh) {
  const int tid = threadIdx.x, lane = tid & 63;
  sel_begin(sh, need);
  for (int shift = 56; shift >= 0; shift -= 8) {
    const uint64_t pre = sh.prefix;
    const uint64_t hmask = shift == 56 ? 0ull : (~0ull << (shift + 8));
    for (int64_t i0 = 0; i0 < cnt; i0 += kFinThreads) {
      const int64_t i = i0 + tid;
      uint64_t v = 0ull;
      bool act = false;
      if (i < cnt) {
        v = get(i);
        act = (v & hmask) == (pre & hmask);
      }
      wave_hist_add(sh.hist, (uint32_t)(v >> shift) & 255u, act, lane);
    }
    sel_pick(sh, shift);
    if (sh.done) break;
  }
  return sh.prefix;
}

__global__ __launch_bounds__(kFinThreads) void finalize_kernel(int64_t m, int64_t k, int64_t sink, int64_t local,
                                                               TopkSel s, int64_t *__restrict__ idx) {
  constexpr int kPer = kCandLds / kFinThreads;
  __shared__ uint64_t cl[kCandLds];
  __shared__ uint64_t ss[kMaxK + 8];
  __shared__ SelShared<uint64_t> sh;
  __shared__ uint32_t s_cnt;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t kk = k - sink - local;
  const int64_t cnt = min((int64_t)s.cand_cnt[row], s.cand_cap);
  const uint64_t *gc = s.cand + row * s.cand_cap;
  int64_t *out = idx + row * k;
  const bool in_lds = cnt <= kCandLds;
  if (in_lds) {
    uint64_t v[kPer];  // all loads in flight before the first store
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int64_t i = tid + (int64_t)u * kFinThreads;
      v[u] = i < cnt ? gc[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int64_t i = tid + (int64_t)u * kFinThreads;
      if (i < cnt) cl[i] = v[u];
    }
  }
  __syncthreads();
  uint64_t thr = 0ull;
  if (cnt >= kk) {
    if (in_lds)
      thr = select_k64([&](int64_t i) { return cl[i]; }, cnt, (uint32_t)kk, sh);
    else
      thr = select_k64([&](int64_t i) { return gc[i]; }, cnt, (uint32_t)kk, sh);
  }
  if (tid == 0) s_cnt = 0u;
  __syncthreads();
  for (int64_t i = tid; i < cnt; i += kFinThreads) {
    const uint64_t v = in_lds ? cl[i] : gc[i];
    if (v >= thr) {
      const uint32_t p = atomicAdd(&s_cnt, 1u);
      if (p < (uint32_t)kMaxK) ss[p] = v;
    }
  }
  __syncthreads();
  // the selected keys are distinct: each one's output position is the number
  // of selected keys above it (every lane of a wave reads the same ss[j])
  const int got = (int)min(s_cnt, (uint32_t)kMaxK);
  for (int i = got + tid; i < ((got + 7) & ~7); i += kFinThreads) ss[i] = 0ull;  // pad to 8 (zero ranks below all)
  __syncthreads();
  for (int i = tid; i < got; i += kFinThreads) {
    const uint64_t v = ss[i];
    int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
    for (int j = 0; j < got; j += 8) {  // independent LDS reads in flight
      const uint64_t a0 = ss[j], a1 = ss[j + 1], a2 = ss[j + 2], a3 = ss[j + 3];
      const uint64_t a4 = ss[j + 4], a5 = ss[j + 5], a6 = ss[j + 6], a7 = ss[j + 7];
      r0 += (a0 > v) + (a4 > v);
      r1 += (a1 > v) + (a5 > v);
      r2 += (a2 > v) + (a6 > v);
      r3 += (a3 > v) + (a7 > v);
    }
    const int rank = (r0 + r1) + (r2 + r3);
    if (rank < kk) out[rank] = (int64_t)(0xFFFFFFFFu - (uint32_t)v);
  }
  for (int i = got + tid; i < (int)kk; i += kFinThreads) out[i] = 0;
  for (int i = tid; i < (int)(sink + local); i += kFinThreads)
    out[kk + i] = (i < sink) ? (int64_t)i : (int64_t)(m - local + (i - sink));
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

size_t topk_sel_layout(int64_t rows, int64_t cand_cap, char *base, TopkSel *s) {
  const size_t thr_b = ws_align((size_t)rows * 4);
  const size_t cnt_b = ws_align((size_t)rows * 4);
  const size_t cand_b = ws_align((size_t)rows * (size_t)cand_cap * 8);
  if (s) {
    s->thr = reinterpret_cast<uint32_t *>(base);
    s->cand_cnt = reinterpret_cast<uint32_t *>(base + thr_b);
    s->cand = reinterpret_cast<uint64_t *>(base + thr_b + cnt_b);
    s->cand_cap = cand_cap;
  }
  return thr_b + cnt_b + cand_b;
}

size_t topk_layout(int64_t rows, int64_t n, int64_t k, char *base, uint32_t **samp, int64_t *samp_cap, TopkSel *sel,
                   int64_t *S_out) {
  const int64_t kk = k > 0 ? k : 0;
  const int64_t S = topk_tile_stride(n, kk);
  const int64_t cap = topk_sample_tiles(n, S) * kTileTok;
  const size_t samp_b = ws_align((size_t)rows * (size_t)cap * 4);
  if (samp) *samp = reinterpret_cast<uint32_t *>(base);
  if (samp_cap) *samp_cap = cap;
  if (S_out) *S_out = S;
  return samp_b + topk_sel_layout(rows, n, base ? base + samp_b : nullptr, sel);
}

int launch_select_keys(const uint32_t *samp, int64_t rows, int64_t samp_cap, int64_t kk, TopkSel s, hipStream_t st) {
  if (samp_cap > kMaxSample) return fail(FATHOM_ERR_INVALID, "select: %lld sampled keys exceed %lld", (long long)samp_cap, (long long)kMaxSample);
  select_keys_kernel<<<(unsigned)rows, kSelThreads, 0, st>>>(samp, samp_cap, (uint32_t)kk, s);
  return launch_status("select_keys_kernel");
}

int launch_sample_scores(const float *scores, int64_t rows, int64_t n, int64_t S, int64_t sink, int64_t lstart,
                         uint32_t *samp, int64_t samp_cap, hipStream_t st) {
  sample_scores_kernel<<<dim3((unsigned)(samp_cap / kTileTok), (unsigned)rows), 256, 0, st>>>(scores, n, S, sink,
                                                                                            lstart, samp, samp_cap);
  return launch_status("sample_scores_kernel");
}

int launch_filter_scores(const float *scores, int64_t rows, int64_t n, int64_t sink, int64_t lstart, TopkSel s,
                         hipStream_t st) {
  filter_scores_kernel<<<dim3((unsigned)cdiv(n, kFilterChunk), (unsigned)rows), kFilterThreads, 0, st>>>(
      scores, n, sink, lstart, s);
  return launch_status("filter_scores_kernel");
}

int launch_finalize(int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, TopkSel s, int64_t *idx,
                    hipStream_t st) {
  finalize_kernel<<<(unsigned)rows, kFinThreads, 0, st>>>(m, k, sink, local, s, idx);
  return launch_status("finalize_kernel");
}

int launch_fixed_only(int64_t rows, int64_t m, int64_t k, int64_t sink, int64_t local, int64_t *idx, hipStream_t st) {
  if (k == 0) return FATHOM_OK;
  fixed_only_kernel<<<(unsigned)min(cdiv(rows * k, 256), (int64_t)65535), 256, 0, st>>>(rows, m, k, sink, local, idx);
  return launch_status("fixed_only_kernel");
}

int check_topk_args(int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink, int64_t local, const char *who) {
  if (rows < 1 || rows > 65535) return fail(FATHOM_ERR_INVALID, "%s: rows=%lld outside [1, 65535]", who, (long long)rows);
  if (n < 1 || n > 0x7FFFFFFFLL) return fail(FATHOM_ERR_INVALID, "%s: n=%lld unsupported", who, (long long)n);
  if (sink < 0 || local < 0 || k < 0) return fail(FATHOM_ERR_INVALID, "%s: negative k/sink/local", who);
  const int64_t kk = k - sink - local;
  if (kk < 0) return fail(FATHOM_ERR_INVALID, "%s: k=%lld < sink+local=%lld", who, (long long)k, (long long)(sink + local));
  if (kk > n) return fail(FATHOM_ERR_INVALID, "%s: k - sink - local = %lld exceeds n=%lld", who, (long long)kk, (long long)n);
  if (kk > kMaxK) return fail(FATHOM_ERR_INVALID, "%s: k - sink - local = %lld exceeds %d", who, (long long)kk, kMaxK);
  if (sink > n || m < n || local > m)
    return fail(FATHOM_ERR_INVALID, "%s: need sink <= n <= m and local <= m (sink=%lld n=%lld m=%lld local=%lld)", who,
                (long long)sink, (long long)n, (long long)m, (long long)local);
  return FATHOM_OK;
}

}  // namespace fathom

using namespace fathom;

extern "C" size_t fathom_topk_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows < 1 || n < 1 || k < 0) return 0;
  return topk_layout(rows, n, k, nullptr, nullptr, nullptr, nullptr, nullptr);
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
  const size_t need = topk_layout(rows, n, k, nullptr, nullptr, nullptr, nullptr, nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "sink_local_topk: workspace %zu bytes, need %zu", workspace_bytes, need);
  TopkSel s;
  uint32_t *samp = nullptr;
  int64_t samp_cap = 0, S = 1;
  topk_layout(rows, n, k, static_cast<char *>(workspace), &samp, &samp_cap, &s, &S);
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  rc = launch_sample_scores(scores, rows, n, S, sink, lstart, samp, samp_cap, st);
  if (rc) return rc;
  rc = launch_select_keys(samp, rows, samp_cap, kk, s, st);
  if (rc) return rc;
  rc = launch_filter_scores(scores, rows, n, sink, lstart, s, st);
  if (rc) return rc;
  return launch_finalize(rows, m, k, sink, local, s, idx, st);
}
