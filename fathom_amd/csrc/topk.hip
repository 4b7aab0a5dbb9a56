// Sink/local-masked exact top-k over score rows (radix select).
//
// Scores map to 32-bit orderable keys; the selection order is the 64-bit key
// K64 = key << 32 | (0xFFFFFFFF - index), so "larger K64" means "larger score,
// then lower index" and all K64 of a row are distinct.
//   init      zero the per-row histogram and counters;
//   hist      one pass over the row: 2048-bin histogram of the top 11 key bits
//             (LDS, then global atomics); the last workgroup of each row picks
//             the bin d1 holding the kk-th largest element;
//   collect   second pass: elements above bin d1 are selected outright, those
//             in bin d1 become candidates (wave-aggregated atomic appends);
//   finalize  one workgroup per row sorts the candidates (bitonic in LDS, or an
//             in-memory radix refinement when the bin is huge), keeps the best
//             kk - |selected|, sorts the selected set, and writes the indices
//             followed by the sink and local positions.
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kBins = 2048;
constexpr int kDigitShift = 21;      // key >> 21 = top 11 bits
constexpr int kChunk = 16384;        // elements per workgroup in the row passes
constexpr int kCandLds = 8192;       // candidates sortable in LDS
constexpr int kMaxK = 2048;          // selected set held in LDS
constexpr int kFinThreads = 1024;

struct RowState {
  uint32_t d1, above, cnt, done;
  uint32_t sel_cnt, cand_cnt, pad0, pad1;
};

struct TopkWs {
  uint32_t *hist;
  RowState *state;
  uint64_t *sel;
  uint64_t *cand;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t ws_layout(int64_t rows, int64_t n, int64_t k, char *base, TopkWs *ws) {
  size_t off = 0;
  const size_t hist_b = align256((size_t)rows * kBins * 4);
  const size_t state_b = align256((size_t)rows * sizeof(RowState));
  const size_t sel_b = align256((size_t)rows * (size_t)k * 8);
  const size_t cand_b = align256((size_t)rows * (size_t)n * 8);
  if (ws) {
    ws->hist = reinterpret_cast<uint32_t *>(base + off);
    ws->state = reinterpret_cast<RowState *>(base + off + hist_b);
    ws->sel = reinterpret_cast<uint64_t *>(base + off + hist_b + state_b);
    ws->cand = reinterpret_cast<uint64_t *>(base + off + hist_b + state_b + sel_b);
  }
  return hist_b + state_b + sel_b + cand_b;
}

__device__ __forceinline__ uint32_t masked_key(const float *row, int64_t i, int64_t sink, int64_t lstart) {
  return (i < sink || i >= lstart) ? kKeyNegInf : score_key(row[i]);
}

__global__ __launch_bounds__(256) void topk_init_kernel(TopkWs ws) {
  const int64_t row = blockIdx.x;
  uint32_t *h = ws.hist + row * kBins;
  for (int d = threadIdx.x; d < kBins; d += 256) h[d] = 0u;
  if (threadIdx.x == 0) {
    RowState s = {};
    ws.state[row] = s;
  }
}

__global__ __launch_bounds__(256) void topk_hist_kernel(const float *__restrict__ scores, int64_t n, int64_t sink,
                                                        int64_t lstart, uint32_t need, TopkWs ws) {
  __shared__ uint32_t h[kBins];
  __shared__ uint32_t part[256];
  __shared__ int is_last;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.y;
  const float *rs = scores + row * n;
  for (int d = tid; d < kBins; d += 256) h[d] = 0u;
  __syncthreads();
  const int64_t start = (int64_t)blockIdx.x * kChunk;
  const int64_t end = min(start + (int64_t)kChunk, n);
  for (int64_t i = start + tid; i < end; i += 256) atomicAdd(&h[masked_key(rs, i, sink, lstart) >> kDigitShift], 1u);
  __syncthreads();
  uint32_t *gh = ws.hist + row * kBins;
  for (int d = tid; d < kBins; d += 256)
    if (h[d]) atomicAdd(&gh[d], h[d]);
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(&ws.state[row].done, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  // this workgroup saw every other workgroup's histogram: pick the bin of the need-th largest
  constexpr int kPer = kBins / 256;
  uint32_t loc[kPer];
  uint32_t sum = 0;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    loc[u] = __hip_atomic_load(&gh[tid * kPer + u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sum += loc[u];
  }
  part[tid] = sum;
  __syncthreads();
  // suffix sums over threads: above[t] = sum of part[t'] for t' > t
  if (tid == 0) {
    uint32_t run = 0;
    for (int t = 255; t >= 0; --t) {
      const uint32_t v = part[t];
      part[t] = run;
      run += v;
    }
  }
  __syncthreads();
  uint32_t cum = part[tid];
#pragma unroll
  for (int u = kPer - 1; u >= 0; --u) {
    if (cum < need && cum + loc[u] >= need) {
      ws.state[row].d1 = (uint32_t)(tid * kPer + u);
      ws.state[row].above = cum;
      ws.state[row].cnt = loc[u];
    }
    cum += loc[u];
  }
}

// Wave-aggregated append of `val` where pred holds; slots past `cap` are
// dropped (the counts of a consistent selection never reach cap).
__device__ __forceinline__ void wave_append(bool pred, uint64_t val, uint32_t *counter, uint64_t *buf, uint64_t cap,
                                            int lane) {
  const uint64_t m = __ballot(pred);
  if (m == 0) return;
  const int leader = __ffsll((unsigned long long)m) - 1;
  uint32_t base = 0;
  if (lane == leader) base = atomicAdd(counter, (uint32_t)__popcll(m));
  base = __shfl(base, leader, kWave);
  const uint64_t slot = (uint64_t)base + __popcll(m & ((1ull << lane) - 1ull));
  if (pred && slot < cap) buf[slot] = val;
}

__global__ __launch_bounds__(256) void topk_collect_kernel(const float *__restrict__ scores, int64_t n, int64_t sink,
                                                           int64_t lstart, int64_t k, TopkWs ws) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t row = blockIdx.y;
  const float *rs = scores + row * n;
  RowState *st = ws.state + row;
  const uint32_t d1 = st->d1;
  uint64_t *sel = ws.sel + row * k;
  uint64_t *cand = ws.cand + row * n;
  const int64_t start = (int64_t)blockIdx.x * kChunk;
  const int64_t end = min(start + (int64_t)kChunk, n);
  for (int64_t i0 = start; i0 < end; i0 += 256) {
    const int64_t i = i0 + tid;
    const bool in = i < end;
    const uint32_t key = in ? masked_key(rs, i, sink, lstart) : 0u;
    const uint32_t d = key >> kDigitShift;
    const uint64_t k64 = ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
    wave_append(in && d > d1, k64, &st->sel_cnt, sel, (uint64_t)k, lane);
    wave_append(in && d == d1, k64, &st->cand_cnt, cand, (uint64_t)n, lane);
  }
}

// Bitonic sort of s[0, P) into descending order (P a power of two).
__device__ void bitonic_desc(uint64_t *s, int P) {
  for (int kk = 2; kk <= P; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = s[i], b = s[ixj];
          const bool swap = ((i & kk) == 0) ? (a < b) : (a > b);
          if (swap) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

__global__ __launch_bounds__(kFinThreads) void topk_finalize_kernel(int64_t n, int64_t m, int64_t k, int64_t sink,
                                                                    int64_t local, TopkWs ws,
                                                                    int64_t *__restrict__ idx) {
  __shared__ uint64_t cs[kCandLds];
  __shared__ uint64_t ss[kMaxK];
  __shared__ uint32_t h8[256];
  __shared__ uint32_t s_cnt;
  __shared__ uint64_t s_prefix;
  __shared__ uint32_t s_need;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t kk = k - sink - local;
  const RowState st = ws.state[row];
  const uint32_t sel_cnt = min(st.sel_cnt, (uint32_t)kk);
  const uint32_t cand_cnt = min(st.cand_cnt, (uint32_t)n);
  const uint32_t need2 = (uint32_t)kk - sel_cnt;
  const uint64_t *cand = ws.cand + row * n;
  const uint64_t *sel = ws.sel + row * k;
  int64_t *out = idx + row * k;

  // --- the best need2 candidates, descending, into cs[0, need2)
  if (cand_cnt <= (uint32_t)kCandLds) {
    const int P = next_pow2((int)cand_cnt);
    for (int i = tid; i < P; i += kFinThreads) cs[i] = (i < (int)cand_cnt) ? cand[i] : 0ull;
    __syncthreads();
    bitonic_desc(cs, P);
  } else {
    // Radix refinement over the low 53 bits (the top 11 equal d1 for every
    // candidate): find the exact need2-th largest K64, then gather all >= it.
    constexpr uint64_t kTop11 = 0xFFE0000000000000ull;
    if (tid == 0) {
      s_prefix = cand[0] & kTop11;
      s_need = need2;
    }
    __syncthreads();
    const int shifts[7] = {45, 37, 29, 21, 13, 5, 0};
    const int widths[7] = {8, 8, 8, 8, 8, 8, 5};
    uint64_t pmask = kTop11;
    for (int lvl = 0; lvl < 7; ++lvl) {
      const int sh = shifts[lvl], wd = widths[lvl];
      const uint32_t dm = (1u << wd) - 1u;
      for (int d = tid; d < 256; d += kFinThreads) h8[d] = 0u;
      __syncthreads();
      const uint64_t pre = s_prefix;
      for (uint32_t i = tid; i < cand_cnt; i += kFinThreads) {
        const uint64_t v = cand[i];
        if ((v & pmask) == pre) atomicAdd(&h8[(v >> sh) & dm], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t cum = 0;
        const uint32_t nd = s_need;
        for (int d = (int)dm; d >= 0; --d) {
          if (cum + h8[d] >= nd) {
            s_prefix = pre | ((uint64_t)d << sh);
            s_need = nd - cum;
            break;
          }
          cum += h8[d];
        }
      }
      __syncthreads();
      pmask |= (uint64_t)dm << sh;
    }
    const uint64_t thr = s_prefix;
    if (tid == 0) s_cnt = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < cand_cnt; i += kFinThreads) {
      const uint64_t v = cand[i];
      if (v >= thr) {
        const uint32_t p = atomicAdd(&s_cnt, 1u);
        if (p < (uint32_t)kMaxK) cs[p] = v;
      }
    }
    __syncthreads();
    const int got = (int)min(s_cnt, (uint32_t)kMaxK);
    const int P = next_pow2(got);
    for (int i = got + tid; i < P; i += kFinThreads) cs[i] = 0ull;
    __syncthreads();
    bitonic_desc(cs, P);
  }
  // --- the selected set, descending
  {
    const int P = next_pow2((int)sel_cnt);
    for (int i = tid; i < P; i += kFinThreads) ss[i] = (i < (int)sel_cnt) ? sel[i] : 0ull;
    __syncthreads();
    bitonic_desc(ss, P);
  }
  for (int i = tid; i < (int)sel_cnt; i += kFinThreads) out[i] = (int64_t)(0xFFFFFFFFu - (uint32_t)ss[i]);
  for (int i = tid; i < (int)need2; i += kFinThreads)
    out[sel_cnt + i] = (int64_t)(0xFFFFFFFFu - (uint32_t)cs[i]);
  for (int i = tid; i < (int)(sink + local); i += kFinThreads)
    out[kk + i] = (i < sink) ? (int64_t)i : (int64_t)(m - local + (i - sink));
}

__global__ __launch_bounds__(256) void topk_fixed_only_kernel(int64_t rows, int64_t m, int64_t k, int64_t sink,
                                                              int64_t local, int64_t *__restrict__ idx) {
  const int64_t total = rows * k;
  for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
    const int64_t i = o % k;
    idx[o] = (i < sink) ? i : (m - local + (i - sink));
  }
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" size_t fathom_topk_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows < 1 || n < 1 || k < 0) return 0;
  return ws_layout(rows, n, k, nullptr, nullptr);
}

extern "C" int fathom_sink_local_topk(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k,
                                      int64_t sink, int64_t local, int64_t *idx, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  if (!scores || !idx) return fail(FATHOM_ERR_INVALID, "sink_local_topk: null pointer");
  if (rows < 1 || rows > 65535) return fail(FATHOM_ERR_INVALID, "sink_local_topk: rows=%lld outside [1, 65535]", (long long)rows);
  if (n < 1 || n > 0x7FFFFFFFLL) return fail(FATHOM_ERR_INVALID, "sink_local_topk: n=%lld unsupported", (long long)n);
  if (sink < 0 || local < 0 || k < 0) return fail(FATHOM_ERR_INVALID, "sink_local_topk: negative k/sink/local");
  const int64_t kk = k - sink - local;
  if (kk < 0) return fail(FATHOM_ERR_INVALID, "sink_local_topk: k=%lld < sink+local=%lld", (long long)k, (long long)(sink + local));
  if (kk > n) return fail(FATHOM_ERR_INVALID, "sink_local_topk: k - sink - local = %lld exceeds n=%lld", (long long)kk, (long long)n);
  if (kk > kMaxK) return fail(FATHOM_ERR_INVALID, "sink_local_topk: k - sink - local = %lld exceeds %d", (long long)kk, kMaxK);
  if (sink > n || m < n || local > m)
    return fail(FATHOM_ERR_INVALID, "sink_local_topk: need sink <= n <= m and local <= m (sink=%lld n=%lld m=%lld local=%lld)",
                (long long)sink, (long long)n, (long long)m, (long long)local);
  hipStream_t st = (hipStream_t)stream;
  if (kk == 0) {
    if (k == 0) return FATHOM_OK;
    topk_fixed_only_kernel<<<(unsigned)min(cdiv(rows * k, 256), (int64_t)65535), 256, 0, st>>>(rows, m, k, sink, local, idx);
    return launch_status("topk_fixed_only_kernel");
  }
  const size_t need_bytes = ws_layout(rows, n, k, nullptr, nullptr);
  if (!workspace || workspace_bytes < need_bytes)
    return fail(FATHOM_ERR_WORKSPACE, "sink_local_topk: workspace %zu bytes, need %zu", workspace_bytes, need_bytes);
  TopkWs ws;
  ws_layout(rows, n, k, static_cast<char *>(workspace), &ws);
  const int64_t lstart = (m - local) > 0 ? (m - local) : 0;
  const int64_t chunks = cdiv(n, kChunk);
  topk_init_kernel<<<(unsigned)rows, 256, 0, st>>>(ws);
  int rc = launch_status("topk_init_kernel");
  if (rc) return rc;
  topk_hist_kernel<<<dim3((unsigned)chunks, (unsigned)rows), 256, 0, st>>>(scores, n, sink, lstart, (uint32_t)kk, ws);
  rc = launch_status("topk_hist_kernel");
  if (rc) return rc;
  topk_collect_kernel<<<dim3((unsigned)chunks, (unsigned)rows), 256, 0, st>>>(scores, n, sink, lstart, k, ws);
  rc = launch_status("topk_collect_kernel");
  if (rc) return rc;
  topk_finalize_kernel<<<(unsigned)rows, kFinThreads, 0, st>>>(n, m, k, sink, local, ws, idx);
  return launch_status("topk_finalize_kernel");
}
