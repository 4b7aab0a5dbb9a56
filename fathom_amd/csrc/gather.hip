// Row gathers of the selected K/V tokens, from HBM or zero-copy from mapped
// pinned host memory.
//
// gather_rows: the reference kernel's semantics, one 16-byte vector per lane.
// gather_union: the decode step's group-union fetch in two launches --
//   dedup   one workgroup per (batch*KV head) sorts the G*k (token, position)
//           pairs in LDS (bitonic, 64-bit keys) and counts distinct host rows;
//   fetch   one wave per sorted slot; the first slot of each distinct token
//           reads the row once (host store, recent-token device buffer, or a
//           zero row for negative tokens) and writes it to every position that
//           selected it, so each distinct host row crosses PCIe exactly once.
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kRowsPerWG = 16;
constexpr int kMaxGK = 16384;
constexpr int kDedupThreads = 1024;
constexpr uint32_t kTokNeg = 0xFFFFFFFEu;   // sort key of negative tokens
constexpr uint32_t kTokPad = 0xFFFFFFFFu;   // sort key of padding slots

template <typename V>
__global__ __launch_bounds__(256) void gather_rows_kernel(const char *__restrict__ src, int64_t cap,
                                                          const int32_t *__restrict__ idx, int64_t R,
                                                          int64_t row_bytes, char *__restrict__ dst) {
  const int64_t bh = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * kRowsPerWG;
  const int64_t nv = row_bytes / (int64_t)sizeof(V);
  for (int64_t f = threadIdx.x; f < kRowsPerWG * nv; f += 256) {
    const int64_t r = r0 + f / nv, v = f % nv;
    if (r >= R) break;
    const int32_t i = idx[bh * R + r];
    V val = {};
    if (i >= 0 && i < cap) val = reinterpret_cast<const V *>(src + (bh * cap + i) * row_bytes)[v];
    reinterpret_cast<V *>(dst + (bh * R + r) * row_bytes)[v] = val;
  }
}

__global__ __launch_bounds__(kDedupThreads) void union_dedup_kernel(const int64_t *__restrict__ idx, int64_t GK,
                                                                   int64_t n, uint64_t *__restrict__ sorted,
                                                                   int32_t *__restrict__ n_unique) {
  __shared__ uint64_t s[kMaxGK];
  __shared__ uint32_t s_cnt;
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x;
  int P = 1;
  while (P < GK) P <<= 1;
  for (int i = tid; i < P; i += kDedupThreads) {
    uint64_t key = ((uint64_t)kTokPad << 32) | 0xFFFFFFFFull;
    if (i < GK) {
      const int64_t v = idx[bh * GK + i];
      const uint32_t tok = v < 0 ? kTokNeg : (uint32_t)(v < (int64_t)kTokNeg - 1 ? v : (int64_t)kTokNeg - 1);
      key = ((uint64_t)tok << 32) | (uint32_t)i;
    }
    s[i] = key;
  }
  if (tid == 0) s_cnt = 0u;
  __syncthreads();
  // ascending bitonic sort: equal tokens end up adjacent, positions ascending
  for (int kk = 2; kk <= P; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P; i += kDedupThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = s[i], b = s[ixj];
          const bool swap = ((i & kk) == 0) ? (a > b) : (a < b);
          if (swap) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  uint32_t local = 0;
  for (int i = tid; i < GK; i += kDedupThreads) {
    const uint64_t key = s[i];
    sorted[bh * GK + i] = key;
    const uint32_t tok = (uint32_t)(key >> 32);
    const bool first = i == 0 || (uint32_t)(s[i - 1] >> 32) != tok;
    local += (first && tok != kTokNeg && (int64_t)tok < n) ? 1u : 0u;
  }
  if (local) atomicAdd(&s_cnt, local);
  __syncthreads();
  if (tid == 0 && n_unique) n_unique[bh] = (int32_t)s_cnt;
}

__global__ __launch_bounds__(256) void union_fetch_kernel(const uint64_t *__restrict__ sorted, int64_t GK, int64_t n,
                                                          const char *__restrict__ Ksrc, const char *__restrict__ Vsrc,
                                                          int64_t cap, const char *__restrict__ Krec,
                                                          const char *__restrict__ Vrec, int64_t nrec,
                                                          int64_t row_bytes, char *__restrict__ Kout,
                                                          char *__restrict__ Vout) {
  const int lane = threadIdx.x & 63;
  const int64_t bh = blockIdx.y;
  const int64_t s = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= GK) return;
  const uint64_t *srt = sorted + bh * GK;
  const uint32_t tok = (uint32_t)(srt[s] >> 32);
  if (s > 0 && (uint32_t)(srt[s - 1] >> 32) == tok) return;  // not the first slot of this token
  const char *ks = nullptr;
  const char *vs = nullptr;
  if (tok != kTokNeg) {
    if ((int64_t)tok < n) {
      if ((int64_t)tok < cap) {
        ks = Ksrc + (bh * cap + tok) * row_bytes;
        vs = Vsrc + (bh * cap + tok) * row_bytes;
      }
    } else if (Krec && Vrec && nrec > 0) {
      int64_t r = (int64_t)tok - n;
      r = r < nrec ? r : nrec - 1;
      ks = Krec + (bh * nrec + r) * row_bytes;
      vs = Vrec + (bh * nrec + r) * row_bytes;
    }
  }
  for (int64_t o = (int64_t)lane * 4; o < row_bytes; o += kWave * 4) {
    const uint32_t kv = ks ? *reinterpret_cast<const uint32_t *>(ks + o) : 0u;
    const uint32_t vv = vs ? *reinterpret_cast<const uint32_t *>(vs + o) : 0u;
    for (int64_t s2 = s; s2 < GK; ++s2) {
      const uint64_t key = srt[s2];
      if ((uint32_t)(key >> 32) != tok) break;
      const int64_t pos = (int64_t)(uint32_t)key;
      *reinterpret_cast<uint32_t *>(Kout + (bh * GK + pos) * row_bytes + o) = kv;
      *reinterpret_cast<uint32_t *>(Vout + (bh * GK + pos) * row_bytes + o) = vv;
    }
  }
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_gather_rows(const void *src, int64_t cap, const int32_t *idx, int64_t BH, int64_t R,
                                  int64_t row_bytes, void *dst, void *stream) {
  if (!src || !idx || !dst) return fail(FATHOM_ERR_INVALID, "gather_rows: null pointer");
  if (BH < 1 || BH > 65535 || R < 0 || cap < 0) return fail(FATHOM_ERR_INVALID, "gather_rows: bad shape");
  if (row_bytes < 4 || row_bytes % 4) return fail(FATHOM_ERR_INVALID, "gather_rows: row_bytes=%lld not a multiple of 4", (long long)row_bytes);
  if (R == 0) return FATHOM_OK;
  dim3 grid((unsigned)cdiv(R, kRowsPerWG), (unsigned)BH);
  hipStream_t st = (hipStream_t)stream;
  const bool vec16 = row_bytes % 16 == 0 && ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
  if (vec16)
    gather_rows_kernel<uint4><<<grid, 256, 0, st>>>((const char *)src, cap, idx, R, row_bytes, (char *)dst);
  else
    gather_rows_kernel<uint32_t><<<grid, 256, 0, st>>>((const char *)src, cap, idx, R, row_bytes, (char *)dst);
  return launch_status("gather_rows_kernel");
}

extern "C" size_t fathom_gather_union_workspace_bytes(int64_t BH, int64_t GK) {
  if (BH < 1 || GK < 1) return 0;
  return (size_t)BH * (size_t)GK * 8;
}

extern "C" int fathom_gather_union(const int64_t *idx, int64_t BH, int64_t GK, int64_t n, const void *Ksrc,
                                   const void *Vsrc, int64_t cap, const void *Krec, const void *Vrec, int64_t nrec,
                                   int64_t row_bytes, void *Kout, void *Vout, int32_t *n_unique, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  if (!idx || !Ksrc || !Vsrc || !Kout || !Vout) return fail(FATHOM_ERR_INVALID, "gather_union: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "gather_union: BH=%lld outside [1, 65535]", (long long)BH);
  if (GK < 1 || GK > kMaxGK) return fail(FATHOM_ERR_INVALID, "gather_union: G*k=%lld outside [1, %d]", (long long)GK, kMaxGK);
  if (n < 0 || cap < 0) return fail(FATHOM_ERR_INVALID, "gather_union: bad n/cap");
  if (row_bytes < 4 || row_bytes % 4) return fail(FATHOM_ERR_INVALID, "gather_union: row_bytes=%lld not a multiple of 4", (long long)row_bytes);
  const size_t need = fathom_gather_union_workspace_bytes(BH, GK);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "gather_union: workspace %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  uint64_t *sorted = static_cast<uint64_t *>(workspace);
  union_dedup_kernel<<<(unsigned)BH, kDedupThreads, 0, st>>>(idx, GK, n, sorted, n_unique);
  int rc = launch_status("union_dedup_kernel");
  if (rc) return rc;
  dim3 grid((unsigned)cdiv(GK, 4), (unsigned)BH);
  union_fetch_kernel<<<grid, 256, 0, st>>>(sorted, GK, n, (const char *)Ksrc, (const char *)Vsrc, cap,
                                           (const char *)Krec, (const char *)Vrec, nrec, row_bytes, (char *)Kout,
                                           (char *)Vout);
  return launch_status("union_fetch_kernel");
}
