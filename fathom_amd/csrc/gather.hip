// Row gathers of the selected K/V tokens, from HBM or zero-copy from mapped
// pinned host memory, and exact attention over the gathered rows.
//
// gather_rows: the reference kernel's semantics, one 16-byte vector per lane.
// Group union (the decode step's fetch of the G query heads' selections):
//   dedup   one workgroup per (batch*KV head) row inserts its G*k tokens into
//           an LDS hash table (open addressing, linear probing).  The positions
//           holding one token form a chain (an atomic exchange on the slot's
//           chain head links each new position to the previous one); the
//           position that ends up at the chain head walks it, counts the
//           token's positions per query head and marks the token's first
//           position.  An ordered compaction of the marks then lists the
//           distinct tokens in first-position order, so everything downstream
//           is deterministic although the hash layout is not;
//   fetch   one wave per distinct token reads its row once (host store,
//           recent-token device buffer, or a zero row for negative tokens) and
//           writes it to every position of its chain, so each distinct host
//           row crosses PCIe exactly once;
//   attend  (gather_attention) one wave per distinct token reads the K and V
//           rows straight into registers and updates a running softmax of
//           every query head that selected it, weighted by the number of times
//           that head selected it; workgroups hold 32 distinct tokens and
//           write partial (max, sum, weighted V) triples that a second kernel
//           merges in a fixed order.
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kRowsPerWG = 16;
constexpr int kMaxGK = 16384;
constexpr int kDedupThreads = 1024;
constexpr int kDedupPer = kMaxGK / kDedupThreads;  // positions per thread at most
constexpr int kHashSlots = 16384;                  // >= kMaxGK: the table never fills
constexpr int kMaxHeads = 8;                       // query heads counted per token
constexpr uint32_t kTokNeg = 0xFFFFFFFEu;          // token key of negative indices
constexpr int kAttnD = 128;                        // head dimension of gather_attention
constexpr int kAttnWaves = 4;
constexpr int kAttnPerWave = 8;                            // distinct tokens per wave
constexpr int kAttnTok = kAttnWaves * kAttnPerWave;        // distinct tokens per workgroup
constexpr int kPartStride = kAttnD + 2;                    // (max, sum, weighted V[128])

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

// ------------------------------------------------------------------ group union
struct UnionWs {
  int32_t *nxt;     // [BH, GK] next position holding the same token (-1: end of chain)
  int32_t *cstart;  // [BH, GK] at a token's first position: the start of its chain
  uint4 *cnt;       // [BH, GK] at a token's first position: positions per query head, 8 x uint16
  uint64_t *ulist;  // [BH, GK] distinct tokens in first-position order: token << 32 | first position
  int32_t *U;       // [BH] number of distinct tokens (the negative-index key included)
};

size_t union_ws_layout(int64_t BH, int64_t GK, char *base, UnionWs *w) {
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t e = (size_t)BH * (size_t)GK;
  const size_t o_nxt = 0, o_cs = o_nxt + al(e * 4), o_cnt = o_cs + al(e * 4), o_ul = o_cnt + al(e * 16),
               o_u = o_ul + al(e * 8), end = o_u + al((size_t)BH * 4);
  if (w) {
    w->nxt = reinterpret_cast<int32_t *>(base + o_nxt);
    w->cstart = reinterpret_cast<int32_t *>(base + o_cs);
    w->cnt = reinterpret_cast<uint4 *>(base + o_cnt);
    w->ulist = reinterpret_cast<uint64_t *>(base + o_ul);
    w->U = reinterpret_cast<int32_t *>(base + o_u);
  }
  return end;
}

__device__ __forceinline__ uint32_t tok_key(int64_t v) {
  return v < 0 ? kTokNeg : (uint32_t)(v < (int64_t)kTokNeg - 1 ? v : (int64_t)kTokNeg - 1);
}

// idx [BH, GK]: position p belongs to query head p / k (k = GK for a plain union).
__global__ __launch_bounds__(kDedupThreads) void union_dedup_kernel(const int64_t *__restrict__ idx, int64_t GK,
                                                                    int64_t k, int64_t n, int hbits, UnionWs w,
                                                                    int32_t *__restrict__ n_unique) {
  __shared__ uint32_t hkey[kHashSlots];  // token + 1 (0: empty)
  __shared__ int32_t hhead[kHashSlots];  // latest position inserted with this token
  __shared__ uint8_t first[kMaxGK];      // 1 at a token's first position
  __shared__ int32_t wsum[kDedupThreads / kWave];
  __shared__ int32_t s_valid;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = blockIdx.x;
  const int HS = 1 << hbits;
  const int E = (int)cdiv(GK, kDedupThreads);  // thread t owns positions [t * E, t * E + E)
  for (int i = tid; i < HS; i += kDedupThreads) {
    hkey[i] = 0u;
    hhead[i] = -1;
  }
  for (int i = tid; i < (int)GK; i += kDedupThreads) first[i] = 0;
  if (tid == 0) s_valid = 0;
  __syncthreads();
  int32_t *nxt = w.nxt + bh * GK;
  uint32_t tok[kDedupPer];
  int slot[kDedupPer];
#pragma unroll
  for (int e = 0; e < kDedupPer; ++e) {
    const int p = tid * E + e;
    tok[e] = 0u;
    slot[e] = -1;
    if (e < E && p < (int)GK) {
      const uint32_t t = tok_key(idx[bh * GK + p]);
      const uint32_t key = t + 1u;  // t <= kTokNeg, so key != 0
      uint32_t s = (t * 2654435761u) >> (32 - hbits);
      for (int it = 0; it < HS; ++it) {  // ends at the token's slot: HS >= GK >= distinct tokens
        const uint32_t old = atomicCAS(&hkey[s], 0u, key);
        if (old == 0u || old == key) break;
        s = (s + 1u) & (uint32_t)(HS - 1);
      }
      tok[e] = t;
      slot[e] = (int)s;
      nxt[p] = atomicExch(&hhead[s], p);
    }
  }
  __syncthreads();  // chains complete (nxt is read back by other waves of this workgroup)
#pragma unroll
  for (int e = 0; e < kDedupPer; ++e) {
    const int p = tid * E + e;
    if (slot[e] >= 0 && hhead[slot[e]] == p) {  // the chain head walks the token's positions
      int q = p, minp = p;
      uint64_t c_lo = 0ull, c_hi = 0ull;  // 16-bit counts of heads 0-3 and 4-7
      for (int it = 0; it < (int)GK && q >= 0; ++it) {
        const int g = (int)((uint32_t)q / (uint32_t)k);
        if (g < 4)
          c_lo += 1ull << (16 * g);
        else if (g < kMaxHeads)
          c_hi += 1ull << (16 * (g - 4));
        minp = q < minp ? q : minp;
        q = nxt[q];
      }
      first[minp] = 1;
      w.cstart[bh * GK + minp] = p;
      w.cnt[bh * GK + minp] = make_uint4((uint32_t)c_lo, (uint32_t)(c_lo >> 32), (uint32_t)c_hi,
                                         (uint32_t)(c_hi >> 32));
    }
  }
  __syncthreads();
  // ordered compaction of the first positions
  int f = 0;
#pragma unroll
  for (int e = 0; e < kDedupPer; ++e) {
    const int p = tid * E + e;
    if (e < E && p < (int)GK && first[p]) ++f;
  }
  const int ex = wave_excl_scan_i(f, lane);
  if (lane == kWave - 1) wsum[wave] = ex + f;
  __syncthreads();
  int base = 0, total = 0;
  for (int w2 = 0; w2 < kDedupThreads / kWave; ++w2) {
    base += w2 < wave ? wsum[w2] : 0;
    total += wsum[w2];
  }
  int u = base + ex, valid = 0;
#pragma unroll
  for (int e = 0; e < kDedupPer; ++e) {
    const int p = tid * E + e;
    if (e < E && p < (int)GK && first[p]) {
      w.ulist[bh * GK + u] = ((uint64_t)tok[e] << 32) | (uint32_t)p;
      ++u;
      valid += (tok[e] != kTokNeg && (int64_t)tok[e] < n) ? 1 : 0;
    }
  }
  valid = wave_sum_i(valid);
  if (lane == 0 && valid) atomicAdd(&s_valid, valid);
  __syncthreads();
  if (tid == 0) {
    w.U[bh] = total;
    if (n_unique) n_unique[bh] = s_valid;
  }
}

// Where a token's row lives: the host store (tokens < min(n, cap)), the recent
// buffer (tokens >= n, clamped to its last row), or nowhere (a zero row).
struct RowSrc {
  const char *K, *V, *Krec, *Vrec;
  int64_t cap, nrec, n, row_bytes;
  __device__ __forceinline__ int64_t locate(uint32_t tok, int64_t bh, bool &rec) const {
    rec = false;
    if (tok == kTokNeg) return -1;
    if ((int64_t)tok < n) return (int64_t)tok < cap ? bh * cap + tok : -1;
    if (!Krec || !Vrec || nrec <= 0) return -1;
    rec = true;
    const int64_t r = (int64_t)tok - n;
    return bh * nrec + (r < nrec ? r : nrec - 1);
  }
};

__global__ __launch_bounds__(256) void union_fetch_kernel(UnionWs w, int64_t GK, RowSrc rs, char *__restrict__ Kout,
                                                          char *__restrict__ Vout) {
  const int lane = threadIdx.x & 63;
  const int64_t bh = blockIdx.y;
  const int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (u >= (int64_t)w.U[bh]) return;
  const uint64_t ent = w.ulist[bh * GK + u];
  const uint32_t tok = (uint32_t)(ent >> 32);
  const int32_t c0 = w.cstart[bh * GK + (uint32_t)ent];
  const int32_t *nxt = w.nxt + bh * GK;
  bool rec;
  const int64_t row = rs.locate(tok, bh, rec);
  const char *ks = row < 0 ? nullptr : (rec ? rs.Krec : rs.K) + row * rs.row_bytes;
  const char *vs = row < 0 ? nullptr : (rec ? rs.Vrec : rs.V) + row * rs.row_bytes;
  for (int64_t o = (int64_t)lane * 4; o < rs.row_bytes; o += kWave * 4) {
    const uint32_t kv = ks ? *reinterpret_cast<const uint32_t *>(ks + o) : 0u;
    const uint32_t vv = vs ? *reinterpret_cast<const uint32_t *>(vs + o) : 0u;
    int q = c0;
    for (int it = 0; it < (int)GK && q >= 0; ++it) {
      *reinterpret_cast<uint32_t *>(Kout + (bh * GK + q) * rs.row_bytes + o) = kv;
      *reinterpret_cast<uint32_t *>(Vout + (bh * GK + q) * rs.row_bytes + o) = vv;
      q = nxt[q];
    }
  }
}

// ------------------------------------------------------------------ attention
__device__ __forceinline__ uint32_t head_count(const uint4 &c, int g) {
  const uint32_t w = g < 2 ? c.x : g < 4 ? c.y : g < 6 ? c.z : c.w;
  return (g & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// Partial softmax attention of one workgroup's 32 distinct tokens for the G
// query heads of row bh.  Lane l holds dimensions 2l and 2l + 1 (bf16 rows of
// 128 elements: one dword of K and one of V per lane and token).
template <int G>
__global__ __launch_bounds__(kAttnWaves * kWave) void attn_partial_kernel(const float *__restrict__ q, UnionWs w,
                                                                          int64_t GK, RowSrc rs, float scale,
                                                                          float *__restrict__ part, int64_t nsplit) {
  __shared__ float sm[kAttnWaves][G], sl[kAttnWaves][G];
  __shared__ float2 so[kAttnWaves][G][kWave];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t bh = blockIdx.y, split = blockIdx.x;
  const int64_t U = w.U[bh];
  float2 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = reinterpret_cast<const float2 *>(q + (bh * G + g) * kAttnD)[lane];
  float m[G], l[G];
  float2 o[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
    o[g] = make_float2(0.0f, 0.0f);
  }
  const int64_t u0 = split * kAttnTok + wave * kAttnPerWave;
  // every row of the wave in flight before the first use
  uint32_t kw[kAttnPerWave], vw[kAttnPerWave];
  uint4 cn[kAttnPerWave];
#pragma unroll
  for (int i = 0; i < kAttnPerWave; ++i) {
    kw[i] = 0u;
    vw[i] = 0u;
    cn[i] = make_uint4(0u, 0u, 0u, 0u);
    const int64_t u = u0 + i;
    if (u < U) {
      const uint64_t ent = w.ulist[bh * GK + u];
      const uint32_t tok = (uint32_t)(ent >> 32);
      cn[i] = w.cnt[bh * GK + (uint32_t)ent];
      bool rec;
      const int64_t row = rs.locate(tok, bh, rec);
      if (row >= 0) {
        kw[i] = reinterpret_cast<const uint32_t *>((rec ? rs.Krec : rs.K) + row * rs.row_bytes)[lane];
        vw[i] = reinterpret_cast<const uint32_t *>((rec ? rs.Vrec : rs.V) + row * rs.row_bytes)[lane];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kAttnPerWave; ++i) {
    const float kx = bf16_bits_to_float((uint16_t)(kw[i] & 0xFFFFu)), ky = bf16_bits_to_float((uint16_t)(kw[i] >> 16));
    const float vx = bf16_bits_to_float((uint16_t)(vw[i] & 0xFFFFu)), vy = bf16_bits_to_float((uint16_t)(vw[i] >> 16));
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = fmaf(qv[g].y, ky, qv[g].x * kx);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
      for (int g = 0; g < G; ++g) s[g] += __shfl_xor(s[g], off, kWave);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t c = head_count(cn[i], g);
      if (c) {
        const float sc = s[g] * scale;
        const float mn = fmaxf(m[g], sc);
        const float a = expf(m[g] - mn);
        const float p = (float)c * expf(sc - mn);
        l[g] = fmaf(l[g], a, p);
        o[g].x = fmaf(o[g].x, a, p * vx);
        o[g].y = fmaf(o[g].y, a, p * vy);
        m[g] = mn;
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) {
      sm[wave][g] = m[g];
      sl[wave][g] = l[g];
    }
    so[wave][g][lane] = o[g];
  }
  __syncthreads();
  // merge the waves in wave order: thread (g, lane) of the first G waves' slots
  for (int e = threadIdx.x; e < G * kWave; e += kAttnWaves * kWave) {
    const int g = e / kWave, ln = e % kWave;
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < kAttnWaves; ++v) M = fmaxf(M, sm[v][g]);
    float L = 0.0f;
    float2 Ov = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int v = 0; v < kAttnWaves; ++v) {
      if (sm[v][g] != -INFINITY) {
        const float wt = expf(sm[v][g] - M);
        L = fmaf(sl[v][g], wt, L);
        Ov.x = fmaf(so[v][g][ln].x, wt, Ov.x);
        Ov.y = fmaf(so[v][g][ln].y, wt, Ov.y);
      }
    }
    float *pp = part + ((bh * nsplit + split) * G + g) * kPartStride;
    if (ln == 0) {
      pp[0] = M;
      pp[1] = L;
    }
    pp[2 + 2 * ln] = Ov.x;
    pp[3 + 2 * ln] = Ov.y;
  }
}

// out[bh, g, d] = sum_s O_s e^(M_s - M) / sum_s L_s e^(M_s - M), splits in order.
__global__ __launch_bounds__(kAttnD) void attn_merge_kernel(const float *__restrict__ part, int64_t G,
                                                            int64_t nsplit, float *__restrict__ out) {
  const int64_t r = blockIdx.x;  // bh * G + g
  const int64_t bh = r / G, g = r % G;
  const int d = threadIdx.x;
  float M = -INFINITY;
  for (int64_t s = 0; s < nsplit; ++s) M = fmaxf(M, part[((bh * nsplit + s) * G + g) * kPartStride]);
  float L = 0.0f, Od = 0.0f;
  for (int64_t s = 0; s < nsplit; ++s) {
    const float *pp = part + ((bh * nsplit + s) * G + g) * kPartStride;
    if (pp[0] != -INFINITY) {
      const float wt = expf(pp[0] - M);
      L = fmaf(pp[1], wt, L);
      Od = fmaf(pp[2 + d], wt, Od);
    }
  }
  out[r * kAttnD + d] = Od / L;
}

int hash_bits(int64_t GK) {
  int b = 6;
  while ((1 << b) < 2 * GK && (1 << b) < kHashSlots) ++b;
  return b;
}

int launch_union(const int64_t *idx, int64_t BH, int64_t GK, int64_t k, int64_t n, const UnionWs &w, int32_t *n_unique,
                 hipStream_t st) {
  union_dedup_kernel<<<(unsigned)BH, kDedupThreads, 0, st>>>(idx, GK, k, n, hash_bits(GK), w, n_unique);
  return launch_status("union_dedup_kernel");
}

template <int G>
void launch_attn_g(const float *q, const UnionWs &w, int64_t BH, int64_t GK, const RowSrc &rs, float scale, float *part,
                   int64_t nsplit, hipStream_t st) {
  attn_partial_kernel<G><<<dim3((unsigned)nsplit, (unsigned)BH), kAttnWaves * kWave, 0, st>>>(q, w, GK, rs, scale,
                                                                                               part, nsplit);
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
  return union_ws_layout(BH, GK, nullptr, nullptr);
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
  UnionWs w;
  union_ws_layout(BH, GK, static_cast<char *>(workspace), &w);
  int rc = launch_union(idx, BH, GK, GK, n, w, n_unique, st);
  if (rc) return rc;
  const RowSrc rs{(const char *)Ksrc, (const char *)Vsrc, (const char *)Krec, (const char *)Vrec,
                  cap, nrec, n, row_bytes};
  dim3 grid((unsigned)cdiv(GK, 4), (unsigned)BH);
  union_fetch_kernel<<<grid, 256, 0, st>>>(w, GK, rs, (char *)Kout, (char *)Vout);
  return launch_status("union_fetch_kernel");
}

extern "C" size_t fathom_gather_attention_workspace_bytes(int64_t BH, int64_t G, int64_t k) {
  if (BH < 1 || G < 1 || k < 1) return 0;
  const int64_t GK = G * k, nsplit = cdiv(GK, kAttnTok);
  return union_ws_layout(BH, GK, nullptr, nullptr) + (size_t)BH * nsplit * G * kPartStride * sizeof(float);
}

extern "C" int fathom_gather_attention(const float *q, const int64_t *idx, int64_t BH, int64_t G, int64_t k, int64_t n,
                                       const void *Ksrc, const void *Vsrc, int64_t cap, const void *Krec,
                                       const void *Vrec, int64_t nrec, float scale, float *out, int32_t *n_unique,
                                       void *workspace, size_t workspace_bytes, void *stream) {
  if (!q || !idx || !Ksrc || !Vsrc || !out) return fail(FATHOM_ERR_INVALID, "gather_attention: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "gather_attention: BH=%lld outside [1, 65535]", (long long)BH);
  if (G < 1 || G > kMaxHeads) return fail(FATHOM_ERR_INVALID, "gather_attention: G=%lld outside [1, %d]", (long long)G, kMaxHeads);
  if (k < 1 || G * k > kMaxGK)
    return fail(FATHOM_ERR_INVALID, "gather_attention: G*k=%lld outside [1, %d]", (long long)(G * k), kMaxGK);
  if (n < 0 || cap < 0 || nrec < 0) return fail(FATHOM_ERR_INVALID, "gather_attention: bad n/cap/nrec");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(Ksrc) | reinterpret_cast<uintptr_t>(Vsrc)) & 7)
    return fail(FATHOM_ERR_INVALID, "gather_attention: q, K and V must be 8-byte aligned");
  const size_t need = fathom_gather_attention_workspace_bytes(BH, G, k);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "gather_attention: workspace %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int64_t GK = G * k, nsplit = cdiv(GK, kAttnTok);
  UnionWs w;
  const size_t off = union_ws_layout(BH, GK, static_cast<char *>(workspace), &w);
  float *part = reinterpret_cast<float *>(static_cast<char *>(workspace) + off);
  int rc = launch_union(idx, BH, GK, k, n, w, n_unique, st);
  if (rc) return rc;
  const RowSrc rs{(const char *)Ksrc, (const char *)Vsrc, (const char *)Krec, (const char *)Vrec,
                  cap, nrec, n, (int64_t)kAttnD * 2};
  switch (G) {
    case 1: launch_attn_g<1>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    case 2: launch_attn_g<2>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    case 3: launch_attn_g<3>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    case 4: launch_attn_g<4>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    case 5: launch_attn_g<5>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    case 6: launch_attn_g<6>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    case 7: launch_attn_g<7>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
    default: launch_attn_g<8>(q, w, BH, GK, rs, scale, part, nsplit, st); break;
  }
  rc = launch_status("attn_partial_kernel");
  if (rc) return rc;
  attn_merge_kernel<<<(unsigned)(BH * G), kAttnD, 0, st>>>(part, G, nsplit, out);
  return launch_status("attn_merge_kernel");
}
