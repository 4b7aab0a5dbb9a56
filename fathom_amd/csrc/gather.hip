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
//   attend  (gather_attention) workgroups of 128 distinct tokens read each
//           token's K and V rows once, straight into registers, and form the
//           softmax numerators of every query head that selected the token,
//           weighted by the number of times that head selected it; each
//           workgroup writes a partial (max, sum, weighted V) triple per head
//           and a second kernel merges a row's triples in split order.
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
constexpr int kAttnWaves = 2;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kAttnTok = kAttnThreads;             // distinct tokens per workgroup (one per thread)
constexpr int kPartStride = kAttnD + 2;            // (max, sum, weighted V[128])
constexpr int kMaxSplit = kMaxGK / kAttnTok;       // workgroups per row at most

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

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

template <int G>
struct AttnShared {
  float q[G][kAttnD];            // the row's query heads
  float p[kAttnTok][G];          // softmax numerators of the workgroup's tokens
  int64_t vrow[kAttnTok];        // V row offset in bytes from its base (-1: zero row)
  uint8_t vrec[kAttnTok];        // 1: the row is in the recent buffer
  float wm[kAttnWaves][G], wl[kAttnWaves][G];
  float2 o[G][kWave];            // the second wave's weighted V sums
};

// Partial softmax attention of one workgroup's 128 distinct tokens for the G
// query heads of row bh, in two phases:
//   scores  thread t owns distinct token u0 + t: it reads the whole 256-byte K
//           row (16 x 16-byte loads) and forms q_g . K for every head g with
//           the query read from LDS (broadcast), so no cross-lane reductions;
//           the workgroup's max M_g and numerators c_g e^(s - M_g) follow;
//   values  lane l of each wave owns dimensions 2l and 2l + 1 and sums
//           p_g(token) V[token] over its wave's 64 tokens (one coalesced
//           256-byte V row per wave and token, 8 rows in flight).
template <int G>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(4))) void attn_partial_kernel(const float *__restrict__ q, UnionWs w,
                                                                    int64_t GK, RowSrc rs, float scale,
                                                                    float *__restrict__ part, int64_t nsplit) {
  __shared__ AttnShared<G> sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = blockIdx.y, split = blockIdx.x;
  const int64_t U = w.U[bh];
  for (int e = tid; e < G * kAttnD; e += kAttnThreads) sh.q[e / kAttnD][e % kAttnD] = q[bh * G * kAttnD + e];
  // ---- scores
  const int64_t u = split * kAttnTok + tid;
  uint4 cn = make_uint4(0u, 0u, 0u, 0u);
  const uint4 *krow = nullptr;
  int64_t vrow = -1;
  bool rec = false;
  if (u < U) {
    const uint64_t ent = w.ulist[bh * GK + u];
    cn = w.cnt[bh * GK + (uint32_t)ent];
    const int64_t row = rs.locate((uint32_t)(ent >> 32), bh, rec);
    if (row >= 0) {
      krow = reinterpret_cast<const uint4 *>((rec ? rs.Krec : rs.K) + row * rs.row_bytes);
      vrow = row * rs.row_bytes;
    }
  }
  sh.vrow[tid] = vrow;
  sh.vrec[tid] = rec ? 1 : 0;
  // unconditional loads (no branch per load): threads without a row read the
  // query array instead and their scores are replaced below
  const uint4 *kp = krow ? krow : reinterpret_cast<const uint4 *>(q);
  uint4 kv[kAttnD / 8];
#pragma unroll
  for (int j = 0; j < kAttnD / 8; ++j) kv[j] = kp[j];
  __syncthreads();  // q staged
  float s[G];
#pragma unroll
  for (int g = 0; g < G; ++g) s[g] = 0.0f;
#pragma unroll
  for (int j = 0; j < kAttnD / 8; ++j) {
    const uint32_t d4[4] = {kv[j].x, kv[j].y, kv[j].z, kv[j].w};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float4 qa = *reinterpret_cast<const float4 *>(&sh.q[g][8 * j]);
      const float4 qb = *reinterpret_cast<const float4 *>(&sh.q[g][8 * j + 4]);
      const float qq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t h = d4[e >> 1];
        const float kf = __uint_as_float((e & 1) ? (h & 0xFFFF0000u) : (h << 16));
        s[g] = fmaf(qq[e], kf, s[g]);
      }
      // keep the query reads of at most 4 heads in flight (hoisting them all
      // costs G * 128 registers)
      if ((g & 3) == 3 || g == G - 1) __builtin_amdgcn_sched_barrier(0);
    }
  }
  // every head's reductions before any lane-0 branch, so no score is computed late
  float c[G], wr[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    c[g] = (float)head_count(cn, g);
    s[g] = c[g] > 0.0f ? (krow ? s[g] * scale : 0.0f) : -INFINITY;  // a zero row scores 0
    wr[g] = wave_max_f(s[g]);
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) sh.wm[wave][g] = wr[g];
  }
  __syncthreads();
  float M[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    M[g] = -INFINITY;
#pragma unroll
    for (int v = 0; v < kAttnWaves; ++v) M[g] = fmaxf(M[g], sh.wm[v][g]);
    const float p = c[g] > 0.0f ? c[g] * expf(s[g] - M[g]) : 0.0f;
    sh.p[tid][g] = p;
    wr[g] = wave_sum_f(p);
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) sh.wl[wave][g] = wr[g];
  }
  __syncthreads();
  // ---- values: wave v sums tokens [64 v, 64 v + 64)
  float2 o[G];
#pragma unroll
  for (int g = 0; g < G; ++g) o[g] = make_float2(0.0f, 0.0f);
  const int t0 = wave * kWave;
#pragma unroll 1
  for (int r0 = 0; r0 < kWave; r0 += 8) {
    uint32_t vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // unconditional loads; rows without data read q and are zeroed
      const int64_t vr = sh.vrow[t0 + r0 + i];
      const char *vb = vr >= 0 ? (sh.vrec[t0 + r0 + i] ? rs.Vrec : rs.V) + vr : reinterpret_cast<const char *>(q);
      vv[i] = reinterpret_cast<const uint32_t *>(vb)[lane];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t vi = sh.vrow[t0 + r0 + i] >= 0 ? vv[i] : 0u;
      const float vx = __uint_as_float(vi << 16), vy = __uint_as_float(vi & 0xFFFF0000u);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = sh.p[t0 + r0 + i][g];
        o[g].x = fmaf(p, vx, o[g].x);
        o[g].y = fmaf(p, vy, o[g].y);
      }
    }
  }
  if (wave == 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) sh.o[g][lane] = o[g];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float *pp = part + ((bh * nsplit + split) * G + g) * kPartStride;
      if (lane == 0) {
        pp[0] = M[g];
        pp[1] = sh.wl[0][g] + sh.wl[1][g];
      }
      pp[2 + 2 * lane] = o[g].x + sh.o[g][lane].x;
      pp[3 + 2 * lane] = o[g].y + sh.o[g][lane].y;
    }
  }
}

// out[bh, g, d] = sum_s O_s e^(M_s - M) / sum_s L_s e^(M_s - M) over the
// row's splits (<= kMaxSplit), in split order.
__global__ __launch_bounds__(kAttnD) void attn_merge_kernel(const float *__restrict__ part, int64_t G,
                                                            int64_t nsplit, float *__restrict__ out) {
  __shared__ float wt[kMaxSplit];
  __shared__ float s_L;
  const int64_t r = blockIdx.x;  // bh * G + g
  const int64_t bh = r / G, g = r % G;
  const int d = threadIdx.x;
  const float *base = part + (bh * nsplit * G + g) * kPartStride;  // split s at + s * G * kPartStride
  const int64_t sstride = G * kPartStride;
  if (d < nsplit) wt[d] = base[d * sstride];
  __syncthreads();
  if (d == 0) {
    float M = -INFINITY;
    for (int s = 0; s < (int)nsplit; ++s) M = fmaxf(M, wt[s]);
    float L = 0.0f;
    for (int s = 0; s < (int)nsplit; ++s) {
      const float e = wt[s] == -INFINITY ? 0.0f : expf(wt[s] - M);
      wt[s] = e;
      L = fmaf(base[s * sstride + 1], e, L);
    }
    s_L = L;
  }
  __syncthreads();
  float Od = 0.0f;
  for (int s0 = 0; s0 < (int)nsplit; s0 += 8) {
    float ov[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ov[i] = s0 + i < nsplit ? base[(s0 + i) * sstride + 2 + d] : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (s0 + i < nsplit) Od = fmaf(ov[i], wt[s0 + i], Od);
  }
  out[r * kAttnD + d] = Od / s_L;
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
  attn_partial_kernel<G><<<dim3((unsigned)nsplit, (unsigned)BH), kAttnThreads, 0, st>>>(q, w, GK, rs, scale, part,
                                                                                         nsplit);
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
