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
//   wide    rows of more than 16384 positions (and distinct-row counts over
//           more than 8 query heads) keep the table in global memory instead:
//           the same rows and counts, no shape limit;
//   attend  (gather_attention) the K and V rows are read 16 lanes per 256-byte
//           row, so every load instruction reads whole rows, and form the
//           softmax numerators of the query heads, weighted by the times a
//           head selected the token.  Over the union (host-resident rows:
//           each row crosses PCIe once), workgroups of 64 distinct tokens
//           write a partial (max, sum, weighted V) triple per head and a
//           second kernel merges a row's triples in split order; without it
//           (rows in device memory), one workgroup per query head folds its
//           own positions 256 at a time and writes the output: one launch.
#include "attn_core.hpp"

namespace fathom {
namespace {

using namespace attn;

constexpr int kRowsPerWG = 16;
constexpr int kMaxGK = 16384;
constexpr int kDedupThreads = 1024;
constexpr int kDedupPer = kMaxGK / kDedupThreads;  // positions per thread at most
constexpr int kHashSlots = 16384;                  // >= kMaxGK: the table never fills
constexpr int kMaxHeads = 8;                       // query heads counted per token
constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kAttnTok = 16 * kAttnWaves;          // distinct tokens per workgroup (16 per wave)

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

// ------------------------------------------------------------------ wide union
// Rows of more than kMaxGK positions, or distinct-row counts over more than
// kMaxHeads query heads: the same semantics from a hash table in global memory
// (2^hbits >= 2 GK slots per row, so a probe always ends at its token's slot).
// The lowest position holding a token (an atomic minimum per slot) fetches its
// row once; the token's other positions copy it from there afterwards.
struct WideUnionWs {
  uint32_t *key;   // [BH, S] token key + 1 (0: empty)
  int32_t *first;  // [BH, S] lowest position holding the slot's token
  int32_t *slot;   // [BH, GK] slot of each position's token
  int64_t S;
  int hbits;
};

size_t wide_union_layout(int64_t BH, int64_t GK, char *base, WideUnionWs *w) {
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  int hb = 6;
  while ((int64_t(1) << hb) < 2 * GK) ++hb;
  const int64_t S = int64_t(1) << hb;
  const size_t o_first = al((size_t)BH * S * 4), o_slot = o_first + al((size_t)BH * S * 4),
               end = o_slot + al((size_t)BH * GK * 4);
  if (w) {
    w->key = reinterpret_cast<uint32_t *>(base);
    w->first = reinterpret_cast<int32_t *>(base + o_first);
    w->slot = reinterpret_cast<int32_t *>(base + o_slot);
    w->S = S;
    w->hbits = hb;
  }
  return end;
}

__global__ __launch_bounds__(256) void wide_union_clear_kernel(WideUnionWs w, int64_t BH, int32_t *__restrict__ n_unique) {
  const int64_t total = BH * w.S;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    w.key[i] = 0u;
    w.first[i] = 0x7FFFFFFF;
    if (n_unique && i < BH) n_unique[i] = 0;
  }
}

__global__ __launch_bounds__(256) void wide_union_insert_kernel(const int64_t *__restrict__ idx, int64_t GK,
                                                                WideUnionWs w) {
  const int64_t bh = blockIdx.y;
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= GK) return;
  const uint32_t t = tok_key(idx[bh * GK + p]);
  const uint32_t key = t + 1u;  // t <= kTokNeg, so key != 0
  uint32_t *hk = w.key + bh * w.S;
  const uint32_t smask = (uint32_t)(w.S - 1);
  uint32_t s = (uint32_t)(((uint64_t)(t * 2654435761u) << w.hbits) >> 32) & smask;
  for (int64_t it = 0; it < w.S; ++it) {  // ends at the token's slot: the table is at most half full
    const uint32_t old = atomicCAS(&hk[s], 0u, key);
    if (old == 0u || old == key) break;
    s = (s + 1u) & smask;
  }
  atomicMin(&w.first[bh * w.S + s], (int32_t)p);
  w.slot[bh * GK + p] = (int32_t)s;
}

// n_unique[bh] += distinct tokens < n (a thread per position, one atomic per workgroup).
__global__ __launch_bounds__(256) void wide_union_count_kernel(const int64_t *__restrict__ idx, int64_t GK, int64_t n,
                                                               WideUnionWs w, int32_t *__restrict__ n_unique) {
  __shared__ int32_t part[256 / kWave];
  const int64_t bh = blockIdx.y;
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int c = 0;
  if (p < GK) {
    const uint32_t t = tok_key(idx[bh * GK + p]);
    c = (t != kTokNeg && (int64_t)t < n && w.first[bh * w.S + w.slot[bh * GK + p]] == (int32_t)p) ? 1 : 0;
  }
  c = wave_sum_i(c);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int tot = part[0] + part[1] + part[2] + part[3];
    if (tot) atomicAdd(&n_unique[bh], tot);
  }
}

// A wave per position: first positions read their token's row (as
// union_fetch_kernel), the others copy it from the first position's output
// row (DUP, launched after the fetch).
template <bool DUP>
__global__ __launch_bounds__(256) void wide_union_fetch_kernel(const int64_t *__restrict__ idx, int64_t GK,
                                                               WideUnionWs w, RowSrc rs, char *__restrict__ Kout,
                                                               char *__restrict__ Vout) {
  const int lane = threadIdx.x & 63;
  const int64_t bh = blockIdx.y;
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (p >= GK) return;
  const int32_t fp = w.first[bh * w.S + w.slot[bh * GK + p]];
  if ((fp != (int32_t)p) != DUP) return;
  const char *ks, *vs;
  if (DUP) {
    ks = Kout + (bh * GK + fp) * rs.row_bytes;
    vs = Vout + (bh * GK + fp) * rs.row_bytes;
  } else {
    bool rec;
    const int64_t row = rs.locate(tok_key(idx[bh * GK + p]), bh, rec);
    ks = row < 0 ? nullptr : (rec ? rs.Krec : rs.K) + row * rs.row_bytes;
    vs = row < 0 ? nullptr : (rec ? rs.Vrec : rs.V) + row * rs.row_bytes;
  }
  char *kd = Kout + (bh * GK + p) * rs.row_bytes;
  char *vd = Vout + (bh * GK + p) * rs.row_bytes;
  for (int64_t o = (int64_t)lane * 4; o < rs.row_bytes; o += kWave * 4) {
    *reinterpret_cast<uint32_t *>(kd + o) = ks ? *reinterpret_cast<const uint32_t *>(ks + o) : 0u;
    *reinterpret_cast<uint32_t *>(vd + o) = vs ? *reinterpret_cast<const uint32_t *>(vs + o) : 0u;
  }
}

// The table of every row, and n_unique when given.
int launch_wide_union(const int64_t *idx, int64_t BH, int64_t GK, int64_t n, const WideUnionWs &w, int32_t *n_unique,
                      hipStream_t st) {
  const int64_t cells = BH * w.S;
  wide_union_clear_kernel<<<(unsigned)min(cdiv(cells, 256), (int64_t)16384), 256, 0, st>>>(w, BH, n_unique);
  int rc = launch_status("wide_union_clear_kernel");
  if (rc) return rc;
  const dim3 grid((unsigned)cdiv(GK, 256), (unsigned)BH);
  wide_union_insert_kernel<<<grid, 256, 0, st>>>(idx, GK, w);
  rc = launch_status("wide_union_insert_kernel");
  if (rc || !n_unique) return rc;
  wide_union_count_kernel<<<grid, 256, 0, st>>>(idx, GK, n, w, n_unique);
  return launch_status("wide_union_count_kernel");
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

// LDS of an attention workgroup of NW waves (16 tokens per wave).
template <int G, int NW = kAttnWaves, int NC = 1>
struct AttnShared {
  float q[G][kAttnD];            // the row's query heads
  uint64_t kaddr[16 * NW * NC];  // K and V row addresses of the workgroup's tokens (0: zero row), NC groups
  uint64_t vaddr[16 * NW * NC];
  uint4 cnt[16 * NW * NC];       // per-head selection counts (0 past the row's distinct tokens)
  float wm[NW][G], wl[NW][G];
  float o[NW][G][kAttnD];        // the waves' weighted V sums
};

// Softmax attention over the 16 NW tokens whose K/V row addresses and
// per-head counts are in sh (kaddr, vaddr, cnt; the whole workgroup calls it,
// after a barrier that completes them).  Wave w takes tokens 16 w .. 16 w +
// 15; lane l reads dims 8 (l & 15) .. + 7 of the rows of tokens 16 w + 4 j +
// (l >> 4), j < 4, so each load instruction reads four whole 256-byte rows,
// and the K and V rows are loaded together.  Then:
//   scores  partial dots of 8 dims per lane, summed over the 16 lanes of a
//           row (DPP); the tokens' maximum M_g and the numerators
//           c_g e^(s - M_g) (c_g: the times head g selected the token);
//   values  each lane sums p V over its dims and tokens, and the four row
//           groups of a wave are summed by row swaps.
// Leaves each wave's maximum, numerator sum and weighted V sums of every head
// in sh.wm, sh.wl and sh.o (complete after the caller's next barrier).  Rows
// without data (address 0) score 0 and add nothing to V; qa: any 256 readable
// bytes, read in their place.
// The lane's K and V row pieces of one group of 16 NW tokens (the group at
// token t0 of the address arrays), loads only.
struct AttnRows {
  u32x4 kv[4], vv[4];
  bool has[4];
};

template <int G, int NW, int NC>
__device__ __forceinline__ void attn_load(const AttnShared<G, NW, NC> &sh, int t0, uint64_t qa, AttnRows &r) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane >> 4, ds = lane & 15;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = t0 + 16 * wave + 4 * j + rg;
    const uint64_t ka = sh.kaddr[t], va = sh.vaddr[t];
    r.has[j] = ka != 0ull;
    r.kv[j] = reinterpret_cast<gptr4>(ka ? ka : qa)[ds];
    r.vv[j] = reinterpret_cast<gptr4>(va ? va : qa)[ds];
  }
}

template <int G, int NW = kAttnWaves>
__device__ __forceinline__ void attn_tokens(AttnShared<G, NW> &sh, uint64_t qa, float scale);

template <int G, int NW, int NC>
__device__ __forceinline__ void attn_compute(AttnShared<G, NW, NC> &sh, int t0, const AttnRows &r, float scale) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = lane >> 4, ds = lane & 15;
  const u32x4(&kv)[4] = r.kv;
  const u32x4(&vv)[4] = r.vv;
  const bool(&has)[4] = r.has;
  // ---- scores
  float s[4][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float4 q0 = *reinterpret_cast<const float4 *>(&sh.q[g][8 * ds]);
    const float4 q1 = *reinterpret_cast<const float4 *>(&sh.q[g][8 * ds + 4]);
    const float qq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d4[4] = {kv[j].x, kv[j].y, kv[j].z, kv[j].w};
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t h = d4[e >> 1];
        a = fmaf(qq[e], __uint_as_float((e & 1) ? (h & 0xFFFF0000u) : (h << 16)), a);
      }
      s[j][g] = a;
    }
  }
  float c[4][G];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 cn = sh.cnt[t0 + 16 * wave + 4 * j + rg];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      c[j][g] = (float)head_count(cn, g);
      const float sc = row16_reduce<false>(s[j][g]);
      s[j][g] = c[j][g] > 0.0f ? (has[j] ? sc * scale : 0.0f) : -INFINITY;  // a zero row scores 0
    }
  }
  // ---- softmax over the tokens
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = fmaxf(fmaxf(s[0][g], s[1][g]), fmaxf(s[2][g], s[3][g]));
    m = across_rows<true>(m);
    if (lane == 0) sh.wm[wave][g] = m;
  }
  __syncthreads();
  float l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) M = fmaxf(M, sh.wm[v][g]);
    float ls = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s[j][g] = c[j][g] > 0.0f ? c[j][g] * expf(s[j][g] - M) : 0.0f;  // the numerator p
      ls += s[j][g];
    }
    l[g] = ls;
  }
  // ---- values: the lane's 8 dims over its 4 tokens, then over the wave's rows
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d4[4] = {vv[j].x, vv[j].y, vv[j].z, vv[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t h = has[j] ? d4[e >> 1] : 0u;
        o[e] = fmaf(s[j][g], __uint_as_float((e & 1) ? (h & 0xFFFF0000u) : (h << 16)), o[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = across_rows<false>(o[e]);
    if (rg == 0) {
      *reinterpret_cast<float4 *>(&sh.o[wave][g][8 * ds]) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4 *>(&sh.o[wave][g][8 * ds + 4]) = make_float4(o[4], o[5], o[6], o[7]);
    }
    const float lw = across_rows<false>(l[g]);
    if (lane == 0) sh.wl[wave][g] = lw;
  }
}

template <int G, int NW>
__device__ __forceinline__ void attn_tokens(AttnShared<G, NW> &sh, uint64_t qa, float scale) {
  AttnRows r;
  attn_load(sh, 0, qa, r);
  attn_compute(sh, 0, r, scale);
}

// Partial attention of one workgroup's kAttnTok distinct tokens of the union
// list (tokens [split * kAttnTok, + kAttnTok) of row bh): the (M, sum,
// weighted V) triple of every head.
template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(const float *__restrict__ q, UnionWs w, int64_t GK,
                                                                    RowSrc rs, float scale, float *__restrict__ part,
                                                                    int64_t nsplit) {
  __shared__ AttnShared<G> sh;
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.y, split = blockIdx.x;
  const int64_t U = w.U[bh];
  for (int e = tid; e < G * kAttnD; e += kAttnThreads) sh.q[e / kAttnD][e % kAttnD] = q[bh * G * kAttnD + e];
  if (tid < kAttnTok) {
    const int64_t u = split * kAttnTok + tid;
    uint4 cn = make_uint4(0u, 0u, 0u, 0u);
    uint64_t ka = 0ull, va = 0ull;
    if (u < U) {
      const uint64_t ent = w.ulist[bh * GK + u];
      cn = w.cnt[bh * GK + (uint32_t)ent];
      bool rec;
      const int64_t row = rs.locate((uint32_t)(ent >> 32), bh, rec);
      if (row >= 0) {
        ka = reinterpret_cast<uint64_t>((rec ? rs.Krec : rs.K) + row * rs.row_bytes);
        va = reinterpret_cast<uint64_t>((rec ? rs.Vrec : rs.V) + row * rs.row_bytes);
      }
    }
    sh.kaddr[tid] = ka;
    sh.vaddr[tid] = va;
    sh.cnt[tid] = cn;
  }
  __syncthreads();
  attn_tokens<G>(sh, reinterpret_cast<uint64_t>(q), scale);
  __syncthreads();
  float *pb = part + (bh * nsplit + split) * G * kPartStride;
  for (int e = tid; e < G * kAttnD; e += kAttnThreads) {
    const int g = e / kAttnD, d = e % kAttnD;
    float acc = 0.0f;
#pragma unroll
    for (int v = 0; v < kAttnWaves; ++v) acc += sh.o[v][g][d];
    pb[g * kPartStride + 2 + d] = acc;
  }
  if (tid < G) {
    float Mg = -INFINITY, Lg = 0.0f;
#pragma unroll
    for (int v = 0; v < kAttnWaves; ++v) {
      Mg = fmaxf(Mg, sh.wm[v][tid]);
      Lg += sh.wl[v][tid];
    }
    pb[tid * kPartStride] = Mg;
    pb[tid * kPartStride + 1] = Lg;
  }
}

// gather_attention over rows per selected position: workgroup (split s, head
// g, row bh) runs attn_stream_block over head g's positions of split s.
template <int NW, bool REC>
__global__ __launch_bounds__(NW * kWave) void attn_stream_kernel(const float *__restrict__ q,
                                                                 const int64_t *__restrict__ idx, int64_t G, int64_t k,
                                                                 RowSrc rs, float scale, float *__restrict__ out,
                                                                 float *__restrict__ part, int64_t nsplit) {
  __shared__ float wm[NW], wl[NW];
  __shared__ float wo[NW][kAttnD];
  const int64_t s = blockIdx.x, g = blockIdx.y, bh = blockIdx.z;
  const int64_t *ig = idx + (bh * G + g) * k;
  attn_stream_block<NW, REC>(q + (bh * G + g) * kAttnD, [&](int64_t j) { return ig[j]; }, k, s, bh, rs, scale, wm, wl,
                             wo, out + (bh * G + g) * kAttnD, part + ((bh * nsplit + s) * G + g) * kPartStride,
                             nsplit == 1);
}

// out[bh, g, d] = sum_s O_s e^(M_s - M) / sum_s L_s e^(M_s - M) over the
// row's splits, by every thread for its own dimension d with no barrier:
// M = max_s M_s first, then the weighted sums in split order, kB splits per
// round of loads (rows of at most kB splits: one round).  A split where a head
// selected nothing (M_s = -inf) adds nothing to it.
__global__ __launch_bounds__(kAttnD) void attn_merge_kernel(const float *__restrict__ part, int64_t G,
                                                            int64_t nsplit, float *__restrict__ out) {
  constexpr int kB = 32;
  const int64_t r = blockIdx.x;  // bh * G + g
  const int64_t bh = r / G, g = r % G;
  const int d = threadIdx.x;
  const float *base = part + (bh * nsplit * G + g) * kPartStride;  // split s at + s * G * kPartStride
  const int64_t sstride = G * kPartStride;
  float M = -INFINITY;
  if (nsplit > kB)
    for (int s = 0; s < (int)nsplit; ++s) M = fmaxf(M, base[s * sstride]);
  float L = 0.0f, O = 0.0f;
  for (int s0 = 0; s0 < (int)nsplit; s0 += kB) {
    float ms[kB], ls[kB], os[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const bool in = s0 + i < nsplit;
      const float *b = base + (in ? (s0 + i) : 0) * sstride;
      ms[i] = in ? b[0] : -INFINITY;
      ls[i] = in ? b[1] : 0.0f;
      os[i] = in ? b[2 + d] : 0.0f;
    }
    if (nsplit <= kB) {
#pragma unroll
      for (int i = 0; i < kB; ++i) M = fmaxf(M, ms[i]);
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const float e = ms[i] == -INFINITY ? 0.0f : expf(ms[i] - M);  // an empty split adds nothing
      L = fmaf(ls[i], e, L);
      O = fmaf(os[i], e, O);
    }
  }
  out[r * kAttnD + d] = O / L;
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
  return GK <= kMaxGK ? union_ws_layout(BH, GK, nullptr, nullptr) : wide_union_layout(BH, GK, nullptr, nullptr);
}

extern "C" int fathom_gather_union(const int64_t *idx, int64_t BH, int64_t GK, int64_t n, const void *Ksrc,
                                   const void *Vsrc, int64_t cap, const void *Krec, const void *Vrec, int64_t nrec,
                                   int64_t row_bytes, void *Kout, void *Vout, int32_t *n_unique, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  if (!idx || !Ksrc || !Vsrc || !Kout || !Vout) return fail(FATHOM_ERR_INVALID, "gather_union: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "gather_union: BH=%lld outside [1, 65535]", (long long)BH);
  if (GK < 1 || GK > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "gather_union: G*k=%lld unsupported", (long long)GK);
  if (n < 0 || cap < 0) return fail(FATHOM_ERR_INVALID, "gather_union: bad n/cap");
  if (row_bytes < 4 || row_bytes % 4) return fail(FATHOM_ERR_INVALID, "gather_union: row_bytes=%lld not a multiple of 4", (long long)row_bytes);
  const size_t need = fathom_gather_union_workspace_bytes(BH, GK);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "gather_union: workspace %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const RowSrc rs{(const char *)Ksrc, (const char *)Vsrc, (const char *)Krec, (const char *)Vrec,
                  cap, nrec, n, row_bytes};
  if (GK > kMaxGK) {  // beyond one workgroup's LDS: the table in the workspace
    WideUnionWs ww;
    wide_union_layout(BH, GK, static_cast<char *>(workspace), &ww);
    int rc = launch_wide_union(idx, BH, GK, n, ww, n_unique, st);
    if (rc) return rc;
    const dim3 grid((unsigned)cdiv(GK, 4), (unsigned)BH);
    wide_union_fetch_kernel<false><<<grid, 256, 0, st>>>(idx, GK, ww, rs, (char *)Kout, (char *)Vout);
    rc = launch_status("wide_union_fetch_kernel");
    if (rc) return rc;
    wide_union_fetch_kernel<true><<<grid, 256, 0, st>>>(idx, GK, ww, rs, (char *)Kout, (char *)Vout);
    return launch_status("wide_union_fetch_kernel");
  }
  UnionWs w;
  union_ws_layout(BH, GK, static_cast<char *>(workspace), &w);
  int rc = launch_union(idx, BH, GK, GK, n, w, n_unique, st);
  if (rc) return rc;
  dim3 grid((unsigned)cdiv(GK, 4), (unsigned)BH);
  union_fetch_kernel<<<grid, 256, 0, st>>>(w, GK, rs, (char *)Kout, (char *)Vout);
  return launch_status("union_fetch_kernel");
}

// The union path (distinct rows, counts per head) holds a row's G * k
// positions in one workgroup's LDS and its counts per head in 16-bit fields
// of 8; rows per selected position have neither limit.
static bool union_fits(int64_t G, int64_t k) { return G <= kMaxHeads && G * k <= kMaxGK; }

extern "C" size_t fathom_gather_attention_workspace_bytes(int64_t BH, int64_t G, int64_t k) {
  if (BH < 1 || G < 1 || k < 1) return 0;
  // per-position partials: at most one split per 128 positions of a head
  const size_t stream = (size_t)BH * cdiv(k, (int64_t)(4 * kStreamTok)) * G * kPartStride * sizeof(float);
  if (!union_fits(G, k)) return wide_union_layout(BH, G * k, nullptr, nullptr) + stream;
  const int64_t GK = G * k, nsplit = cdiv(GK, kAttnTok);
  const size_t uni = (size_t)BH * nsplit * G * kPartStride * sizeof(float);
  return union_ws_layout(BH, GK, nullptr, nullptr) + (uni > stream ? uni : stream);
}

extern "C" int fathom_gather_attention(const float *q, const int64_t *idx, int64_t BH, int64_t G, int64_t k, int64_t n,
                                       const void *Ksrc, const void *Vsrc, int64_t cap, const void *Krec,
                                       const void *Vrec, int64_t nrec, float scale, float *out, int32_t *n_unique,
                                       void *workspace, size_t workspace_bytes, void *stream) {
  if (!q || !idx || !Ksrc || !Vsrc || !out) return fail(FATHOM_ERR_INVALID, "gather_attention: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "gather_attention: BH=%lld outside [1, 65535]", (long long)BH);
  if (G < 1 || G > 65535 || k < 1) return fail(FATHOM_ERR_INVALID, "gather_attention: G=%lld k=%lld", (long long)G, (long long)k);
  if (G * k > 0x7FFFFFFF) return fail(FATHOM_ERR_INVALID, "gather_attention: G*k=%lld unsupported", (long long)(G * k));
  if (n < 0 || cap < 0 || nrec < 0) return fail(FATHOM_ERR_INVALID, "gather_attention: bad n/cap/nrec");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(Ksrc) | reinterpret_cast<uintptr_t>(Vsrc)) & 7)
    return fail(FATHOM_ERR_INVALID, "gather_attention: q, K and V must be 8-byte aligned");
  const size_t need = fathom_gather_attention_workspace_bytes(BH, G, k);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "gather_attention: workspace %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int64_t GK = G * k, nsplit = cdiv(GK, kAttnTok);
  UnionWs w{};
  WideUnionWs ww{};
  const bool fits = union_fits(G, k);
  const size_t off = fits ? union_ws_layout(BH, GK, static_cast<char *>(workspace), &w)
                          : wide_union_layout(BH, GK, static_cast<char *>(workspace), &ww);
  float *part = reinterpret_cast<float *>(static_cast<char *>(workspace) + off);
  const RowSrc rs{(const char *)Ksrc, (const char *)Vsrc, (const char *)Krec, (const char *)Vrec,
                  cap, nrec, n, (int64_t)kAttnD * 2};
  int rc;
  if (n_unique && !fits) {  // the distinct-row count from the table in the workspace; rows per position below
    rc = launch_wide_union(idx, BH, GK, n, ww, n_unique, st);
    if (rc) return rc;
  }
  if (!n_unique || !fits) {
    // rows per selected position, streamed (attn_wide: 16 or 4 waves per
    // workgroup), split heads merged by attn_merge_kernel
    const bool wide = attn_wide(BH, G, k);
    const int64_t ns = cdiv(k, (int64_t)(kStreamTok * (wide ? 16 : 4)));
    const dim3 grid((unsigned)ns, (unsigned)G, (unsigned)BH);
    const bool rec = Krec && Vrec && nrec > 0;
    if (wide && rec)
      attn_stream_kernel<16, true><<<grid, 16 * kWave, 0, st>>>(q, idx, G, k, rs, scale, out, part, ns);
    else if (wide)
      attn_stream_kernel<16, false><<<grid, 16 * kWave, 0, st>>>(q, idx, G, k, rs, scale, out, part, ns);
    else if (rec)
      attn_stream_kernel<4, true><<<grid, 4 * kWave, 0, st>>>(q, idx, G, k, rs, scale, out, part, ns);
    else
      attn_stream_kernel<4, false><<<grid, 4 * kWave, 0, st>>>(q, idx, G, k, rs, scale, out, part, ns);
    rc = launch_status("attn_stream_kernel");
    if (rc || ns == 1) return rc;
    attn_merge_kernel<<<(unsigned)(BH * G), kAttnD, 0, st>>>(part, G, ns, out);
    return launch_status("attn_merge_kernel");
  } else {
    // the union list (each distinct row read once), then its groups of kAttnTok tokens
    rc = launch_union(idx, BH, GK, k, n, w, n_unique, st);
    if (rc) return rc;
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
  }
  if (rc) return rc;
  attn_merge_kernel<<<(unsigned)(BH * G), kAttnD, 0, st>>>(part, G, nsplit, out);
  return launch_status("attn_merge_kernel");
}
