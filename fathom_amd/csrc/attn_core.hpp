// Attention over selected K/V rows, shared by gather_attention (gather.hip) and
// the decode step's fused selection + attention (topk.hip): the row source,
// the lane reductions and the streamed per-head attention block.
#pragma once

#include "common.hpp"

namespace fathom {
namespace attn {

constexpr uint32_t kTokNeg = 0xFFFFFFFEu;  // token key of negative indices
constexpr int kAttnD = 128;                // head dimension of gather_attention
constexpr int kPartStride = kAttnD + 2;    // (max, sum, weighted V[128])
constexpr int kStreamWide = 16;            // waves of a workgroup that takes 512 positions of a head

// gather_attention's choice for rows per selected position: workgroups of 16
// waves (512 positions, one split per head for k <= 512) when that gives the
// chip about 128 workgroups or more, else of 4 waves (128 positions).
inline bool attn_wide(int64_t BH, int64_t G, int64_t k) { return BH * G * cdiv(k, (int64_t)(32 * kStreamWide)) >= 96; }

__device__ __forceinline__ uint32_t tok_key(int64_t v) {
  return v < 0 ? kTokNeg : (uint32_t)(v < (int64_t)kTokNeg - 1 ? v : (int64_t)kTokNeg - 1);
}

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

// Sum (MAX = false) or maximum over the 16 lanes of a DPP row: quad_perm
// [1,0,3,2], [2,3,0,1], then row_half_mirror and row_mirror, each pairing
// halves whose lanes already agree.
template <bool MAX>
__device__ __forceinline__ float row16_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));
  return op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));
}

// Sum or maximum of the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the same lane of
// the four DPP rows): the gfx950 row swaps v_permlane32_swap and
// v_permlane16_swap give each lane its partner's value.
template <bool MAX>
__device__ __forceinline__ float across_rows(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  const uint32_t x = __float_as_uint(v);
  const auto p32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  v = op(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
  const uint32_t y = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(y, y, false, false);
  return op(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4 *gptr4;

// Attention of one query head's positions streamed through registers (no
// union, rows in device memory): a workgroup of NW waves takes positions
// [32 NW s, 32 NW (s + 1)) of the head's k selected tokens tok_at(j) of row
// bh, each with a count of one (a row selected twice counts twice).  Wave w
// holds 32 of them: lane l works on dims 8 (l & 15) .. + 7 of the rows of
// positions 4 t + (l >> 4), t < 8.  Every K and V row piece of the wave is
// requested before the first score is formed (K first), so the scores follow
// the K rows as they arrive and the values the V rows.  A position without a
// row (negative token, beyond the cache) scores 0 and reads kZeroRow, which
// adds nothing to V.  The wave's softmax is taken against its own maximum, so no
// barrier is needed until the waves' (M, sum, weighted V) triples are
// combined (LDS wm[NW], wl[NW], wo[NW][kAttnD]).  single: the workgroup
// writes the head's output out_row; else its (M, sum, weighted V) triple to
// pb for attn_merge_kernel.
constexpr int kStreamTok = 32;               // positions per wave
constexpr uint64_t kRowBytes = 2 * kAttnD;   // a bf16 row
__device__ const u32x4 kZeroRow[kRowBytes / 16] = {};
template <int NW, bool REC, typename TokAt>
__device__ __forceinline__ void attn_stream_block(const float *__restrict__ qg, TokAt tok_at, int64_t k, int64_t s,
                                                  int64_t bh, const RowSrc &rs, float scale, float *wm, float *wl,
                                                  float (*wo)[kAttnD], float *__restrict__ out_row,
                                                  float *__restrict__ pb, bool single) {
  constexpr int kSteps = kStreamTok / 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = lane >> 4, ds = lane & 15;
  const int64_t p0 = (s * NW + wave) * kStreamTok + rg;
  const float4 qa = *reinterpret_cast<const float4 *>(qg + 8 * ds);
  const float4 qb = *reinterpret_cast<const float4 *>(qg + 8 * ds + 4);
  int64_t tk[kSteps];  // positions past k read the last one (and are masked)
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    const int64_t j = p0 + 4 * t;
    tk[t] = tok_at(j < k ? j : k - 1);
  }
  const float qq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  // RowSrc::locate without branches: a device row (token < min(n, cap)), a
  // recent row (token >= n, the last one for tokens past nrec) or none
  const int64_t dlim = rs.n < rs.cap ? rs.n : rs.cap;
  const uint64_t kdev = reinterpret_cast<uint64_t>(rs.K) + (uint64_t)(bh * rs.cap) * kRowBytes;
  const uint64_t vdev = reinterpret_cast<uint64_t>(rs.V) + (uint64_t)(bh * rs.cap) * kRowBytes;
  const uint64_t zero = reinterpret_cast<uint64_t>(kZeroRow);
  uint64_t ka[kSteps], va[kSteps];
  bool in[kSteps], has[kSteps];
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    in[t] = p0 + 4 * t < k;
    const uint32_t tok = tok_key(tk[t]);
    const bool dv = tok != kTokNeg && (int64_t)tok < dlim;
    has[t] = dv;
    ka[t] = dv ? kdev + (uint64_t)tok * kRowBytes : zero;
    va[t] = dv ? vdev + (uint64_t)tok * kRowBytes : zero;
    if (REC && !dv && tok != kTokNeg && (int64_t)tok >= rs.n) {
      has[t] = true;
      const int64_t r = bh * rs.nrec + ((int64_t)tok - rs.n < rs.nrec - 1 ? (int64_t)tok - rs.n : rs.nrec - 1);
      ka[t] = reinterpret_cast<uint64_t>(rs.Krec) + (uint64_t)r * kRowBytes;
      va[t] = reinterpret_cast<uint64_t>(rs.Vrec) + (uint64_t)r * kRowBytes;
    }
  }
  u32x4 kv[kSteps], vv[kSteps];
#pragma unroll
  for (int t = 0; t < kSteps; ++t) kv[t] = reinterpret_cast<gptr4>(ka[t])[ds];
  __builtin_amdgcn_sched_barrier(0);  // the K pieces first, in position order
#pragma unroll
  for (int t = 0; t < kSteps; ++t) vv[t] = reinterpret_cast<gptr4>(va[t])[ds];
  __builtin_amdgcn_sched_barrier(0);  // every row piece requested before the first score
  // ---- scores; a position past k is absent
  float sc[kSteps];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    const uint32_t d4[4] = {kv[t].x, kv[t].y, kv[t].z, kv[t].w};
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = d4[e >> 1];
      a = fmaf(qq[e], __uint_as_float((e & 1) ? (h & 0xFFFF0000u) : (h << 16)), a);
    }
    a = row16_reduce<false>(a);
    sc[t] = in[t] ? (has[t] ? a * scale : 0.0f) : -INFINITY;
    m = fmaxf(m, sc[t]);
  }
  m = across_rows<true>(m);  // the wave's maximum
  __builtin_amdgcn_sched_barrier(0);  // the V pieces are awaited only from here
  // ---- the wave's sum and weighted V against its own maximum
  float l = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    const float p = in[t] ? expf(sc[t] - m) : 0.0f;
    l += p;
    const uint32_t d4[4] = {vv[t].x, vv[t].y, vv[t].z, vv[t].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = d4[e >> 1];
      o[e] = fmaf(p, __uint_as_float((e & 1) ? (h & 0xFFFF0000u) : (h << 16)), o[e]);
    }
  }
  l = across_rows<false>(l);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = across_rows<false>(o[e]);
  if (rg == 0) {
    *reinterpret_cast<float4 *>(&wo[wave][8 * ds]) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4 *>(&wo[wave][8 * ds + 4]) = make_float4(o[4], o[5], o[6], o[7]);
  }
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
  __syncthreads();
  if (tid < kAttnD) {
    // lane v < NW: wave v's factor e^(M_v - M); every lane reads them by readlane
    const float mv = lane < NW ? wm[lane] : -INFINITY;
    float M = mv;
#pragma unroll
    for (int sh = 1; sh < NW; sh <<= 1) M = fmaxf(M, __shfl_xor(M, sh));
    const float ev = mv == -INFINITY ? 0.0f : expf(mv - M);  // a wave past k adds nothing
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float e = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(ev), v));
      L = fmaf(wl[v], e, L);
      O = fmaf(wo[v][tid], e, O);
    }
    if (single) {
      out_row[tid] = O / L;
    } else {
      pb[2 + tid] = O;
      if (tid == 0) {
        pb[0] = M;
        pb[1] = L;
      }
    }
  }
}

}  // namespace attn
}  // namespace fathom
