// Partial-depth bit-plane scan (PlaneStore.scan) and the fused scan + top-k.
//
// Score of token i of row (bh, g), with depth t_j planes read for channel j:
//   s = sum_j q_gj * a_bj * 2^(1 - t_j) * x_j(i),   x = c_t - (2^t - 1) / 2,
// where c_t is the top-t-bit code and a_bj the block absmax.  This is the
// reference's dequantised value (c_t + 0.5 - 2^(t-1)) * a / 2^(t-1)
// (kernels/bitplane.py:34-42) with the constant term folded into x.  Each
// factor is exact up to the final products: the kernel builds y = a * x' with
// x' = -x for depth 1 (x' = +-0.5 from the bit as a sign) and x' = 2x for
// deeper channels (x' = 2c_t - 2^t + 1, an integer), and the head weights
// w_gj = -q_gj (depth 1) or q_gj * 2^(-t_j) absorb the sign and the power of
// two, so w * y is exactly q * a * 2^(1-t) * x.
//
// Layout of the work: a workgroup (4 waves) owns a tile of 32 blocks (2048
// tokens) of one row bh; wave w owns blocks 8w..8w+7, lane = token.  The
// plan's channels are visited in chunks of at most 16 (channel, plane) units
// of one depth class.  A chunk's plane words (32 blocks each) and scales are
// read with coalesced vector loads (every (channel, plane) run of the tile is
// whole 128-byte segments: HBM, or PCIe for a store in mapped host memory)
// and stored in LDS with each word split into its low dword (tokens 0-31) and
// high dword (tokens 32-63), so a lane reads only the dwords holding its own
// bits, four blocks per 16-byte LDS read.  Chunks are double buffered: the
// loads of chunk k + 1 are in flight while chunk k is computed.
//
// Per (channel, block) the VALU extracts the lane's t bits and forms y (3
// instructions at depth 1, 2t + 2 deeper); the head contraction acc_g += w_gj
// * y runs on the matrix cores: one v_mfma_f32_4x4x1_16b_f32 per (channel,
// block) multiplies the lane's y (B operand: lane = token) by the four heads'
// weights (A operand: lane l holds head l & 3) and adds into four fp32
// accumulators per lane (head h in component h).  Each step is an fp32 fused
// multiply-add, the operation of v_fmac_f32: the score is one fp32 FMA chain
// over the channels in plan order, whatever the store's location, so scans of
// a store in HBM and of the same store in host memory are bit-identical.
// G > 4 takes a second MFMA for heads 4..7.
//
// Output modes: scores [BH, G, n] (PlaneStore.scan), sampled keys (every S-th
// tile, for the top-k threshold), or candidate emission (key >= threshold ->
// per-row candidate list, aggregated per workgroup in LDS), the last two
// fusing the scan with the top-k.
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr int kGB = 8;             // blocks per wave
constexpr int kWaves = 4;          // waves per workgroup
constexpr int kTB = kGB * kWaves;  // blocks per tile
constexpr int kMaxD = 256;
constexpr int kWUnits = 32;        // (channel, plane) units per wave chunk
static_assert(kTB * kBlk == kTileTok, "scan tile and top-k sample tile must agree");
constexpr int kThreads = 64 * kWaves;
static_assert(2 * kWUnits == kWave, "two staging lanes per unit");
static_assert(kGB == 8, "a wave stages two groups of four blocks");
static_assert(kGB * kBlk == kRegTok, "a candidate region is one wave's blocks");

// Tile geometry by NG, the block groups of four a wave computes: NG = 2 (8
// blocks per wave, 4 waves per tile, two staging lanes per unit) everywhere but
// the sample pass, which is latency-bound (a few workgroups per row) and uses
// NG = 1 (4 blocks per wave, 8 waves per tile, one lane per unit): half a
// wave's work per tile, the same scores bit for bit.
template <int NG>
struct Geo {
  static constexpr int GB = 4 * NG;          // blocks per wave
  static constexpr int WAVES = kTB / GB;     // waves per tile
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int WUNITS = kWave / NG;  // units per wave chunk
};
static_assert(Geo<2>::GB == kGB && Geo<2>::THREADS == kThreads && Geo<2>::WUNITS == kWUnits, "NG = 2 is the tile");

enum : int { kEmitScores = 0, kEmitSample = 1, kEmitFilter = 2, kEmitFallback = 3 };

struct Emit {
  float *out;        // scores [BH, G, n]
  uint32_t *samp;    // sampled keys [BH*G, samp_cap]
  int64_t samp_cap;
  TopkSel sel;       // thresholds + candidate lists
  int64_t sink, lstart;
  int fallback;      // candidate mode: the fallback pass (threshold T_lo, rows whose first pass found < kk)
};

struct ScanArgs {
  const float *q;          // [BH, G, D]
  const int32_t *cls;      // [BH, bmax, D]
  const int32_t *clsn;     // [BH, bmax]
  const uint64_t *planes;  // [BH, nsb, D, 4, sub]
  const uint16_t *scales;  // [BH, nsb, D, sub] fp16 bits
  int64_t n, nsb, sub;
  int64_t blk0, blk_end;   // blocks [blk0, blk_end) are emitted
  int64_t tile0;           // tile of blockIdx.x == 0 (tile T = blocks [32T, 32T + 32))
  int64_t tile_stride;     // tiles between consecutive list entries
  int64_t ntiles;          // list entries (tile0 + L * tile_stride, L < ntiles)
  int D, bmax, ncls;       // classes 1..ncls are scanned (ncls = min(bmax, 4))
  int fast;                // sub % 4 == 0 and 16-byte (planes) / 8-byte (scales) aligned: vector staging loads
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Wave-uniform loads through the constant address space: scalar loads into
// SGPRs (the plan is read-only for the kernel's lifetime).
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// ----------------------------------------------------------------- head weights
// w_gj for every listed channel, QS floats per channel (heads >= G are zero),
// so the MFMA A operand of lane l is w[j][4h + (l & 3)].
template <int G>
struct QShared {
  static constexpr int QS = G <= 4 ? 4 : 8;
  float w[kMaxD * QS];
};

// Per-channel head operand: the lane's MFMA A value(s).
template <int G>
struct QOp {
  static constexpr int NQ = (G + 3) / 4;
  float a[NQ];
};

template <int G>
__device__ __forceinline__ QOp<G> load_qop(const QShared<G> &qs, int j, int lane) {
  QOp<G> o;
#pragma unroll
  for (int h = 0; h < QOp<G>::NQ; ++h) o.a[h] = qs.w[j * QShared<G>::QS + 4 * h + (lane & 3)];
  return o;
}

// Four fp32 accumulators per lane and head quad: component h of v[b][hq] is the
// score of head 4*hq + h for the lane's token of block b.
template <int G, int GB = kGB>
struct Acc {
  static constexpr int NQ = (G + 3) / 4;
  f32x4 v[GB][NQ];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int b = 0; b < GB; ++b)
#pragma unroll
      for (int h = 0; h < NQ; ++h) v[b][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __device__ __forceinline__ float get(int b, int g) const { return v[b][g >> 2][g & 3]; }
};

template <int G, int GB>
__device__ __forceinline__ void accum(Acc<G, GB> &acc, int b, const QOp<G> &q, float y) {
#pragma unroll
  for (int h = 0; h < QOp<G>::NQ; ++h) acc.v[b][h] = __builtin_amdgcn_mfma_f32_4x4x1f32(q.a[h], y, acc.v[b][h], 0, 0, 0);
}

// ----------------------------------------------------------------- value of a lane
// y = a * x' of a lane's token from its plane bits and the block's staged
// scale pair (P, Q):
//  * depth 1: y = -a * x = (bit ? -a/2 : +a/2), the bit put into the sign of
//    P = a/2 (a >= 0);
//  * deeper: y = 2a * x = c * P + Q with P = 2a, Q = -(2^C - 1) a and c the
//    C-bit code: one fused multiply-add of exact operands (c < 16, a fp16).
// (compute_chunk below forms both from the octet-layout dwords.)

// --------------------------------------------------------------------- emission
// Threshold of a row as a float for "key >= thr": every element whose key is
// >= thr has !(v < thr_f) (thr at or below -inf's key: everything passes; thr
// in the NaN range: NaN and +inf pass -- extra candidates never change the
// exact selection, they only cost time).
__device__ __forceinline__ float threshold_value(uint32_t thr) {
  if (thr <= kKeyNegInf) return -INFINITY;
  if (thr > 0xFF800000u) return INFINITY;  // above +inf's key
  return key_value(thr);
}

// Candidate emission of a wave's 8 blocks into its region of each row's
// candidate buffer (region gb0 / kGB: tokens [gb0 * kBlk, + kRegTok)): one
// compare + ballot per (block, head) ranks the passing tokens, each writes its
// K64 at its rank, and lane 0 writes the region's count.  The wave touches no
// other wave's memory and no shared counter.  Heads in skipm emit nothing.
template <int G>
__device__ __forceinline__ void emit_filter(const Emit &em, const Acc<G> &acc, int64_t bh, int64_t gb0, int64_t blk0,
                                            int64_t blk_end, int64_t n, int lane, uint32_t skipm) {
  const int64_t t0 = gb0 * kBlk, t1 = t0 + kGB * kBlk;
  // no per-lane validity or sink/local masking anywhere in the wave's blocks
  const bool plain = gb0 >= blk0 && gb0 + kGB <= blk_end && t1 <= n && t0 >= em.sink && t1 <= em.lstart;
  const uint32_t *const thr = em.fallback ? em.sel.thr_lo : em.sel.thr;
  uint32_t *const rc = em.fallback ? em.sel.rc2 : em.sel.rc1;
  const int64_t region = gb0 / kGB;
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if ((skipm >> g) & 1u) continue;
    const int64_t row = bh * G + g;
    const float thr_f = threshold_value(ld_uniform(thr + row));
    uint64_t *dst = em.sel.cand + row * em.sel.cand_cap + t0;
    uint32_t off = 0u;
#pragma unroll
    for (int r = 0; r < kGB; ++r) {
      const float v = acc.get(r, g);
      const int64_t tok = (gb0 + r) * kBlk + lane;
      bool valid = true;
      float vm = v;
      if (!plain) {
        valid = gb0 + r >= blk0 && gb0 + r < blk_end && tok < n;
        vm = (tok < em.sink || tok >= em.lstart) ? -INFINITY : v;
      }
      const bool pass = valid && !(vm < thr_f);
      const uint64_t m = __ballot(pass);
      if (pass) dst[off + (uint32_t)__popcll(m & lt)] = k64_of(vm == -INFINITY ? kKeyNegInf : score_key(vm), tok);
      off += (uint32_t)__popcll(m);
    }
    if (lane == 0) rc[row * em.sel.nreg + region] = off;
  }
}

template <int G, int MODE, int GB = kGB>
__device__ __forceinline__ void emit_group(const Emit &em, const Acc<G, GB> &acc, int64_t bh, int64_t gb0, int64_t blk0,
                                           int64_t blk_end, int64_t n, int wave, int lane, int64_t samp_tile,
                                           uint32_t skipm) {
  if constexpr (MODE == kEmitFilter) {
    static_assert(GB == kGB, "candidate regions are 8-block waves");
    emit_filter<G>(em, acc, bh, gb0, blk0, blk_end, n, lane, skipm);
    return;
  }
#pragma unroll
  for (int r = 0; r < GB; ++r) {
    const int64_t b = gb0 + r;
    const int64_t tok = b * kBlk + lane;
    const bool valid = b >= blk0 && b < blk_end && tok < n;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = acc.get(r, g);
      const int64_t row = bh * G + g;
      if (MODE == kEmitScores) {
        if (valid) em.out[row * n + tok] = v;
      } else {
        const bool masked = tok < em.sink || tok >= em.lstart;
        const uint32_t key = valid ? (masked ? kKeyNegInf : score_key(v)) : 0u;
        em.samp[row * em.samp_cap + samp_tile * kTileTok + (wave * GB + r) * kBlk + lane] = key;
      }
    }
  }
}

// --------------------------------------------------------------------- tile kernel
// The plan as two streams, built once per workgroup: channel slots in class
// order (class 1 list, then 2, 3, 4; SF[c] = end of class c's slots) and their
// (channel, plane) units (slot s of class c owns units UE[c-1] + (s -
// SF[c-1]) * (c + 1) + p, p < c + 1; UE[c] = end of class c's units).
struct PlanStreams {
  int SF[4], UE[4];
};

__device__ __forceinline__ PlanStreams plan_streams(const int (&nc)[4]) {
  PlanStreams ps;
  int s = 0, u = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    s += nc[c];
    u += nc[c] * (c + 1);
    ps.SF[c] = s;
    ps.UE[c] = u;
  }
  return ps;
}

// A wave chunk: plan slots [s0, s1) (whole channels), their units [u0, u1),
// at most kWUnits units.
struct Chunk {
  int s0, s1, u0, u1;
};

// The chunk starting at slot s (s < SF[3]).
template <int WU = kWUnits>
__device__ __forceinline__ Chunk chunk_from(const PlanStreams &ps, int s) {
  Chunk ck;
  ck.s0 = s;
  int used = 0, u0 = -1;
  bool open = true;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int lo = c ? ps.SF[c - 1] : 0;
    if (open && s < ps.SF[c]) {
      if (u0 < 0) u0 = (c ? ps.UE[c - 1] : 0) + (s - lo) * (c + 1);
      const int take = min(ps.SF[c] - s, (WU - used) / (c + 1));
      used += take * (c + 1);
      s += take;
      if (s < ps.SF[c]) open = false;
    }
  }
  ck.s1 = s;
  ck.u0 = u0;
  ck.u1 = u0 + used;
  return ck;
}

// A wave's staged chunk in the octet layout.  For unit u, block group g
// (blocks 4g..4g+3 of the wave) and token octet o (tokens 8o..8o+7 of a
// block), dword oct[u][g][o] holds byte o of the four blocks' plane words,
// block k in byte k: bit 8k + t is token 8o + t of block 4g + k.  A lane
// (token 8o + t) reads one dword per (unit, group) and finds its bit of the
// four blocks at bits t, 8 + t, 16 + t, 24 + t.  A channel of depth C > 1
// stores plane p rotated left by C - 1 - p: masking the C dwords at the lane's
// positions, OR-ing them and one rotation right by t leave the lane's C-bit
// code of block k in byte k.  P, Q: the scale pair of each channel slot and
// block (see lane_value).
template <int NG = 2>
struct WaveBuf {
  alignas(16) uint32_t oct[Geo<NG>::WUNITS][NG][8];
  alignas(16) float P[Geo<NG>::WUNITS][Geo<NG>::GB];
  alignas(16) float Q[Geo<NG>::WUNITS][Geo<NG>::GB];
};

template <int G, int NG = 2>
struct TileShared {
  alignas(16) float w[kMaxD][QShared<G>::QS];  // head weights by plan slot
  uint16_t unit[4 * kMaxD];                    // plan unit -> (j * 4 + p) << 2 | (C - 1 - p)
  uint16_t slot[kMaxD];                        // plan slot -> j | class << 8
  WaveBuf<NG> wb[Geo<NG>::WAVES];
};

// What a lane loads for one chunk: the four plane words of its (unit, group)
// with the rotation its plane needs, and the four scales of its (channel
// slot, group) with the slot's class.
struct Staged {
  uint64_t w[4];
  uint32_t s[2];
  uint32_t rot;
  int scls;
};

// A lane's staging addresses: element offsets of the first block of its plane
// group (lane & 1) and of its scale group (lane >> 5), with the channel term
// left out; all four blocks of a group share them when the store qualifies
// for vector loads (sub % 4 == 0).
struct LaneAddr {
  int64_t pbase, sbase;
  bool pin, sin;  // the group lies inside the store's nsb * sub blocks
};

__device__ __forceinline__ void group_base(const ScanArgs &a, int64_t bh, int64_t blk, int64_t &pb, int64_t &sb_off) {
  const uint32_t s = (uint32_t)a.sub;
  const uint32_t sb = (uint32_t)blk / s, off = (uint32_t)blk - sb * s;
  pb = ((bh * a.nsb + sb) * a.D * 4) * a.sub + off;
  sb_off = ((bh * a.nsb + sb) * a.D) * a.sub + off;
}

// Issues the global loads of chunk ck: lane l stages unit l >> 1 for block
// group l & 1 and the scales of channel slot l & 31 for group l >> 5.
template <int G, bool FAST, int NG = 2>
__device__ __forceinline__ void stage_load(Staged &r, const ScanArgs &a, const TileShared<G, NG> &sh, const Chunk &ck,
                                           const LaneAddr &la, int64_t gb0, int64_t bh, int lane) {
  const int u = ck.u0 + (NG == 2 ? lane >> 1 : lane), g = NG == 2 ? lane & 1 : 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) r.w[k] = 0ull;
  r.rot = 0u;
  if (u < ck.u1) {
    const uint32_t d = sh.unit[u];
    const int64_t jp = d >> 2;
    r.rot = (32u - (d & 3u)) & 31u;  // alignbit amount of the left rotation by C - 1 - p
    if (FAST) {
      if (la.pin) {
        const uint4 *src = reinterpret_cast<const uint4 *>(a.planes + la.pbase + jp * a.sub);
        const uint4 v0 = src[0], v1 = src[1];
        r.w[0] = ((uint64_t)v0.y << 32) | v0.x;
        r.w[1] = ((uint64_t)v0.w << 32) | v0.z;
        r.w[2] = ((uint64_t)v1.y << 32) | v1.x;
        r.w[3] = ((uint64_t)v1.w << 32) | v1.z;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t blk = gb0 + 4 * g + k;
        if (blk < a.nsb * a.sub) {
          int64_t pb, sbo;
          group_base(a, bh, blk, pb, sbo);
          r.w[k] = a.planes[pb + jp * a.sub];
        }
      }
    }
  }
  const int cs = ck.s0 + (NG == 2 ? lane & 31 : lane), gs = NG == 2 ? lane >> 5 : 0;
  r.s[0] = r.s[1] = 0u;
  r.scls = 0;
  if (cs < ck.s1) {
    const uint32_t sd = sh.slot[cs];
    const int64_t j = sd & 0xFFu;
    r.scls = (int)(sd >> 8);
    if (FAST) {
      if (la.sin) {
        const uint2 v = *reinterpret_cast<const uint2 *>(a.scales + la.sbase + j * a.sub);
        r.s[0] = v.x;
        r.s[1] = v.y;
      }
    } else {
      uint32_t h[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t blk = gb0 + 4 * gs + k;
        if (blk < a.nsb * a.sub) {
          int64_t pb, sbo;
          group_base(a, bh, blk, pb, sbo);
          h[k] = a.scales[sbo + j * a.sub];
        }
      }
      r.s[0] = h[0] | (h[1] << 16);
      r.s[1] = h[2] | (h[3] << 16);
    }
  }
}

// Writes a loaded chunk to the wave's buffer: plane words as octet dwords
// (two 4 x 4 byte transposes per lane, rotated for the unit's plane) and the
// scale pairs.
template <int NG = 2>
__device__ __forceinline__ void stage_store(WaveBuf<NG> &wb, const Staged &r, const Chunk &ck, int lane) {
  const int u = NG == 2 ? lane >> 1 : lane, g = NG == 2 ? lane & 1 : 0;
  if (ck.u0 + u < ck.u1) {
    uint32_t out[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // h = 0: tokens 0-31 (octets 0-3), h = 1: tokens 32-63
      const uint32_t x0 = (uint32_t)(r.w[0] >> (32 * h)), x1 = (uint32_t)(r.w[1] >> (32 * h));
      const uint32_t x2 = (uint32_t)(r.w[2] >> (32 * h)), x3 = (uint32_t)(r.w[3] >> (32 * h));
      const uint32_t e0 = __builtin_amdgcn_perm(x1, x0, 0x06020400u);  // x0.b0 x1.b0 x0.b2 x1.b2
      const uint32_t e1 = __builtin_amdgcn_perm(x1, x0, 0x07030501u);  // x0.b1 x1.b1 x0.b3 x1.b3
      const uint32_t e2 = __builtin_amdgcn_perm(x3, x2, 0x06020400u);
      const uint32_t e3 = __builtin_amdgcn_perm(x3, x2, 0x07030501u);
      out[4 * h + 0] = __builtin_amdgcn_perm(e2, e0, 0x05040100u);  // byte 0 of x0..x3
      out[4 * h + 1] = __builtin_amdgcn_perm(e3, e1, 0x05040100u);  // byte 1
      out[4 * h + 2] = __builtin_amdgcn_perm(e2, e0, 0x07060302u);  // byte 2
      out[4 * h + 3] = __builtin_amdgcn_perm(e3, e1, 0x07060302u);  // byte 3
    }
#pragma unroll
    for (int o = 0; o < 8; ++o) out[o] = __builtin_amdgcn_alignbit(out[o], out[o], r.rot);
    uint4 *dst = reinterpret_cast<uint4 *>(&wb.oct[u][g][0]);
    dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
    dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
  }
  const int cs = NG == 2 ? lane & 31 : lane, gs = NG == 2 ? lane >> 5 : 0;
  if (ck.s0 + cs < ck.s1) {
    float P[4], Q[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = __half2float(__ushort_as_half((uint16_t)(r.s[k >> 1] >> (16 * (k & 1)))));
      P[k] = r.scls == 0 ? 0.5f * a : 2.0f * a;
      Q[k] = r.scls == 0 ? 0.0f : -(float)((2 << r.scls) - 1) * a;
    }
    *reinterpret_cast<float4 *>(&wb.P[cs][4 * gs]) = make_float4(P[0], P[1], P[2], P[3]);
    *reinterpret_cast<float4 *>(&wb.Q[cs][4 * gs]) = make_float4(Q[0], Q[1], Q[2], Q[3]);
  }
}

// Orders the wave's LDS accesses around a staging store: every lane's writes
// complete before any lane reads the chunk, and the reads of the previous chunk
// before the writes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The wave's 8 blocks of chunk slots [s0, s1), all of depth C, whose units
// start at chunk unit u0; w: the head weights of those slots.  In slot order,
// four blocks per group: one dword read per (plane, group) brings the lane's
// bits of the group's four blocks, two 16-byte reads the scale pairs.
template <int C, int G, int NG = 2>
__device__ __forceinline__ void compute_slots(const WaveBuf<NG> &wb, const float (*w)[QShared<G>::QS], int s0, int s1,
                                              int u0, int lane, uint32_t sign, Acc<G, Geo<NG>::GB> &acc) {
  const int o = lane >> 3, t = lane & 7;
  // depth 1: the shift bringing block k's bit to bit 31; deeper: plane p's mask
  uint32_t sh[4], mk[C];
#pragma unroll
  for (int k = 0; k < 4; ++k) sh[k] = (uint32_t)(31 - 8 * k - t);
#pragma unroll
  for (int p = 0; p < C; ++p) mk[p] = 0x01010101u << ((t + C - 1 - p) & 7);
  const uint32_t *ob = &wb.oct[u0][0][o];
  for (int ci = s0; ci < s1; ++ci, ob += C * NG * 8) {
    QOp<G> q;
#pragma unroll
    for (int h = 0; h < QOp<G>::NQ; ++h) q.a[h] = w[ci][4 * h + (lane & 3)];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const float4 P4 = *reinterpret_cast<const float4 *>(&wb.P[ci][4 * g]);
      float4 Q4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (C > 1) Q4 = *reinterpret_cast<const float4 *>(&wb.Q[ci][4 * g]);
      const float P[4] = {P4.x, P4.y, P4.z, P4.w}, Q[4] = {Q4.x, Q4.y, Q4.z, Q4.w};
      uint32_t d[C];
#pragma unroll
      for (int p = 0; p < C; ++p) d[p] = ob[p * NG * 8 + g * 8];
      float y[4];
      if (C == 1) {
#pragma unroll
        for (int k = 0; k < 4; ++k) y[k] = __uint_as_float(((d[0] << sh[k]) & sign) | __float_as_uint(P[k]));
      } else {
        uint32_t x = d[0] & mk[0];
#pragma unroll
        for (int p = 1; p < C; ++p) x |= d[p] & mk[p];
        x = __builtin_amdgcn_alignbit(x, x, (uint32_t)t);
#pragma unroll
        for (int k = 0; k < 4; ++k) y[k] = fmaf((float)((x >> (8 * k)) & 0xFFu), P[k], Q[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) accum<G>(acc, 4 * g + k, q, y[k]);
    }
  }
}

// Workgroup prologue: the plan streams in LDS -- per slot its channel and
// class and the head weights (w = -q at depth 1, q * 2^-C deeper: exact
// power-of-two scalings), per unit its plane word index and rotation.
template <int G, int NG = 2>
__device__ __forceinline__ void tile_prologue(TileShared<G, NG> &sh, const ScanArgs &a, const int (&nc)[4],
                                              const PlanStreams &ps, int64_t bh) {
  constexpr int QS = QShared<G>::QS;
  for (int e = threadIdx.x; e < ps.SF[3]; e += Geo<NG>::THREADS) {
    const int c = (e >= ps.SF[0]) + (e >= ps.SF[1]) + (e >= ps.SF[2]);
    const int lo = c == 0 ? 0 : c == 1 ? ps.SF[0] : c == 2 ? ps.SF[1] : ps.SF[2];
    const int ub = (c == 0 ? 0 : c == 1 ? ps.UE[0] : c == 2 ? ps.UE[1] : ps.UE[2]) + (e - lo) * (c + 1);
    const int jr = a.cls[(bh * a.bmax + c) * a.D + (e - lo)];
    const int j = min(max(jr, 0), a.D - 1);  // memory-safe; make_plan lists only valid channels
    sh.slot[e] = (uint16_t)(j | (c << 8));
    for (int p = 0; p <= c; ++p) sh.unit[ub + p] = (uint16_t)(((j * 4 + p) << 2) | (c - p));
#pragma unroll
    for (int g = 0; g < QS; ++g) {
      const float qv = g < G ? a.q[(bh * G + g) * a.D + j] : 0.0f;
      sh.w[e][g] = c == 0 ? -qv : ldexpf(qv, -(c + 1));
    }
  }
}

// One tile (list entry L of the launch) of a workgroup: the plan streams are in
// LDS; each wave stages and computes its own 8 blocks, then emits them.
template <int G, int MODE, bool FAST, int NG = 2>
__device__ __forceinline__ void scan_one(const ScanArgs &a, const Emit &em, TileShared<G, NG> &sh,
                                         const PlanStreams &ps, int64_t L, int wave, int lane, uint32_t skipm) {
  constexpr int GB = Geo<NG>::GB;
  const int64_t bh = blockIdx.y;
  const int64_t tb0 = (a.tile0 + L * a.tile_stride) * kTB;
  const int64_t gb0 = tb0 + wave * GB;  // the wave's first block
  LaneAddr la{0, 0, false, false};
  {
    const int64_t pblk = gb0 + (NG == 2 ? 4 * (lane & 1) : 0), sblk = gb0 + (NG == 2 ? 4 * (lane >> 5) : 0);
    int64_t unused;
    la.pin = pblk < a.nsb * a.sub;
    la.sin = sblk < a.nsb * a.sub;
    if (la.pin) group_base(a, bh, pblk, la.pbase, unused);
    if (la.sin) group_base(a, bh, sblk, unused, la.sbase);
  }
  Acc<G, GB> acc;
  acc.zero();
  WaveBuf<NG> &wb = sh.wb[wave];
  if (tb0 < a.blk_end && tb0 + kTB > a.blk0 && ps.SF[3] > 0) {  // uniform over the workgroup
    Staged r;
    // the sign-bit mask as an opaque VGPR value (VOP3 encodings take no literal)
    uint32_t sign;
    asm("v_mov_b32 %0, 0x80000000" : "=v"(sign));
    Chunk cur = chunk_from<Geo<NG>::WUNITS>(ps, 0);
    stage_load<G, FAST, NG>(r, a, sh, cur, la, gb0, bh, lane);
    // chunks in plan order; the next chunk is loaded while the current one is
    // computed.  Waves run independently: each stages and computes its own blocks.
    while (true) {
      wave_lds_sync();  // the previous chunk's reads are done
      stage_store<NG>(wb, r, cur, lane);
      wave_lds_sync();
      const bool more = cur.s1 < ps.SF[3];
      Chunk nxt = cur;
      if (more) {
        nxt = chunk_from<Geo<NG>::WUNITS>(ps, cur.s1);
        stage_load<G, FAST, NG>(r, a, sh, nxt, la, gb0, bh, lane);
      }
      const float (*w)[QShared<G>::QS] = sh.w + cur.s0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int lo = max(cur.s0, c ? ps.SF[c - 1] : 0), hi = min(cur.s1, ps.SF[c]);
        if (lo < hi) {
          const int ul = (c ? ps.UE[c - 1] : 0) + (lo - (c ? ps.SF[c - 1] : 0)) * (c + 1) - cur.u0;
          if (c == 0) compute_slots<1, G, NG>(wb, w, lo - cur.s0, hi - cur.s0, ul, lane, sign, acc);
          if (c == 1) compute_slots<2, G, NG>(wb, w, lo - cur.s0, hi - cur.s0, ul, lane, sign, acc);
          if (c == 2) compute_slots<3, G, NG>(wb, w, lo - cur.s0, hi - cur.s0, ul, lane, sign, acc);
          if (c == 3) compute_slots<4, G, NG>(wb, w, lo - cur.s0, hi - cur.s0, ul, lane, sign, acc);
        }
      }
      if (!more) break;
      cur = nxt;
    }
  }
  emit_group<G, MODE, GB>(em, acc, bh, gb0, a.blk0, a.blk_end, a.n, wave, lane, L, skipm);
}

// One tile per workgroup (grid.x = list entries), except the fallback pass:
// a grid-stride loop of few workgroups over the list, so that rows which need
// no fallback (every row, normally) cost only those workgroups' launches.
template <int G, int MODE, bool FAST, int NG>
__global__ __launch_bounds__(Geo<NG>::THREADS) __attribute__((amdgpu_waves_per_eu(G <= 4 && MODE != kEmitFallback ? 5 : 4))) void scan_tile_kernel(ScanArgs a, Emit em) {
  __shared__ TileShared<G, NG> sh;
  __shared__ uint32_t s_tot[G];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = blockIdx.y;
  uint32_t skipm = 0u;
  if (MODE == kEmitFallback) {  // heads whose first pass found kk candidates skip the pass
    if (tid < G) s_tot[tid] = 0u;
    __syncthreads();
    const int64_t nq = em.sel.nreg / 4;  // regions per row: a multiple of 4
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint4 *rc = reinterpret_cast<const uint4 *>(em.sel.rc1 + (bh * G + g) * em.sel.nreg);
      uint32_t part = 0u;
      for (int64_t i = tid; i < nq; i += Geo<NG>::THREADS) {
        const uint4 c = rc[i];
        part += c.x + c.y + c.z + c.w;
      }
      part = __builtin_amdgcn_readlane(wave_incl_scan_u32(part), kWave - 1);
      if (lane == 0 && part) atomicAdd(&s_tot[g], part);
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) skipm |= (s_tot[g] >= em.sel.kk ? 1u : 0u) << g;
    if (skipm == (1u << G) - 1u) return;  // uniform
  }
  int nc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) nc[c] = c < a.ncls ? min(max(ld_uniform(a.clsn + bh * a.bmax + c), 0), a.D) : 0;
  const PlanStreams ps = plan_streams(nc);
  tile_prologue<G, NG>(sh, a, nc, ps, bh);
  __syncthreads();  // plan streams ready
  if constexpr (MODE == kEmitFallback) {
    for (int64_t L = blockIdx.x; L < a.ntiles; L += gridDim.x) scan_one<G, kEmitFilter, FAST, NG>(a, em, sh, ps, L, wave, lane, skipm);
  } else {
    scan_one<G, MODE, FAST, NG>(a, em, sh, ps, blockIdx.x, wave, lane, 0u);
  }
}

// --------------------------------------------------------------------- chan4 baseline scan
// The channel-major 4-bit store (kernels/bitplane.py:67-74 pack_chan4,
// :175-198 scan_chan4_kernel): word m of (channel j, block b) holds the codes of
// tokens 8m..8m+7 of the block, nibble k = token 8m + k.  Every listed channel
// is read at full depth, 32 + 2 bytes per (channel, block).  Same tile and
// head contraction as the plane scan: y = 2a (c - 7.5) = c * 2a - 15a (one
// FMA of exact operands), w = q / 16, acc += w * y on the matrix cores, in
// list order, so a chan4 scan equals the plane scan of a plan with t = 4 on
// the same channels bit for bit.
constexpr int kC4Chan = 8;                 // channels per staged chunk
constexpr int kC4Row = kTB + 4;            // padded LDS row of one word index over the tile's blocks

struct Chan4Args {
  const float *q;            // [BH, G, D]
  const int32_t *act;        // [BH, D] listed channels first
  const int32_t *nact;       // [BH]
  const uint4 *chan;         // [BH, nsb, D, sub, 8] uint32 words as 16-byte halves
  const uint16_t *scales;    // [BH, nsb, D, sub] fp16 bits
  int64_t n, nsb, sub, blk0, blk_end, tile0;
  int D;
};

template <int G>
struct C4Buf {
  alignas(16) uint32_t w[kC4Chan][8][kC4Row];  // [channel slot][word m][block]
  alignas(16) float P[kC4Chan][kTB];           // 2a
  alignas(16) float Q[kC4Chan][kTB];           // -15a
  alignas(16) float wq[kC4Chan][QShared<G>::QS];
};

template <int G>
struct C4Shared {
  QShared<G> qs;
  uint8_t lst[kMaxD];
  C4Buf<G> buf[2];
};

// A thread stages two 16-byte halves (item e = tid + 256 h: channel slot e / 64,
// block (e / 2) % 32, half e % 2) and the scale of (slot tid / 32, block tid % 32).
struct C4Staged {
  uint4 v[2];
  uint16_t s;
};

__device__ __forceinline__ void c4_load(C4Staged &r, const Chan4Args &a, const uint8_t *lst, int i0, int m, int64_t bh,
                                        int64_t tb0, int tid) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = tid + kThreads * h, ci = e >> 6, b = (e >> 1) & (kTB - 1), half = e & 1;
    const int64_t blk = tb0 + b;
    r.v[h] = make_uint4(0u, 0u, 0u, 0u);
    if (ci < m && blk < a.nsb * a.sub) {
      const int64_t sb = blk / a.sub, off = blk - sb * a.sub;
      r.v[h] = a.chan[(((bh * a.nsb + sb) * a.D + lst[i0 + ci]) * a.sub + off) * 2 + half];
    }
  }
  const int ci = tid >> 5, b = tid & (kTB - 1);
  const int64_t blk = tb0 + b;
  r.s = 0;
  if (ci < m && blk < a.nsb * a.sub) {
    const int64_t sb = blk / a.sub, off = blk - sb * a.sub;
    r.s = a.scales[((bh * a.nsb + sb) * a.D + lst[i0 + ci]) * a.sub + off];
  }
}

template <int G>
__device__ __forceinline__ void c4_store(C4Buf<G> &bf, const C4Staged &r, const QShared<G> &qs, const uint8_t *lst,
                                         int i0, int m, int tid) {
  constexpr int QS = QShared<G>::QS;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = tid + kThreads * h, ci = e >> 6, b = (e >> 1) & (kTB - 1), half = e & 1;
    bf.w[ci][4 * half + 0][b] = r.v[h].x;
    bf.w[ci][4 * half + 1][b] = r.v[h].y;
    bf.w[ci][4 * half + 2][b] = r.v[h].z;
    bf.w[ci][4 * half + 3][b] = r.v[h].w;
  }
  const int ci = tid >> 5, b = tid & (kTB - 1);
  const float a = __half2float(__ushort_as_half(r.s));
  bf.P[ci][b] = 2.0f * a;
  bf.Q[ci][b] = -15.0f * a;
  if (b < QS && ci < m) bf.wq[ci][b] = qs.w[lst[i0 + ci] * QS + b];
}

template <int G>
__device__ __forceinline__ void c4_compute(const C4Buf<G> &bf, int m, int wave, int lane, Acc<G> &acc) {
  const int wm = lane >> 3, sh = 4 * (lane & 7);
  for (int ci = 0; ci < m; ++ci) {
    QOp<G> q;
#pragma unroll
    for (int h = 0; h < QOp<G>::NQ; ++h) q.a[h] = bf.wq[ci][4 * h + (lane & 3)];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint4 w4 = *reinterpret_cast<const uint4 *>(&bf.w[ci][wm][wave * kGB + 4 * hf]);
      const float4 P4 = *reinterpret_cast<const float4 *>(&bf.P[ci][wave * kGB + 4 * hf]);
      const float4 Q4 = *reinterpret_cast<const float4 *>(&bf.Q[ci][wave * kGB + 4 * hf]);
      const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
      const float P[4] = {P4.x, P4.y, P4.z, P4.w}, Q[4] = {Q4.x, Q4.y, Q4.z, Q4.w};
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = fmaf((float)__builtin_amdgcn_ubfe(wd[r], sh, 4), P[r], Q[r]);
#pragma unroll
      for (int r = 0; r < 4; ++r) accum<G>(acc, 4 * hf + r, q, y[r]);
    }
  }
}

template <int G>
__global__ __launch_bounds__(kThreads) void scan_chan4_kernel(Chan4Args a, Emit em) {
  constexpr int QS = QShared<G>::QS;
  __shared__ C4Shared<G> sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = blockIdx.y;
  const int64_t tb0 = (a.tile0 + (int64_t)blockIdx.x) * kTB;
  const int na = min(max(ld_uniform(a.nact + bh), 0), a.D);
  for (int i = tid; i < na; i += kThreads) {
    const int j = min(max(a.act[bh * a.D + i], 0), a.D - 1);  // memory-safe
    sh.lst[i] = (uint8_t)j;
#pragma unroll
    for (int g = 0; g < QS; ++g) sh.qs.w[j * QS + g] = g < G ? ldexpf(a.q[(bh * G + g) * a.D + j], -4) : 0.0f;
  }
  Acc<G> acc;
  acc.zero();
  if (tb0 < a.blk_end && tb0 + kTB > a.blk0 && na > 0) {
    __syncthreads();
    C4Staged r;
    const int nk = (na + kC4Chan - 1) / kC4Chan;
    c4_load(r, a, sh.lst, 0, min(kC4Chan, na), bh, tb0, tid);
    c4_store<G>(sh.buf[0], r, sh.qs, sh.lst, 0, min(kC4Chan, na), tid);
    __syncthreads();
    for (int k = 0; k < nk; ++k) {
      const int i0 = k * kC4Chan, m = min(kC4Chan, na - i0);
      const bool more = k + 1 < nk;
      const int i1 = i0 + kC4Chan, m1 = min(kC4Chan, na - i1);
      if (more) c4_load(r, a, sh.lst, i1, m1, bh, tb0, tid);
      c4_compute<G>(sh.buf[k & 1], m, wave, lane, acc);
      if (more) c4_store<G>(sh.buf[(k + 1) & 1], r, sh.qs, sh.lst, i1, m1, tid);
      __syncthreads();
    }
  }
  emit_group<G, kEmitScores>(em, acc, bh, tb0 + wave * kGB, a.blk0, a.blk_end, a.n, wave, lane, blockIdx.x, 0u);
}

template <int G>
void launch_chan4_g(const Chan4Args &a, int64_t tiles, int64_t BH, const Emit &em, hipStream_t st) {
  scan_chan4_kernel<G><<<dim3((unsigned)tiles, (unsigned)BH), kThreads, 0, st>>>(a, em);
}

// --------------------------------------------------------------------- launch
template <int G, int MODE>
void launch_g(const ScanArgs &a, int64_t tiles, int64_t BH, const Emit &em, hipStream_t st) {
  constexpr int NG = MODE == kEmitSample ? 1 : 2;
  constexpr int NT = Geo<NG>::THREADS;
  if (a.fast)
    scan_tile_kernel<G, MODE, true, NG><<<dim3((unsigned)tiles, (unsigned)BH), NT, 0, st>>>(a, em);
  else
    scan_tile_kernel<G, MODE, false, NG><<<dim3((unsigned)tiles, (unsigned)BH), NT, 0, st>>>(a, em);
}

constexpr int64_t kFallbackWGs = 64;  // workgroups per row of the fallback pass

template <int MODE>
int launch_scan(const ScanArgs &a0, int64_t G, int64_t tiles, int64_t BH, const Emit &em, hipStream_t st) {
  if (tiles <= 0) return FATHOM_OK;
  ScanArgs a = a0;
  a.ntiles = tiles;
  if (MODE == kEmitFallback && tiles > kFallbackWGs) tiles = kFallbackWGs;
  switch (G) {
    case 1: launch_g<1, MODE>(a, tiles, BH, em, st); break;
    case 2: launch_g<2, MODE>(a, tiles, BH, em, st); break;
    case 3: launch_g<3, MODE>(a, tiles, BH, em, st); break;
    case 4: launch_g<4, MODE>(a, tiles, BH, em, st); break;
    case 5: launch_g<5, MODE>(a, tiles, BH, em, st); break;
    case 6: launch_g<6, MODE>(a, tiles, BH, em, st); break;
    case 7: launch_g<7, MODE>(a, tiles, BH, em, st); break;
    default: launch_g<8, MODE>(a, tiles, BH, em, st); break;
  }
  return launch_status("scan_tile_kernel");
}

int check_scan(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax,
               const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, const char *who) {
  if (!q || !cls || !clsn || !planes_sb || !scales_sb) return fail(FATHOM_ERR_INVALID, "%s: null pointer", who);
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "%s: BH=%lld outside [1, 65535]", who, (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "%s: G=%lld outside [1, 8]", who, (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "%s: D=%lld outside [1, %d]", who, (long long)D, kMaxD);
  if (bmax < 1 || bmax > 8) return fail(FATHOM_ERR_INVALID, "%s: bmax=%d outside [1, 8]", who, bmax);
  if (n < 1 || n > (1LL << 31) || sub < 1)
    return fail(FATHOM_ERR_INVALID, "%s: n=%lld sub=%lld unsupported", who, (long long)n, (long long)sub);
  if (nsb < 1 || nsb * sub < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "%s: store holds %lld blocks (nsb=%lld x sub=%lld), n needs %lld", who,
                (long long)(nsb * sub), (long long)nsb, (long long)sub, (long long)cdiv(n, kBlk));
  return FATHOM_OK;
}

ScanArgs make_args(const float *q, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax, const void *planes_sb,
                   const void *scales_sb, int64_t n, int64_t nsb, int64_t sub) {
  ScanArgs a{};
  a.q = q;
  a.cls = cls;
  a.clsn = clsn;
  a.planes = static_cast<const uint64_t *>(planes_sb);
  a.scales = static_cast<const uint16_t *>(scales_sb);
  a.n = n;
  a.nsb = nsb;
  a.sub = sub;
  a.D = (int)D;
  a.bmax = bmax;
  a.ncls = bmax < 4 ? bmax : 4;
  a.tile_stride = 1;
  a.fast = sub % 4 == 0 && (reinterpret_cast<uintptr_t>(planes_sb) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(scales_sb) & 7) == 0;
  return a;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_planes(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                  const int32_t *clsn, int bmax, const void *planes_sb, const void *scales_sb,
                                  int64_t n, int64_t nsb, int64_t sub, int64_t blk0, int64_t blk1, float *out,
                                  void *stream) {
  int rc = check_scan(q, BH, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub, "scan_planes");
  if (rc) return rc;
  if (!out) return fail(FATHOM_ERR_INVALID, "scan_planes: null output");
  if (blk0 < 0 || blk1 < blk0)
    return fail(FATHOM_ERR_INVALID, "scan_planes: bad block range [%lld, %lld)", (long long)blk0, (long long)blk1);
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t blk_end = blk1 < nblk ? blk1 : nblk;
  if (blk_end <= blk0) return FATHOM_OK;
  ScanArgs a = make_args(q, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = blk0;
  a.blk_end = blk_end;
  a.tile0 = blk0 / kTB;
  const int64_t tiles = cdiv(blk_end, kTB) - a.tile0;
  Emit em{};
  em.out = out;
  return launch_scan<kEmitScores>(a, G, tiles, BH, em, (hipStream_t)stream);
}

namespace fathom {
namespace {
// Workspace of the fused scan + top-k: rows up to kRowSelectMax keep their
// scores ([rows, n] fp32) for one row-select launch; longer rows the sampled
// keys and the candidate regions.
size_t scan_topk_ws(int64_t rows, int64_t n, int64_t k) {
  if (n <= kRowSelectMax) return ws_align((size_t)rows * (size_t)n * 4);
  return topk_layout(rows, n, k, true, nullptr, nullptr, nullptr, nullptr, nullptr);
}
}  // namespace
}  // namespace fathom

extern "C" size_t fathom_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t n, int64_t k, int64_t sink,
                                                   int64_t local) {
  const int64_t kk = k - sink - local;
  if (BH < 1 || G < 1 || n < 1 || kk < 0) return 0;
  return scan_topk_ws(BH * G, n, k);
}

extern "C" int fathom_scan_topk(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                const int32_t *clsn, int bmax, const void *planes_sb, const void *scales_sb,
                                int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink,
                                int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_scan(q, BH, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub, "scan_topk");
  if (rc) return rc;
  if (!idx) return fail(FATHOM_ERR_INVALID, "scan_topk: null output");
  const int64_t rows = BH * G;
  rc = check_topk_args(rows, n, m, k, sink, local, "scan_topk");
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int64_t kk = k - sink - local;
  if (kk == 0) return launch_fixed_only(rows, m, k, sink, local, idx, st);
  const size_t need = scan_topk_ws(rows, n, k);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "scan_topk: workspace %zu bytes, need %zu", workspace_bytes, need);
  const int64_t nblk = cdiv(n, kBlk);
  ScanArgs a = make_args(q, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = 0;
  a.blk_end = nblk;
  a.tile0 = 0;
  if (n <= kRowSelectMax) {
    // short rows: the scores in the workspace, then the whole rows selected
    // in one launch (two kernels instead of the five of the chain below)
    Emit es{};
    es.out = static_cast<float *>(workspace);
    rc = launch_scan<kEmitScores>(a, G, cdiv(nblk, kTB), BH, es, st);
    if (rc) return rc;
    return launch_rowselect(es.out, rows, n, m, k, sink, local, idx, st);
  }
  Emit em{};
  int64_t S = 1;
  topk_layout(rows, n, k, true, static_cast<char *>(workspace), &em.samp, &em.samp_cap, &em.sel, &S);
  em.sel.kk = (uint32_t)kk;
  const int64_t r_hi = topk_hi_rank(n, S, kk);
  em.sink = sink;
  em.lstart = (m - local) > 0 ? (m - local) : 0;
  a.tile_stride = S;
  rc = launch_scan<kEmitSample>(a, G, topk_sample_tiles(n, S), BH, em, st);
  if (rc) return rc;
  rc = launch_select_keys(em.samp, rows, em.samp_cap, kk, r_hi, em.sel, st);
  if (rc) return rc;
  a.tile_stride = 1;
  rc = launch_scan<kEmitFilter>(a, G, cdiv(nblk, kTB), BH, em, st);
  if (rc) return rc;
  if (r_hi < kk) {  // T_hi may exceed a row's kk-th largest key: rows with < kk candidates scan again with T_lo
    em.fallback = 1;
    rc = launch_scan<kEmitFallback>(a, G, cdiv(nblk, kTB), BH, em, st);
    if (rc) return rc;
  }
  return launch_finalize(rows, m, k, sink, local, em.sel, idx, st);
}

extern "C" int fathom_scan_chan4(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *act,
                                 const int32_t *nact, const void *chan_sb, const void *scales_sb, int64_t n,
                                 int64_t nsb, int64_t sub, int64_t blk0, int64_t blk1, float *out, void *stream) {
  if (!q || !act || !nact || !chan_sb || !scales_sb || !out) return fail(FATHOM_ERR_INVALID, "scan_chan4: null pointer");
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "scan_chan4: BH=%lld outside [1, 65535]", (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "scan_chan4: G=%lld outside [1, 8]", (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "scan_chan4: D=%lld outside [1, %d]", (long long)D, kMaxD);
  if (n < 1 || sub < 1 || nsb < 1 || nsb * sub < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "scan_chan4: store of nsb=%lld x sub=%lld blocks does not cover n=%lld",
                (long long)nsb, (long long)sub, (long long)n);
  if ((reinterpret_cast<uintptr_t>(chan_sb) & 15) != 0)
    return fail(FATHOM_ERR_INVALID, "scan_chan4: the nibble store must be 16-byte aligned");
  if (blk0 < 0 || blk1 < blk0)
    return fail(FATHOM_ERR_INVALID, "scan_chan4: bad block range [%lld, %lld)", (long long)blk0, (long long)blk1);
  const int64_t nblk = cdiv(n, kBlk);
  const int64_t blk_end = blk1 < nblk ? blk1 : nblk;
  if (blk_end <= blk0) return FATHOM_OK;
  Chan4Args a{};
  a.q = q;
  a.act = act;
  a.nact = nact;
  a.chan = static_cast<const uint4 *>(chan_sb);
  a.scales = static_cast<const uint16_t *>(scales_sb);
  a.n = n;
  a.nsb = nsb;
  a.sub = sub;
  a.blk0 = blk0;
  a.blk_end = blk_end;
  a.tile0 = blk0 / kTB;
  a.D = (int)D;
  const int64_t tiles = cdiv(blk_end, kTB) - a.tile0;
  Emit em{};
  em.out = out;
  hipStream_t st = (hipStream_t)stream;
  switch (G) {
    case 1: launch_chan4_g<1>(a, tiles, BH, em, st); break;
    case 2: launch_chan4_g<2>(a, tiles, BH, em, st); break;
    case 3: launch_chan4_g<3>(a, tiles, BH, em, st); break;
    case 4: launch_chan4_g<4>(a, tiles, BH, em, st); break;
    case 5: launch_chan4_g<5>(a, tiles, BH, em, st); break;
    case 6: launch_chan4_g<6>(a, tiles, BH, em, st); break;
    case 7: launch_chan4_g<7>(a, tiles, BH, em, st); break;
    default: launch_chan4_g<8>(a, tiles, BH, em, st); break;
  }
  return launch_status("scan_chan4_kernel");
}
