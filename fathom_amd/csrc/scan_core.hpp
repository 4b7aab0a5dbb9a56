// The wave-tile machinery of the bit-plane scan (PlaneStore.scan): plan tables,
// the (channel, plane) contraction on the matrix cores, and the emission modes.
// Shared by the scan kernels and the fused top-k's finalize (its fallback rescan).
//
// Score of token i of row (bh, g), with depth t_j planes read for channel j
// (the dequantised value of kernels/bitplane.py:34-42, code bits b_jp, p = 0
// the most significant):
//   s = sum_j q_gj a_bj ((c_t + 0.5) / 2^(t_j - 1) - 1)
//     = sum_(j, p < t_j) W_gbu b_u(i)  +  C_gb,
//   W_gbu = q_gj a_bj 2^-p  for unit u = (j, p),   C_gb = sum_j q_gj a_bj (2^-t_j - 1),
// with a_bj the absmax scale of token block b (64 tokens).  The first sum is a
// [heads x units] by [units x tokens] product with a weight matrix per block.
//
// Matrix-core mapping (v_mfma_f32_4x4x4_16b_f16: 16 independent 4x4x4
// products; product k of an instruction reads lanes 4k..4k+3).  A wave owns a
// wave-tile of 16 consecutive token blocks (1024 tokens); product k is token
// block k, and lane 4k + i holds
//   A  row i (head i) of W_b for four units, as f16 hi + lo parts: hi = W
//      truncated to f16, lo = W - hi (two instructions; 21 significant bits);
//   B  the four units' bits of its token 16 i + r, as the f16 numbers
//      bit * 2^e_r, one pair of instructions per r = 0..15 with the same A;
//   D  the four heads' sums for that token (acc[r]).
// B takes one AND per dword and token: the lane's 16 bits of a unit (its
// quarter of the 64-bit plane word) are one f16 half of a dword, two units
// per dword (one byte permute), and each half is shifted once per group of
// four tokens so that the bits of tokens r = 4v..4v+3 sit on f16 exponent
// bits 11..14: masking one of them leaves 0 or the normal number 2^e_r,
// e_r = -13, -11, -7, 1.  (Subnormal B operands, bits 0..9, lose precision in
// the products: their error grows as 2^-e_r.)  A's parts and B are exact f16
// numbers, so every product is exact and the accumulation is fp32 (round to
// nearest even, measured).
//
// Range: before the split, W is scaled by 2^-(sigma_g + s_b): sigma_g from the
// head's largest |q|, s_b from the block's largest scale among the plan's
// channels, so |W| < 2^13.  The score is acc * 2^(sigma_g + s_b - e_r) + C_gb
// (one fused multiply-add of an exact power-of-two product).  Every output
// mode runs the same arithmetic, so scores, sampled keys and candidates agree
// bit for bit, whether the store is in HBM or in mapped host memory.
//
// A workgroup of 4 waves shares the plan tables (built once: per unit its
// plane word index, channel slot and the heads' q 2^-(p + sigma)); its waves
// then run independently over wave-tiles in a grid-stride loop.  Per
// wave-tile: the listed channels' scales of the 16 blocks are loaded into the
// wave's LDS (the four lanes of a block split the channels and reduce the
// block's largest scale and the constant C for every head with quad DPP
// sums), rescaled by 2^-s_b; then the plane dwords are loaded 8 units at a
// time (the next 8 in flight while the current ones are computed), one dword
// per lane and unit: 64 lanes read the unit's 16 blocks as one 128-byte run
// of a superblock store.  Stores in mapped host memory with superblocks of a
// multiple of 32 blocks are read two adjacent wave-tiles per instruction (256
// contiguous bytes, scan_tile_pair).
#pragma once
#include "topk_internal.hpp"

namespace fathom {
namespace sc {

constexpr int kWB = 16;                // token blocks per wave-tile: one MFMA product each
constexpr int kWTok = kWB * kBlk;      // tokens per wave-tile
constexpr int kR = 16;                 // tokens per lane (16 i + r)
static_assert(kR == kGroupTok, "a lane's tokens are one group of the group maxima");
constexpr int kWaves = 4;              // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxD = 128;             // the reference's head dimension (kernels/bitplane.py:313)
constexpr int kMaxUnits = 4 * kMaxD;   // (channel, plane) units of a plan
constexpr int kChunk = 8;              // units per load chunk
static_assert(kWTok == kRegTok, "a candidate region is one wave-tile");
static_assert(kMaxUnits % kChunk == 0, "unit tables pad to whole chunks");

typedef __fp16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
struct h2x2 {
  h2 a, b;
};

enum : int { kEmitScores = 0, kEmitSample = 1, kEmitFilter = 2, kEmitScoresMax = 3 };

struct ScanArgs {
  const float *q;          // [BH, G, D]
  const int32_t *cls;      // [BH, bmax, D]
  const int32_t *clsn;     // [BH, bmax]
  const uint32_t *planes;  // [BH, nsb, D, 4, sub] 64-bit words, read as dwords
  const uint16_t *scales;  // [BH, nsb, D, sub] fp16 bits
  int64_t n, nsb, sub;
  int64_t blk0, blk_end;   // blocks [blk0, blk_end) are emitted
  int64_t wt0;             // wave-tile of list entry 0 (wave-tile T = blocks [16T, 16T + 16))
  int64_t wt_stride;       // wave-tiles between consecutive list entries
  int64_t nwt;             // list entries per row
  int D, G, bmax, ncls;    // classes 1..ncls are scanned (ncls = min(bmax, 4))
};

struct Emit {
  float *out;        // scores [BH, G, n]
  uint32_t *gmax;    // kEmitScoresMax: [BH * G, ceil(n / 16)] each 16-token group's largest masked key
  uint32_t *samp;    // sampled keys [BH * G, samp_cap]: list entry L at L * kWTok
  int64_t samp_cap;
  TopkSel sel;       // thresholds + candidate regions
  int64_t sink, lstart;
};

// Wave-uniform loads through the constant address space (scalar loads).
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// e_r: the f16 number 2^e_r that token step r's bit stands for once masked
// (exponent bit 11 + (r & 3) of a half).
__host__ __device__ constexpr int bit_exp(int r) {
  return (r & 3) == 0 ? -13 : (r & 3) == 1 ? -11 : (r & 3) == 2 ? -7 : 1;
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The dword x with each 16-bit half shifted so that bits 4v..4v+3 land on
// bits 11..14 (higher bits of the half are dropped, lower ones stay below).
template <int V>
__device__ __forceinline__ uint32_t half_shift(uint32_t x) {
  const u16x2 h = __builtin_bit_cast(u16x2, x);
  constexpr int L = 11 - 4 * V;
  u16x2 r;
  if constexpr (L >= 0) r = h << (unsigned short)L;
  else r = h >> (unsigned short)(-L);
  return __builtin_bit_cast(uint32_t, r);
}

template <int NQ>
struct Shared {
  float qt[4 * NQ][kMaxUnits];     // q_gj 2^-(p + sigma_g) per unit (0: padding units, heads >= G)
  float qc[4 * NQ][kMaxD];         // q_gj (2^-t_j - 1) per channel slot
  uint32_t desc[kMaxUnits];        // unit -> plane word index (j * 4 + p) | slot << 16
  uint16_t schan[kMaxD];           // channel slot -> channel
  uint16_t a[kWaves][kMaxD][kWB];  // per wave: scales of the slots' channels by block (f16 bits)
  float qs[4 * NQ][kMaxD];         // the queries (0 for heads >= G)
  int sig[4 * NQ];                 // sigma_g: the exponent of the head's largest |q|
};

// Quad (4-lane) reductions: every lane of the quad gets the same value, summed
// in the fixed order (l0 + l1) + (l2 + l3).
__device__ __forceinline__ float quad_sum(float v) {
  v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
}
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
  return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
}

// A CU's waves of equal priority issue oldest first, so the workgroups placed
// first on a CU race ahead and the last ones run the kernel's tail at low
// occupancy.  Waves with more tiles left take a higher priority instead.
__device__ __forceinline__ void set_priority_by_tiles_left(int64_t left) {
  if (left >= 3) __builtin_amdgcn_s_setprio(3);
  else if (left == 2) __builtin_amdgcn_s_setprio(2);
  else if (left == 1) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Orders a wave's LDS accesses: every lane's writes before any lane's reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup prologue: the plan tables in LDS (units in class order: the class
// 1 list, then 2, 3, 4; a channel's planes consecutive), padded with zero
// weights to a whole number of chunks.  One round of global loads: the
// queries (32 threads per head, which also reduce the head's largest |q|)
// and the class lists, then the tables from LDS.  Returns the unit count.
template <int NQ>
__device__ __forceinline__ int plan_tables(Shared<NQ> &sh, const ScanArgs &a, int64_t bh, int &nact) {
  const int tid = threadIdx.x;
  int nc[4], SF[4], UE[4];
  int s = 0, u = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    nc[c] = c < a.ncls ? min(max(ld_uniform(a.clsn + bh * a.bmax + c), 0), a.D) : 0;
    nc[c] = min(nc[c], a.D - s);  // at most D slots in all
    s += nc[c];
    u += nc[c] * (c + 1);
    SF[c] = s;
    UE[c] = u;
  }
  nact = s;
  static_assert(4 * NQ * 32 <= kThreads, "32 threads per head");
  {
    const int h = tid >> 5, part = tid & 31;
    if (h < 4 * NQ) {
      float qv[kMaxD / 32];
#pragma unroll
      for (int k = 0; k < kMaxD / 32; ++k) {
        const int j = part + 32 * k;
        qv[k] = (h < a.G && j < a.D) ? a.q[(bh * a.G + h) * a.D + j] : 0.0f;
      }
      float m = 0.0f;
#pragma unroll
      for (int k = 0; k < kMaxD / 32; ++k) {
        sh.qs[h][part + 32 * k] = qv[k];
        m = fmaxf(m, fabsf(qv[k]));
      }
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 32));
      if (part == 0) sh.sig[h] = __builtin_amdgcn_frexp_expf(m);
    }
  }
  for (int e = tid; e < nact; e += kThreads) {
    const int c = (e >= SF[0]) + (e >= SF[1]) + (e >= SF[2]);
    const int lo = c == 0 ? 0 : SF[c - 1];
    const int jr = a.cls[(bh * a.bmax + c) * a.D + (e - lo)];
    sh.schan[e] = (uint16_t)min(max(jr, 0), a.D - 1);  // memory-safe; make_plan lists only valid channels
  }
  __syncthreads();
  for (int e = tid; e < nact; e += kThreads) {
    const int c = (e >= SF[0]) + (e >= SF[1]) + (e >= SF[2]);
    const int lo = c == 0 ? 0 : SF[c - 1];
    const int ub = (c == 0 ? 0 : UE[c - 1]) + (e - lo) * (c + 1);
    const int j = sh.schan[e];
    const float cf = ldexpf(1.0f, -(c + 1)) - 1.0f;
#pragma unroll
    for (int h = 0; h < 4 * NQ; ++h) {
      const float qv = sh.qs[h][j];
      sh.qc[h][e] = qv * cf;
      for (int p = 0; p <= c; ++p) sh.qt[h][ub + p] = ldexpf(qv, -(p + sh.sig[h]));
    }
    for (int p = 0; p <= c; ++p) sh.desc[ub + p] = (uint32_t)(j * 4 + p) | ((uint32_t)e << 16);
  }
  // zero-weight padding units (plane word 0) up to a whole chunk of every pass
  const int upad = (u + kChunk - 1) / kChunk * kChunk;
  for (int v = u + tid; v < upad; v += kThreads) {
    sh.desc[v] = 0u;
#pragma unroll
    for (int h = 0; h < 4 * NQ; ++h) sh.qt[h][v] = 0.0f;
  }
  __syncthreads();
  return u;
}

// Per-lane state of a wave-tile.  A wave computes the token steps r = r0 +
// RS k (k < kR / RS): all 16 (RS = 1), or one step class r & 3 = r0 (RS = 4,
// four waves sharing a tile); every step's accumulator sees the same MFMA
// sequence either way.
template <int NQ, int RS>
struct Tile {
  static constexpr int NR = kR / RS;
  f4 acc[NQ][NR];      // acc[hq][k][h]: head 4 hq + h, token 16 i + r0 + RS k of the lane's block
  float cst[4 * NQ];   // C of every head for the lane's block
  int sx;              // s_b of the lane's block
  int r0;              // first token step
};

// The wave-uniform descriptors of a chunk's units (in SGPRs): four broadcast
// LDS reads, then one readfirstlane per unit.
template <int CH>
struct ChunkDesc {
  uint32_t w[CH];
};

template <int CH>
__device__ __forceinline__ void read_descs(ChunkDesc<CH> &cd, const uint32_t *desc, int u0) {
  const uint4 *p = reinterpret_cast<const uint4 *>(desc + u0);
  uint4 v[CH / 4];
#pragma unroll
  for (int k = 0; k < CH / 4; ++k) v[k] = p[k];
#pragma unroll
  for (int k = 0; k < CH / 4; ++k) {
    cd.w[4 * k + 0] = __builtin_amdgcn_readfirstlane(v[k].x);
    cd.w[4 * k + 1] = __builtin_amdgcn_readfirstlane(v[k].y);
    cd.w[4 * k + 2] = __builtin_amdgcn_readfirstlane(v[k].z);
    cd.w[4 * k + 3] = __builtin_amdgcn_readfirstlane(v[k].w);
  }
}

// A lane's addressing of one wave-tile: buffer resources based at the row's
// superblock sb0 (the tile's first), a 32-bit lane offset, and the unit or
// channel offset in an SGPR (buffer soffset), so a load costs no address
// arithmetic.  Lanes whose block lies past the store (only in a tile that
// runs past n) read the tile's first block instead: every value a lane
// computes stays within its own block's four lanes, and tokens past n are
// never emitted.
struct TileAddr {
  __amdgpu_buffer_rsrc_t pr, sr;  // plane and scale buffers of superblock sb0 of row bh
  uint32_t poff, soff;            // lane byte offsets
};

constexpr int kBufFlags = 0x00020000;  // raw 32-bit buffer (gfx9 resource word 3)

// Loads the plane dwords of the chunk's units (unit offset w * sub * 8 bytes).
template <int CH>
__device__ __forceinline__ void load_chunk(uint32_t (&d)[CH], const ChunkDesc<CH> &cd, const TileAddr &ta,
                                           uint32_t sub8) {
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    d[k] = __builtin_amdgcn_raw_buffer_load_b32(ta.pr, ta.poff, (cd.w[k] & 0xFFFFu) * sub8, 0);
  }
}

// w - hi for the low (hi_half = false) or high f16 half of h: one mixed-precision
// FMA (exact: hi is w truncated to f16).
template <bool HI>
__device__ __forceinline__ float residual(h2 h, float w) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(w));
  else
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(w));
  return r;
}

// One chunk of units: per group of four units the weights (f16 hi/lo) and the
// token steps of B and the MFMAs.  FIRST: the tile's first chunk, whose first
// MFMA of every accumulator adds to zero (no separate clearing).
template <int NQ, int RS, int CH, bool FIRST = false>
__device__ __forceinline__ void compute_chunk(Tile<NQ, RS> &t, const uint32_t (&d)[CH], const ChunkDesc<CH> &cd,
                                              const Shared<NQ> &sh, const uint16_t *awb, int u0, int i, uint32_t sel) {
#pragma unroll
  for (int g = 0; g < CH / 4; ++g) {
    __fp16 av[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) av[k] = __builtin_bit_cast(__fp16, awb[(cd.w[4 * g + k] >> 16) * kWB]);
    h4 Ah[NQ], Al[NQ];
#pragma unroll
    for (int hq = 0; hq < NQ; ++hq) {
      const float4 qv = *reinterpret_cast<const float4 *>(&sh.qt[4 * hq + i][u0 + 4 * g]);
      // W = q' a' (the f16 scale as a mixed-precision FMA operand)
      const float W[4] = {__builtin_fmaf(qv.x, (float)av[0], 0.0f), __builtin_fmaf(qv.y, (float)av[1], 0.0f),
                          __builtin_fmaf(qv.z, (float)av[2], 0.0f), __builtin_fmaf(qv.w, (float)av[3], 0.0f)};
      const h2 h01 = __builtin_amdgcn_cvt_pkrtz(W[0], W[1]), h23 = __builtin_amdgcn_cvt_pkrtz(W[2], W[3]);
      const h2 l01 = __builtin_amdgcn_cvt_pkrtz(residual<false>(h01, W[0]), residual<true>(h01, W[1]));
      const h2 l23 = __builtin_amdgcn_cvt_pkrtz(residual<false>(h23, W[2]), residual<true>(h23, W[3]));
      Ah[hq] = __builtin_bit_cast(h4, (h2x2{h01, h23}));
      Al[hq] = __builtin_bit_cast(h4, (h2x2{l01, l23}));
    }
    const uint32_t x01 = __builtin_amdgcn_perm(d[4 * g + 1], d[4 * g], sel);
    const uint32_t x23 = __builtin_amdgcn_perm(d[4 * g + 3], d[4 * g + 2], sel);
    if constexpr (RS == 1) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t y01 = v == 0 ? half_shift<0>(x01) : v == 1 ? half_shift<1>(x01) : v == 2 ? half_shift<2>(x01) : half_shift<3>(x01);
        const uint32_t y23 = v == 0 ? half_shift<0>(x23) : v == 1 ? half_shift<1>(x23) : v == 2 ? half_shift<2>(x23) : half_shift<3>(x23);
        // two token steps at a time: both B operands first, then the hi products
        // of both, then the lo products (no MFMA waits on the one before it)
#pragma unroll
        for (int w = 0; w < 4; w += 2) {
          const int r = 4 * v + w;
          h4 B0, B1;
          {
            const uint32_t m0 = 0x08000800u << w, m1 = 0x08000800u << (w + 1);
            const uint32_t b0[2] = {y01 & m0, y23 & m0}, b1[2] = {y01 & m1, y23 & m1};
            __builtin_memcpy(&B0, b0, sizeof(B0));
            __builtin_memcpy(&B1, b1, sizeof(B1));
          }
#pragma unroll
          for (int hq = 0; hq < NQ; ++hq) {
            t.acc[hq][r] = __builtin_amdgcn_mfma_f32_4x4x4f16(Ah[hq], B0, FIRST && g == 0 ? f4{} : t.acc[hq][r], 0, 0, 0);
            t.acc[hq][r + 1] =
                __builtin_amdgcn_mfma_f32_4x4x4f16(Ah[hq], B1, FIRST && g == 0 ? f4{} : t.acc[hq][r + 1], 0, 0, 0);
          }
#pragma unroll
          for (int hq = 0; hq < NQ; ++hq) {
            t.acc[hq][r] = __builtin_amdgcn_mfma_f32_4x4x4f16(Al[hq], B0, t.acc[hq][r], 0, 0, 0);
            t.acc[hq][r + 1] = __builtin_amdgcn_mfma_f32_4x4x4f16(Al[hq], B1, t.acc[hq][r + 1], 0, 0, 0);
          }
        }
      }
    } else {
      static_assert(RS == 4, "token-step strides 1 and 4");
      // steps r = r0 + 4k: variant k, mask bit 11 + r0 of each half
      const uint32_t m = 0x08000800u << t.r0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t y01 = k == 0 ? half_shift<0>(x01) : k == 1 ? half_shift<1>(x01) : k == 2 ? half_shift<2>(x01) : half_shift<3>(x01);
        const uint32_t y23 = k == 0 ? half_shift<0>(x23) : k == 1 ? half_shift<1>(x23) : k == 2 ? half_shift<2>(x23) : half_shift<3>(x23);
        const uint32_t bb[2] = {y01 & m, y23 & m};
        h4 B;
        __builtin_memcpy(&B, bb, sizeof(B));
#pragma unroll
        for (int hq = 0; hq < NQ; ++hq)
          t.acc[hq][k] = __builtin_amdgcn_mfma_f32_4x4x4f16(Ah[hq], B, FIRST && g == 0 ? f4{} : t.acc[hq][k], 0, 0, 0);
#pragma unroll
        for (int hq = 0; hq < NQ; ++hq) t.acc[hq][k] = __builtin_amdgcn_mfma_f32_4x4x4f16(Al[hq], B, t.acc[hq][k], 0, 0, 0);
      }
    }
  }
}

// Output factors of head h for the lane's block: the score of token step r is
// acc * f[r & 3] + C with f[w] = 2^(sigma_h + s_b - e_w), one fused
// multiply-add of an exact power-of-two product.
template <int NQ, int RS>
__device__ __forceinline__ void head_factors(float (&f)[4], const Tile<NQ, RS> &t, const Shared<NQ> &sh, int h) {
#pragma unroll
  for (int w = 0; w < 4; ++w) f[w] = ldexpf(1.0f, sh.sig[h] + t.sx - bit_exp(w));
}

// Score of head h at the wave's k-th token step (RS = 1: step k).
template <int NQ, int RS>
__device__ __forceinline__ float tile_score(const Tile<NQ, RS> &t, const float (&f)[4], int k, int h) {
  const float fk = RS == 1 ? f[k & 3] : (t.r0 == 0 ? f[0] : t.r0 == 1 ? f[1] : t.r0 == 2 ? f[2] : f[3]);
  return fmaf(t.acc[h >> 2][k][h & 3], fk, t.cst[h]);
}

constexpr int kScaleBatch = 8;  // scale loads in flight per lane

// The tile's scale pass: lane i of a block takes the slots s = i (mod 4),
// kScaleBatch loads in flight; the per-head constants C, the block exponent
// s_b, and the scales rescaled by 2^-s_b into the wave's LDS buffer.
template <int NQ, int RS>
__device__ __forceinline__ void scale_pass(Tile<NQ, RS> &t, const Shared<NQ> &sh, uint16_t (*aw)[kWB],
                                           __amdgpu_buffer_rsrc_t sr, uint32_t soff, uint32_t sub2, int nact, int lane) {
  const int b = lane >> 2, i = lane & 3;
  float amax = 0.0f;
#pragma unroll
  for (int h = 0; h < 4 * NQ; ++h) t.cst[h] = 0.0f;
  for (int s0 = 0; s0 < nact; s0 += 4 * kScaleBatch) {
    uint16_t raw[kScaleBatch];
    uint32_t jo[kScaleBatch];
#pragma unroll
    for (int m = 0; m < kScaleBatch; ++m) {
      const int s = s0 + 4 * m + i;
      jo[m] = (s < nact ? sh.schan[s] : 0u) * sub2 + soff;
    }
#pragma unroll
    for (int m = 0; m < kScaleBatch; ++m) {
      raw[m] = __builtin_amdgcn_raw_buffer_load_b16(sr, jo[m], 0, 0);
    }
#pragma unroll
    for (int m = 0; m < kScaleBatch; ++m) {
      const int s = s0 + 4 * m + i;
      if (s < nact) {
        aw[s][b] = raw[m];
        const float av = f16_bits_to_float(raw[m]);
        amax = fmaxf(amax, av);
#pragma unroll
        for (int h = 0; h < 4 * NQ; ++h) t.cst[h] = fmaf(sh.qc[h][s], av, t.cst[h]);
      }
    }
  }
  amax = quad_max(amax);
#pragma unroll
  for (int h = 0; h < 4 * NQ; ++h) t.cst[h] = quad_sum(t.cst[h]);
  t.sx = __builtin_amdgcn_frexp_expf(amax) - 13;  // a * 2^-sx < 2^13
  wave_lds_sync();
  for (int s = i; s < nact; s += 4)
    aw[s][b] = float_to_f16_bits(ldexpf(f16_bits_to_float(aw[s][b]), -t.sx));
  wave_lds_sync();
}

// Scans one wave-tile (blocks beta0 .. beta0 + 15 of row bh) into t.  The first
// chunk's plane loads are issued before the scale pass, so the two round
// trips overlap.
template <int NQ, int RS, int CH>
__device__ __forceinline__ void scan_tile(Tile<NQ, RS> &t, const ScanArgs &a, const Shared<NQ> &sh, uint16_t (*aw)[kWB],
                                          int64_t bh, int64_t beta0, int U, int nact, int lane) {
  const int b = lane >> 2, i = lane & 3;
  TileAddr ta;
  {
    // block indices fit 32 bits (n <= 2^31); the lane's block is beta0 + b, so
    // its superblock is sb0 + (off0 + b) / sub, one step past sb0 at most when
    // sub >= 16
    const uint32_t sub = (uint32_t)a.sub, D = (uint32_t)a.D;
    const uint32_t sb0 = (uint32_t)beta0 / sub, off0 = (uint32_t)beta0 - sb0 * sub;
    const uint32_t x = off0 + (uint32_t)b;
    const uint32_t dq = sub >= (uint32_t)kWB ? (x >= sub ? 1u : 0u) : x / sub;
    const uint32_t off = x - dq * sub;
    const uint32_t *pb = a.planes + ((bh * a.nsb + sb0) * a.D * 4) * a.sub * 2;
    const uint16_t *sbp = a.scales + ((bh * a.nsb + sb0) * a.D) * a.sub;
    ta.pr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(pb), (short)0, 0x7FFFFFFF, kBufFlags);
    ta.sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(sbp), (short)0, 0x7FFFFFFF, kBufFlags);
    ta.poff = ta.soff = 0u;
    if ((int64_t)sb0 + dq < a.nsb) {
      ta.poff = ((dq * D * 4u) * sub + off) * 8u + (uint32_t)(i >> 1) * 4u;
      ta.soff = ((dq * D) * sub + off) * 2u;
    }
  }
  const uint32_t sub8 = (uint32_t)(a.sub * 8), sub2 = (uint32_t)(a.sub * 2);
  const int nck = (U + CH - 1) / CH;
  uint32_t d[CH], dn[CH];
  ChunkDesc<CH> cur, nxt;
  if (nck > 0) {
    read_descs(cur, sh.desc, 0);
    load_chunk(d, cur, ta, sub8);
  }
  scale_pass<NQ, RS>(t, sh, aw, ta.sr, ta.soff, sub2, nact, lane);
  const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;  // the lane's 16-bit half of each dword
  const uint16_t *awb = &aw[0][b];
  if (nck == 0) {
#pragma unroll
    for (int hq = 0; hq < NQ; ++hq)
#pragma unroll
      for (int k = 0; k < Tile<NQ, RS>::NR; ++k) t.acc[hq][k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    return;
  }
  // chunk 0 starts the accumulators
  if (nck > 1) {
    read_descs(nxt, sh.desc, CH);
    load_chunk(dn, nxt, ta, sub8);
  }
  compute_chunk<NQ, RS, CH, true>(t, d, cur, sh, awb, 0, i, sel);
#pragma unroll
  for (int k = 0; k < CH; ++k) d[k] = dn[k];
  cur = nxt;
  for (int ck = 1; ck < nck; ++ck) {
    if (ck + 1 < nck) {
      read_descs(nxt, sh.desc, (ck + 1) * CH);
      load_chunk(dn, nxt, ta, sub8);
    }
    compute_chunk<NQ, RS, CH>(t, d, cur, sh, awb, ck * CH, i, sel);
#pragma unroll
    for (int k = 0; k < CH; ++k) d[k] = dn[k];
    cur = nxt;
  }
}

// Scans the two adjacent wave-tiles of blocks beta0 .. beta0 + 31 (beta0 a
// multiple of 32, within one superblock: sub a multiple of 32) into tA and tB,
// for stores in mapped host memory: each load instruction reads one unit of
// both tiles, 256 contiguous bytes, which zero-copy reads over PCIe serve at
// the link's rate (128-byte reads run at about 70 % of it).  Lanes 4k, 4k + 1
// load block k of tile A, lanes 4k + 2, 4k + 3 block k of tile B (8 bytes
// each); a DPP swap of lane pairs then gives every lane its dword of both.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int CH>
__device__ __forceinline__ void load_chunk_pair(u32x2 (&d)[CH], const ChunkDesc<CH> &cd, __amdgpu_buffer_rsrc_t pr,
                                                uint32_t poff, uint32_t sub8) {
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(pr, poff, (cd.w[k] & 0xFFFFu) * sub8, 0);
    d[k] = u32x2{v[0], v[1]};
  }
}

template <int CH>
__device__ __forceinline__ void split_pair(const u32x2 (&d)[CH], uint32_t (&dA)[CH], uint32_t (&dB)[CH], int i) {
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const uint32_t px = (uint32_t)__builtin_amdgcn_mov_dpp((int)d[k][0], 0x4E, 0xF, 0xF, false);  // lane i ^ 2
    const uint32_t py = (uint32_t)__builtin_amdgcn_mov_dpp((int)d[k][1], 0x4E, 0xF, 0xF, false);
    dA[k] = i < 2 ? d[k][0] : py;  // dword i >> 1 of tile A's block
    dB[k] = i < 2 ? px : d[k][1];  // dword i >> 1 of tile B's block
  }
}

template <int NQ, int CH>
__device__ __forceinline__ void scan_tile_pair(Tile<NQ, 1> &tA, Tile<NQ, 1> &tB, const ScanArgs &a,
                                               const Shared<NQ> &sh, uint16_t (*awA)[kWB], uint16_t (*awB)[kWB],
                                               int64_t bh, int64_t beta0, int U, int nact, int lane) {
  const int b = lane >> 2, i = lane & 3;
  const uint32_t sub = (uint32_t)a.sub, sb0 = (uint32_t)beta0 / sub, off0 = (uint32_t)beta0 - sb0 * sub;
  const uint32_t *pb = a.planes + ((bh * a.nsb + sb0) * a.D * 4) * a.sub * 2;
  const uint16_t *sbp = a.scales + ((bh * a.nsb + sb0) * a.D) * a.sub;
  const __amdgpu_buffer_rsrc_t pr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(pb), (short)0, 0x7FFFFFFF, kBufFlags);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(sbp), (short)0, 0x7FFFFFFF, kBufFlags);
  const uint32_t poff = (off0 + (uint32_t)b + (i >= 2 ? (uint32_t)kWB : 0u)) * 8u;
  const uint32_t sub8 = (uint32_t)(a.sub * 8), sub2 = (uint32_t)(a.sub * 2);
  const int nck = (U + CH - 1) / CH;
  u32x2 d[CH], dn[CH];
  ChunkDesc<CH> cur, nxt;
  if (nck > 0) {
    read_descs(cur, sh.desc, 0);
    load_chunk_pair(d, cur, pr, poff, sub8);
  }
#pragma unroll
  for (int hq = 0; hq < NQ; ++hq)
#pragma unroll
    for (int k = 0; k < kR; ++k) tA.acc[hq][k] = tB.acc[hq][k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  scale_pass<NQ, 1>(tA, sh, awA, sr, (off0 + (uint32_t)b) * 2u, sub2, nact, lane);
  scale_pass<NQ, 1>(tB, sh, awB, sr, (off0 + kWB + (uint32_t)b) * 2u, sub2, nact, lane);
  const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;  // the lane's 16-bit half of each dword
  const uint16_t *awbA = &awA[0][b], *awbB = &awB[0][b];
  for (int ck = 0; ck < nck; ++ck) {
    if (ck + 1 < nck) {
      read_descs(nxt, sh.desc, (ck + 1) * CH);
      load_chunk_pair(dn, nxt, pr, poff, sub8);
    }
    uint32_t dA[CH], dB[CH];
    split_pair(d, dA, dB, i);
    compute_chunk<NQ, 1, CH>(tA, dA, cur, sh, awbA, ck * CH, i, sel);
    compute_chunk<NQ, 1, CH>(tB, dB, cur, sh, awbB, ck * CH, i, sel);
#pragma unroll
    for (int k = 0; k < CH; ++k) d[k] = dn[k];
    cur = nxt;
  }
}

// --------------------------------------------------------------------- emission
// Threshold of a row as a float for "key >= thr" (see filter below).
__device__ __forceinline__ float threshold_value(uint32_t thr) {
  if (thr <= kKeyNegInf) return -INFINITY;
  if (thr > 0xFF800000u) return INFINITY;  // above +inf's key: NaN and +inf pass
  return key_value(thr);
}

// Scores [BH, G, n]: the lane's 16 tokens of a head are 64 contiguous bytes.
// Largest key of the lane's 16 scores, sink/local-masked (-inf), past n
// excluded: a max over the floats (which passes NaN over) and a NaN test of
// pairs, then one key -- the maximum of the 16 keys.
__device__ __forceinline__ uint32_t group_max_key(const float (&s)[kR], int64_t tok0, int64_t n, int64_t sink,
                                                  int64_t lstart, bool plain) {
  float v[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t tok = tok0 + r;
    v[r] = plain || (tok < n && tok >= sink && tok < lstart) ? s[r] : -INFINITY;
  }
  float mx = -INFINITY;
  bool nan = false;
#pragma unroll
  for (int r = 0; r < kR; r += 2) {
    mx = fmaxf(mx, fmaxf(v[r], v[r + 1]));
    nan |= __builtin_isunordered(v[r], v[r + 1]);
  }
  return nan ? 0xFFFFFFFFu : score_key(mx);
}

// Scores of a wave-tile wholly inside its row and block range: lane l holds
// tokens 16 l .. 16 l + 15 of each head (the MFMA layout), so a store
// instruction straight from the registers would write four 16-byte pieces 64
// bytes apart per lane quad.  Instead each head's 4 KB goes through the wave's
// scale buffer (free once the tile's chunks are computed): float4 f (tokens
// 4f .. 4f + 3) in slot f ^ ((f >> 4) & 3), which spreads the sixteen lanes of
// each LDS phase over distinct banks both ways; then each store instruction
// writes 1 KB of consecutive tokens, with the non-temporal hint (the scores are
// read once, by the next kernel or the caller).
template <int NQ, bool GMAX>
__device__ __forceinline__ void emit_scores_staged(const Emit &em, const Tile<NQ, 1> &t, const Shared<NQ> &sh,
                                                   const ScanArgs &a, int64_t bh, int64_t beta0, int lane, void *stage) {
  const int b = lane >> 2, i = lane & 3;
  const int64_t beta = beta0 + b;
  const int64_t tok0 = beta * kBlk + 16 * i;
  const bool plain = tok0 >= em.sink && tok0 + kR <= em.lstart;
  const int64_t ngrp = (a.n + kR - 1) / kR;
  f4 *slots = reinterpret_cast<f4 *>(stage);
#pragma unroll
  for (int h = 0; h < 4 * NQ; ++h) {
    if (h >= a.G) break;
    float f[4], s[kR];
    head_factors(f, t, sh, h);
#pragma unroll
    for (int r = 0; r < kR; ++r) s[r] = tile_score<NQ, 1>(t, f, r, h);
    if (GMAX) em.gmax[(bh * a.G + h) * ngrp + beta * 4 + i] = group_max_key(s, tok0, a.n, em.sink, em.lstart, plain);
    wave_lds_sync();  // the buffer's last readers (the chunks, or the previous head) are done
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int fi = 4 * lane + c;
      slots[fi ^ ((fi >> 4) & 3)] = f4{s[4 * c], s[4 * c + 1], s[4 * c + 2], s[4 * c + 3]};
    }
    wave_lds_sync();
    float *dst = em.out + (bh * a.G + h) * a.n + beta0 * kBlk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int fi = 64 * j + lane;
      __builtin_nontemporal_store(slots[fi ^ ((fi >> 4) & 3)], reinterpret_cast<f4 *>(dst + 4 * fi));
    }
    __builtin_amdgcn_sched_barrier(0);  // one head's values live at a time
  }
}

// Scores [BH, G, n] of a wave-tile (and, GMAX, the 16-token group maxima
// beside them).  STAGED (kernels with registers to spare for it): whole tiles
// go out through stage, the wave's 4 KB LDS scale buffer, free at this point.
template <int NQ, bool GMAX = false, bool STAGED = false>
__device__ __forceinline__ void emit_scores(const Emit &em, const Tile<NQ, 1> &t, const Shared<NQ> &sh, const ScanArgs &a,
                                            int64_t bh, int64_t beta0, int lane, void *stage = nullptr) {
  static_assert(sizeof(sh.a[0]) == kWTok * sizeof(float), "a wave's scale buffer holds one head of a wave-tile");
  if constexpr (STAGED) {
    if (beta0 >= a.blk0 && beta0 + kWB <= a.blk_end && (beta0 + kWB) * kBlk <= a.n && (a.n & 3) == 0 &&
        ((uintptr_t)stage & 15) == 0) {  // uniform
      emit_scores_staged<NQ, GMAX>(em, t, sh, a, bh, beta0, lane, stage);
      return;
    }
  }
  const int b = lane >> 2, i = lane & 3;
  const int64_t beta = beta0 + b;
  if (beta < a.blk0 || beta >= a.blk_end) return;
  const int64_t tok0 = beta * kBlk + 16 * i;
  const bool whole = tok0 + kR <= a.n && (a.n & 3) == 0;
  const bool plain = tok0 + kR <= a.n && tok0 >= em.sink && tok0 + kR <= em.lstart;
  const int64_t ngrp = (a.n + kR - 1) / kR;
#pragma unroll
  for (int h = 0; h < 4 * NQ; ++h) {
    if (h >= a.G) break;
    float *dst = em.out + (bh * a.G + h) * a.n + tok0;
    float f[4], s[kR];
    head_factors(f, t, sh, h);
#pragma unroll
    for (int r = 0; r < kR; ++r) s[r] = tile_score<NQ, 1>(t, f, r, h);
    if (GMAX && tok0 < a.n)
      em.gmax[(bh * a.G + h) * ngrp + beta * 4 + i] = group_max_key(s, tok0, a.n, em.sink, em.lstart, plain);
    if (whole) {
#pragma unroll
      for (int r = 0; r < kR; r += 4) *reinterpret_cast<float4 *>(dst + r) = make_float4(s[r], s[r + 1], s[r + 2], s[r + 3]);
    } else {
#pragma unroll
      for (int r = 0; r < kR; ++r)
        if (tok0 + r < a.n) dst[r] = s[r];
    }
  }
}

// Sampled keys of list entry L (sink/local masked, 0 beyond the row): the
// wave's token steps of the lane's 16 tokens.
template <int NQ, int RS>
__device__ __forceinline__ void emit_sample(const Emit &em, const Tile<NQ, RS> &t, const Shared<NQ> &sh,
                                            const ScanArgs &a, int64_t bh, int64_t beta0, int64_t L, int lane) {
  const int b = lane >> 2, i = lane & 3;
  const int64_t tok0 = (beta0 + b) * kBlk + 16 * i;
#pragma unroll
  for (int h = 0; h < 4 * NQ; ++h) {
    if (h >= a.G) break;
    uint32_t *dst = em.samp + (bh * a.G + h) * em.samp_cap + L * kWTok + b * kBlk + 16 * i;
    float f[4];
    head_factors(f, t, sh, h);
#pragma unroll
    for (int k = 0; k < Tile<NQ, RS>::NR; ++k) {
      const int r = t.r0 + RS * k;
      const int64_t tok = tok0 + r;
      const bool masked = tok < em.sink || tok >= em.lstart;
      dst[r] = tok < a.n ? (masked ? kKeyNegInf : score_key(tile_score<NQ, RS>(t, f, k, h))) : 0u;
    }
  }
}

// Candidate emission of a wave-tile into its region (tokens [beta0 * 64, +
// 1024)) of each row: keys >= the row's threshold, ranked within the wave by
// ballots, and the region's count.  Heads in skipm emit nothing.
//
// In a tile with no masked token, a token step first runs a prefilter, one
// compare of the accumulators with a threshold in their own domain, T_w =
// ((thr - C) - margin) / f_w.  The score is RN(acc f_w + C) with acc f_w exact,
// so a score >= thr needs acc f_w + C >= thr - ulp(thr); the margin covers
// that ulp and the rounding of thr - C, so no passing token fails the
// prefilter (NaN passes both).  Only steps where some lane passes it compute
// scores and keys.
// f_w = 2^fe_w exactly, fe_w = fe0 - e_w, so dividing by it is an exact ldexp
// of the one numerator X = (thr - C) - margin when every f_w is a normal power
// of two (e_w spans [-13, 1]); otherwise T is NaN and every token of the tile
// takes the exact path.
__device__ __forceinline__ void acc_thresholds(float (&T)[4], float thr, float C, int fe0) {
  const float margin = (fabsf(thr) + fabsf(C)) * 0x1p-20f + 0x1p-126f;
  const bool ok = fabsf(C) < INFINITY && fe0 - bit_exp(3) >= -126 && fe0 - bit_exp(0) <= 127;
  const float X = ok ? (thr - C) - margin : __int_as_float(0x7FC00000);  // NaN: all pass
#pragma unroll
  for (int w = 0; w < 4; ++w) T[w] = ldexpf(X, bit_exp(w) - fe0);
}

template <int NQ>
__device__ __forceinline__ void emit_filter(const Emit &em, const Tile<NQ, 1> &t, const Shared<NQ> &sh,
                                            const ScanArgs &a, int64_t bh, int64_t beta0, int lane, bool fallback,
                                            uint32_t skipm, uint32_t (&tot)[4 * NQ]) {
  const int b = lane >> 2, i = lane & 3;
  const int64_t region = beta0 / kWB;
  const int64_t tok0 = (beta0 + b) * kBlk + 16 * i;
  const int64_t t0 = beta0 * kBlk, t1 = t0 + kWTok;
  // no per-lane validity or sink/local masking anywhere in the wave-tile
  const bool plain = beta0 >= a.blk0 && beta0 + kWB <= a.blk_end && t1 <= a.n && t0 >= em.sink && t1 <= em.lstart;
  const uint32_t *thr = fallback ? em.sel.thr_lo : em.sel.thr;
  uint32_t *rc = fallback ? em.sel.rc2 : em.sel.rc1;
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int h = 0; h < 4 * NQ; ++h) {
    if (h >= a.G) break;
    if ((skipm >> h) & 1u) continue;
    const int64_t row = bh * a.G + h;
    const float thr_f = threshold_value(ld_uniform(thr + row));
    const int fe0 = sh.sig[h] + t.sx;
    float T[4];
    if (plain) {
      acc_thresholds(T, thr_f, t.cst[h], fe0);
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) T[w] = __int_as_float(0x7FC00000);
    }
    uint64_t *dst = em.sel.cand + row * em.sel.cand_cap + t0;
    uint32_t off = 0u;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      if (__ballot(!(t.acc[h >> 2][r][h & 3] < T[r & 3])) == 0ull) continue;  // uniform
      const int64_t tok = tok0 + r;
      // the score as tile_score forms it: acc * 2^(sigma + s_b - e_r) + C
      const float v = fmaf(t.acc[h >> 2][r][h & 3], ldexpf(1.0f, fe0 - bit_exp(r)), t.cst[h]);
      bool valid = true;
      float vm = v;
      if (!plain) {
        const int64_t blk = beta0 + b;
        valid = blk >= a.blk0 && blk < a.blk_end && tok < a.n;
        vm = (tok < em.sink || tok >= em.lstart) ? -INFINITY : v;
      }
      const bool pass = valid && !(vm < thr_f);
      const uint64_t msk = __ballot(pass);
      if (pass) dst[off + (uint32_t)__popcll(msk & lt)] = k64_of(vm == -INFINITY ? kKeyNegInf : score_key(vm), tok);
      off += (uint32_t)__popcll(msk);
    }
    if (lane == 0) rc[row * em.sel.nreg + region] = off;
    tot[h] += off;
  }
}

// The tile loop of the one-tile modes: list entries L0, L0 + Ls, ... < nlist.
// FB: the candidate pass's fallback rescan (T_lo, second count array; heads in
// skipm emit nothing).
template <int NQ, int MODE, bool FB>
__device__ __forceinline__ void tile_pass(Tile<NQ, 1> &t, const ScanArgs &a, const Emit &em, const Shared<NQ> &sh,
                                          uint16_t (*aw)[kWB], int64_t bh, int U, int nact, int lane, int64_t L0,
                                          int64_t Ls, int64_t nlist, uint32_t skipm, uint32_t (&tot)[4 * NQ]) {
  constexpr bool kCand = MODE == kEmitFilter;
  uint32_t *rcp = FB ? em.sel.rc2 : em.sel.rc1;
  for (int64_t L = L0; L < nlist; L += Ls) {
    if (kCand && L >= a.nwt) {
      if (lane < a.G && !((skipm >> lane) & 1u)) rcp[(bh * a.G + lane) * em.sel.nreg + L] = 0u;
      continue;
    }
    const int64_t beta0 = (a.wt0 + L * a.wt_stride) * kWB;
    if (beta0 >= a.blk_end || beta0 + kWB <= a.blk0) continue;  // uniform per wave
    set_priority_by_tiles_left((nlist - 1 - L) / Ls);
    scan_tile<NQ, 1, kChunk>(t, a, sh, aw, bh, beta0, U, nact, lane);
    if constexpr (MODE == kEmitScores || MODE == kEmitScoresMax)
      emit_scores<NQ, MODE == kEmitScoresMax, NQ == 1 || MODE == kEmitScores>(em, t, sh, a, bh, beta0, lane, aw);
    if constexpr (MODE == kEmitFilter) emit_filter<NQ>(em, t, sh, a, bh, beta0, lane, FB, skipm, tot);
    wave_lds_sync();  // the wave's scale buffer is rewritten by its next tile
  }
}

}  // namespace sc

// Exact top kk of every row of the fused scan + top-k from its candidate
// regions; a row whose first pass holds fewer than kk candidates (a sample that
// misled T_hi) is first rescanned with T_lo by its finalize workgroup.
int launch_finalize_fused(const sc::ScanArgs &a, const sc::Emit &em, int64_t rows, int64_t m, int64_t k, int64_t sink,
                          int64_t local, int64_t *idx, hipStream_t st);

}  // namespace fathom
