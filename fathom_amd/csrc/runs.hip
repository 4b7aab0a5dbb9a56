// Run copies of the copy-index path: contiguous runs of a store in mapped
// pinned host memory are moved into an HBM staging store at the same offsets,
// then scanned there (scripts/B_e2e_offload_v2.py:62-71 gather_runs_kernel,
// :190-197 the copy-index run list).
//
// In the whole-sequence layout (sub = nblk, one superblock) the first t planes
// of channel j are one run of t * nblk words and its scales one run of nblk
// halves, so a plan needs one plane run and one scale run per listed channel:
// a few hundred runs of 32-512 KB for a 1M-token layer.  Each workgroup moves a
// 64 KB piece of one run with 16-byte lane loads (8 in flight per lane), a
// stream of whole 4 KB requests that keeps the PCIe link busy.  Run lengths
// come from the device (the plan's t, or a run list), so nothing waits on the
// host; empty runs cost a workgroup that exits at once.
#include "common.hpp"

namespace fathom {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kUnroll = 8;                                        // vectors in flight per lane
constexpr int64_t kPieceVec = (int64_t)kCopyThreads * kUnroll * 4;  // vectors per workgroup piece (4 rounds)

// Register form of a copy unit: clang vector types, which stay in VGPRs (an
// array of HIP's struct vector types is spilled to scratch memory).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <typename V> struct Reg { typedef V type; };
template <> struct Reg<uint4> { typedef u32x4 type; };
template <> struct Reg<uint2> { typedef u32x2 type; };

// Copies vectors [b, e) of src to dst (same offsets), kUnroll loads in flight per lane.
template <typename V>
__device__ __forceinline__ void copy_vectors(const V *__restrict__ src_v, V *__restrict__ dst_v, int64_t b, int64_t e) {
  typedef typename Reg<V>::type R;
  static_assert(sizeof(R) == sizeof(V), "register form must match the vector size");
  const R *__restrict__ src = reinterpret_cast<const R *>(src_v);
  R *__restrict__ dst = reinterpret_cast<R *>(dst_v);
  for (int64_t i0 = b; i0 < e; i0 += (int64_t)kCopyThreads * kUnroll) {
    R v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * kCopyThreads + threadIdx.x;
      v[u] = i < e ? src[i] : R{};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * kCopyThreads + threadIdx.x;
      if (i < e) dst[i] = v[u];
    }
  }
}

// Generic run list: run r covers vectors [off[r], off[r] + len[r]) (in units of V).
template <typename V>
__global__ __launch_bounds__(kCopyThreads) void gather_runs_kernel(const V *__restrict__ src, V *__restrict__ dst,
                                                                   const int64_t *__restrict__ off,
                                                                   const int64_t *__restrict__ len,
                                                                   const int32_t *__restrict__ nrun) {
  const int64_t r = blockIdx.y;
  if (r >= (int64_t)*nrun) return;
  const int64_t l = len[r];
  const int64_t b = (int64_t)blockIdx.x * kPieceVec;
  if (l <= 0 || b >= l) return;
  const int64_t o = off[r];
  copy_vectors(src, dst, o + b, o + (l < b + kPieceVec ? l : b + kPieceVec));
}

// Plan-driven runs: slot s (= bh * D + channel) covers vectors
// [s * stride, s * stride + unit * w(t_s)) with w(t) = min(t, 4) (plane runs:
// the store holds 4 planes) or [t > 0] (scale runs).
template <typename V>
__global__ __launch_bounds__(kCopyThreads) void copy_index_kernel(const V *__restrict__ src, V *__restrict__ dst,
                                                                  const int8_t *__restrict__ t, int64_t stride,
                                                                  int64_t unit, int per_plane) {
  const int64_t s = blockIdx.y;
  const int ts = t[s];
  const int64_t l = (per_plane ? (ts > 0 ? (ts < 4 ? ts : 4) : 0) : (ts > 0 ? 1 : 0)) * unit;
  const int64_t b = (int64_t)blockIdx.x * kPieceVec;
  if (b >= l) return;
  const int64_t o = s * stride;
  copy_vectors(src, dst, o + b, o + (l < b + kPieceVec ? l : b + kPieceVec));
}

// One block range of the plan-selected runs (the chunked copy/scan pipeline):
// slot y = s * P + p (s = bh * D + channel, p < P) covers [y * stride + off,
// y * stride + off + len) in units of V and is copied when its plan depth t_s
// selects it: p < min(t_s, 4) for plane slots (P = 4), t_s > 0 otherwise.
template <typename V>
__global__ __launch_bounds__(kCopyThreads) void copy_range_kernel(const V *__restrict__ src, V *__restrict__ dst,
                                                                  const int8_t *__restrict__ t, int P,
                                                                  int64_t stride, int64_t off, int64_t len) {
  const int64_t y = blockIdx.y;
  const int ts = t[y / P];
  const int p = (int)(y % P);
  const bool on = P == 4 ? p < (ts < 4 ? ts : 4) : ts > 0;
  const int64_t b = (int64_t)blockIdx.x * kPieceVec;
  if (!on || b >= len) return;
  const int64_t o = y * stride + off;
  copy_vectors(src, dst, o + b, o + (len < b + kPieceVec ? len : b + kPieceVec));
}

template <typename V>
void launch_copy_range_v(const void *src, void *dst, const int8_t *t, int64_t slots, int P, int64_t stride_b,
                         int64_t off_b, int64_t len_b, hipStream_t st) {
  const int64_t sz = (int64_t)sizeof(V);
  const int64_t pieces = cdiv(len_b / sz, kPieceVec);
  if (pieces == 0) return;
  copy_range_kernel<V><<<dim3((unsigned)pieces, (unsigned)(slots * P)), kCopyThreads, 0, st>>>(
      static_cast<const V *>(src), static_cast<V *>(dst), t, P, stride_b / sz, off_b / sz, len_b / sz);
}

int launch_copy_range(const void *src, void *dst, const int8_t *t, int64_t slots, int P, int64_t stride_b,
                      int64_t off_b, int64_t len_b, hipStream_t st) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | (uintptr_t)stride_b |
                      (uintptr_t)off_b | (uintptr_t)len_b;
  if ((a & 15) == 0)
    launch_copy_range_v<uint4>(src, dst, t, slots, P, stride_b, off_b, len_b, st);
  else if ((a & 7) == 0)
    launch_copy_range_v<uint2>(src, dst, t, slots, P, stride_b, off_b, len_b, st);
  else if ((a & 3) == 0)
    launch_copy_range_v<uint32_t>(src, dst, t, slots, P, stride_b, off_b, len_b, st);
  else
    launch_copy_range_v<uint16_t>(src, dst, t, slots, P, stride_b, off_b, len_b, st);
  return launch_status("copy_range_kernel");
}

template <typename V>
void launch_copy_index_v(const void *src, void *dst, const int8_t *t, int64_t slots, int64_t stride_bytes,
                         int64_t unit_bytes, int max_w, bool per_plane, hipStream_t st) {
  const int64_t unit = unit_bytes / (int64_t)sizeof(V), stride = stride_bytes / (int64_t)sizeof(V);
  const int64_t pieces = cdiv(unit * max_w, kPieceVec);
  if (pieces == 0) return;
  copy_index_kernel<V><<<dim3((unsigned)pieces, (unsigned)slots), kCopyThreads, 0, st>>>(
      static_cast<const V *>(src), static_cast<V *>(dst), t, stride, unit, per_plane ? 1 : 0);
}

// Vector width: 16 bytes when every run start and length allows, else 4 or 2.
int launch_copy_index(const void *src, void *dst, const int8_t *t, int64_t slots, int64_t stride_bytes,
                      int64_t unit_bytes, int max_w, bool per_plane, hipStream_t st) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                      (uintptr_t)stride_bytes | (uintptr_t)unit_bytes;
  if ((a & 15) == 0)
    launch_copy_index_v<uint4>(src, dst, t, slots, stride_bytes, unit_bytes, max_w, per_plane, st);
  else if ((a & 3) == 0)
    launch_copy_index_v<uint32_t>(src, dst, t, slots, stride_bytes, unit_bytes, max_w, per_plane, st);
  else
    launch_copy_index_v<uint16_t>(src, dst, t, slots, stride_bytes, unit_bytes, max_w, per_plane, st);
  return launch_status("copy_index_kernel");
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_gather_runs(const void *src, void *dst, const int64_t *off, const int64_t *len,
                                  const int32_t *nrun, int64_t R, int64_t max_len, void *stream) {
  if (!src || !dst || !off || !len || !nrun) return fail(FATHOM_ERR_INVALID, "gather_runs: null pointer");
  if (R < 0 || R > 65535 || max_len < 0)
    return fail(FATHOM_ERR_INVALID, "gather_runs: R=%lld (at most 65535) max_len=%lld", (long long)R,
                (long long)max_len);
  if (R == 0 || max_len == 0) return FATHOM_OK;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 3)
    return fail(FATHOM_ERR_INVALID, "gather_runs: src and dst must be 4-byte aligned");
  const dim3 grid((unsigned)cdiv(max_len, kPieceVec), (unsigned)R);
  gather_runs_kernel<uint32_t><<<grid, kCopyThreads, 0, (hipStream_t)stream>>>(
      static_cast<const uint32_t *>(src), static_cast<uint32_t *>(dst), off, len, nrun);
  return launch_status("gather_runs_kernel");
}

extern "C" int fathom_copy_index(const int8_t *t, int64_t BH, int64_t D, int64_t nblk, const void *planes_src,
                                 const void *scales_src, void *planes_dst, void *scales_dst, void *stream) {
  if (!t || !planes_src || !scales_src || !planes_dst || !scales_dst)
    return fail(FATHOM_ERR_INVALID, "copy_index: null pointer");
  if (BH < 1 || D < 1 || BH * D > 65535 || nblk < 1)
    return fail(FATHOM_ERR_INVALID, "copy_index: BH=%lld D=%lld nblk=%lld unsupported (BH * D <= 65535)",
                (long long)BH, (long long)D, (long long)nblk);
  hipStream_t st = (hipStream_t)stream;
  // planes [BH, 1, D, 4, nblk] uint64: slot stride 4 * nblk words, plane unit nblk words
  int rc = launch_copy_index(planes_src, planes_dst, t, BH * D, 32 * nblk, 8 * nblk, 4, true, st);
  if (rc) return rc;
  // scales [BH, 1, D, nblk] fp16: slot stride = unit = nblk halves
  return launch_copy_index(scales_src, scales_dst, t, BH * D, 2 * nblk, 2 * nblk, 1, false, st);
}

extern "C" int fathom_copy_index_range(const int8_t *t, int64_t BH, int64_t D, int64_t nblk, int64_t b0, int64_t b1,
                                       int64_t block_bytes, int planes, const void *data_src, const void *scales_src,
                                       void *data_dst, void *scales_dst, void *stream) {
  if (!t || !data_src || !scales_src || !data_dst || !scales_dst)
    return fail(FATHOM_ERR_INVALID, "copy_index_range: null pointer");
  if (planes != 1 && planes != 4) return fail(FATHOM_ERR_INVALID, "copy_index_range: planes=%d (1 or 4)", planes);
  if (BH < 1 || D < 1 || BH * D * planes > 65535 || nblk < 1 || block_bytes < 2 || block_bytes % 2)
    return fail(FATHOM_ERR_INVALID, "copy_index_range: BH=%lld D=%lld nblk=%lld block_bytes=%lld unsupported",
                (long long)BH, (long long)D, (long long)nblk, (long long)block_bytes);
  if (b0 < 0 || b1 < b0 || b1 > nblk)
    return fail(FATHOM_ERR_INVALID, "copy_index_range: blocks [%lld, %lld) outside [0, %lld)", (long long)b0,
                (long long)b1, (long long)nblk);
  if (b1 == b0) return FATHOM_OK;
  hipStream_t st = (hipStream_t)stream;
  // data runs: planes [BH, 1, D, 4, nblk] words (planes = 4) or chan4 words [BH, 1, D, nblk, 8] (planes = 1)
  int rc = launch_copy_range(data_src, data_dst, t, BH * D, planes, nblk * block_bytes, b0 * block_bytes,
                             (b1 - b0) * block_bytes, st);
  if (rc) return rc;
  // scale runs [BH, 1, D, nblk] fp16
  return launch_copy_range(scales_src, scales_dst, t, BH * D, 1, nblk * 2, b0 * 2, (b1 - b0) * 2, st);
}
