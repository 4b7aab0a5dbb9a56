// Partial-depth bit-plane scan (PlaneStore.scan) and the fused scan + top-k:
// the kernels and launches over the wave-tile machinery of scan_core.hpp.
#include <type_traits>

#include "scan_core.hpp"
#include "scan_internal.hpp"
#include "attn_core.hpp"

namespace fathom {
namespace {

using namespace sc;

// --------------------------------------------------------------------- kernel
// Grid (workgroups, BH); the waves of the grid's row take the list entries L
// in a grid-stride loop.  Nothing waits on another wave: a candidate pass
// that found fewer than kk candidates for a row is completed by the row's
// finalize workgroup (launch_finalize_fused).  The sample pass gives each of
// its tiles four waves, one quarter of every block each.
// NSMAX (2..4 at four waves per SIMD, 6 at two): the plan slices (16 units
// each) held in registers; ACC (1 or 4): step groups whose accumulators a
// larger plan keeps over its register groups (4: fewer reloads, more
// registers).  The scores are the same for any
// choice; the launch picks them from the plan's units bound.  HOST (the
// candidate pass over a store in mapped host memory, superblocks of a
// multiple of 64 blocks): workgroups stage groups of four wave-tiles in LDS
// (two workgroups per CU).
template <int MODE, int NSMAX, int ACC, bool HOST = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(
    ACC == 4 || HOST ? 2 : 4))) void scan_wave_kernel(ScanArgs a, Emit em, int split) {
  __shared__ Shared sh;
  __shared__ std::conditional_t<HOST, HostStage, char> hst;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = blockIdx.y;
  // the candidate pass starts from the tables its sample pass left, every
  // other launch builds them
  if (MODE != kEmitFilter || !em.tab || !load_tables(sh, a, em.tab + bh, NSMAX * kSlice))
    plan_tables(sh, a, bh, NSMAX * kSlice);
  if (MODE == kEmitSample && em.tab && blockIdx.x == 0) save_tables(sh, em.tab + bh, NSMAX * kSlice);
  if (MODE == kEmitSample || (MODE != kEmitFilter && split == 4)) {
    // few tiles (the sample pass, short rows): four waves per tile, one
    // quarter each; the candidate pass keeps whole tiles (a region per tile)
    static_assert(kWaves == kQS, "a wave per quarter of a tile");
    tile_pass<MODE, ACC, false, NSMAX>(a, em, sh, bh, lane, (int64_t)blockIdx.x, (int64_t)gridDim.x, a.nwt,
                                       wave, wave + 1, 0u);
  } else if (MODE != kEmitFilter && split == 2) {
    // short rows on the two-waves-per-SIMD kernels: two tiles per workgroup,
    // two quarters per wave (every wave of the launch resident at once)
    const int q0 = (wave & 1) * 2;
    tile_pass<MODE, ACC, false, NSMAX>(a, em, sh, bh, lane, (int64_t)blockIdx.x * 2 + (wave >> 1),
                                       (int64_t)gridDim.x * 2, a.nwt, q0, q0 + 2, 0u);
  } else {
    // the candidate pass also writes the (zero) counts of the padding regions past the row
    constexpr bool kCand = MODE == kEmitFilter;
    const int64_t nlist = kCand && em.sel.nreg > a.nwt ? em.sel.nreg : a.nwt;
    if constexpr (HOST) {
      static_assert(kCand, "staged host tiles in the candidate pass");
      const int nsl = __builtin_amdgcn_readfirstlane(sh.U) / kSlice;
      const int ureal = __builtin_amdgcn_readfirstlane(sh.ureal);
      if (nsl <= NSMAX) {  // uniform; larger plans read the store directly
        if (a.G <= kMaxG / 2)
          host_tile_loop<MODE, NSMAX, false, true>(a, em, sh, hst, bh, lane, wave, nlist, 0u, nsl, ureal);
        else
          host_tile_loop<MODE, NSMAX, false, false>(a, em, sh, hst, bh, lane, wave, nlist, 0u, nsl, ureal);
        return;
      }
    }
    const int64_t L0 = (int64_t)blockIdx.x * kWaves + wave, Ls = (int64_t)gridDim.x * kWaves;
    tile_pass<MODE, ACC, false, NSMAX>(a, em, sh, bh, lane, L0, Ls, nlist, 0, kQS, 0u);
  }
}

// --------------------------------------------------------------------- launch
constexpr int64_t kTargetWaves = 4096;  // waves of a full launch (4 per SIMD on 256 CUs)

template <int MODE>
int launch_scan(const ScanArgs &a0, int64_t nwt, int64_t BH, const Emit &em, int64_t units_max, hipStream_t st) {
  if (nwt <= 0) return FATHOM_OK;
  ScanArgs a = a0;
  a.nwt = nwt;
  int64_t wgs;
  int split = 0;
  const int64_t nsl = cdiv(units_max, kSlice);
  if (MODE == kEmitSample || (MODE != kEmitFilter && nwt * BH < kTargetWaves)) {
    // fewer tiles than wave slots: waves split the tiles' quarters, two
    // quarters (one quarter pair of the plane dwords) per wave in the score
    // modes, one per wave in the sample pass
    split = MODE != kEmitSample ? 2 : 4;
    wgs = split == 4 ? nwt : cdiv(nwt, 2);
  } else {
    // enough waves to fill the chip, each taking a whole number of tiles
    const int64_t per = cdiv(nwt * BH, kTargetWaves);
    wgs = cdiv(cdiv(nwt, per), kWaves);
  }
  // the layout of stores in mapped host memory (superblocks of a multiple of
  // 64 blocks, shorter than the row; 16-byte aligned): the candidate pass
  // stages its tiles, two workgroups per CU.  The whole-row layout of the
  // copy-index staging store (in HBM) reads directly.
  const bool host = MODE == kEmitFilter && nsl <= kGS && a.sub % kHostBlk == 0 && a.sub < cdiv(a.n, kBlk) &&
                    (reinterpret_cast<uintptr_t>(a.planes) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.scales) & 15) == 0;
  if (host) {
    const int64_t per = cdiv(nwt * BH, kTargetWaves / 2);
    const dim3 hgrid((unsigned)cdiv(cdiv(nwt, per), kWaves), (unsigned)BH);
    if (MODE == kEmitFilter) {
      if (nsl == 4)
        scan_wave_kernel<kEmitFilter, 4, 1, true><<<hgrid, kThreads, 0, st>>>(a, em, split);
      else if (nsl == 3)
        scan_wave_kernel<kEmitFilter, 3, 1, true><<<hgrid, kThreads, 0, st>>>(a, em, split);
      else
        scan_wave_kernel<kEmitFilter, 2, 1, true><<<hgrid, kThreads, 0, st>>>(a, em, split);
    }
    return launch_status("scan_wave_kernel");
  }
  const dim3 grid((unsigned)wgs, (unsigned)BH);
  if (nsl > kGS)
    scan_wave_kernel<MODE, kMaxNS, 4><<<grid, kThreads, 0, st>>>(a, em, split);
  else if (nsl == 4)
    scan_wave_kernel<MODE, 4, 1><<<grid, kThreads, 0, st>>>(a, em, split);
  else if (nsl == 3)
    scan_wave_kernel<MODE, 3, 1><<<grid, kThreads, 0, st>>>(a, em, split);
  else
    scan_wave_kernel<MODE, 2, 1><<<grid, kThreads, 0, st>>>(a, em, split);
  return launch_status("scan_wave_kernel");
}

// The plan's units bound: the caller's, else every channel at full depth.
int64_t units_bound(int64_t units_max, int64_t D, int bmax) {
  const int64_t full = D * (bmax < 4 ? bmax : 4);
  return units_max > 0 && units_max < full ? units_max : full;
}

int check_scan(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax,
               const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, const char *who,
               bool own_plan = false) {
  if (!q || (!own_plan && (!cls || !clsn)) || !planes_sb || !scales_sb)
    return fail(FATHOM_ERR_INVALID, "%s: null pointer", who);
  if (BH < 1 || BH > 65535) return fail(FATHOM_ERR_INVALID, "%s: BH=%lld outside [1, 65535]", who, (long long)BH);
  if (G < 1 || G > 8) return fail(FATHOM_ERR_INVALID, "%s: G=%lld outside [1, 8]", who, (long long)G);
  if (D < 1 || D > kMaxD) return fail(FATHOM_ERR_INVALID, "%s: D=%lld outside [1, %d]", who, (long long)D, kMaxD);
  if (bmax < 1 || bmax > 8) return fail(FATHOM_ERR_INVALID, "%s: bmax=%d outside [1, 8]", who, bmax);
  if (n < 1 || n > (1LL << 31) || sub < 1)
    return fail(FATHOM_ERR_INVALID, "%s: n=%lld sub=%lld unsupported", who, (long long)n, (long long)sub);
  if (nsb < 1 || nsb * sub < cdiv(n, kBlk))
    return fail(FATHOM_ERR_INVALID, "%s: store holds %lld blocks (nsb=%lld x sub=%lld), n needs %lld", who,
                (long long)(nsb * sub), (long long)nsb, (long long)sub, (long long)cdiv(n, kBlk));
  if ((reinterpret_cast<uintptr_t>(planes_sb) & 3) != 0 || (reinterpret_cast<uintptr_t>(scales_sb) & 1) != 0)
    return fail(FATHOM_ERR_INVALID, "%s: planes must be 4-byte and scales 2-byte aligned", who);
  // a wave-tile's loads are 32-bit offsets from its first superblock
  if (D * 4 * sub * 8 * (kWB / sub + 2) > 0x7FFFFFFFLL)
    return fail(FATHOM_ERR_INVALID, "%s: superblocks of sub=%lld blocks exceed the 2 GiB addressing of a scan tile", who,
                (long long)sub);
  return FATHOM_OK;
}

ScanArgs make_args(const float *q, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax,
                   const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub) {
  ScanArgs a{};
  a.q = q;
  a.cls = cls;
  a.clsn = clsn;
  a.planes = static_cast<const uint32_t *>(planes_sb);
  a.scales = static_cast<const uint16_t *>(scales_sb);
  a.n = n;
  a.nsb = nsb;
  a.sub = sub;
  a.D = (int)D;
  a.G = (int)G;
  a.bmax = bmax;
  a.ncls = bmax < 4 ? bmax : 4;
  a.wt_stride = 1;
  return a;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_planes(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                  const int32_t *clsn, int bmax, int64_t units_max, const void *planes_sb,
                                  const void *scales_sb,
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
  ScanArgs a = make_args(q, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = blk0;
  a.blk_end = blk_end;
  a.wt0 = blk0 / kWB;
  Emit em{};
  em.out = out;
  return launch_scan<kEmitScores>(a, cdiv(blk_end, kWB) - a.wt0, BH, em, units_bound(units_max, D, bmax),
                                  (hipStream_t)stream);
}

namespace fathom {
// Workspace of the fused scan + top-k: rows up to kRowSelectMax keep their
// scores ([rows, n] fp32) for one row-select launch; longer rows the sampled
// keys, the candidate regions and the plan tables (one per row: at least one
// per (batch, KV head)).  kk above kSelMaxK: the scores and the wide path's
// selection state.
size_t scan_topk_ws(int64_t rows, int64_t n, int64_t k, int64_t kk) {
  if (kk > kSelMaxK) return ws_align((size_t)rows * (size_t)n * 4) + wide_topk_bytes(rows, n, k);
  if (n <= kRowSelectMax) return ws_align((size_t)rows * (size_t)n * 4) + ws_align((size_t)rows * cdiv(n, kGroupTok) * 4);
  return topk_layout(rows, n, k, true, nullptr, nullptr, nullptr, nullptr, nullptr) +
         ws_align((size_t)rows * sizeof(sc::PlanTab));
}
}  // namespace fathom

extern "C" size_t fathom_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t n, int64_t k, int64_t sink,
                                                   int64_t local) {
  const int64_t kk = k - sink - local;
  if (BH < 1 || G < 1 || n < 1 || kk < 0) return 0;
  return scan_topk_ws(BH * G, n, k, kk);
}

namespace fathom {
int scan_topk_run(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax,
                  int64_t units_max, const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t m,
                  int64_t k, int64_t sink, int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes,
                  int stages, void *stream) {
  int rc = check_scan(q, BH, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub, "scan_topk");
  if (rc) return rc;
  if (!idx) return fail(FATHOM_ERR_INVALID, "scan_topk: null output");
  if (stages & ~FATHOM_STAGE_ALL) return fail(FATHOM_ERR_INVALID, "scan_topk: unknown stage bits 0x%x", stages);
  const int64_t rows = BH * G;
  rc = check_topk_args(rows, n, m, k, sink, local, "scan_topk");
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int64_t kk = k - sink - local;
  if (kk == 0) return (stages & FATHOM_STAGE_FINALIZE) ? launch_fixed_only(rows, m, k, sink, local, idx, st) : FATHOM_OK;
  const size_t need = scan_topk_ws(rows, n, k, kk);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "scan_topk: workspace %zu bytes, need %zu", workspace_bytes, need);
  const int64_t nblk = cdiv(n, kBlk);
  ScanArgs a = make_args(q, G, D, cls, clsn, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = 0;
  a.blk_end = nblk;
  a.wt0 = 0;
  const int64_t nwt = cdiv(nblk, kWB);
  const int64_t um = units_bound(units_max, D, bmax);
  if (kk > kSelMaxK) {
    // kk beyond the LDS-resident selections: the scores in the workspace (the
    // candidate stage), then the score-row chain and the wide selection over
    // its candidate lists (the finalize stage)
    Emit es{};
    es.out = static_cast<float *>(workspace);
    const size_t sb = ws_align((size_t)rows * (size_t)n * 4);
    if (stages & FATHOM_STAGE_CANDIDATES) {
      rc = launch_scan<kEmitScores>(a, nwt, BH, es, um, st);
      if (rc) return rc;
    }
    return (stages & FATHOM_STAGE_FINALIZE)
               ? wide_topk_run(es.out, rows, n, m, k, sink, local, idx, static_cast<char *>(workspace) + sb,
                               workspace_bytes - sb, st)
               : FATHOM_OK;
  }
  if (n <= kRowSelectMax) {
    // short rows: the scores and their 16-token group maxima in the workspace
    // (the candidate stage), then the rows selected in one launch from the
    // groups that can hold a top-kk key (the finalize stage)
    Emit es{};
    es.out = static_cast<float *>(workspace);
    es.gmax = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + ws_align((size_t)rows * (size_t)n * 4));
    es.sink = sink;
    es.lstart = (m - local) > 0 ? (m - local) : 0;
    if (stages & FATHOM_STAGE_CANDIDATES) {
      rc = launch_scan<kEmitScoresMax>(a, nwt, BH, es, um, st);
      if (rc) return rc;
    }
    return (stages & FATHOM_STAGE_FINALIZE) ? launch_rowselect_gmax(es.out, es.gmax, rows, n, m, k, sink, local, idx, st)
                                            : FATHOM_OK;
  }
  Emit em{};
  int64_t S = 1;
  const size_t tab_at = topk_layout(rows, n, k, true, static_cast<char *>(workspace), &em.samp, &em.samp_cap, &em.sel, &S);
  em.tab = reinterpret_cast<sc::PlanTab *>(static_cast<char *>(workspace) + tab_at);
  em.sel.kk = (uint32_t)kk;
  const int64_t r_hi = topk_hi_rank(n, S, kk, kRegTok);
  em.sink = sink;
  em.lstart = (m - local) > 0 ? (m - local) : 0;
  if (stages & FATHOM_STAGE_SAMPLE) {
    a.wt_stride = S;
    rc = launch_scan<kEmitSample>(a, topk_sample_tiles(n, S, kRegTok), BH, em, um, st);
    if (rc) return rc;
  }
  if (stages & FATHOM_STAGE_SELECT) {
    rc = launch_select_groups(em.samp, rows, em.samp_cap, kk, r_hi, em.sel, st);
    if (rc) return rc;
  }
  if (stages & FATHOM_STAGE_CANDIDATES) {
    a.wt_stride = 1;
    rc = launch_scan<kEmitFilter>(a, nwt, BH, em, um, st);
    if (rc) return rc;
  }
  // T_hi may exceed a row's kk-th largest key (r_hi < kk): the finalize
  // workgroup of a row with fewer than kk candidates rescans it with T_lo
  a.wt_stride = 1;
  a.nwt = nwt;
  return (stages & FATHOM_STAGE_FINALIZE) ? launch_finalize_fused(a, em, rows, m, k, sink, local, idx, st)
                                          : FATHOM_OK;
}
}  // namespace fathom

extern "C" int fathom_scan_topk(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                const int32_t *clsn, int bmax, int64_t units_max, const void *planes_sb, const void *scales_sb,
                                int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink,
                                int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes, void *stream) {
  return scan_topk_run(q, BH, G, D, cls, clsn, bmax, units_max, planes_sb, scales_sb, n, nsb, sub, m, k, sink, local, idx,
                       workspace, workspace_bytes, FATHOM_STAGE_ALL, stream);
}

extern "C" int fathom_scan_topk_stages(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                       const int32_t *clsn, int bmax, int64_t units_max, const void *planes_sb, const void *scales_sb,
                                       int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink,
                                       int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes,
                                       int stages, void *stream) {
  return scan_topk_run(q, BH, G, D, cls, clsn, bmax, units_max, planes_sb, scales_sb, n, nsb, sub, m, k, sink, local, idx,
                       workspace, workspace_bytes, stages, stream);
}

namespace fathom {
namespace {
// make_plan's arrays for plan_scan_topk's long rows, past the scan's workspace.
size_t plan_arrays_ws(int64_t BH, int64_t D, int bmax) {
  return ws_align((size_t)(BH * D)) + ws_align((size_t)(BH * D * bmax) * 4) + 2 * ws_align((size_t)BH * 4) +
         ws_align((size_t)(BH * D) * 4) + ws_align((size_t)(BH * bmax * D) * 4) + ws_align((size_t)(BH * bmax) * 4);
}
}  // namespace
}  // namespace fathom

extern "C" size_t fathom_plan_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t D, int bmax, int64_t n, int64_t k,
                                                        int64_t sink, int64_t local) {
  const int64_t kk = k - sink - local;
  if (BH < 1 || G < 1 || D < 1 || bmax < 1 || n < 1 || kk < 0) return 0;
  return scan_topk_ws(BH * G, n, k, kk) + plan_arrays_ws(BH, D, bmax);
}

namespace fathom {
namespace {
// The attention of fathom_plan_scan_topk_attention (null: none).
struct AttnOut {
  const void *K, *V;
  int64_t cap;
  float scale;
  float *out;
};

int plan_scan_topk_run(const float *q, const float *g, const float *budget, float budget_value, int64_t BH, int64_t G,
                       int64_t D, int bmax, int iters, int64_t units_max, const void *planes_sb, const void *scales_sb,
                       int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink, int64_t local,
                       int64_t *idx, int8_t *t_out, void *workspace, size_t workspace_bytes, const AttnOut *att,
                       void *stream) {
  if (!g) return fail(FATHOM_ERR_INVALID, "plan_scan_topk: null pointer");
  if (iters < 0 || iters > 200) return fail(FATHOM_ERR_INVALID, "plan_scan_topk: iters=%d outside [0, 200]", iters);
  int rc = check_scan(q, BH, G, D, nullptr, nullptr, bmax, planes_sb, scales_sb, n, nsb, sub, "plan_scan_topk", true);
  if (rc) return rc;
  if (!idx) return fail(FATHOM_ERR_INVALID, "plan_scan_topk: null output");
  const int64_t rows = BH * G;
  rc = check_topk_args(rows, n, m, k, sink, local, "plan_scan_topk");
  if (rc) return rc;
  const size_t need = fathom_plan_scan_topk_workspace_bytes(BH, G, D, bmax, n, k, sink, local);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "plan_scan_topk: workspace %zu bytes, need %zu", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int64_t kk = k - sink - local;
  const size_t sws = scan_topk_ws(rows, n, k, kk);
  if (n > kRowSelectMax || kk == 0 || kk > kSelMaxK) {
    // make_plan into the workspace, then the fused scan + top-k
    char *p = static_cast<char *>(workspace) + sws;
    int8_t *t = t_out ? t_out : reinterpret_cast<int8_t *>(p);
    p += ws_align((size_t)(BH * D));
    int32_t *pairs = reinterpret_cast<int32_t *>(p);
    p += ws_align((size_t)(BH * D * bmax) * 4);
    int32_t *npairs = reinterpret_cast<int32_t *>(p);
    p += ws_align((size_t)BH * 4);
    int32_t *nact = reinterpret_cast<int32_t *>(p);
    p += ws_align((size_t)BH * 4);
    int32_t *act = reinterpret_cast<int32_t *>(p);
    p += ws_align((size_t)(BH * D) * 4);
    int32_t *cls = reinterpret_cast<int32_t *>(p);
    p += ws_align((size_t)(BH * bmax * D) * 4);
    int32_t *clsn = reinterpret_cast<int32_t *>(p);
    rc = make_plan_run(g, budget, budget_value, BH, D, bmax, iters, t, pairs, npairs, act, nact, cls, clsn, stream);
    if (rc) return rc;
    return scan_topk_run(q, BH, G, D, cls, clsn, bmax, units_max, planes_sb, scales_sb, n, nsb, sub, m, k, sink, local,
                         idx, workspace, sws, FATHOM_STAGE_ALL, stream);
  }
  // short rows: every workgroup of the scan plans its row in the prologue
  // (the plan kernel's arithmetic), then the rows are selected as in scan_topk
  const int64_t nblk = cdiv(n, kBlk);
  ScanArgs a = make_args(q, G, D, nullptr, nullptr, bmax, planes_sb, scales_sb, n, nsb, sub);
  a.blk0 = 0;
  a.blk_end = nblk;
  a.wt0 = 0;
  a.g = g;
  a.budget = budget;
  a.budget_value = budget_value;
  a.iters = iters;
  a.t_out = t_out;
  Emit es{};
  es.out = static_cast<float *>(workspace);
  es.gmax = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + ws_align((size_t)rows * (size_t)n * 4));
  es.sink = sink;
  es.lstart = (m - local) > 0 ? (m - local) : 0;
  rc = launch_scan<kEmitScoresMax>(a, cdiv(nblk, kWB), BH, es, units_bound(units_max, D, bmax), st);
  if (rc) return rc;
  if (att)  // the selection's workgroups go on to their head's attention
    return launch_rowselect_gmax_attn(es.out, es.gmax, rows, n, m, k, sink, local, idx, q, G, att->K, att->V, att->cap,
                                      att->scale, att->out, st);
  return launch_rowselect_gmax(es.out, es.gmax, rows, n, m, k, sink, local, idx, st);
}
}  // namespace
}  // namespace fathom

extern "C" int fathom_plan_scan_topk(const float *q, const float *g, const float *budget, float budget_value, int64_t BH,
                                     int64_t G, int64_t D, int bmax, int iters, int64_t units_max, const void *planes_sb,
                                     const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k,
                                     int64_t sink, int64_t local, int64_t *idx, int8_t *t_out, void *workspace,
                                     size_t workspace_bytes, void *stream) {
  return plan_scan_topk_run(q, g, budget, budget_value, BH, G, D, bmax, iters, units_max, planes_sb, scales_sb, n, nsb,
                            sub, m, k, sink, local, idx, t_out, workspace, workspace_bytes, nullptr, stream);
}

extern "C" size_t fathom_plan_scan_topk_attention_workspace_bytes(int64_t BH, int64_t G, int64_t D, int bmax, int64_t n,
                                                                  int64_t k, int64_t sink, int64_t local) {
  const size_t base = fathom_plan_scan_topk_workspace_bytes(BH, G, D, bmax, n, k, sink, local);
  return base ? base + ws_align(fathom_gather_attention_workspace_bytes(BH, G, k)) : 0;
}

extern "C" int fathom_plan_scan_topk_attention(const float *q, const float *g, const float *budget, float budget_value,
                                               int64_t BH, int64_t G, int64_t D, int bmax, int iters, int64_t units_max,
                                               const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb,
                                               int64_t sub, int64_t m, int64_t k, int64_t sink, int64_t local,
                                               int64_t *idx, int8_t *t_out, const void *Ksrc, const void *Vsrc,
                                               int64_t cap, float scale, float *out, void *workspace,
                                               size_t workspace_bytes, void *stream) {
  if (!Ksrc || !Vsrc || !out) return fail(FATHOM_ERR_INVALID, "plan_scan_topk_attention: null pointer");
  if (D != 128) return fail(FATHOM_ERR_INVALID, "plan_scan_topk_attention: D=%lld, attention needs 128", (long long)D);
  if (cap < 0) return fail(FATHOM_ERR_INVALID, "plan_scan_topk_attention: cap=%lld", (long long)cap);
  const size_t need = fathom_plan_scan_topk_attention_workspace_bytes(BH, G, D, bmax, n, k, sink, local);
  if (!workspace || workspace_bytes < need)
    return fail(FATHOM_ERR_WORKSPACE, "plan_scan_topk_attention: workspace %zu bytes, need %zu", workspace_bytes, need);
  const size_t pws = fathom_plan_scan_topk_workspace_bytes(BH, G, D, bmax, n, k, sink, local);
  const int64_t kk = k - sink - local;
  // fused where gather_attention would take one 16-wave split per head, so
  // the outputs are the two calls' bit for bit
  const bool fused = n <= kRowSelectMax && kk > 0 && k <= 512 && attn::attn_wide(BH, G, k) &&
                     ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(Ksrc) |
                       reinterpret_cast<uintptr_t>(Vsrc)) & 7) == 0;
  if (fused) {
    const AttnOut att{Ksrc, Vsrc, cap, scale, out};
    return plan_scan_topk_run(q, g, budget, budget_value, BH, G, D, bmax, iters, units_max, planes_sb, scales_sb, n, nsb,
                              sub, m, k, sink, local, idx, t_out, workspace, pws, &att, stream);
  }
  // the two calls: the selection, then gather_attention over its indices
  int rc = plan_scan_topk_run(q, g, budget, budget_value, BH, G, D, bmax, iters, units_max, planes_sb, scales_sb, n, nsb,
                              sub, m, k, sink, local, idx, t_out, workspace, pws, nullptr, stream);
  if (rc) return rc;
  return fathom_gather_attention(q, idx, BH, G, k, n, Ksrc, Vsrc, cap, nullptr, nullptr, 0, scale, out, nullptr,
                                 static_cast<char *>(workspace) + pws, need - pws, stream);
}
