/*
 * fathom_hip.h -- C ABI of the MI355X (gfx950) bit-plane key-scan library.
 *
 * The reference exposes this path as the Python module kernels/bitplane.py
 * (imported as `from bitplane import *`, scripts/B_e2e_offload_v2.py:12-17,
 * scripts/B_kernel_bench.py:8-12) plus the gather kernels and ctypes host
 * mapping of scripts/B_e2e_offload_v2.py.  Each entry point below replaces one
 * of those; the replaced reference interface is cited above it.
 *
 * Conventions (all entry points):
 *   - every pointer is device-visible: HBM, or pinned host memory mapped into
 *     the GPU address space (fathom_host_alloc_mapped); the caller owns every
 *     buffer, including workspaces;
 *   - tensors are dense, row-major (C order), with the shapes documented;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t, NULL = the
 *     default stream); no entry point synchronises the host;
 *   - the return value is a status: FATHOM_OK (0) or an error code; the text
 *     of the last error on the calling thread is fathom_last_error();
 *   - no state is kept between calls: entry points are thread-safe as long as
 *     concurrent calls do not share output or workspace buffers.
 */
#ifndef FATHOM_HIP_H
#define FATHOM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define FATHOM_OK 0
#define FATHOM_ERR_INVALID 1   /* shape or argument rejected before any launch */
#define FATHOM_ERR_HIP 2       /* HIP runtime error (launch, copy, query) */
#define FATHOM_ERR_ALLOC 3     /* host allocation failed */
#define FATHOM_ERR_WORKSPACE 4 /* workspace missing or too small */

/* element types of key and scale tensors */
#define FATHOM_DT_F32 0
#define FATHOM_DT_F16 1
#define FATHOM_DT_BF16 2

/* Library version string and last error text (per calling thread). */
const char *fathom_version(void);
const char *fathom_last_error(void);

/*
 * Quantise keys to 4-bit codes and pack them as bit planes, in one pass.
 * Replaces quantise_u4 + pack_planes + to_superblocks as PlaneStore.__init__
 * chains them (kernels/bitplane.py:23-32, 44-50, 60-65, 312-316).
 *   K           [lead, n, D] of k_dtype (FATHOM_DT_*)
 *   scale_dtype FATHOM_DT_* the block absmax is rounded to (reference default f16)
 *   outputs (each may be NULL to skip it):
 *   code        [lead, n, D] uint8 in [0, 16)
 *   scales_blk  [lead, nblk, D] of scale_dtype (nblk = ceil(n / 64))
 *   planes_log  [lead, nblk, D, 4] uint64 (bit i = token 64b+i, plane 0 = MSB)
 *   planes_sb   [lead, nsb, D, 4, sub] uint64, nsb = ceil(nblk / sub), zero padded
 *   scales_sb   [lead, nsb, D, sub] fp16 bits; required iff planes_sb != NULL
 */
int fathom_quantise_pack(const void *K, int k_dtype, int64_t lead, int64_t n, int64_t D, int scale_dtype,
                         int64_t sub, uint8_t *code, void *scales_blk, uint64_t *planes_log, uint64_t *planes_sb,
                         uint16_t *scales_sb, void *stream);

/* pack_planes (kernels/bitplane.py:44-50): code [lead, n, D] uint8 -> planes [lead, nblk, D, 4]. */
int fathom_pack_planes(const uint8_t *code, int64_t lead, int64_t n, int64_t D, uint64_t *planes, void *stream);

/* unpack_planes (kernels/bitplane.py:52-58): planes [lead, nblk, D, 4] -> code [lead, n, D] uint8. */
int fathom_unpack_planes(const uint64_t *planes, int64_t lead, int64_t nblk, int64_t D, int64_t n, uint8_t *code,
                         void *stream);

/*
 * to_superblocks (kernels/bitplane.py:60-65): logical planes [lead, nblk, D, 4] and
 * scales [lead, nblk, D] (elements of scale_bytes = 2 or 4 bytes) -> planes_sb
 * [lead, nsb, D, 4, sub] and scales_sb [lead, nsb, D, sub], zero padded.
 */
int fathom_to_superblocks(const uint64_t *planes, const void *scales, int scale_bytes, int64_t lead, int64_t nblk,
                          int64_t D, int64_t sub, uint64_t *planes_sb, void *scales_sb, void *stream);

/*
 * dequant_planes (kernels/bitplane.py:34-42): value of the top t[j] planes,
 * out [lead, n, D] float32 from code [lead, n, D], scales [lead, nblk, D] of
 * scale_dtype and t [D] int32 (device).
 */
int fathom_dequant_planes(const uint8_t *code, const void *scales, int scale_dtype, const int32_t *t, int64_t lead,
                          int64_t n, int64_t D, float *out, void *stream);

/*
 * make_plan (kernels/bitplane.py:83-116, plan_kernel + make_plan): per
 * (batch, KV head) reverse water-filling.  g [BH, D] float32 gains, budget [BH]
 * float32 (code bits).  Outputs, all fully written (zero padded):
 *   t [BH, D] int8; pairs [BH, D*bmax] int32 (channel*bmax + plane);
 *   npairs [BH]; act [BH, D]; nact [BH]; cls [BH, bmax, D]; clsn [BH, bmax].
 * 1 <= bmax <= 8, D <= 256.
 */
int fathom_make_plan(const float *g, const float *budget, int64_t BH, int64_t D, int bmax, int iters, int8_t *t,
                     int32_t *pairs, int32_t *npairs, int32_t *act, int32_t *nact, int32_t *cls, int32_t *clsn,
                     void *stream);

/*
 * make_plan with one budget for every row (kernels/bitplane.py:83-116 called
 * with a float budget, as scripts/B_kernel_bench.py:74 does): the value is a
 * kernel argument, so no device copy of it is made per call.  Outputs and
 * limits as fathom_make_plan.
 */
int fathom_make_plan_uniform(const float *g, float budget, int64_t BH, int64_t D, int bmax, int iters, int8_t *t,
                             int32_t *pairs, int32_t *npairs, int32_t *act, int32_t *nact, int32_t *cls,
                             int32_t *clsn, void *stream);

/*
 * PlaneStore.scan (kernels/bitplane.py:319-338, scan_planes_cls_kernel :275-307):
 * out[bh, g, tok] = sum_j q[bh, g, j] * value_{t_j}(tok, j) over the channels of
 * the plan's depth classes 1..min(bmax, 4), for the 64-token blocks [blk0, blk1)
 * (tokens < n); other tokens of `out` are not written.
 *   q         [BH, G, D] float32, 1 <= G <= 8, D <= 128 (the reference's D = 128,
 *             kernels/bitplane.py:313)
 *   cls, clsn from fathom_make_plan ([BH, bmax, D] and [BH, bmax] int32)
 *   units_max an upper bound on the plan's (channel, plane) units of every row,
 *             sum_j t_j (make_plan keeps it within the bit budget), or 0 when
 *             none is known.  It only picks the kernel's register layout
 *             (plans above 64 units keep more accumulators live); results are
 *             the same for any value, a wrong bound included.
 *   planes_sb [BH, nsb, D, 4, sub] uint64, scales_sb [BH, nsb, D, sub] fp16
 *             (HBM, or mapped pinned host memory: the scan then reads over PCIe)
 *   out       [BH, G, n] float32
 */
int fathom_scan_planes(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn,
                       int bmax, int64_t units_max, const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub,
                       int64_t blk0, int64_t blk1, float *out, void *stream);

/*
 * The chan4 baseline store: channel-major 4-bit codes, word m of (channel j,
 * block b) holding tokens 8m..8m+7 of the block, nibble k = token 8m + k.
 *   pack_chan4 (kernels/bitplane.py:67-74): code [lead, n, D] uint8 ->
 *     chan_sb [lead, nsb, D, sub, 8] uint32 (16-byte aligned), zero padded,
 *     nsb = ceil(ceil(n / 64) / sub).
 *   quantise_chan4 (Chan4Store.__init__, kernels/bitplane.py:342-347): keys ->
 *     codes and block scales (optional outputs, as fathom_quantise_pack),
 *     chan_sb and the fp16 superblock scales scales_sb [lead, nsb, D, sub].
 *   channel_list (kernels/bitplane.py:128-132): active [BH, D] (bytes, 0 or 1)
 *     -> act [BH, D] int32 (listed channels first, then the others, both
 *     ascending) and nact [BH] int32.
 *   scan_chan4 (Chan4Store.scan, kernels/bitplane.py:348-353, kernel :175-198):
 *     scores [BH, G, n] over the first nact[bh] channels of act at full depth,
 *     blocks [blk0, blk1) only.
 */
int fathom_pack_chan4(const uint8_t *code, int64_t lead, int64_t n, int64_t D, int64_t sub, uint32_t *chan_sb,
                      void *stream);
int fathom_quantise_chan4(const void *K, int k_dtype, int64_t lead, int64_t n, int64_t D, int scale_dtype,
                          int64_t sub, uint8_t *code, void *scales_blk, uint32_t *chan_sb, uint16_t *scales_sb,
                          void *stream);
int fathom_channel_list(const uint8_t *active, int64_t BH, int64_t D, int32_t *act, int32_t *nact, void *stream);
int fathom_scan_chan4(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *act, const int32_t *nact,
                      const void *chan_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t blk0,
                      int64_t blk1, float *out, void *stream);

/*
 * Query side of the KLT-rotated store (scripts/R_ruler.py:82-84, planesK):
 * qr[bh, g] = q[bh, g] @ Vt[bh] and gain[bh, e] = sum_g qr[bh, g, e]^2 * lam[bh, e]
 * (the make_plan gains of the rotated coordinates).  q [BH, G, D], Vt [BH, D, D]
 * row-major (column e = basis vector e), lam [BH, D], qr [BH, G, D], gain [BH, D],
 * all float32; G <= 32, D <= 256.
 */
int fathom_klt_query(const float *q, const float *Vt, const float *lam, int64_t BH, int64_t G, int64_t D, float *qr,
                     float *gain, void *stream);

/*
 * Fused scan + sink/local top-k: the selection of fathom_scan_planes followed by
 * fathom_sink_local_topk on its scores (kernels/bitplane.py:319-338 then
 * :372-378, as chained by scripts/B_kernel_bench.py:74 and
 * scripts/B_e2e_offload_v2.py:203, 224-227), without materialising the score
 * tensor for rows longer than 32768 (shorter rows keep their scores in the
 * workspace for one selection launch).  Same arguments as fathom_scan_planes
 * over the whole sequence, plus the top-k arguments of fathom_sink_local_topk;
 * idx [BH * G, k] int64 is identical to running the two entry points.
 * workspace: fathom_scan_topk_workspace_bytes(BH, G, n, k, sink, local) bytes.
 */
size_t fathom_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t n, int64_t k, int64_t sink, int64_t local);
int fathom_scan_topk(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn,
                     int bmax, int64_t units_max, const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub,
                     int64_t m, int64_t k, int64_t sink, int64_t local, int64_t *idx, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * The stages of fathom_scan_topk, run separately on one workspace: `stages` is
 * a bitmask of FATHOM_STAGE_*; fathom_scan_topk runs FATHOM_STAGE_ALL, in the
 * order sample, select, candidates, finalize.  A stage reads what the earlier
 * stages left in the workspace, so a partial call repeats a later stage over
 * the state of the last full one (same arguments).  Rows of at most 32768
 * tokens have two stages only: candidates (the scores into the workspace) and
 * finalize (the selection over them).  It exists for stage timing (bench.py
 * times the candidate pass, the dominant kernel, on its own) and has no
 * counterpart in the reference.
 */
#define FATHOM_STAGE_SAMPLE 1
#define FATHOM_STAGE_SELECT 2
#define FATHOM_STAGE_CANDIDATES 4
#define FATHOM_STAGE_FINALIZE 8
#define FATHOM_STAGE_ALL 15
int fathom_scan_topk_stages(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                            const int32_t *clsn, int bmax, int64_t units_max, const void *planes_sb, const void *scales_sb, int64_t n,
                            int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink, int64_t local,
                            int64_t *idx, void *workspace, size_t workspace_bytes, int stages, void *stream);

/*
 * make_plan followed by the fused scan + top-k in one call: idx is identical
 * to fathom_make_plan (budget [BH], or budget_value for every row when budget
 * is null; bmax, iters as there) then fathom_scan_topk with that plan's cls and
 * clsn (kernels/bitplane.py:83-116 then :319-338 and :372-378, the plan ->
 * scan -> top-k stages of scripts/B_kernel_bench.py:74).  For rows of at most
 * 32768 tokens (D <= 128) every workgroup of the scan makes its row's plan in
 * its prologue with the plan kernel's arithmetic, so no plan launch and no
 * plan arrays precede the scan: the decode form of the chain.  Longer rows run
 * the plan kernel into the workspace first.  t_out [BH, D] int8 (nullable)
 * receives the plan's depths.  It composes reference stages and has no single
 * counterpart in the reference.
 * workspace: fathom_plan_scan_topk_workspace_bytes(BH, G, D, bmax, n, k, sink,
 * local) bytes.
 */
size_t fathom_plan_scan_topk_workspace_bytes(int64_t BH, int64_t G, int64_t D, int bmax, int64_t n, int64_t k,
                                             int64_t sink, int64_t local);
int fathom_plan_scan_topk(const float *q, const float *g, const float *budget, float budget_value, int64_t BH, int64_t G,
                          int64_t D, int bmax, int iters, int64_t units_max, const void *planes_sb, const void *scales_sb,
                          int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink, int64_t local,
                          int64_t *idx, int8_t *t_out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * fathom_plan_scan_topk followed by fathom_gather_attention over its indices
 * (rows in device memory: Ksrc, Vsrc bf16 [BH, cap, 128], no recent rows),
 * the decode step's plan -> scan -> top-k -> gather + attention chain of
 * scripts/B_kernel_bench.py:64-101 in one call.  For rows of at most 32768
 * tokens and k <= 512 each selection workgroup goes on to its query head's
 * attention over the indices it wrote (the arithmetic of gather_attention), so
 * idx and out equal the two calls'.  Other shapes run the two calls.  It
 * composes reference stages and has no single counterpart in the reference.
 * workspace: fathom_plan_scan_topk_attention_workspace_bytes(BH, G, D, bmax,
 * n, k, sink, local) bytes.
 */
size_t fathom_plan_scan_topk_attention_workspace_bytes(int64_t BH, int64_t G, int64_t D, int bmax, int64_t n, int64_t k,
                                                       int64_t sink, int64_t local);
int fathom_plan_scan_topk_attention(const float *q, const float *g, const float *budget, float budget_value, int64_t BH,
                                    int64_t G, int64_t D, int bmax, int iters, int64_t units_max, const void *planes_sb,
                                    const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t m, int64_t k,
                                    int64_t sink, int64_t local, int64_t *idx, int8_t *t_out, const void *Ksrc,
                                    const void *Vsrc, int64_t cap, float scale, float *out, void *workspace,
                                    size_t workspace_bytes, void *stream);

/*
 * fathom_scan_topk without a workspace argument, for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The workspace is a static device array of the library, of
 * FATHOM_NOALLOC_SCRATCH_BYTES, one per device that calls it (held until the
 * process ends); shapes whose fathom_scan_topk_workspace_bytes exceed it are
 * rejected with FATHOM_ERR_WORKSPACE before any launch.  The call allocates
 * nothing (no hipMalloc, no library allocation).  Calls that overlap on one
 * device (several streams or threads) share the array and race.  Results are
 * those of fathom_scan_topk on the same arguments.  The array's device address
 * is looked up on a device's first call and kept: make one call on a device
 * before capturing the call in a graph, and do not call it again on a device
 * after hipDeviceReset (the kept address no longer names the array).
 */
#define FATHOM_NOALLOC_SCRATCH_BYTES (64ull << 20)
int fathom_scan_topk_noalloc(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                             const int32_t *clsn, int bmax, int64_t units_max, const void *planes_sb, const void *scales_sb, int64_t n,
                             int64_t nsb, int64_t sub, int64_t m, int64_t k, int64_t sink, int64_t local,
                             int64_t *idx, void *stream);

/*
 * sink_local_topk (kernels/bitplane.py:372-378; inline form with the current
 * length m at scripts/B_e2e_offload_v2.py:224-227).  For each of `rows` rows of
 * scores [rows, n] float32: mask [0, sink) and [max(m - local, 0), n) to -inf,
 * select the top kk = k - sink - local by (score descending, index ascending;
 * NaN above +inf, -0.0 == +0.0), then append 0..sink-1 and m-local..m-1.
 *   idx [rows, k] int64.  Requires 0 <= kk <= n, sink <= n, local <= m, n <= m
 * (any kk, as torch.topk: kk above 2048 takes an exact 64-bit radix select over
 * the rows' candidate lists, then a counting sort of up to 8192 values or a
 * bitonic sort).
 * workspace: fathom_topk_workspace_bytes(rows, n, k) bytes of device memory,
 * contents arbitrary on entry.
 */
size_t fathom_topk_workspace_bytes(int64_t rows, int64_t n, int64_t k);
int fathom_sink_local_topk(const float *scores, int64_t rows, int64_t n, int64_t m, int64_t k, int64_t sink,
                           int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes, void *stream);

/*
 * gather_rows (scripts/B_e2e_offload_v2.py:73-83, gather_rows_kernel):
 * dst[bh, r, :] = src[bh, idx[bh, r], :] for idx >= 0, zero row for idx < 0.
 *   src [BH, cap, row_bytes] (HBM or mapped host), idx [BH, R] int32,
 *   dst [BH, R, row_bytes]; row_bytes % 4 == 0.
 */
int fathom_gather_rows(const void *src, int64_t cap, const int32_t *idx, int64_t BH, int64_t R, int64_t row_bytes,
                       void *dst, void *stream);

/*
 * Group-union row gather (scripts/B_e2e_offload_v2.py:228-241): for idx
 * [BH, GK] int64 (GK = G*k, any size: up to 16384 the dedup runs in one
 * workgroup's LDS, above in a hash table in the workspace), fetch every distinct token < n of a row
 * once from Ksrc/Vsrc [BH, cap, row_bytes] (usually mapped host memory), tokens
 * >= n from the device buffers Krec/Vrec [BH, nrec, row_bytes] at row
 * clamp(idx - n, 0, nrec - 1), negative tokens as zero rows, and write
 * Kout/Vout [BH, GK, row_bytes] in the order of idx.  n_unique [BH] int32
 * (may be NULL) receives the number of distinct host rows fetched.
 * workspace: fathom_gather_union_workspace_bytes(BH, GK) bytes.
 */
size_t fathom_gather_union_workspace_bytes(int64_t BH, int64_t GK);
int fathom_gather_union(const int64_t *idx, int64_t BH, int64_t GK, int64_t n, const void *Ksrc, const void *Vsrc,
                        int64_t cap, const void *Krec, const void *Vrec, int64_t nrec, int64_t row_bytes, void *Kout,
                        void *Vout, int32_t *n_unique, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Exact attention over the selected rows (scripts/B_kernel_bench.py:22-27
 * gather_attn; scripts/B_e2e_offload_v2.py:228-244, the gather + attention of
 * offload_attn): for every query head g of row bh,
 *   out[bh, g] = softmax_j(scale * q[bh, g] . K[t_j]) . V[t_j]   over the k
 * positions j of idx[bh, g] (fp32 math on bf16 rows; a token selected twice
 * counts twice).  Rows come from the same sources as fathom_gather_union
 * (Ksrc/Vsrc [BH, cap, 128] bf16 for tokens < n, Krec/Vrec [BH, nrec, 128]
 * for tokens >= n, zero rows for negative tokens).  With n_unique set, the
 * row's union is formed first and each distinct token is read once (the
 * host-resident case: every row crosses PCIe once), and n_unique is as in
 * fathom_gather_union; with n_unique NULL the rows are read per selected
 * position, with no union pass (rows in device memory: one launch fewer).
 * Both give the same attention up to fp32 summation order.  q [BH, G, 128]
 * fp32, idx [BH, G, k] int64, out [BH, G, 128] fp32.  With G > 8 or G*k >
 * 16384 the rows are read per selected position also when n_unique is set,
 * and n_unique comes from a hash table in the workspace.
 * workspace: fathom_gather_attention_workspace_bytes(BH, G, k) bytes.
 */
size_t fathom_gather_attention_workspace_bytes(int64_t BH, int64_t G, int64_t k);
int fathom_gather_attention(const float *q, const int64_t *idx, int64_t BH, int64_t G, int64_t k, int64_t n,
                            const void *Ksrc, const void *Vsrc, int64_t cap, const void *Krec, const void *Vrec,
                            int64_t nrec, float scale, float *out, int32_t *n_unique, void *workspace,
                            size_t workspace_bytes, void *stream);

/*
 * One chunk of the chunked copy/scan pipeline (scripts/B_e2e_offload_v2.py:
 * 105-133, stream_planes / stream_chan4 with chunk_bounds): copies blocks
 * [b0, b1) of every plan-selected run of a whole-sequence store (sub = nblk,
 * nsb = 1) from data_src/scales_src to the same places of data_dst/scales_dst.
 *   planes = 4: bit-plane store, data [BH, 1, D, 4, nblk] uint64
 *               (block_bytes = 8), plane p of channel j copied when p < min(t, 4);
 *   planes = 1: chan4 store, data [BH, 1, D, nblk, 8] uint32 (block_bytes = 32),
 *               channel j copied when t > 0 (t = the active mask as int8);
 *   scales [BH, 1, D, nblk] fp16, copied for channels with t > 0.
 * t [BH, D] int8 (device).  BH * D * planes <= 65535.
 */
int fathom_copy_index_range(const int8_t *t, int64_t BH, int64_t D, int64_t nblk, int64_t b0, int64_t b1,
                            int64_t block_bytes, int planes, const void *data_src, const void *scales_src,
                            void *data_dst, void *scales_dst, void *stream);

/*
 * gather_runs (scripts/B_e2e_offload_v2.py:62-71, gather_runs_kernel): copy run r,
 * the 4-byte words [off[r], off[r] + len[r]) of src, to the same words of dst,
 * for r < *nrun (off, len [R] int64 and nrun [1] int32 in device memory, so the
 * run list can be built on the device without a host sync; len <= 0 skips a
 * run).  src is usually mapped host memory, dst HBM; max_len bounds every
 * len[r] (words); R <= 65535; src and dst 4-byte aligned.
 */
int fathom_gather_runs(const void *src, void *dst, const int64_t *off, const int64_t *len, const int32_t *nrun,
                       int64_t R, int64_t max_len, void *stream);

/*
 * The copy-index gather of a plan (scripts/B_e2e_offload_v2.py:190-197: the run
 * list of every (bh, channel) slot -- first t planes, and the scales of active
 * channels -- passed to gather_runs for planes and scales).  Stores in the
 * whole-sequence layout (sub = nblk, nsb = 1): planes [BH, 1, D, 4, nblk]
 * uint64 and scales [BH, 1, D, nblk] fp16.  For every slot with t > 0 the first
 * min(t, 4) planes and the scales are copied from *_src (usually mapped host
 * memory) to the same offsets of *_dst (HBM staging); other bytes of *_dst are
 * left unchanged.  t [BH, D] int8 (device); BH * D <= 65535.
 */
int fathom_copy_index(const int8_t *t, int64_t BH, int64_t D, int64_t nblk, const void *planes_src,
                      const void *scales_src, void *planes_dst, void *scales_dst, void *stream);

/*
 * Pinned, GPU-mapped host memory (scripts/B_e2e_offload_v2.py:33-39,
 * host_mapped / free_host through cudaHostAlloc(flags=3) and
 * cudaHostGetDevicePointer).  coherent != 0 asks for fine-grained (coherent)
 * memory, 0 for non-coherent.  *dev_ptr is the address kernels use.
 */
int fathom_host_alloc_mapped(size_t bytes, int coherent, void **host_ptr, void **dev_ptr);
int fathom_host_free(void *host_ptr);

/* Asynchronous copy between any two device-visible or host buffers (hipMemcpyAsync, kind default). */
int fathom_memcpy(void *dst, const void *src, size_t bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FATHOM_HIP_H */
