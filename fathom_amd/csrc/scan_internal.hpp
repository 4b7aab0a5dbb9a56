// Host-side pieces of the fused scan + top-k shared between translation units.
#pragma once
#include "common.hpp"

namespace fathom {

// Workspace bytes of the fused scan + top-k over rows = BH * G score rows of n
// tokens, kk = k - sink - local.
size_t scan_topk_ws(int64_t rows, int64_t n, int64_t k, int64_t kk);

// The fused scan + top-k (stages: FATHOM_STAGE_* mask) on a caller-provided workspace.
int scan_topk_run(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls, const int32_t *clsn, int bmax,
                  int64_t units_max, const void *planes_sb, const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t m,
                  int64_t k, int64_t sink, int64_t local, int64_t *idx, void *workspace, size_t workspace_bytes,
                  int stages, void *stream);

// make_plan on the device (budget [BH], or budget_value when budget is null).
int make_plan_run(const float *g, const float *budget, float budget_value, int64_t BH, int64_t D, int bmax, int iters,
                  int8_t *t, int32_t *pairs, int32_t *npairs, int32_t *act, int32_t *nact, int32_t *cls, int32_t *clsn,
                  void *stream);

}  // namespace fathom
