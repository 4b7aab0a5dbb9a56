"""Config 3 at its full size (8 KV heads, G = 4, n = 2^20, B = 48, k = 512): the
headline workload checked against the oracle where the oracle can follow it,
the way the reference checks its copy at the real shape (PLANES_CHECK,
scripts/B_e2e_offload_v2.py:184-202):

* the plan, bit for bit;
* the scores of 16 random 2048-token tiles per row and of the blocks of every
  selected token, within 1e-3 of oracle.scan_planes over those blocks (the
  quantiser works per 64-token block, so quantising the gathered blocks gives
  the full store's codes and scales);
* the fused scan + top-k == sink_local_topk(scan) == the oracle's top-k of the
  same scores, at k = 512 and at k above the LDS-resident selections (4096,
  20036);
* the zero-copy (host-mapped index) and copy-index (staged runs) paths select
  the HBM path's indices;
* the union-gathered K/V rows == oracle.gather_union.
"""
import math

import numpy as np
import pytest
import torch

from fathom_amd import bitplane as bp
from fathom_amd import offload as off
from fathom_amd import workloads as W
from oracle import fathom_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


@pytest.fixture(scope="module")
def c3():
    print("[c3-full] building the 2^20-token store", flush=True)
    x = W.config_inputs(3, device=DEV)
    st = bp.PlaneStore(x["K"])
    plan = bp.make_plan(x["g"], x["budget"])
    q = x["q"]
    scores = st.scan(q, plan)
    idx = st.scan_topk(q, plan, x["k"], x["sink"], x["local"])
    torch.cuda.synchronize()
    yield {"x": x, "st": st, "plan": plan, "q": q, "scores": scores, "idx": idx}
    del st, scores
    torch.cuda.empty_cache()


def test_c3_plan_bitexact(c3):
    x = c3["x"]
    assert x["n"] == 1 << 20 and x["BH"] == 8 and x["G"] == 4
    pr = O.make_plan(x["g"].cpu().numpy(), x["budget"])
    np.testing.assert_array_equal(c3["plan"]["t"].cpu().numpy(), pr["t"])


def test_c3_scores_on_tiles_and_selected_tokens(c3):
    print("[c3-full] scores vs oracle on sampled blocks", flush=True)
    x, scores = c3["x"], c3["scores"]
    n, BH = x["n"], x["BH"]
    rng = np.random.default_rng(2026)
    t = c3["plan"]["t"].cpu().numpy()
    idx = c3["idx"].cpu().numpy()
    q = x["q"].cpu().numpy()
    nblk = n // 64
    for r in range(BH):
        tiles = rng.choice(n // 2048, 16, replace=False)
        blocks = set((tiles[:, None] * 32 + np.arange(32)[None]).ravel().tolist())
        blocks |= set((idx[r].ravel() // 64).tolist())
        blocks = np.array(sorted(b for b in blocks if 0 <= b < nblk))
        tok = (blocks[:, None] * 64 + np.arange(64)[None]).ravel()
        Kr = x["K"][r, torch.from_numpy(tok).to(DEV)].float().cpu().numpy()[None]
        code, sc = O.quantise_u4(Kr)
        ref = O.scan_planes(q[r:r + 1], code, sc.astype(np.float16).astype(np.float32), t[r:r + 1])[0]
        got = scores[r][:, torch.from_numpy(tok).to(DEV)].cpu().numpy().astype(np.float64)
        floor = 1e-4 * np.abs(ref).max(-1, keepdims=True)
        err = np.abs(got - ref)
        bad = err > 1e-3 * np.abs(ref) + floor
        assert not bad.any(), f"row {r}: {int(bad.sum())} of {bad.size} scores off; max err {err.max():.3e}"


def test_c3_fused_topk_equals_unfused_and_oracle(c3):
    print("[c3-full] top-k parity", flush=True)
    x = c3["x"]
    unfused = bp.sink_local_topk(c3["scores"], x["k"], x["sink"], x["local"])
    torch.testing.assert_close(c3["idx"], unfused, rtol=0, atol=0)
    ref = O.sink_local_topk(c3["scores"].cpu().numpy().reshape(-1, x["n"]), x["k"], x["sink"], x["local"])
    np.testing.assert_array_equal(c3["idx"].cpu().numpy().reshape(-1, x["k"]), ref)


@pytest.mark.parametrize("k", [4096, 20036])
def test_c3_wide_topk_equals_oracle(c3, k):
    """k - sink - local above 2048 at full size (kk = 4060: the counting-sort
    ranking; kk = 20000: the bitonic sort with its global merge steps): the
    fused call == sink_local_topk(scan) == the oracle's top-k of the same
    scores (torch.topk has no limit on k, kernels/bitplane.py:376)."""
    print(f"[c3-full] wide top-k k={k}", flush=True)
    x = c3["x"]
    got = c3["st"].scan_topk(c3["q"], c3["plan"], k, x["sink"], x["local"])
    unfused = bp.sink_local_topk(c3["scores"], k, x["sink"], x["local"])
    assert torch.equal(got, unfused)
    ref = O.sink_local_topk(c3["scores"].cpu().numpy().reshape(-1, x["n"]), k, x["sink"], x["local"])
    np.testing.assert_array_equal(got.cpu().numpy().reshape(-1, k), ref)


def test_c3_zero_copy_and_copy_index_equal_hbm(c3):
    print("[c3-full] zero-copy and copy-index", flush=True)
    x, st, plan, q = c3["x"], c3["st"], c3["plan"], c3["q"]
    k, sink, local = x["k"], x["sink"], x["local"]
    hps = []
    try:
        _, pl_dev, h = off.host_mapped(st.planes_k)
        hps.append(h)
        _, sc_dev, h = off.host_mapped(st.scales_k)
        hps.append(h)
        hst = bp.PlaneStore.__new__(bp.PlaneStore)
        hst.BH, hst.n, hst.nsb, hst.sub = st.BH, st.n, st.nsb, st.sub
        hst.planes32, hst.scales_k = pl_dev, sc_dev
        got = hst.scan_topk(q, plan, k, sink, local)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, c3["idx"], rtol=0, atol=0)
    finally:
        for h in hps:
            off.free_host(h)
    nb = math.ceil(x["n"] / 64)
    bp.SUB = nb
    try:
        full = bp.PlaneStore(x["K"], keep_code=False)
    finally:
        bp.SUB = 16
    hs, hps = off.host_store(full)
    try:
        stg = off.staging_store(full)
        del full
        off.copy_index(hs, stg, plan)
        got = stg.scan_topk(q, plan, k, sink, local)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, c3["idx"], rtol=0, atol=0)
    finally:
        for h in hps:
            off.free_host(h)


def test_c3_union_rows_match_oracle(c3):
    print("[c3-full] union gather", flush=True)
    x = c3["x"]
    n = x["n"]
    V = W.synth_values(x["BH"], n, device=DEV)
    Ks, Vs, nu = off.gather_union(c3["idx"], n, x["K"], V, n)
    torch.cuda.synchronize()
    idx = c3["idx"].cpu().numpy()
    rK, rV, rnu = O.gather_union(idx, n, x["K"].cpu().view(torch.int16).numpy(), V.cpu().view(torch.int16).numpy())
    np.testing.assert_array_equal(nu.cpu().numpy(), rnu)
    np.testing.assert_array_equal(Ks.cpu().view(torch.int16).numpy(), rK)
    np.testing.assert_array_equal(Vs.cpu().view(torch.int16).numpy(), rV)
