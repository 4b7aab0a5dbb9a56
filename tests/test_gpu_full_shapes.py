"""Configs 2, 4 and 5 at their full sizes, checked against the oracle where the
oracle can follow them (as the config-3 file does for the 2^20-token layer):

* config 2: 8 KV heads, G = 4, n = 131072, k = 512;
* config 4: 8 KV heads, G = 7, n = 131072, k = 2048, RoPE-rotated keys (kk = 2012:
  the finalize's largest list);
* config 5: one layer of the 36-layer decode step, 32 rows, G = 4, n = 32768
  (the short-row path: scan with group maxima, then the row selection), at the
  first layer's budget and at the last layer's.

Per case: the plan bit for bit; the fused scan + top-k == sink_local_topk(scan)
== the oracle's top-k of the same scores; the scores of 8 random 2048-token
tiles per row and of the blocks of up to 512 selected tokens per row within
1e-3 of oracle.scan_planes over those blocks (the quantiser works per 64-token
block, so quantising the gathered blocks gives the full store's codes and
scales); exact attention over the selected rows (union and per-position
reads) within 1e-4 relative + 2e-5 absolute of the float64 oracle, with the
union's distinct-row counts equal.
"""
import numpy as np
import pytest
import torch

from fathom_amd import bitplane as bp
from fathom_amd import offload as off
from fathom_amd import workloads as W
from oracle import fathom_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

CASES = [(2, 0), (4, 0), (5, 0), (5, 35)]


@pytest.fixture(scope="module", params=CASES, ids=[f"c{c}-layer{l}" for c, l in CASES])
def full(request):
    cfg, layer = request.param
    print(f"[full-shape] config {cfg} layer {layer}: building the store", flush=True)
    x = W.config_inputs(cfg, device=DEV, layer=layer)
    st = bp.PlaneStore(x["K"], keep_code=False)
    plan = bp.make_plan(x["g"], x["budget"])
    scores = st.scan(x["q"], plan)
    idx = st.scan_topk(x["q"], plan, x["k"], x["sink"], x["local"])
    torch.cuda.synchronize()
    yield {"cfg": cfg, "x": x, "plan": plan, "scores": scores, "idx": idx}
    del st, scores
    torch.cuda.empty_cache()


def test_full_shape_plan_bitexact(full):
    x = full["x"]
    pr = O.make_plan(x["g"].cpu().numpy(), x["budget"])
    np.testing.assert_array_equal(full["plan"]["t"].cpu().numpy(), pr["t"])


def test_full_shape_fused_equals_unfused_and_oracle(full):
    print(f"[full-shape] config {full['cfg']}: top-k parity", flush=True)
    x = full["x"]
    unfused = bp.sink_local_topk(full["scores"], x["k"], x["sink"], x["local"])
    torch.testing.assert_close(full["idx"], unfused, rtol=0, atol=0)
    ref = O.sink_local_topk(full["scores"].cpu().numpy().reshape(-1, x["n"]), x["k"], x["sink"], x["local"])
    np.testing.assert_array_equal(full["idx"].cpu().numpy().reshape(-1, x["k"]), ref)


def test_full_shape_scores_on_tiles_and_selected_tokens(full):
    print(f"[full-shape] config {full['cfg']}: scores vs oracle on sampled blocks", flush=True)
    x, scores = full["x"], full["scores"]
    n, BH = x["n"], x["BH"]
    rng = np.random.default_rng(7 + full["cfg"])
    t = full["plan"]["t"].cpu().numpy()
    idx = full["idx"].cpu().numpy()
    q = x["q"].float().cpu().numpy()
    nblk = (n + 63) // 64
    for r in range(BH):
        tiles = rng.choice(n // 2048, 8, replace=False)
        blocks = set((tiles[:, None] * 32 + np.arange(32)[None]).ravel().tolist())
        sel = idx[r].ravel()
        sel = rng.choice(sel, min(512, sel.size), replace=False)
        blocks |= set((sel // 64).tolist())
        blocks = np.array(sorted(b for b in blocks if 0 <= b < nblk))
        tok = (blocks[:, None] * 64 + np.arange(64)[None]).ravel()
        tok = tok[tok < n]
        Kr = x["K"][r, torch.from_numpy(tok).to(DEV)].float().cpu().numpy()[None]
        code, sc = O.quantise_u4(Kr)
        ref = O.scan_planes(q[r:r + 1], code, sc.astype(np.float16).astype(np.float32), t[r:r + 1])[0]
        got = scores[r][:, torch.from_numpy(tok).to(DEV)].cpu().numpy().astype(np.float64)
        floor = 1e-4 * np.abs(ref).max(-1, keepdims=True)
        err = np.abs(got - ref)
        bad = err > 1e-3 * np.abs(ref) + floor
        assert not bad.any(), f"row {r}: {int(bad.sum())} of {bad.size} scores off; max err {err.max():.3e}"


def test_full_shape_attention_matches_oracle(full):
    print(f"[full-shape] config {full['cfg']}: attention vs oracle", flush=True)
    x, idx = full["x"], full["idx"]
    n = x["n"]
    V = W.synth_values(x["BH"], n, device=DEV)
    q = x["q"].float().contiguous()
    ref, rnu = O.gather_attention(q.cpu().numpy(), idx.cpu().numpy(), n, x["K"].float().cpu().numpy(),
                                  V.float().cpu().numpy())
    for unique in (True, False):
        out, nu = off.gather_attention(q, idx, n, x["K"], V, n, unique=unique)
        torch.cuda.synchronize()
        got = out.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref)
        bad = err > 1e-4 * np.abs(ref) + 2e-5
        assert not bad.any(), f"unique={unique}: {int(bad.sum())} outputs off; max err {err.max():.3e}"
        if unique:
            np.testing.assert_array_equal(nu.cpu().numpy(), rnu)
