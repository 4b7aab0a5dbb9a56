"""GPU parity tests: the gfx950 kernels (through the C ABI) against the CPU oracle.

Bit-exact: codes, scales, plane words (logical and superblock order), plans,
top-k index sets given the same scores, gathered rows.  Scores: within 1e-3
relative of the float64 oracle, with an absolute floor of 1e-4 x the row's
largest |score| (summation-order noise near zero crossings).
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
SDT = {"f16": torch.float16, "f32": torch.float32, "bf16": torch.bfloat16}


def _u64(t):
    return t.cpu().numpy().view(np.uint64)


def _scores_close(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = 1e-4 * np.abs(ref).max(-1, keepdims=True)
    err = np.abs(got - ref)
    bad = err > 1e-3 * np.abs(ref) + floor
    assert not bad.any(), f"{int(bad.sum())} scores off; max err {err.max():.3e}"


def _keys(BH, n, d=128, seed=0, dtype=torch.float32, edge=True):
    g = torch.Generator().manual_seed(seed)
    sigma = torch.exp(torch.randn(BH, d, generator=g))
    K = torch.randn(BH, n, d, generator=g) * sigma[:, None, :]
    if edge:
        K[0, :64, 0] = 0.0                       # all-zero block: 0/0 codes
        K[0, :, 1] = 1e-9                        # fp16 absmax underflow
        K[0, min(70, n - 1), 2] = float("nan")   # NaN poisons a block
        if BH > 1:
            K[1, :, 3] = 7.0e4                   # fp16 absmax overflow
        if n >= 164:
            K[0, 100:164, 5] = torch.linspace(-2, 2, 64)
    return K.to(dtype)


# ----------------------------------------------------------------------------- store build
@pytest.mark.parametrize("kdtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("sdt", ["f16", "f32", "bf16"])
@pytest.mark.parametrize("n", [64, 1000, 4097])
def test_quantise_and_pack_bitexact(kdtype, sdt, n):
    print(f"[quantise] kdtype={kdtype} sdt={sdt} n={n}", flush=True)
    K = _keys(2, n, dtype=kdtype, edge=kdtype != torch.float16)
    code_r, sc_r = O.quantise_u4(K.float().numpy(), sdt)
    code, sc = bp.quantise_u4(K.to(DEV), SDT[sdt])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(code.cpu().numpy(), code_r)
    np.testing.assert_array_equal(sc.float().cpu().numpy(), sc_r)
    planes = bp.pack_planes(code)
    np.testing.assert_array_equal(_u64(planes), O.pack_planes(code_r))
    np.testing.assert_array_equal(bp.unpack_planes(planes, n).cpu().numpy(), code_r)


@pytest.mark.parametrize("sub", [16, 1, 3, "whole"])
@pytest.mark.parametrize("n", [1000, 70001])
def test_planestore_superblocks_bitexact(sub, n, monkeypatch):
    print(f"[planestore] sub={sub} n={n}", flush=True)
    nb = math.ceil(n / 64)
    s = nb if sub == "whole" else sub
    monkeypatch.setattr(bp, "SUB", s)
    K = _keys(3, n, seed=1, dtype=torch.bfloat16)
    st = bp.PlaneStore(K.to(DEV))
    code_r, sc_r = O.quantise_u4(K.float().numpy())
    pl_r, scs_r = O.to_superblocks(O.pack_planes(code_r), sc_r.astype(np.float16), s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(st.code.cpu().numpy(), code_r)
    np.testing.assert_array_equal(_u64(st.planes_k), pl_r)
    np.testing.assert_array_equal(st.scales_k.cpu().numpy(), scs_r)
    # the standalone permutation gives the same store
    pl2, sc2 = bp.to_superblocks(bp.pack_planes(st.code), st.scales_blk)
    np.testing.assert_array_equal(_u64(pl2), pl_r)
    np.testing.assert_array_equal(sc2.cpu().numpy(), scs_r)


def test_dequant_bitexact():
    K = _keys(2, 777, seed=2, edge=False)
    code_r, sc_r = O.quantise_u4(K.numpy())
    code, sc = bp.quantise_u4(K.to(DEV))
    for tv in [0, 1, 3, 4, np.arange(128) % 5]:
        t = torch.as_tensor(tv)
        got = bp.dequant_planes(code[1], sc[1], t).cpu().numpy()
        np.testing.assert_array_equal(got, O.dequant_planes(code_r[1], sc_r[1], np.asarray(tv)))


# ----------------------------------------------------------------------------- plan
@pytest.mark.parametrize("d", [128, 64, 100, 256])
@pytest.mark.parametrize("bmax", [4, 1, 2, 8])
def test_make_plan_bitexact(d, bmax):
    print(f"[plan] d={d} bmax={bmax}", flush=True)
    rng = np.random.default_rng(d * 10 + bmax)
    BH = 37
    g = (np.exp(rng.standard_normal((BH, d)) * 3) * rng.random((BH, d))).astype(np.float32)
    g[0, :5] = 0
    g[1, :] = 0
    g[2, 3] = np.nan
    g[3, :] = 1.0                                    # all tied
    budget = rng.integers(0, d * bmax + 20, BH).astype(np.float32)
    ref = O.make_plan(g, budget, bmax=bmax)
    got = bp.make_plan(torch.from_numpy(g).to(DEV), torch.from_numpy(budget).to(DEV), bmax=bmax)
    for key in ("t", "pairs", "npairs", "act", "nact", "cls", "clsn"):
        np.testing.assert_array_equal(got[key].cpu().numpy(), ref[key], err_msg=key)


def test_make_plan_torch_is_the_plan_depths():
    """make_plan_torch (the reference's torch plan, kernels/bitplane.py:118-126):
    the float depths [BH, D] of make_plan, equal to the oracle's plan."""
    x = W.config_inputs(2, n=128, BH=4)
    t = bp.make_plan_torch(x["g"].to(DEV), x["budget"])
    assert t.dtype == torch.float32 and tuple(t.shape) == (4, 128)
    np.testing.assert_array_equal(t.cpu().numpy(), O.make_plan(x["g"].numpy(), x["budget"])["t"].astype(np.float32))
    assert torch.equal(t, bp.make_plan(x["g"].to(DEV), x["budget"])["t"].float())


def test_make_plan_scalar_budget_and_iters():
    """The scalar-budget entry point (fathom_make_plan_uniform) and every
    bisection count modulo the kernel's three-step rounds (30, 29, 28, ...):
    the oracle's one-step bisection bit for bit, and the tensor-budget call."""
    rng = np.random.default_rng(9)
    g = np.exp(rng.standard_normal((8, 128)) * 2).astype(np.float32)
    gd = torch.from_numpy(g).to(DEV)
    for budget in (48.0, 47.5, 0.3, 700.0):
        for it in (30, 29, 28, 10, 2, 1, 0):
            ref = O.make_plan(g, budget, iters=it)
            got = bp.make_plan(gd, budget, iters=it)
            tens = bp.make_plan(gd, torch.full((8,), budget, device=DEV), iters=it)
            for key in ("t", "pairs", "npairs", "act", "nact", "cls", "clsn"):
                np.testing.assert_array_equal(got[key].cpu().numpy(), ref[key], err_msg=f"{key} {budget} {it}")
                assert torch.equal(got[key], tens[key])


def test_make_plan_boundary_gains_and_long_bisections():
    """Gains on exact depth boundaries (powers of two: log2 g an integer, so
    lg - mid hits the rounding ties of the depth at dyadic mids; channels tied
    in groups) and bisection counts past the kernel's line-count checkpoints
    (steps 15, 18, 21, ...): the oracle's plan bit for bit."""
    rng = np.random.default_rng(21)
    BH, d = 16, 128
    g = (np.float32(2.0) ** rng.integers(-12, 12, (BH, d))).astype(np.float32)
    g[2] = np.exp(rng.standard_normal(d) * 4).astype(np.float32)
    g[3, :64] = np.float32(8.0)
    gd = torch.from_numpy(g).to(DEV)
    for bmax in (4, 2, 3):
        for it in (16, 17, 18, 19, 31, 40, 60):
            budget = (rng.integers(0, d * bmax, BH) + 0.5 * (it % 2)).astype(np.float32)
            ref = O.make_plan(g, budget, bmax=bmax, iters=it)
            got = bp.make_plan(gd, torch.from_numpy(budget).to(DEV), bmax=bmax, iters=it)
            for key in ("t", "pairs", "npairs", "act", "nact", "cls", "clsn"):
                np.testing.assert_array_equal(got[key].cpu().numpy(), ref[key], err_msg=f"{key} bmax={bmax} iters={it}")


def test_make_plan_worked_example():
    K = np.array([[1.8, 0.4, -0.2, 0.05], [-1.1, 0.9, 0.3, -0.02], [0.3, -1.2, 0.1, 0.04],
                  [1.2, 0.7, 0.4, 0.01], [-0.6, -0.3, -0.5, 0.03], [0.9, 1.1, -0.3, -0.05]], np.float32)
    g = (np.float32([3, 1, 2, 0.1]) ** 2 + np.float32([1, 2, -1, 0.2]) ** 2) * K.var(0, ddof=1)
    for B, t in ((8, [4, 3, 1, 0]), (6, [3, 2, 1, 0])):
        got = bp.make_plan(torch.from_numpy(g[None]).to(DEV), float(B))
        assert got["t"][0].tolist() == t


# ----------------------------------------------------------------------------- scan
def _scan_case(cfg, n, BH, sub=None, seed=0, budget=None):
    x = W.config_inputs(cfg, seed=seed, n=n, BH=BH)
    if sub is not None:
        bp.SUB = sub
    try:
        st = bp.PlaneStore(x["K"].to(DEV))
    finally:
        bp.SUB = 16
    plan = bp.make_plan(x["g"].to(DEV), budget if budget is not None else x["budget"])
    return x, st, plan


@pytest.mark.parametrize("cfg,n,BH,sub", [(1, 16384, None, None), (2, 16421, 2, None), (2, 8192, 2, 128),
                                          (4, 8192, 2, None), (3, 20000, 1, 7)])
def test_scan_matches_oracle(cfg, n, BH, sub):
    print(f"[scan] cfg={cfg} n={n} BH={BH} sub={sub}", flush=True)
    x, st, plan = _scan_case(cfg, n, BH, sub)
    scores = st.scan(x["q"].to(DEV), plan).cpu().numpy()
    t = plan["t"].cpu().numpy()
    code_r, sc_r = O.quantise_u4(x["K"].float().numpy())
    ref = O.scan_planes(x["q"].numpy(), code_r, sc_r.astype(np.float16).astype(np.float32), t)
    _scores_close(scores, ref)


@pytest.mark.parametrize("G,n,k", [(12, 9000, 512), (16, 40000, 300)])
def test_store_methods_more_than_8_query_heads(G, n, k):
    """G > 8 query heads per KV head (the scan kernels take 8 per launch; the
    store methods run groups of at most 8): scores within tolerance of the
    float64 oracle, and scan_topk, plan_scan_topk and plan_scan_topk_attention
    equal the oracle's top-k of those scores and gather_attention over it."""
    print(f"[G>8] G={G} n={n} k={k}", flush=True)
    x = W.config_inputs(2, seed=3, n=n, BH=2)
    K = x["K"]
    gen = torch.Generator().manual_seed(G)
    q = torch.randn(2, G, 128, generator=gen)
    g = x["g"].to(DEV)
    st = bp.PlaneStore(K.to(DEV))
    plan = bp.make_plan(g, 48.0)
    qd = q.to(DEV)
    sc = st.scan(qd, plan)
    code_r, sc_r = O.quantise_u4(K.float().numpy())
    _scores_close(sc.cpu().numpy(), O.scan_planes(q.numpy(), code_r, sc_r.astype(np.float16).astype(np.float32),
                                                   plan["t"].cpu().numpy()))
    ref = O.sink_local_topk(sc.cpu().numpy(), k, 4, 32)
    np.testing.assert_array_equal(st.scan_topk(qd, plan, k).cpu().numpy(), ref)
    got, t = st.plan_scan_topk(qd, g, 48.0, k, return_t=True)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    assert torch.equal(t, plan["t"])
    Kb = K.to(torch.bfloat16).to(DEV).contiguous()
    Vb = torch.randn(K.shape, generator=gen).to(torch.bfloat16).to(DEV)
    idx, out = st.plan_scan_topk_attention(qd, g, 48.0, k, Kb, Vb)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref)
    ref_out, _ = off.gather_attention(qd, idx, n, Kb, Vb, n)
    _attn_close(out.cpu().numpy(), ref_out.cpu().numpy())  # launch shapes differ per head group


@pytest.mark.parametrize("budget,umax", [(16.0, None), (24.0, None), (40.0, None), (48.0, None), (48.0, 64),
                                         (48.0, 16), (64.0, None), (80.0, None), (90.0, None), (90.0, 200),
                                         (100.0, None), (100.0, 64)])
def test_scan_stacked_classes_equal_unstacked(budget, umax):
    """Rows of at most four heads run stacked step classes (two classes per
    accumulator, an odd last slice of both classes in one instruction); rows of
    more heads do not.  Heads 0..3 scanned in a G = 4 call equal the same heads
    scanned in a G = 8 call (heads 4..7 a copy) bit for bit, for plans of 1 to
    7 slices (up to 6 held in registers), kernels picked for smaller or larger
    plans included; so do the fused top-k indices (long rows, the candidate
    pass and its sample)."""
    print(f"[stacked] budget={budget} umax={umax}", flush=True)
    x = W.config_inputs(2, n=40000, BH=2)
    st = bp.PlaneStore(x["K"].to(DEV))
    plan = bp.make_plan(x["g"].to(DEV), budget)
    if umax is not None:
        plan = dict(plan, units_max=umax)
    q4 = x["q"].to(DEV)
    assert q4.shape[1] == 4
    q8 = torch.cat([q4, q4], 1).contiguous()
    s4, s8 = st.scan(q4, plan), st.scan(q8, plan)
    torch.testing.assert_close(s4, s8[:, :4], rtol=0, atol=0)
    torch.testing.assert_close(s8[:, 4:], s8[:, :4], rtol=0, atol=0)
    i4, i8 = st.scan_topk(q4, plan, 512, 4, 64), st.scan_topk(q8, plan, 512, 4, 64)
    torch.testing.assert_close(i4, i8[:, :4], rtol=0, atol=0)
    torch.testing.assert_close(i4, bp.sink_local_topk(s4, 512, 4, 64), rtol=0, atol=0)
    for G in (1, 2, 3):  # fewer heads: rows 2G..7 of each half are zero
        torch.testing.assert_close(st.scan(q4[:, :G].contiguous(), plan), s4[:, :G], rtol=0, atol=0)


@pytest.mark.parametrize("G,n", [(2, 40000), (3, 20000), (5, 40000), (6, 20000), (8, 40000), (8, 20000)])
def test_scan_and_fused_topk_every_group_size(G, n):
    """The scan is instantiated per head count G (1-8) and the configurations
    reach only G = 1, 4, 7: scores against the oracle, and the fused top-k
    (chain above 32768 tokens, row select below) against the unfused one, bit
    for bit.  (PlaneStore keeps D = 128, kernels/bitplane.py:313.)"""
    print(f"[scan-G] G={G} n={n}", flush=True)
    BH, k = 2, 256
    x = W.synth_layer(BH, n, G, seed=100 * G + n % 7)
    g = ((x["q"] ** 2) * x["var"][:, None, :]).sum(1)
    st = bp.PlaneStore(x["K"].to(DEV))
    plan = bp.make_plan(g.to(DEV), 48.0)
    q = x["q"].to(DEV)
    scores = st.scan(q, plan)
    code_r, sc_r = O.quantise_u4(x["K"].float().numpy())
    ref = O.scan_planes(x["q"].numpy(), code_r, sc_r.astype(np.float16).astype(np.float32), plan["t"].cpu().numpy())
    _scores_close(scores.cpu().numpy(), ref)
    want = bp.sink_local_topk(scores, k, 4, 32)
    got = st.scan_topk(q, plan, k, 4, 32)
    torch.testing.assert_close(got, want, rtol=0, atol=0)


@pytest.mark.parametrize("budget", [40.0, 48.0, 80.0, 0.0, 512.0])
def test_scan_budgets_c4_shape(budget):
    x, st, plan = _scan_case(4, 4096, 2, budget=budget)
    scores = st.scan(x["q"].to(DEV), plan).cpu().numpy()
    code_r, sc_r = O.quantise_u4(x["K"].float().numpy())
    ref = O.scan_planes(x["q"].numpy(), code_r, sc_r, plan["t"].cpu().numpy())
    _scores_close(scores, ref)


def test_scan_block_range_writes_only_its_tokens():
    x, st, plan = _scan_case(2, 9000, 2)
    q = x["q"].to(DEV)
    full = st.scan(q, plan)
    out = torch.full_like(full, 12345.0)
    st.scan(q, plan, out=out, blocks=(3, 40))
    lo, hi = 3 * 64, min(40 * 64, 9000)
    torch.testing.assert_close(out[..., lo:hi], full[..., lo:hi], rtol=0, atol=0)
    assert (out[..., :lo] == 12345.0).all() and (out[..., hi:] == 12345.0).all()


def test_scan_host_resident_equals_hbm():
    """Same kernel reading the store zero-copy from mapped pinned host memory."""
    x, st, plan = _scan_case(2, 33000, 2)
    q = x["q"].to(DEV)
    ref = st.scan(q, plan).clone()
    _, pl_dev, hp1 = off.host_mapped(st.planes_k)
    _, sc_dev, hp2 = off.host_mapped(st.scales_k)
    try:
        st.planes32, st.scales_k = pl_dev, sc_dev
        got = st.scan(q, plan)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, ref, rtol=0, atol=0)
    finally:
        off.free_host(hp1)
        off.free_host(hp2)


# ----------------------------------------------------------------------------- top-k
def _topk_case(rows, k, sink, local, m=None):
    got = bp.sink_local_topk(torch.from_numpy(rows).to(DEV), k, sink, local, m=m).cpu().numpy()
    ref = O.sink_local_topk(rows, k, sink, local, m=m)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("n,k,sink,local", [(1000, 128, 4, 64), (16384, 128, 4, 64), (131072, 512, 4, 32),
                                            (100000, 2048, 4, 32), (3000, 2048, 4, 32), (600, 40, 0, 0),
                                            (32768, 512, 4, 32), (32769, 512, 4, 32), (32768, 2048, 0, 0),
                                            (65536, 1024, 0, 0), (600000, 40, 4, 32), (1000000, 64, 4, 32)])
def test_topk_random_bitexact(n, k, sink, local):
    """Rows up to 32768 take the one-kernel row selection, longer rows the
    sample / select / filter / finalize chain; both must equal the oracle.
    Small k on long rows (kk = 4 of 600000, 28 of 10^6) needs the sample's
    tile stride rounded up, or the sample would outgrow its 65536 keys."""
    print(f"[topk] n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + k)
    rows = rng.standard_normal((2, 3, n)).astype(np.float32)
    _topk_case(rows, k, sink, local)


def test_topk_edge_k_and_errors():
    """kk = k - sink - local at its edges: 0 (only the fixed positions), the
    whole row, one token, more than the unmasked tokens (masked -inf keys fill
    the rest by index); then the argument errors."""
    rng = np.random.default_rng(7)
    rows = rng.standard_normal((2, 3, 5000)).astype(np.float32)
    _topk_case(rows[..., :1000], 36, 4, 32)     # kk = 0
    _topk_case(rows[..., :300], 300, 0, 0)      # kk = n
    _topk_case(rows[..., :1], 1, 0, 0)          # one token
    _topk_case(rows[..., :40], 50, 4, 32)       # kk = 14, four unmasked tokens
    t = torch.from_numpy(rows).to(DEV)
    for n, k, sink, local in ((1000, 30, 4, 32),     # k < sink + local
                              (1000, 1037, 4, 32)):  # kk > n
        with pytest.raises(ValueError):
            bp.sink_local_topk(t[..., :n].contiguous(), k, sink, local)
    x, st, plan = _scan_case(2, 2000, 2)
    q = x["q"].to(DEV)
    sc = st.scan(q, plan)
    for k, sink, local in ((36, 4, 32), (2000, 0, 0), (100, 4, 32)):
        torch.testing.assert_close(st.scan_topk(q, plan, k, sink, local), bp.sink_local_topk(sc, k, sink, local),
                                   rtol=0, atol=0)
    with pytest.raises(ValueError):
        st.scan_topk(q, plan, 30, 4, 32)


def test_topk_ties_nan_inf_negzero():
    rng = np.random.default_rng(1)
    n = 5000
    rows = rng.integers(-3, 4, size=(4, n)).astype(np.float32)     # huge tie groups
    rows[0, rng.integers(0, n, 20)] = np.nan
    rows[1, rng.integers(0, n, 20)] = -np.inf
    rows[1, rng.integers(0, n, 20)] = np.inf
    rows[2, rng.integers(0, n, 300)] = -0.0
    rows[3] = 0.0
    _topk_case(rows, 512, 4, 32)
    _topk_case(rows, 100, 3, 5, m=n + 2)


@pytest.mark.parametrize("n,k", [(20000, 512), (100000, 512), (100000, 2048)])
def test_topk_final_ranking_spread_and_crowded(n, k):
    """The final ranking of the selected values counts them into 2048 bins over
    their range: spread values (row 0) take the counting sort; a far outlier
    per row squeezes the rest into few bins (rows 1-2: +1e30, +inf), which
    takes the block rank sort instead.  Both orders equal the oracle's."""
    print(f"[topk-rank] n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + 3 * k)
    rows = rng.standard_normal((3, n)).astype(np.float32)
    rows[1, n // 3] = 1e30
    rows[2, n // 2] = np.inf
    _topk_case(rows, k, 4, 32)


@pytest.mark.parametrize("n,k,sink,local,m", [(5000, 2049, 0, 0, None), (5000, 5000, 0, 0, None),
                                                (40000, 20036, 4, 32, None), (70000, 40000, 4, 32, 70010),
                                                (300000, 4100, 4, 32, None), (16385, 16385, 0, 0, None)])
def test_topk_wide_bitexact(n, k, sink, local, m):
    """kk above the LDS-resident selections' 2048 (torch.topk has no limit):
    the 64-bit radix select + bitonic sort.  One LDS sort chunk (P = 4096), the
    whole row, P = 32768 and 65536 (global merge steps between LDS merges), the
    local window partly past the row (m > n), a long row, P = 32768 with
    kk = P / 2 + 1."""
    print(f"[topk-wide] n={n} k={k} m={m}", flush=True)
    rng = np.random.default_rng(n + k)
    rows = rng.standard_normal((2, 2, n)).astype(np.float32)
    _topk_case(rows, k, sink, local, m=m)


def test_topk_wide_ties_nan_inf():
    """Wide kk over rows of seven distinct values (the index rounds break the
    ties), NaN, +-inf, -0.0, and more selected than unmasked tokens (the masked
    -inf keys fill the rest by index)."""
    rng = np.random.default_rng(11)
    n = 12000
    rows = rng.integers(-3, 4, size=(4, n)).astype(np.float32)
    rows[0, rng.integers(0, n, 20)] = np.nan
    rows[1, rng.integers(0, n, 20)] = -np.inf
    rows[1, rng.integers(0, n, 20)] = np.inf
    rows[2, rng.integers(0, n, 300)] = -0.0
    rows[3] = 0.0
    _topk_case(rows, 6000, 4, 32)
    _topk_case(rows, 2100, 3, 5, m=n + 2)
    _topk_case(rows, 12004, 0, 5, m=n + 2)  # kk = 11999 of 11997 unmasked


@pytest.mark.parametrize("cfg,n,BH,k", [(2, 9000, 2, 4000), (2, 40000, 2, 3000), (5, 32768, 2, 6000)])
def test_scan_topk_wide_equals_scan_then_topk(cfg, n, BH, k):
    """The fused entries with kk above 2048: scan_topk and plan_scan_topk (short
    and long rows) equal sink_local_topk of the scan's scores, which equals the
    oracle's top-k of those scores."""
    print(f"[scan-topk-wide] cfg={cfg} n={n} k={k}", flush=True)
    x = W.config_inputs(cfg, seed=2, n=n, BH=BH)
    st = bp.PlaneStore(x["K"].to(DEV), keep_code=False)
    q, g = x["q"].to(DEV), x["g"].to(DEV)
    sink, local = x["sink"], x["local"]
    plan = bp.make_plan(g, x["budget"])
    sc = st.scan(q, plan)
    ref = bp.sink_local_topk(sc, k, sink, local)
    np.testing.assert_array_equal(ref.cpu().numpy(), O.sink_local_topk(sc.cpu().numpy(), k, sink, local))
    for _ in range(2):
        assert torch.equal(st.scan_topk(q, plan, k, sink, local), ref)
        assert torch.equal(st.plan_scan_topk(q, g, x["budget"], k, sink, local), ref)


def test_topk_huge_tie_bucket_slow_path():
    """All scores inside one first-level bucket (> 8192 candidates)."""
    rng = np.random.default_rng(2)
    n = 200000
    rows = (1.0 + rng.integers(0, 50, size=(2, n)) * 1e-7).astype(np.float32)
    _topk_case(rows, 512, 4, 32)
    _topk_case(np.ones((1, 70000), np.float32), 300, 4, 32)
    _topk_case(np.ones((2, 32768), np.float32), 300, 4, 32)  # one tie group, row-selection path


@pytest.mark.parametrize("order", ["falling", "rising", "front_block"])
def test_topk_tight_threshold_fallback(order):
    """Score orders the sampled tiles misrepresent: falling scores put the row's
    top in sampled tile 0, so the tight first-pass threshold admits fewer than
    kk elements and the fallback pass runs; the result stays exact."""
    print(f"[topk] order={order}", flush=True)
    n = 120000
    idx = np.arange(n, dtype=np.float32)
    if order == "falling":
        row = -idx
    elif order == "rising":
        row = idx.copy()
    else:  # a large block of equal top scores at the start, noise after
        row = np.random.default_rng(4).standard_normal(n).astype(np.float32)
        row[: 3000] = 10.0
    rows = np.stack([row, row[::-1].copy()])[None].astype(np.float32)
    _topk_case(rows, 512, 4, 32)
    _topk_case(rows, 2048, 4, 32)


def test_topk_config3_rows():
    print("[topk] 32 x 1M", flush=True)
    rng = np.random.default_rng(3)
    rows = rng.standard_normal((8, 4, 1 << 20)).astype(np.float32)
    _topk_case(rows, 512, 4, 32)


# ----------------------------------------------------------------------------- gathers
def test_gather_rows_matches_oracle():
    rng = np.random.default_rng(4)
    BH, cap, R = 3, 5000, 700
    src = torch.randn(BH, cap, 128).to(torch.bfloat16)
    idx = rng.integers(-2, cap + 3, size=(BH, R)).astype(np.int32)
    got = off.gather_rows(src.to(DEV), cap, torch.from_numpy(idx).to(DEV), BH)
    ref = O.gather_rows(src.view(torch.int16).numpy(), idx)
    np.testing.assert_array_equal(got.cpu().view(torch.int16).numpy(), ref)


@pytest.mark.parametrize("host,G,k", [(False, 7, 2048), (True, 7, 2048), (False, 12, 2048), (True, 16, 1100)])
def test_gather_union_matches_oracle(host, G, k):
    """Rows, order and distinct-row counts of the group union; G * k above
    16384 positions (12 x 2048, 16 x 1100) takes the table in global memory."""
    print(f"[gather_union] host={host} G={G} k={k}", flush=True)
    rng = np.random.default_rng(5 + G)
    BH, n, nrec = 4, 20000, 6
    K = torch.randn(BH, n, 128).to(torch.bfloat16)
    V = torch.randn(BH, n, 128).to(torch.bfloat16)
    Kr = torch.randn(BH, nrec, 128).to(torch.bfloat16)
    Vr = torch.randn(BH, nrec, 128).to(torch.bfloat16)
    idx = rng.integers(0, 3000, size=(BH, G, k))                   # heavy overlap across heads
    idx[:, :, -3:] = n + rng.integers(0, nrec + 2, size=(BH, G, 3))
    idx[0, 0, 0] = -4
    hps = []
    try:
        if host:
            _, Ksrc, h1 = off.host_mapped(K)
            _, Vsrc, h2 = off.host_mapped(V)
            hps = [h1, h2]
        else:
            Ksrc, Vsrc = K.to(DEV), V.to(DEV)
        Ks, Vs, nu = off.gather_union(torch.from_numpy(idx).to(DEV), n, Ksrc, Vsrc, n, Kr.to(DEV), Vr.to(DEV))
        torch.cuda.synchronize()
        rK, rV, rnu = O.gather_union(idx, n, K.view(torch.int16).numpy(), V.view(torch.int16).numpy(),
                                     Kr.view(torch.int16).numpy(), Vr.view(torch.int16).numpy())
        np.testing.assert_array_equal(Ks.cpu().view(torch.int16).numpy(), rK)
        np.testing.assert_array_equal(Vs.cpu().view(torch.int16).numpy(), rV)
        np.testing.assert_array_equal(nu.cpu().numpy(), rnu)
    finally:
        for h in hps:
            off.free_host(h)


@pytest.mark.parametrize("host", [False, True])
def test_select_and_gather_matches_oracle(host):
    """select_and_gather (one decode step's selection, scripts/B_e2e_offload_v2.py:
    181, 203, 224-241) over an HBM or host-resident store: plan, scores, indices
    and union rows against the oracle (indices given the GPU scores, rows given
    the indices); the default fused selection returns the same indices and rows."""
    print(f"[select_and_gather] host={host}", flush=True)
    x = W.config_inputs(2, n=40000, BH=2)
    K = x["K"]
    V = W.synth_values(2, x["n"])
    st = bp.PlaneStore(K.to(DEV))
    hps = []
    try:
        if host:
            _, pl, h = off.host_mapped(st.planes_k)
            hps.append(h)
            _, sc, h = off.host_mapped(st.scales_k)
            hps.append(h)
            st.planes32, st.scales_k = pl, sc
            _, Ksrc, h = off.host_mapped(K)
            hps.append(h)
            _, Vsrc, h = off.host_mapped(V)
            hps.append(h)
        else:
            Ksrc, Vsrc = K.to(DEV), V.to(DEV)
        r = off.select_and_gather(st, x["q"].to(DEV), x["var"].to(DEV), x["budget"], 512, Ksrc, Vsrc,
                                  x["sink"], x["local"], scores=True)
        fused = off.select_and_gather(st, x["q"].to(DEV), x["var"].to(DEV), x["budget"], 512, Ksrc, Vsrc,
                                      x["sink"], x["local"])
        torch.cuda.synchronize()
        assert fused["scores"] is None
        for key in ("idx", "K", "V", "n_unique"):  # the default (fused) selection is the same
            torch.testing.assert_close(fused[key], r[key], rtol=0, atol=0)
        qd, vd = x["q"].to(DEV).float(), x["var"].to(DEV)
        g = ((qd ** 2) * vd[:, None, :]).sum(1)          # the gain as select_and_gather forms it
        pr = O.make_plan(g.cpu().numpy(), x["budget"])
        np.testing.assert_array_equal(r["plan"]["t"].cpu().numpy(), pr["t"])
        code, scl = O.quantise_u4(K.float().numpy())
        ref_s = O.scan_planes(x["q"].numpy(), code, scl.astype(np.float16).astype(np.float32), pr["t"])
        _scores_close(r["scores"].cpu().numpy(), ref_s)
        idx = r["idx"].cpu().numpy()
        np.testing.assert_array_equal(idx, O.sink_local_topk(r["scores"].cpu().numpy(), 512, x["sink"], x["local"]))
        rK, rV, rnu = O.gather_union(idx, x["n"], K.view(torch.int16).numpy(), V.view(torch.int16).numpy())
        np.testing.assert_array_equal(r["n_unique"].cpu().numpy(), rnu)
        np.testing.assert_array_equal(r["K"].cpu().view(torch.int16).numpy(), rK)
        np.testing.assert_array_equal(r["V"].cpu().view(torch.int16).numpy(), rV)
    finally:
        for h in hps:
            off.free_host(h)


# ----------------------------------------------------------------------------- end to end
@pytest.mark.parametrize("host", [False, True])
def test_gather_runs_matches_oracle(host):
    """Random runs (empty, negative-length and beyond-nrun ones included) from HBM
    or mapped host memory into a pre-filled device buffer."""
    print(f"[gather_runs] host={host}", flush=True)
    rng = np.random.default_rng(11)
    W, R = 50000, 40
    src = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, W, dtype=np.int64).astype(np.int32))
    dst0 = torch.full((W,), -7, dtype=torch.int32)
    starts = rng.integers(0, W - 3000, R)
    lens = rng.integers(-5, 3000, R)
    lens[:4] = 0
    nrun = R - 3
    ref = O.gather_runs(src.numpy(), dst0.numpy(), starts, lens, nrun)
    dst = dst0.to(DEV)
    hp = None
    try:
        if host:
            _, s_src, hp = off.host_mapped(src)
        else:
            s_src = src.to(DEV)
        off.gather_runs(s_src, dst, torch.from_numpy(starts).to(DEV), torch.from_numpy(lens).to(DEV),
                        torch.tensor([nrun], dtype=torch.int32, device=DEV), int(max(lens.max(), 0)))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(dst.cpu().numpy(), ref)
    finally:
        if hp:
            off.free_host(hp)


def _whole_sequence_store(x):
    nb = math.ceil(x["n"] / 64)
    bp.SUB = nb
    try:
        return bp.PlaneStore(x["K"].to(DEV))
    finally:
        bp.SUB = 16


@pytest.mark.parametrize("cfg,n,BH", [(2, 40000, 2), (4, 20001, 2), (1, 16384, None)])
def test_copy_index_staging_equals_store(cfg, n, BH):
    """The copy-index path: the plan's runs copied from mapped host memory into a
    zeroed HBM staging store; scanning the staging store equals scanning the full
    store bit for bit (the reference's PLANES_CHECK, scripts/B_e2e_offload_v2.py:
    184-202, at tolerance 0), fused top-k included, and no other word is written."""
    print(f"[copy_index] cfg={cfg} n={n} BH={BH}", flush=True)
    x = W.config_inputs(cfg, n=n, BH=BH)
    st = _whole_sequence_store(x)
    plan = bp.make_plan(x["g"].to(DEV), x["budget"])
    q = x["q"].to(DEV)
    hs, hps = off.host_store(st)
    try:
        stg = off.staging_store(st)
        off.copy_index(hs, stg, plan)
        torch.testing.assert_close(stg.scan(q, plan), st.scan(q, plan), rtol=0, atol=0)
        k = min(512, x["n"] - 40)
        torch.testing.assert_close(stg.scan_topk(q, plan, k), st.scan_topk(q, plan, k), rtol=0, atol=0)
        t = plan["t"].cpu().numpy()
        nb = st.sub
        offp, lenp, offs, lens = O.copy_index_runs(t, nb, 128)
        ref_p = O.gather_runs(st.planes_k.view(torch.int32).cpu().numpy().ravel(),
                              np.zeros(st.planes_k.numel() * 2, np.int32), offp, lenp, len(offp))
        np.testing.assert_array_equal(stg.planes_k.view(torch.int32).cpu().numpy().ravel(), ref_p)
        sc_words = st.scales_k.view(torch.int16).cpu().numpy().ravel()
        got_sc = stg.scales_k.view(torch.int16).cpu().numpy().ravel()
        for s_ in range(t.size):
            on = t.ravel()[s_] > 0
            seg = slice(s_ * nb, (s_ + 1) * nb)
            np.testing.assert_array_equal(got_sc[seg], sc_words[seg] if on else 0)
    finally:
        for h in hps:
            off.free_host(h)


def test_config1_pipeline_matches_oracle():
    """Config 1 end to end: store, plan, scan, sink/local top-k on the GPU vs the oracle."""
    x = W.config_inputs(1)
    st = bp.PlaneStore(x["K"].to(DEV))
    plan = bp.make_plan(x["g"].to(DEV), x["budget"])
    scores = st.scan(x["q"].to(DEV), plan)
    idx = bp.sink_local_topk(scores, x["k"], x["sink"], x["local"]).cpu().numpy()
    code_r, sc_r = O.quantise_u4(x["K"].numpy())
    pr = O.make_plan(x["g"].numpy(), x["budget"])
    np.testing.assert_array_equal(plan["t"].cpu().numpy(), pr["t"])
    ref_s = O.scan_planes(x["q"].numpy(), code_r, sc_r, pr["t"])
    _scores_close(scores.cpu().numpy(), ref_s)
    # same scores -> same index set, bit for bit
    np.testing.assert_array_equal(idx, O.sink_local_topk(scores.cpu().numpy(), x["k"], x["sink"], x["local"]))
    # against the float64 oracle scores, any difference must sit at the selection boundary
    ref_idx = O.sink_local_topk(ref_s.astype(np.float32), x["k"], x["sink"], x["local"])
    diff = set(idx[0, 0].tolist()) ^ set(ref_idx[0, 0].tolist())
    if diff:
        s = ref_s[0, 0]
        kth = np.sort(s[x["sink"]:x["n"] - x["local"]])[::-1][x["k"] - x["sink"] - x["local"] - 1]
        assert all(abs(s[i] - kth) <= 1e-4 * np.abs(s).max() for i in diff)
    # planted keys (0.8 q + noise) score well above the typical key; with these
    # channel scales they sit near 1.6 sigma, so they are a sanity signal only
    sc = scores.cpu().numpy()[0, 0]
    assert (sc[x["planted"][0].numpy()] > np.median(sc)).all()


def test_config2_full_size_invariants():
    """Config 2 at its full size: store round trip, plan parity, scores vs a float32
    torch reference from the dequantised keys, top-k parity given the scores."""
    print("[c2] full size", flush=True)
    x = W.config_inputs(2, device=DEV)
    st = bp.PlaneStore(x["K"])
    n = x["n"]
    nb = math.ceil(n / 64)
    logical = st.planes_k.permute(0, 1, 4, 2, 3).reshape(x["BH"], -1, 128, 4)[:, :nb]
    assert torch.equal(bp.unpack_planes(logical, n), st.code)
    plan = bp.make_plan(x["g"], x["budget"])
    pr = O.make_plan(x["g"].cpu().numpy(), x["budget"])
    np.testing.assert_array_equal(plan["t"].cpu().numpy(), pr["t"])
    scores = st.scan(x["q"], plan)
    ref = bp.scan_planes_reference(x["q"], st.code, st.scales_blk, plan["t"])
    err = (scores - ref).abs()
    tol = 1e-3 * ref.abs() + 1e-4 * ref.abs().amax(-1, keepdim=True)
    assert bool((err <= tol).all()), float(err.max())
    idx = bp.sink_local_topk(scores, x["k"])
    np.testing.assert_array_equal(idx.cpu().numpy(), O.sink_local_topk(scores.cpu().numpy(), x["k"]))


# ----------------------------------------------------------------------------- fused scan + top-k
@pytest.mark.parametrize("cfg,n,BH,k,sub", [(1, 16384, None, 128, None), (2, 40000, 2, 512, None),
                                            (4, 30000, 2, 2048, None), (2, 5000, 3, 300, 7), (2, 700, 1, 60, None),
                                            (2, 4097, 2, 512, None), (3, 32768, 2, 512, None), (2, 30001, 1, 2048, None)])
def test_scan_topk_fused_equals_unfused(cfg, n, BH, k, sub):
    print(f"[fused] cfg={cfg} n={n} BH={BH} k={k} sub={sub}", flush=True)
    x, st, plan = _scan_case(cfg, n, BH, sub)
    q = x["q"].to(DEV)
    sink, local = x["sink"], x["local"]
    ref = bp.sink_local_topk(st.scan(q, plan), k, sink, local)
    got = st.scan_topk(q, plan, k, sink, local)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)
    m = n + 3  # the local window partly past the scanned row
    ref = bp.sink_local_topk(st.scan(q, plan), k, sink, local, m=m)
    got = st.scan_topk(q, plan, k, sink, local, m=m)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


@pytest.mark.parametrize("cfg,n,BH,k,budget", [(5, 32768, 4, 512, None), (5, 32768, 3, 512, 92.0),
                                               (2, 16421, 2, 512, "rows"), (1, 16384, None, 128, None),
                                               (4, 20000, 2, 2048, 40.0), (2, 5000, 3, 300, 17.5), (2, 700, 1, 36, None),
                                               (2, 40000, 2, 512, "rows")])
def test_plan_scan_topk_equals_plan_then_scan_topk(cfg, n, BH, k, budget):
    """make_plan + scan_topk in one call: rows of at most 32768 tokens planned
    in the scan's prologue (C5 at the config budget and at 92 bits, per-row
    budgets, G = 1, 4, 7, kk = 0), longer rows through the plan kernel.  The
    indices and the plan's depths equal the two-call chain's, on two calls in a
    row."""
    print(f"[plan-scan-topk] cfg={cfg} n={n} BH={BH} k={k} budget={budget}", flush=True)
    x = W.config_inputs(cfg, seed=1, n=n, BH=BH)
    st = bp.PlaneStore(x["K"].to(DEV), keep_code=False)
    q, g = x["q"].to(DEV), x["g"].to(DEV)
    bh = q.shape[0]
    if budget == "rows":
        budget = torch.linspace(20.0, 100.0, bh, device=DEV)
    elif budget is None:
        budget = x["budget"]
    sink, local = x["sink"], x["local"]
    plan = bp.make_plan(g, budget)
    ref = st.scan_topk(q, plan, k, sink, local)
    for _ in range(2):
        got, t = st.plan_scan_topk(q, g, budget, k, sink, local, return_t=True)
        torch.testing.assert_close(got, ref, rtol=0, atol=0)
        torch.testing.assert_close(t, plan["t"], rtol=0, atol=0)
    assert torch.equal(st.plan_scan_topk(q, g, budget, k, sink, local), ref)


@pytest.mark.parametrize("cfg,n,BH,k,budget", [(5, 32768, 32, 512, None), (5, 32768, 24, 512, 92.0),
                                               (2, 16421, 24, 300, "rows"), (5, 32768, 4, 512, None),
                                               (1, 16384, None, 128, None), (4, 20000, 2, 2048, 40.0),
                                               (2, 700, 1, 36, None), (2, 40000, 2, 512, None)])
def test_plan_scan_topk_attention_equals_separate_calls(cfg, n, BH, k, budget):
    """Selection + attention in one call: the same workgroups for rows of at
    most 32768 tokens, k <= 512 and at least 96 query heads (C5's 128, 96 at 92
    bits and per-row budgets); the two calls otherwise (16 heads, G = 1,
    k = 2048, kk = 0, long rows).  The indices equal plan_scan_topk's and the
    outputs equal gather_attention's over them bit for bit, on two calls in a
    row."""
    print(f"[plan-scan-topk-attn] cfg={cfg} n={n} BH={BH} k={k} budget={budget}", flush=True)
    x = W.config_inputs(cfg, seed=2, n=n, BH=BH)
    K = x["K"].to(DEV)
    st = bp.PlaneStore(K, keep_code=False)
    q, g = x["q"].to(DEV), x["g"].to(DEV)
    bh = q.shape[0]
    if budget == "rows":
        budget = torch.linspace(24.0, 90.0, bh, device=DEV)
    elif budget is None:
        budget = x["budget"]
    sink, local = x["sink"], x["local"]
    Kb = K.to(torch.bfloat16).contiguous()
    V = W.synth_values(bh, n, seed=5, device=DEV)
    ref_idx = st.plan_scan_topk(q, g, budget, k, sink, local)
    ref_out = off.gather_attention(q, ref_idx, n, Kb, V, n)[0]
    for _ in range(2):
        idx, out = st.plan_scan_topk_attention(q, g, budget, k, Kb, V, sink, local)
        assert torch.equal(idx, ref_idx)
        assert torch.equal(out, ref_out)


@pytest.mark.parametrize("umax", [16, 48, 0, None])
def test_scan_topk_fused_plan_tables(umax):
    """Long rows: the candidate pass starts from the plan tables the sample
    pass left for rows whose plan fits the kernel's register layout, and builds
    its own for the others (a units bound below a row's plan, or per-row
    budgets of 24, 48 and 100 bits under one launch).  Equal to scan + top-k
    in every case."""
    print(f"[fused-tables] umax={umax}", flush=True)
    budget = torch.tensor([24.0, 48.0, 100.0], device=DEV) if umax is None else None
    x, st, plan = _scan_case(2, 70000, 3, budget=budget)
    if umax is not None:
        plan = dict(plan, units_max=umax)
    q = x["q"].to(DEV)
    ref = bp.sink_local_topk(st.scan(q, plan), 512, 4, 64)
    for _ in range(2):  # a repeated call (its workspace may hold the first call's tables)
        got = st.scan_topk(q, plan, 512, 4, 64)
        torch.testing.assert_close(got, ref, rtol=0, atol=0)


@pytest.mark.parametrize("n,k", [(600000, 40), (1000000, 64)])
def test_scan_topk_fused_small_k_long_rows(n, k):
    """The fused call with kk = k - 36 small against n (4 of 600000, 28 of
    10^6): the sample stride rounds up, the call equals scan + top-k."""
    print(f"[fused-small-k] n={n} k={k}", flush=True)
    x, st, plan = _scan_case(2, n, 1)
    q = x["q"].to(DEV)
    ref = bp.sink_local_topk(st.scan(q, plan), k, 4, 32)
    got = st.scan_topk(q, plan, k, 4, 32)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


def test_scan_topk_fused_host_resident():
    x, st, plan = _scan_case(2, 50000, 2)
    q = x["q"].to(DEV)
    ref = st.scan_topk(q, plan, 512)
    _, pl_dev, hp1 = off.host_mapped(st.planes_k)
    _, sc_dev, hp2 = off.host_mapped(st.scales_k)
    try:
        st.planes32, st.scales_k = pl_dev, sc_dev
        got = st.scan_topk(q, plan, 512)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, ref, rtol=0, atol=0)
    finally:
        off.free_host(hp1)
        off.free_host(hp2)


@pytest.mark.parametrize("cfg,n,sub,G", [(2, 50000, 32, None), (2, 65536, 64, None), (3, 33000, 32, None),
                                         (3, 100000, 64, None), (2, 40000, "whole", None), (1, 50000, 32, None),
                                         (2, 50000, 32, 8), (2, 20000, 64, None), (3, 4097, 32, None)])
def test_scan_host_resident_paired_tiles(cfg, n, sub, G):
    """Stores with superblocks of a multiple of 64 blocks (meant for mapped
    host memory) take the staged candidate pass (each workgroup copies four
    wave-tiles' 512-byte plane runs into LDS), 32-block superblocks the direct
    one: in host memory the scores and the fused top-k equal the HBM store's
    bit for bit, and the fused top-k equals the scores' top-k, for tile counts
    that are and are not a multiple of four, G = 8 and the whole-sequence
    layout."""
    print(f"[paired-host] cfg={cfg} n={n} sub={sub} G={G}", flush=True)
    s = math.ceil(n / 64) if sub == "whole" else sub
    x, st, plan = _scan_case(cfg, n, 2, sub=s)
    q = x["q"].to(DEV)
    if G is not None:
        q = torch.randn(2, G, q.shape[-1], generator=torch.Generator().manual_seed(3)).to(DEV)
    k = 512 if n > 32768 else 128
    ref_s = st.scan(q, plan).clone()
    ref_i = st.scan_topk(q, plan, k)
    _, pl_dev, hp1 = off.host_mapped(st.planes_k)
    _, sc_dev, hp2 = off.host_mapped(st.scales_k)
    try:
        st.planes32, st.scales_k = pl_dev, sc_dev
        got_s = st.scan(q, plan)
        got_i = st.scan_topk(q, plan, k)
        torch.cuda.synchronize()
        torch.testing.assert_close(got_s, ref_s, rtol=0, atol=0)
        torch.testing.assert_close(got_i, ref_i, rtol=0, atol=0)
        torch.testing.assert_close(got_i, bp.sink_local_topk(ref_s, k, 4, 32), rtol=0, atol=0)
    finally:
        off.free_host(hp1)
        off.free_host(hp2)


def test_scan_topk_fallback_pass_host_paired():
    """The fallback pass (direct tiles) after a staged first pass: a falling
    row in a host-mapped store of 64-block superblocks."""
    BH, d, n = 2, 128, 90000
    K = torch.zeros(BH, n, d)
    K[:, :, 0] = torch.linspace(1, -1, n)[None] * 3.0
    K[:, :, 1] = torch.randn(BH, n, generator=torch.Generator().manual_seed(5)) * 0.01
    bp.SUB = 64
    try:
        st = bp.PlaneStore(K.to(DEV))
    finally:
        bp.SUB = 16
    q = torch.zeros(BH, 4, d)
    q[:, :, 0] = 1.0
    q[:, 1::2, 1] = 1.0
    g = torch.ones(BH, d)
    g[:, 0] = 1000.0
    g[:, 1] = 10.0
    plan = bp.make_plan(g.to(DEV), 6.0)
    q = q.to(DEV)
    ref = bp.sink_local_topk(st.scan(q, plan), 512)
    _, pl_dev, hp1 = off.host_mapped(st.planes_k)
    _, sc_dev, hp2 = off.host_mapped(st.scales_k)
    try:
        st.planes32, st.scales_k = pl_dev, sc_dev
        got = st.scan_topk(q, plan, 512)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, ref, rtol=0, atol=0)
    finally:
        off.free_host(hp1)
        off.free_host(hp2)


@pytest.mark.parametrize("direction,n,BH,G", [(1.0, 90000, 2, 4), (-1.0, 90000, 2, 4), (1.0, 300000, 2, 4),
                                               (-1.0, 200000, 8, 4), (-1.0, 90000, 2, 8), (-1.0, 40000, 1, 3)])
def test_scan_topk_fallback_pass(direction, n, BH, G):
    """Fused path with scores falling (or rising) along the sequence: a falling
    row has its top kk inside the first sampled tile, so the tight threshold
    falls short and the row's finalize workgroup rescans it with T_lo; the
    result equals the unfused one.  The scores are coarse (few distinct
    values), so the rescan's candidates at the longer length outgrow one
    workgroup's LDS and are selected from the regions in place.  BH = 8 at
    n = 200000: eight rows of rescans; G = 8: the two-tile-row rescan."""
    print(f"[fused-fallback] direction={direction} n={n} BH={BH} G={G}", flush=True)
    d = 128
    K = torch.zeros(BH, n, d)
    K[:, :, 0] = torch.linspace(1, -1, n)[None] * 3.0 * direction
    K[:, :, 1] = torch.randn(BH, n) * 0.01
    st = bp.PlaneStore(K.to(DEV))
    q = torch.zeros(BH, G, d)
    q[:, :, 0] = 1.0
    q[:, 1::2, 1] = 1.0
    g = torch.ones(BH, d)
    g[:, 0] = 1000.0
    g[:, 1] = 10.0
    plan = bp.make_plan(g.to(DEV), 6.0)
    ref = bp.sink_local_topk(st.scan(q.to(DEV), plan), 512)
    got = st.scan_topk(q.to(DEV), plan, 512)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


@pytest.mark.parametrize("fallback", [False, True])
def test_scan_topk_stages_repeat(fallback):
    """The stage entry point: the stages run one by one on one workspace, and the
    candidate pass run again on its own over the state the last full call left
    (the way bench.py times it), give the fused call's indices -- also for rows
    whose tight threshold falls short, which the finalize stage rescans each
    time it runs."""
    print(f"[fused-stages] fallback={fallback}", flush=True)
    if fallback:
        BH, d, n = 2, 128, 90000
        K = torch.zeros(BH, n, d)
        K[:, :, 0] = torch.linspace(3, -3, n)[None]
        K[:, :, 1] = torch.randn(BH, n, generator=torch.Generator().manual_seed(3)) * 0.01
        st = bp.PlaneStore(K.to(DEV))
        q = torch.zeros(BH, 4, d)
        q[:, :, 0] = 1.0
        q[:, 1::2, 1] = 1.0
        g = torch.ones(BH, d)
        g[:, 0], g[:, 1] = 1000.0, 10.0
        q, plan = q.to(DEV), bp.make_plan(g.to(DEV), 6.0)
        sink, local = 4, 32
    else:
        x, st, plan = _scan_case(2, 100000, 2)
        q, sink, local = x["q"].to(DEV), x["sink"], x["local"]
    ref = bp.sink_local_topk(st.scan(q, plan), 512, sink, local)
    idx, ws = None, None
    for stage in (bp.STAGE_SAMPLE, bp.STAGE_SELECT, bp.STAGE_CANDIDATES, bp.STAGE_FINALIZE):
        idx, ws = st.scan_topk_stages(q, plan, 512, stage, ws, idx, sink, local)
    torch.testing.assert_close(idx, ref, rtol=0, atol=0)
    for rep in range(3):
        for _ in range(rep + 1):
            st.scan_topk_stages(q, plan, 512, bp.STAGE_CANDIDATES, ws, idx, sink, local)
        idx.fill_(-1)
        st.scan_topk_stages(q, plan, 512, bp.STAGE_FINALIZE, ws, idx, sink, local)
        torch.testing.assert_close(idx, ref, rtol=0, atol=0, msg=f"repeat {rep}")
    torch.testing.assert_close(st.scan_topk(q, plan, 512, sink, local), ref, rtol=0, atol=0)


def test_scan_topk_graph_replays():
    """The fused call captured in a HIP graph (as bench.py times it): every replay,
    with eager work and synchronisations between replays, equals the eager call."""
    print("[fused-graph]", flush=True)
    x, st, plan = _scan_case(2, 100000, 2)
    q = x["q"].to(DEV)
    ref = st.scan_topk(q, plan, 512, x["sink"], x["local"])
    torch.cuda.synchronize()
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        got = st.scan_topk(q, plan, 512, x["sink"], x["local"])
    for rep in range(4):
        gph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(got, ref, rtol=0, atol=0, msg=f"replay {rep}")
        eager = st.scan_topk(q, plan, 512, x["sink"], x["local"])  # eager work between replays
        torch.cuda.synchronize()
        torch.testing.assert_close(eager, ref, rtol=0, atol=0)


@pytest.mark.parametrize("n", [70000, 16000, 32768])
def test_scan_topk_all_ties(n):
    """Every score equal (all-zero keys): every element reaches the threshold,
    so a row has n candidates -- more than one workgroup's LDS holds at n =
    70000, when the selection reads the candidate regions in place, and at
    n = 32768, when the short-row selection from group maxima takes the whole
    row.  Ties go to the lowest index."""
    print(f"[fused-ties] n={n}", flush=True)
    BH, d = 2, 128
    st = bp.PlaneStore(torch.zeros(BH, n, d, device=DEV))
    q = torch.randn(BH, 4, d, generator=torch.Generator().manual_seed(5)).to(DEV)
    plan = bp.make_plan(torch.ones(BH, d, device=DEV), 12.0)
    ref = bp.sink_local_topk(st.scan(q, plan), 512)
    got = st.scan_topk(q, plan, 512)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)
    expect = O.sink_local_topk(np.zeros((BH * 4, n), np.float32), 512).reshape(BH, 4, 512)
    np.testing.assert_array_equal(got.cpu().numpy(), expect)


@pytest.mark.parametrize("n", [60000, 30000])
def test_scan_topk_adversarial_order(n):
    """Scores rising along the sequence: the sampled threshold admits far more
    candidates than usual (n = 60000), and on a short row the top-kk keys lie
    in the last groups, all of whose maxima reach T (n = 30000); the result
    stays exact."""
    BH, d = 1, 128
    K = torch.zeros(BH, n, d)
    K[0, :, 0] = torch.linspace(-1, 1, n) * 3.0
    K[0, :, 1] = torch.randn(n) * 0.01
    st = bp.PlaneStore(K.to(DEV))
    q = torch.zeros(BH, 2, d)
    q[0, :, 0] = 1.0
    q[0, 1, 1] = 1.0
    g = torch.ones(BH, d)
    g[0, 0] = 1000.0
    g[0, 1] = 10.0
    plan = bp.make_plan(g.to(DEV), 6.0)
    ref = bp.sink_local_topk(st.scan(q.to(DEV), plan), 512)
    got = st.scan_topk(q.to(DEV), plan, 512)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


# ----------------------------------------------------------------------------- attention over gathered rows
def _attn_close(got, ref):
    """fp32 kernel against the float64 oracle: summation order and exp rounding
    only (scores ~1, k <= 16384 terms)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bad = err > 1e-4 * np.abs(ref) + 2e-5
    assert not bad.any(), f"{int(bad.sum())} outputs off; max err {err.max():.3e}"


def _torch_gather_attn(q, K, V, idx):
    """The reference formula in plain torch fp32 on the CPU (scripts/B_kernel_bench.py:22-27)."""
    BH, G, k = idx.shape
    d = q.shape[-1]
    flat = idx.reshape(BH, G * k)
    Ks = torch.gather(K, 1, flat.unsqueeze(-1).expand(-1, -1, d)).view(BH, G, k, d).float()
    Vs = torch.gather(V, 1, flat.unsqueeze(-1).expand(-1, -1, d)).view(BH, G, k, d).float()
    s = torch.einsum("bgd,bgkd->bgk", q, Ks) * d ** -0.5
    return torch.einsum("bgk,bgkd->bgd", torch.softmax(s, -1), Vs)


@pytest.mark.parametrize("host", [False, True])
@pytest.mark.parametrize("G,k", [(4, 512), (7, 2048), (1, 3), (8, 2000)])
def test_gather_attention_matches_oracle(host, G, k):
    print(f"[gather_attention] host={host} G={G} k={k}", flush=True)
    rng = np.random.default_rng(17 + G)
    BH, n, nrec = 3, 12000, 5
    K = torch.randn(BH, n, 128).to(torch.bfloat16)
    V = torch.randn(BH, n, 128).to(torch.bfloat16)
    Kr = torch.randn(BH, nrec, 128).to(torch.bfloat16)
    Vr = torch.randn(BH, nrec, 128).to(torch.bfloat16)
    q = torch.randn(BH, G, 128)
    idx = rng.integers(0, min(n, 3 * k), size=(BH, G, k))          # heavy overlap across heads
    if k >= 8:
        idx[:, :, -3:] = n + rng.integers(0, nrec + 2, size=(BH, G, 3))
        idx[0, 0, 1] = -2
        idx[1, G - 1, :4] = idx[1, G - 1, 4]                        # a token selected 5 times by one head
    hps = []
    try:
        if host:
            _, Ksrc, h1 = off.host_mapped(K)
            _, Vsrc, h2 = off.host_mapped(V)
            hps = [h1, h2]
        else:
            Ksrc, Vsrc = K.to(DEV), V.to(DEV)
        it = torch.from_numpy(idx).to(DEV)
        ref, rnu = O.gather_attention(q.numpy(), idx, n, K.float().numpy(), V.float().numpy(),
                                      Kr.float().numpy(), Vr.float().numpy())
        # over the union (each distinct row once) and per selected position
        for unique in (True, False):
            out, nu = off.gather_attention(q.to(DEV), it, n, Ksrc, Vsrc, n, Kr.to(DEV), Vr.to(DEV), unique=unique)
            out2, _ = off.gather_attention(q.to(DEV), it, n, Ksrc, Vsrc, n, Kr.to(DEV), Vr.to(DEV), unique=unique)
            torch.cuda.synchronize()
            _attn_close(out.cpu().numpy(), ref)
            if unique:
                np.testing.assert_array_equal(nu.cpu().numpy(), rnu)
            else:
                assert nu is None
            assert torch.equal(out, out2), f"two calls on the same input differ (unique={unique})"
    finally:
        for h in hps:
            off.free_host(h)


@pytest.mark.parametrize("G,k", [(12, 2048), (16, 1100)])
def test_gather_attention_beyond_the_union_limits(G, k):
    """Per-position rows (device and mapped host) need neither G <= 8 nor
    G * k <= 16384 (12 x 2048 = 24576 positions, 16 query heads): the output
    is within tolerance of the float64 oracle, and the distinct-row counts
    (from the table in global memory there) equal the oracle's."""
    print(f"[gather_attention-big] G={G} k={k}", flush=True)
    rng = np.random.default_rng(5 + G)
    BH, n = 2, 9000
    K = torch.randn(BH, n, 128).to(torch.bfloat16)
    V = torch.randn(BH, n, 128).to(torch.bfloat16)
    q = torch.randn(BH, G, 128)
    idx = rng.integers(-1, n, size=(BH, G, k))
    ref, rnu = O.gather_attention(q.numpy(), idx, n, K.float().numpy(), V.float().numpy())
    it = torch.from_numpy(idx).to(DEV)
    out, nu = off.gather_attention(q.to(DEV), it, n, K.to(DEV), V.to(DEV), n)
    assert nu is None
    _attn_close(out.cpu().numpy(), ref)
    hps = []
    try:
        _, Ksrc, h1 = off.host_mapped(K)
        _, Vsrc, h2 = off.host_mapped(V)
        hps = [h1, h2]
        out2, nu2 = off.gather_attention(q.to(DEV), it, n, Ksrc, Vsrc, n)  # default: per position here
        torch.cuda.synchronize()
        assert nu2 is None
        _attn_close(out2.cpu().numpy(), ref)
        for _ in range(2):
            out3, nu3 = off.gather_attention(q.to(DEV), it, n, Ksrc, Vsrc, n, unique=True)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(nu3.cpu().numpy(), rnu)
            assert torch.equal(out3, out2)
    finally:
        for h in hps:
            off.free_host(h)


def test_gather_attn_dropin_equals_torch_formula():
    """gather_attn(q, Kc, Vc, idx) against the reference formula in torch fp32."""
    BH, G, n, k = 4, 4, 9000, 512
    gen = torch.Generator().manual_seed(4)
    Kc = torch.randn(BH, n, 128, generator=gen).to(torch.bfloat16)
    Vc = torch.randn(BH, n, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(BH, G, 128, generator=gen)
    idx = torch.randint(0, n, (BH, G, k), generator=gen)
    ref = _torch_gather_attn(q, Kc, Vc, idx)
    got = off.gather_attn(q.to(DEV), Kc.to(DEV), Vc.to(DEV), idx.to(DEV)).cpu()
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("layer", [0, 7])
def test_decode_layer_c5(layer):
    """One layer of the config-5 decode step at a reduced size: plan, fused scan +
    top-k and the fused gather + attention, against the oracle's attention over the
    unfused path's index set."""
    print(f"[decode-c5] layer={layer}", flush=True)
    x = W.config_inputs(5, device="cpu", n=8192, BH=4, layer=layer)
    K = x["K"]
    V = W.synth_values(4, 8192, seed=100 + layer)
    st = bp.PlaneStore(K.to(DEV))
    q = x["q"].to(DEV)
    plan = bp.make_plan(x["g"].to(DEV), x["budget"])
    idx = st.scan_topk(q, plan, x["k"], x["sink"], x["local"])
    ref_idx = bp.sink_local_topk(st.scan(q, plan), x["k"], x["sink"], x["local"])
    torch.testing.assert_close(idx, ref_idx, rtol=0, atol=0)
    out, _ = off.gather_attention(q, idx, 8192, K.to(DEV), V.to(DEV), 8192)
    out_u, nu = off.gather_attention(q, idx, 8192, K.to(DEV), V.to(DEV), 8192, unique=True)
    ref, rnu = O.gather_attention(x["q"].numpy(), idx.cpu().numpy(), 8192, K.float().numpy(), V.float().numpy())
    _attn_close(out.cpu().numpy(), ref)
    _attn_close(out_u.cpu().numpy(), ref)
    np.testing.assert_array_equal(nu.cpu().numpy(), rnu)


def test_decode_layer_graph_replays_equal_eager():
    """plan -> fused scan + top-k -> gather + attention captured in one HIP graph:
    every replay (with eager work and synchronisations between replays) equals
    the eager result bit for bit."""
    x = W.config_inputs(5, device="cpu", n=6000, BH=2, layer=3)
    K, q, g = x["K"].to(DEV), x["q"].to(DEV), x["g"].to(DEV)
    V = W.synth_values(2, 6000, seed=7).to(DEV)
    st = bp.PlaneStore(K)

    def layer():
        plan = bp.make_plan(g, x["budget"])
        idx = st.scan_topk(q, plan, x["k"], x["sink"], x["local"])
        return idx, off.gather_attention(q, idx, 6000, K, V, 6000)[0]

    ref_idx, ref_out = layer()
    torch.cuda.synchronize()
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        gi, go = layer()
    for rep in range(3):
        gi.zero_()
        go.zero_()
        gph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gi, ref_idx), f"replay {rep}: index sets differ"
        assert torch.equal(go, ref_out), f"replay {rep}: attention output differs"
        e_idx, e_out = layer()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(e_idx, ref_idx) and torch.equal(e_out, ref_out)


# ----------------------------------------------------------------------------- chan4 baseline store
@pytest.mark.parametrize("n,sub", [(1000, 16), (4097, 3), (700, 11)])
def test_chan4_store_bitexact(n, sub):
    print(f"[chan4-store] n={n} sub={sub}", flush=True)
    K = _keys(2, n, dtype=torch.bfloat16)
    code_r, sc_r = O.quantise_u4(K.float().numpy())
    old = bp.SUB
    bp.SUB = sub
    try:
        st = bp.Chan4Store(K.to(DEV))
        words = bp.pack_chan4(torch.from_numpy(code_r).to(DEV))
    finally:
        bp.SUB = old
    torch.cuda.synchronize()
    ref = O.pack_chan4(code_r, sub).view(np.int32)
    np.testing.assert_array_equal(st.code.cpu().numpy(), code_r)
    np.testing.assert_array_equal(st.chan_k.cpu().numpy(), ref)
    np.testing.assert_array_equal(words.cpu().numpy(), ref)
    _, sc_sb = O.to_superblocks(O.pack_planes(code_r), sc_r, sub)
    np.testing.assert_array_equal(st.scales_k.cpu().float().numpy(), sc_sb.astype(np.float16).astype(np.float32))


def test_channel_list_matches_oracle():
    rng = np.random.default_rng(2)
    active = rng.random((37, 128)) < 0.3
    active[0] = False
    active[1] = True
    act, nact = bp.channel_list(torch.from_numpy(active).to(DEV))
    ra, rn = O.channel_list(active)
    np.testing.assert_array_equal(act.cpu().numpy(), ra)
    np.testing.assert_array_equal(nact.cpu().numpy(), rn)


def _full_depth_plan(act, nact, D=128):
    """A plan dict whose only class is depth 4 over the listed channels (in list order)."""
    BH = act.shape[0]
    cls = torch.zeros(BH, 4, D, dtype=torch.int32, device=act.device)
    cls[:, 3] = act
    clsn = torch.zeros(BH, 4, dtype=torch.int32, device=act.device)
    clsn[:, 3] = nact
    return {"cls": cls, "clsn": clsn}


@pytest.mark.parametrize("G,n,r", [(4, 5000, 32), (7, 3000, 16), (1, 700, 128), (3, 2100, 0), (12, 3000, 32)])
def test_scan_chan4_matches_oracle_and_plane_scan(G, n, r):
    """Chan4 scores against the float64 oracle, and the plane scan of a plan with
    t = 4 on the same channels against the same oracle scores (the two stores hold
    the same codes; their kernels sum in different orders).  G = 12: both store
    methods run their heads in groups of at most 8, the block sub-range too."""
    print(f"[scan-chan4] G={G} n={n} r={r}", flush=True)
    BH = 3
    K = _keys(BH, n, dtype=torch.bfloat16, edge=False)
    q = torch.randn(BH, G, 128, generator=torch.Generator().manual_seed(G))
    Kd, qd = K.to(DEV), q.to(DEV)
    # SparQ-style lists: top-r channels of sum_g |q_g| (scripts/B_kernel_bench.py:54-56)
    active = torch.zeros(BH, 128, dtype=torch.bool)
    if r:
        active.scatter_(1, q.abs().sum(1).topk(r, -1).indices, True)
    act, nact = bp.channel_list(active.to(DEV))
    cs = bp.Chan4Store(Kd)
    got = cs.scan(qd, act, nact)
    ps = bp.PlaneStore(Kd)
    plane = ps.scan(qd, _full_depth_plan(act, nact))
    torch.cuda.synchronize()
    code, sc = O.quantise_u4(K.float().numpy())
    ref = O.scan_chan4(q.numpy(), code, sc, act.cpu().numpy(), nact.cpu().numpy())
    _scores_close(got.cpu().numpy(), ref)
    _scores_close(plane.cpu().numpy(), ref)
    # a block sub-range leaves the rest of `out` untouched
    out = torch.full_like(got, 7.0)
    cs.scan(qd, act, nact, out=out, blocks=(3, 9))
    torch.cuda.synchronize()
    assert torch.equal(out[..., 3 * 64:min(9 * 64, n)], got[..., 3 * 64:min(9 * 64, n)])
    assert (out[..., :3 * 64] == 7.0).all() and (out[..., 9 * 64:] == 7.0).all()


def test_scan_chan4_reference_matches_oracle():
    """scan_chan4_reference (the reference's dense formula, kernels/bitplane.py:365-370:
    full-depth dequantisation masked to the active channels, then q @ .T) against
    the float64 chan4 oracle, and against the chan4 kernel."""
    BH, G, n = 2, 4, 3000
    K = _keys(BH, n, dtype=torch.bfloat16, edge=False)
    q = torch.randn(BH, G, 128, generator=torch.Generator().manual_seed(9))
    active = torch.zeros(BH, 128, dtype=torch.bool)
    active.scatter_(1, q.abs().sum(1).topk(40, -1).indices, True)
    cs = bp.Chan4Store(K.to(DEV))
    got = bp.scan_chan4_reference(q.to(DEV), cs.code, cs.scales_blk, active.to(DEV))
    act, nact = bp.channel_list(active.to(DEV))
    code, sc = O.quantise_u4(K.float().numpy())
    ref = O.scan_chan4(q.numpy(), code, sc, act.cpu().numpy(), nact.cpu().numpy())
    _scores_close(got.cpu().numpy(), ref)
    _scores_close(cs.scan(q.to(DEV), act, nact).cpu().numpy(), ref)


def test_scan_chan4_host_resident():
    K = _keys(2, 9000, dtype=torch.bfloat16, edge=False)
    q = torch.randn(2, 4, 128).to(DEV)
    cs = bp.Chan4Store(K.to(DEV), keep_code=False)
    active = torch.zeros(2, 128, dtype=torch.bool, device=DEV)
    active[:, :32] = True                                   # a contiguous 32-channel (Loki / DS) store
    act, nact = bp.channel_list(active)
    ref = cs.scan(q, act, nact)
    _, ch_dev, h1 = off.host_mapped(cs.chan_k)
    _, sc_dev, h2 = off.host_mapped(cs.scales_k)
    try:
        cs.chan_k, cs.scales_k = ch_dev, sc_dev
        got = cs.scan(q, act, nact)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    finally:
        off.free_host(h1)
        off.free_host(h2)


# ----------------------------------------------------------------------------- KLT-rotated store
def _klt_case(n=6000, BH=2, G=7, seed=0):
    x = W.config_inputs(4, device="cpu", n=n, BH=BH, seed=seed)       # RoPE-rotated keys (config 4)
    gen = torch.Generator().manual_seed(seed + 1)
    Qcal = torch.randn(BH, 16 * G, 128, generator=gen)
    return x, Qcal


def test_klt_params_and_query_match_oracle():
    from fathom_amd import klt
    x, Qcal = _klt_case()
    K = x["K"].float()
    p = klt.klt_params(K.to(DEV), Qcal.to(DEV))
    r = O.klt_params(K.numpy(), Qcal.numpy())
    for b in range(K.shape[0]):
        # same components up to sign (distinct eigenvalues on this data)
        M = p["Vt"][b].cpu().double().numpy().T @ r["Vt"][b]
        np.testing.assert_allclose(np.abs(M), np.eye(128), atol=2e-4)
    np.testing.assert_allclose(p["lam"].cpu().numpy(), r["lam"], rtol=1e-5)
    np.testing.assert_allclose(p["mu"].cpu().numpy(), r["mu"], rtol=1e-5, atol=1e-6)
    q = x["q"]
    qr, gain = klt.klt_query(q.to(DEV), p["Vt"], p["lam"])
    rq, rg = O.klt_query(q.numpy(), p["Vt"].cpu().numpy(), p["lam"].cpu().numpy())
    np.testing.assert_allclose(qr.cpu().numpy(), rq, rtol=1e-5, atol=1e-5 * np.abs(rq).max())
    np.testing.assert_allclose(gain.cpu().numpy(), rg, rtol=1e-5, atol=1e-6 * np.abs(rg).max())


def test_klt_query_and_scan_more_than_8_heads():
    """G = 12 query heads: the query kernel's wider instance (up to 32 heads,
    the gains still summed in head order) and the rotated store's scan in head
    groups, against the oracle."""
    from fathom_amd import klt
    x, Qcal = _klt_case()
    Kd = x["K"].to(DEV)
    p = klt.klt_params(Kd, Qcal.to(DEV))
    st = klt.KLTPlaneStore(Kd, p)
    q = torch.randn(Kd.shape[0], 12, 128, generator=torch.Generator().manual_seed(12))
    qr, gain = st.query(q.to(DEV))
    rq, rg = O.klt_query(q.numpy(), p["Vt"].cpu().numpy(), p["lam"].cpu().numpy())
    np.testing.assert_allclose(qr.cpu().numpy(), rq, rtol=1e-5, atol=1e-5 * np.abs(rq).max())
    np.testing.assert_allclose(gain.cpu().numpy(), rg, rtol=1e-5, atol=1e-6 * np.abs(rg).max())
    plan = st.plan(q.to(DEV), 48.0)
    Kr = torch.matmul(Kd.float() - p["mu"][:, None, :], p["Vt"]).cpu()
    code_r, sc_r = O.quantise_u4(Kr.numpy())
    s = st.scan(q.to(DEV), plan)
    _scores_close(s.cpu().numpy(), O.scan_planes(qr.cpu().numpy(), code_r, sc_r, plan["t"].cpu().numpy()))


@pytest.mark.parametrize("budget", [40.0, 48.0, 80.0])
def test_klt_store_scan_and_topk(budget):
    """The rotated store: codes of the rotated keys bit-exact, scores within tolerance of
    the oracle scan over them with the rotated query, plan bit-exact from the kernel's
    gains, fused top-k equal to the unfused one."""
    print(f"[klt] budget={budget}", flush=True)
    from fathom_amd import klt
    x, Qcal = _klt_case()
    Kd = x["K"].to(DEV)
    p = klt.klt_params(Kd, Qcal.to(DEV))
    st = klt.KLTPlaneStore(Kd, p)
    Kr = torch.matmul(Kd.float() - p["mu"][:, None, :], p["Vt"]).cpu()    # the store's own rotation
    code_r, sc_r = O.quantise_u4(Kr.numpy())
    np.testing.assert_array_equal(st.code.cpu().numpy(), code_r)
    q = x["q"].to(DEV)
    qr, gain = st.query(q)
    plan = st.plan(q, budget)
    rp = O.make_plan(gain.cpu().numpy(), budget)
    np.testing.assert_array_equal(plan["t"].cpu().numpy(), rp["t"])
    s = st.scan(q, plan)
    ref = O.scan_planes(qr.cpu().numpy(), code_r, sc_r, rp["t"])
    _scores_close(s.cpu().numpy(), ref)
    idx = st.scan_topk(q, plan, 2048, 4, 32)
    torch.testing.assert_close(idx, bp.sink_local_topk(s, 2048, 4, 32), rtol=0, atol=0)


def test_klt_full_depth_within_quantisation_bound():
    """A full-depth KLT store (budget 512 = 4 bits on all 128 rotated channels)
    scores q.(K - mu) to within the 4-bit quantiser's bound: every rotated key
    value lies within a_be / 16 of its dequantised code (a_be the block scale of
    rotated channel e), so |score - q.(K - mu)| <= sum_e |qr_e| a_be / 16, with
    qr = q Vt.  The bound holds because Vt is orthonormal (q.(K - mu) = qr.Kr)
    and is met with a slack only for the fp16 rounding of the scales and fp32
    summation."""
    print("[klt] full depth bound", flush=True)
    from fathom_amd import klt
    x, Qcal = _klt_case()
    Kd = x["K"].to(DEV)
    p = klt.klt_params(Kd, Qcal.to(DEV))
    st = klt.KLTPlaneStore(Kd, p)
    q = x["q"].to(DEV)
    plan = st.plan(q, 512.0)
    assert (plan["t"] == 4).all()
    s = st.scan(q, plan).cpu().double().numpy()
    qr, _ = st.query(q)
    qr = qr.cpu().double().numpy()
    mu = p["mu"].cpu().double().numpy()
    Kc = x["K"].double().numpy() - mu[:, None, :]
    exact = np.einsum("bgd,bnd->bgn", x["q"].double().numpy(), Kc)
    a = st.scales_blk.cpu().double().numpy()                       # [BH, nblk, D]
    bound_blk = np.einsum("bgd,bkd->bgk", np.abs(qr), a) / 16.0
    bound = np.repeat(bound_blk, 64, axis=-1)[..., :x["n"]]
    err = np.abs(s - exact)
    slack = 2e-3 * bound + 1e-5 * np.abs(exact).max(-1, keepdims=True)
    assert (err <= bound + slack).all(), f"max err/bound {(err / bound).max():.4f}"
    assert (err / bound).max() > 0.3                                # the bound is not vacuous here


# ----------------------------------------------------------------------------- chunked copy/scan pipeline
@pytest.mark.parametrize("n,parts", [(300000, 4), (50001, 3), (9000, 1), (130000, 8)])
def test_stream_planes_equals_full_scan(n, parts):
    """Chunks copied on one stream and scanned on another give the scores of the full
    store bit for bit (the reference's PLANES_CHECK, with a zeroed staging store)."""
    print(f"[stream_planes] n={n} parts={parts}", flush=True)
    x = W.config_inputs(2, device="cpu", n=n, BH=2)
    nb = math.ceil(n / 64)
    old = bp.SUB
    bp.SUB = nb
    try:
        full = bp.PlaneStore(x["K"].to(DEV), keep_code=False)
    finally:
        bp.SUB = old
    q = x["q"].to(DEV)
    plan = bp.make_plan(x["g"].to(DEV), x["budget"])
    ref = full.scan(q, plan)
    hs, hps = off.host_store(full)
    try:
        stg = off.staging_store(full)
        got = off.stream_planes(hs, stg, q, plan, parts=parts)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        # unselected runs stay zero in the staging store
        t = plan["t"].cpu()
        for b in range(2):
            off_ch = (t[b] == 0).nonzero().flatten()[:3]
            for j in off_ch.tolist():
                assert int(stg.planes_k[b, 0, j].abs().sum().item()) == 0
    finally:
        for h in hps:
            off.free_host(h)


def test_stream_chan4_equals_full_scan():
    n = 70000
    K = _keys(2, n, dtype=torch.bfloat16, edge=False)
    q = torch.randn(2, 4, 128).to(DEV)
    old = bp.SUB
    bp.SUB = math.ceil(n / 64)
    try:
        full = bp.Chan4Store(K.to(DEV), keep_code=False)
    finally:
        bp.SUB = old
    active = torch.zeros(2, 128, dtype=torch.bool, device=DEV)
    active.scatter_(1, q.abs().sum(1).topk(32, -1).indices, True)
    act, nact = bp.channel_list(active)
    ref = full.scan(q, act, nact)
    hs, hps = off.host_store(full)
    try:
        stg = off.staging_store(full)
        got = off.stream_chan4(hs, stg, q, active, act, nact, parts=4)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    finally:
        for h in hps:
            off.free_host(h)
