"""Benchmark of the key-scan hot path on one MI355X.

Workload (BASELINE.json metric "scanned tokens/s/GPU (scan+top-k) at 1M ctx"):
config 3's layer shape -- 8 KV heads, G = 4 query heads per KV head, n = 2^20
tokens, D = 128, "56-bit" plan (budget B = 48 code bits), k = 512 with 4 sink +
32 local -- on seeded synthetic bf16 keys.  One step = make_plan -> fused
scan + sink/local top-k -> exact attention over the selected rows (fused with
their union gather) over all 8 KV heads.  The unfused pair (scan writing scores,
then sink_local_topk) and the reference-structured union row gather are timed in
the same steps; the unfused pair must select the same indices.

`value` counts scanned token*heads per second of scan + top-k with the index
resident in HBM (n * BH / t_scan_topk, t_scan_topk the GPU time of one fused
call: 20 calls captured in one HIP graph, replayed for 30 ms before 10 timed
replays, checked equal to the eager call).
The roofline object is for the dominant kernel of that call, the candidate
pass (scan_wave_kernel<2, NS, 1>, NS the plan's slices of 16 units held in
registers), run on its own through the stage entry point
(20 launches in one HIP graph, events on the launching stream; algorithmic
bytes = bytes_planes), with the whole call's and the whole step's fractions
and the instruction-issue ceiling beside it.  The same step with the plane
index and the K/V rows in mapped pinned host memory (the scan reads over PCIe)
is reported under "host_resident", and config 5's full decode step (36 layers,
batch 4 x 8 KV heads, n = 32768, per-layer budgets) under "decode_step".  Every
index set measured (host-resident, copy-index, pipelined, graph replays) must
equal the HBM path's, or the run raises.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-host] [--no-cpu]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E
PCIE_PEAK_GBPS = 64.0         # PCIe 5.0 x16, per direction
HOST_SUB = 64                 # superblock of the host-resident store (a multiple of 64 blocks)
# The HBM store of the headline: the whole-sequence superblock layout (one
# superblock per row, SUB = n / 64 blocks), the layout of the reference's own
# 1M-token HBM scan benchmark (scripts/bench_scan_cfg.py:10).  Each active
# channel's scales are then one contiguous run, so the four wave-tiles of a
# candidate-pass workgroup share each 128-byte scale line.
SIMDS = 256 * 4               # MI355X: 256 CUs x 4 SIMDs
CLOCK_HZ = 2.4e9              # MI355X peak engine clock
VALU_CYCLES = 4               # a wave64 VALU instruction occupies a 16-lane SIMD 4 cycles


def cand_kernel(units_max):
    """The candidate pass's kernel for a plan bound (scan.hip launch_scan)."""
    nsl = -(-int(units_max) // 16)
    if units_max <= 0 or nsl > 4:
        return "scan_wave_kernel<2, 6, 4, false>"
    return f"scan_wave_kernel<2, {max(nsl, 2)}, 1, false>"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--n", type=int, default=None, help="override the token count (testing only)")
    ap.add_argument("--no-host", action="store_true", help="skip the host-resident measurement")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decode step")
    ap.add_argument("--stages-only", action="store_true", help="scan + top-k only (for profiling runs)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only config 5's 36-layer decode step (for rocprofv3 kernel traces of its stages)")
    ap.add_argument("--decode-form", choices=["all", "one"], default="all",
                    help="decode step forms timed: all three (default), or only the one-call form (for a kernel "
                         "trace of exactly the reported step)")
    ap.add_argument("--host-scan-only", action="store_true",
                    help="only the fused scan + top-k over the host-mapped store, --steps calls after --warmup "
                         "(for rocprofv3 --pmc runs of the zero-copy scan); raises if its indices differ from "
                         "the HBM store's")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the run, launch a plain fp32 device copy kernel of this many MiB 3 times "
                         "(the known-size kernel that scales rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class StageTimer:
    """HIP events on the current stream around each stage of each step."""

    def __init__(self, torch, names):
        self.torch = torch
        self.names = names
        self.ms = {n: [] for n in names}
        self.evs = []

    def step(self, fns):
        t = self.torch
        evs = [t.cuda.Event(enable_timing=True)]
        evs[0].record()
        out = {}
        for name in self.names:
            fns[name](out)
            e = t.cuda.Event(enable_timing=True)
            e.record()
            evs.append(e)
        self.evs.append(evs)
        return out

    def collect(self):
        for evs in self.evs:
            for name, (a, b) in zip(self.names, zip(evs[:-1], evs[1:])):
                self.ms[name].append(a.elapsed_time(b))
        self.evs = []
        return {n: statistics.mean(v) for n, v in self.ms.items()}


def run_regime(torch, bp, off, x, store, Ksrc, Vsrc, steps, warmup, stages_only=False):
    """Times one decode-step selection per step.  Stages: plan, the unfused scan
    (scores to HBM) and top-k over those scores (the reference's two calls), the
    fused scan+top-k (what the step uses), and the union row gather."""
    q, g = x["q"], x["g"]
    n, BH, k = x["n"], x["BH"], x["k"]

    def s_plan(o):
        o["plan"] = bp.make_plan(g, x["budget"])

    def s_scan(o):
        o["scores"] = store.scan(q, o["plan"])

    def s_topk(o):
        o["idx_unfused"] = bp.sink_local_topk(o["scores"], k, x["sink"], x["local"])

    def s_fused(o):
        o["idx"] = store.scan_topk(q, o["plan"], k, x["sink"], x["local"])

    def s_gather(o):
        o["rows"] = off.gather_union(o["idx"], n, Ksrc, Vsrc, n)

    def s_attn(o):
        o["attn"] = off.gather_attention(q, o["idx"], n, Ksrc, Vsrc, n)

    names = ["plan", "scan", "topk", "scan_topk"] + ([] if stages_only else ["gather", "attn"])
    fns = {"plan": s_plan, "scan": s_scan, "topk": s_topk, "scan_topk": s_fused, "gather": s_gather,
           "attn": s_attn}
    timer = StageTimer(torch, names)
    for _ in range(warmup):
        timer.step(fns)
    torch.cuda.synchronize()
    timer.evs = []
    t0 = time.perf_counter()
    for _ in range(steps):
        out = timer.step(fns)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    stage = timer.collect()
    plan = out["plan"]
    if not bool(torch.equal(out["idx"], out["idx_unfused"])):
        raise RuntimeError("fused scan+top-k disagrees with scan then sink_local_topk")
    scan_bytes = bp.bytes_planes(plan["t"], n)
    uniq = int(out["rows"][2].sum().item()) if "rows" in out else 0
    row_bytes = 2 * uniq * 128 * 2
    return {"stage_ms": stage, "wall_ms_per_step": wall, "scan_bytes": scan_bytes, "row_bytes": row_bytes,
            "unique_rows": uniq, "bits_per_token": scan_bytes * 8 / (n * BH),
            "nact_mean": float(plan["nact"].float().mean().item()), "idx": out["idx"], "plan": plan}


def run_copy_index(torch, bp, off, x, K_dev, V_dev, steps, warmup):
    """The host-resident step in the reference's published method (copy-index,
    scripts/B_e2e_offload_v2.py:190-197): the plane index in mapped host memory in
    the whole-sequence layout; per step the plan's runs are copied into an HBM
    staging store (PCIe), scanned there with the fused scan + top-k, and the
    selected K/V rows gathered zero-copy from host memory (PCIe)."""
    q, g, n, k = x["q"], x["g"], x["n"], x["k"]
    nb = -(-n // 64)
    old_sub = bp.SUB
    bp.SUB = nb
    try:
        full = bp.PlaneStore(x["K"], keep_code=False)
    finally:
        bp.SUB = old_sub
    hs, hps = off.host_store(full)
    stg = off.staging_store(full)
    del full
    torch.cuda.empty_cache()
    try:
        names = ["plan", "copy", "scan_topk", "attn"]
        fns = {"plan": lambda o: o.__setitem__("plan", bp.make_plan(g, x["budget"])),
               "copy": lambda o: off.copy_index(hs, stg, o["plan"]),
               "scan_topk": lambda o: o.__setitem__("idx", stg.scan_topk(q, o["plan"], k, x["sink"], x["local"])),
               "attn": lambda o: o.__setitem__("rows", off.gather_attention(q, o["idx"], n, K_dev, V_dev, n))}
        timer = StageTimer(torch, names)
        for _ in range(warmup):
            timer.step(fns)
        torch.cuda.synchronize()
        timer.evs = []
        for _ in range(steps):
            out = timer.step(fns)
        torch.cuda.synchronize()
        st = timer.collect()
        scan_bytes = bp.bytes_planes(out["plan"]["t"], n)
        uniq = int(out["rows"][1].sum().item())
        # the reference's pipelined form (B_e2e_offload_v2.py:116-130): the copy of chunk
        # c + 1 overlaps the scan of chunk c, then top-k over the scores
        pnames = ["plan", "stream_scan", "topk", "attn"]
        pfns = {"plan": fns["plan"],
                "stream_scan": lambda o: o.__setitem__("scores", off.stream_planes(hs, stg, q, o["plan"], parts=4)),
                "topk": lambda o: o.__setitem__("idx", bp.sink_local_topk(o["scores"], k, x["sink"], x["local"])),
                "attn": fns["attn"]}
        ptimer = StageTimer(torch, pnames)
        for _ in range(warmup):
            ptimer.step(pfns)
        torch.cuda.synchronize()
        ptimer.evs = []
        for _ in range(steps):
            pout = ptimer.step(pfns)
        torch.cuda.synchronize()
        pst = ptimer.collect()
        return {"stage_ms": st, "scan_bytes": scan_bytes, "row_bytes": 2 * uniq * 128 * 2, "unique_rows": uniq,
                "idx": out["idx"], "pipelined_stage_ms": pst, "pipelined_idx": pout["idx"]}
    finally:
        for h in hps:
            off.free_host(h)


def run_decode_step(torch, bp, off, W, dev, steps, warmup, forms="all"):
    """Config 5: one decode step of a 36-layer model with every layer's index and
    K/V rows in HBM -- per layer the plan (the layer's own budget), fused scan +
    top-k and exact attention over the selected rows.  As scripts/B_kernel_bench.py
    does, each stage (over all 36 layers) is captured in a HIP graph and timed
    around graph replays; the eager time per step is reported beside it.  The
    step is timed in three forms: one call per layer
    (PlaneStore.plan_scan_topk_attention: the plan made in the scan's
    prologue, the selection's workgroups going on to the attention; the
    reported step), two calls (plan_scan_topk, gather_attention) and the three
    separate calls make_plan, scan_topk, gather_attention.  Every replayed
    output must equal the eager one bit for bit, and the three forms must give
    the same indices and outputs."""
    c = W.CONFIGS[5]
    layers = []
    for L in range(c["layers"]):
        x = W.config_inputs(5, device=dev, layer=L)
        layers.append({"q": x["q"], "g": x["g"], "budget": x["budget"], "K": x["K"],
                       "V": W.synth_values(x["BH"], x["n"], seed=100 + L, device=dev),
                       "store": bp.PlaneStore(x["K"], keep_code=False)})
        del x
    torch.cuda.synchronize()
    n, BH, k, sink, local = c["n"], c["BH"], c["k"], c["sink"], c["local"]

    def timed(stages, st):
        # eager steps: reference outputs and the per-call (launch-bound) time
        for _ in range(warmup):
            for _, fn in stages:
                fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            for _, fn in stages:
                fn()
        e1.record()
        torch.cuda.synchronize()
        eager_ms = e0.elapsed_time(e1) / steps
        ref = [(s["idx"].clone(), s["out"].clone()) for s in st]
        graphs = []
        for _, fn in stages:
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                fn()
            graphs.append(gph)
        torch.cuda.synchronize()
        ms = {name: 0.0 for name, _ in stages}
        evs = []
        for it in range(warmup + steps):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(len(graphs) + 1)]
            e[0].record()
            for j, gph in enumerate(graphs):
                gph.replay()
                e[j + 1].record()
            if it >= warmup:
                evs.append(e)
        torch.cuda.synchronize()
        for e in evs:
            for j, (name, _) in enumerate(stages):
                ms[name] += e[j].elapsed_time(e[j + 1]) / steps
        for (ri, ro), s in zip(ref, st):
            if not (torch.equal(ri, s["idx"]) and torch.equal(ro, s["out"])):
                raise RuntimeError("decode step: a graph replay differs from the eager step")
        del graphs
        return ms, eager_ms

    fa = [{} for _ in layers]  # one call: plan, scan, top-k and attention

    def s_decode():
        for i, ly in enumerate(layers):
            fa[i]["idx"], fa[i]["out"] = ly["store"].plan_scan_topk_attention(ly["q"], ly["g"], ly["budget"], k, ly["K"],
                                                                              ly["V"], sink, local)

    fu = [{} for _ in layers]  # two calls: the plan made inside the scan, then gather_attention

    def s_plan_scan_topk():
        for i, ly in enumerate(layers):
            fu[i]["idx"] = ly["store"].plan_scan_topk(ly["q"], ly["g"], ly["budget"], k, sink, local)

    def s_attn_fu():
        for i, ly in enumerate(layers):
            fu[i]["out"] = off.gather_attention(ly["q"], fu[i]["idx"], n, ly["K"], ly["V"], n)[0]

    sp = [{} for _ in layers]  # the three separate calls

    def s_plan():
        for i, ly in enumerate(layers):
            sp[i]["plan"] = bp.make_plan(ly["g"], ly["budget"])

    def s_scan_topk():
        for i, ly in enumerate(layers):
            sp[i]["idx"] = ly["store"].scan_topk(ly["q"], sp[i]["plan"], k, sink, local)

    def s_attn_sp():
        for i, ly in enumerate(layers):
            sp[i]["out"] = off.gather_attention(ly["q"], sp[i]["idx"], n, ly["K"], ly["V"], n)[0]

    ms, eager_ms = timed([("plan_scan_topk_attention", s_decode)], fa)
    scan_bytes = sum(bp.bytes_planes(bp.make_plan(ly["g"], ly["budget"])["t"], n) for ly in layers)
    base = {"workload": c["name"], "layers": c["layers"], "BH": BH, "n": n, "k": k,
            "budgets": [float(b) for b in W.C5_BUDGETS], "timing": "HIP graph per stage over all layers",
            "ms_per_step": sum(ms.values()), "eager_ms_per_step": eager_ms,
            "form": "PlaneStore.plan_scan_topk_attention: one call per layer", "scan_bytes_per_step": scan_bytes}
    if forms == "one":
        del layers, fa
        torch.cuda.empty_cache()
        return base
    ms_fu, eager_fu = timed([("plan_scan_topk", s_plan_scan_topk), ("attn", s_attn_fu)], fu)
    ms_sp, eager_sp = timed([("plan", s_plan), ("scan_topk", s_scan_topk), ("attn", s_attn_sp)], sp)
    for a, b, c2 in zip(fa, fu, sp):
        if not all(torch.equal(a[key], b[key]) and torch.equal(a[key], c2[key]) for key in ("idx", "out")):
            raise RuntimeError("decode step: the one-call, two-call and three-call forms differ")
    del layers, fa, fu, sp
    torch.cuda.empty_cache()
    return {**base,
            "scanned_tokens_per_s": c["layers"] * BH * n / (ms_fu["plan_scan_topk"] * 1e-3),
            "scan_topk_GBps": scan_bytes / (ms_fu["plan_scan_topk"] * 1e-3) / 1e9,
            "two_calls": {"ms_per_step": sum(ms_fu.values()), "eager_ms_per_step": eager_fu,
                          "stage_ms_per_step": {s: round(v, 4) for s, v in ms_fu.items()}},
            "separate_calls": {"ms_per_step": sum(ms_sp.values()), "eager_ms_per_step": eager_sp,
                               "stage_ms_per_step": {s: round(v, 4) for s, v in ms_sp.items()}},
            "outputs_equal_across_forms": True}


def _graph_run(torch, fn, reps=20, warm_ms=30.0, timed=10):
    """GPU time of one fn() call: reps calls captured in one HIP graph, replayed
    back to back for at least warm_ms first (the clocks settle under load),
    then `timed` replays between events.  Returns (ms, the last call's output
    after the replays)."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        for _ in range(reps):
            r = fn()
    gph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(4):
            gph.replay()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(timed):
        gph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (timed * reps), r


def _graph_ms(torch, fn, reps=20):
    return _graph_run(torch, fn, reps)[0]


def run_kernel_table(torch, bp, W, dev):
    """The reference's scan-kernel comparison (paper/tables/tab_kernel.tex:6-10, measured
    by scripts/B_kernel_bench.py at n = 131072, batch 4 x 8 KV heads, G = 4): the
    bit-plane scan at B = 48 and the chan4 nibble scans over 16 (SparQ r = 16), 32
    and all 128 channels, each a single scan kernel, GB/s = algorithmic bytes / time."""
    x = W.config_inputs(2, device=dev, BH=32)
    q, n = x["q"], x["n"]
    ps = bp.PlaneStore(x["K"], keep_code=False)
    cs = bp.Chan4Store(x["K"], keep_code=False)
    plan = bp.make_plan(x["g"], x["budget"])
    out = torch.empty(32, x["G"], n, device=dev, dtype=torch.float32)
    rows = {}
    ms = _graph_ms(torch, lambda: ps.scan(q, plan, out=out))
    by = bp.bytes_planes(plan["t"], n)
    rows["planes_B48"] = {"ms": ms, "bytes": by, "GBps": by / (ms * 1e-3) / 1e9,
                          "bits_per_token": by * 8 / (n * 32)}
    abs_sum = q.abs().sum(1)
    for r in (16, 32, 128):
        active = torch.zeros(32, 128, dtype=torch.bool, device=dev)
        active.scatter_(1, abs_sum.topk(r, -1).indices, True)
        act, nact = bp.channel_list(active)
        ms = _graph_ms(torch, lambda: cs.scan(q, act, nact, out=out))
        by = bp.bytes_chan4(nact, n)
        rows[f"chan4_r{r}"] = {"ms": ms, "bytes": by, "GBps": by / (ms * 1e-3) / 1e9}
    del ps, cs, x
    torch.cuda.empty_cache()
    return {"shape": "n=131072, BH=32 (batch 4 x 8 KV heads), G=4, synthetic config-2 keys",
            "timing": "HIP graph of 20 launches, 10 replays after 30 ms of warm-up replays", "scans": rows,
            "reference_A100": "paper/tables/tab_kernel.tex:6-10 at 128k: Fathom 48 0.415 ms (102 GB/s); "
                              "16-ch / 32-ch / full 4-bit nibble scans 218 / 245 / 282 GB/s"}


def run_config4(torch, bp, W, dev):
    """Config 4 (Qwen2.5-7B layer: batch 2 x 4 KV heads, G = 7, n = 131072, RoPE keys
    with 8 outlier channels, k = 2048): plan + fused scan/top-k at budgets B = 40,
    48, 80 code bits (47 / 56 / 92 bits per token with scales) over the raw-channel
    store and the KLT-rotated store (calibrated on the layer's first 16384 keys and
    16 synthetic queries per head), each stage timed as a HIP graph."""
    from fathom_amd import klt
    x = W.config_inputs(4, device=dev)
    q, n, k = x["q"], x["n"], x["k"]
    gen = torch.Generator(device=dev).manual_seed(44)
    Qcal = torch.randn(x["BH"], 16 * x["G"], 128, generator=gen, device=dev)
    p = klt.klt_params(x["K"][:, :16384], Qcal)
    stores = {"raw": bp.PlaneStore(x["K"], keep_code=False), "klt": klt.KLTPlaneStore(x["K"], p, keep_code=False)}
    res = {}
    for name, st in stores.items():
        for B in x["budgets"]:
            if name == "raw":
                plan_fn = lambda: bp.make_plan(x["g"], B)
            else:
                plan_fn = lambda: st.plan(q, B)
            plan = plan_fn()
            ms_plan = _graph_ms(torch, plan_fn, reps=10)
            ms_st = _graph_ms(torch, lambda: st.scan_topk(q, plan, k, x["sink"], x["local"]), reps=10)
            by = bp.bytes_planes(plan["t"], n)
            res[f"{name}_B{int(B)}"] = {"plan_ms": ms_plan, "scan_topk_ms": ms_st,
                                        "bits_per_token": by * 8 / (n * x["BH"]),
                                        "scanned_tokens_per_s": n * x["BH"] / (ms_st * 1e-3)}
    del stores, x
    torch.cuda.empty_cache()
    return {"workload": W.CONFIGS[4]["name"], "k": 2048, "timing": "HIP graph of 10 launches, 10 replays after 30 ms of warm-up replays",
            "runs": res}


def run_wide_topk(torch, bp, store, x, plan, k=4096):
    """The fused call with k - sink - local above 2048 (the reference's
    torch.topk has no limit on k): the scores mode, then the wide selection
    (64-bit radix select over each score row, bitonic sort of the selected),
    timed as a HIP graph, beside the standalone sink_local_topk of the same
    scores.  The fused indices must equal sink_local_topk of the scan's scores."""
    q, sink, local = x["q"], x["sink"], x["local"]
    scores = store.scan(q, plan)
    ref = bp.sink_local_topk(scores, k, sink, local)
    idx = store.scan_topk(q, plan, k, sink, local)
    torch.cuda.synchronize()
    if not bool(torch.equal(idx, ref)):
        raise RuntimeError("wide fused scan+top-k disagrees with sink_local_topk of the scores")
    ms = _graph_ms(torch, lambda: store.scan_topk(q, plan, k, sink, local), reps=10)
    ms_sel = _graph_ms(torch, lambda: bp.sink_local_topk(scores, k, sink, local), reps=10)
    del scores
    torch.cuda.empty_cache()
    return {"k": k, "kk": k - sink - local, "rows": int(q.shape[0] * q.shape[1]), "n": int(store.n),
            "scan_topk_ms": ms, "sink_local_topk_ms": ms_sel, "equal_to_topk_of_scores": True,
            "timing": "HIP graph of 10 launches, 10 replays after 30 ms of warm-up replays"}


def run_stages(torch, bp, store, x, plan, ref_idx):
    """GPU time of each stage of the fused call (sample, select, candidates,
    finalize), each repeated over the state of one full call on one workspace
    (20 launches in one HIP graph).  The indices after the repeats must equal
    the fused call's."""
    q, k, sink, local = x["q"], x["k"], x["sink"], x["local"]
    idx, ws = store.scan_topk_stages(q, plan, k, bp.STAGE_ALL, sink=sink, local=local)
    torch.cuda.synchronize()
    if not bool(torch.equal(idx, ref_idx)):
        raise RuntimeError("stage entry point (all stages) disagrees with the fused call")
    ms = {}
    for name, stage in (("sample", bp.STAGE_SAMPLE), ("select", bp.STAGE_SELECT),
                        ("candidates", bp.STAGE_CANDIDATES), ("finalize", bp.STAGE_FINALIZE)):
        ms[name] = _graph_ms(torch, lambda stage=stage: store.scan_topk_stages(q, plan, k, stage, ws, idx, sink, local))
    idx.fill_(-1)
    store.scan_topk_stages(q, plan, k, bp.STAGE_CANDIDATES | bp.STAGE_FINALIZE, ws, idx, sink, local)
    torch.cuda.synchronize()
    if not bool(torch.equal(idx, ref_idx)):
        raise RuntimeError("repeated candidate passes changed the selected indices")
    return ms


def run_step_graph(torch, bp, off, x, store, K, V, ref_idx):
    """GPU time of one whole step (make_plan -> fused scan + top-k -> attention
    over the gathered rows, all 8 KV heads) as a HIP graph; its indices must
    equal the eager step's."""
    q = x["q"]
    box = {}

    def step():
        plan = bp.make_plan(x["g"], x["budget"])
        box["idx"] = store.scan_topk(q, plan, x["k"], x["sink"], x["local"])
        box["out"] = off.gather_attention(q, box["idx"], x["n"], K, V, x["n"])
        return box["idx"]

    ms, idx = _graph_run(torch, step)
    if not bool(torch.equal(idx, ref_idx)):
        raise RuntimeError("graph-replayed step disagrees with the eager step")
    return ms


def _profile_lines(name):
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return {}
    out = {}
    for line in open(p):
        if ":" in line and not line.startswith(("|", "#", " ")):
            key, val = line.split(":", 1)
            try:
                out[key.strip()] = float(val.split()[0])
            except (ValueError, IndexError):
                pass
    return out


def read_traffic():
    """HBM bytes per candidate-pass launch from rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE (committed summary, scaled by the copy-kernel calibration), or None."""
    return _profile_lines("scan_c3_candidate_hbm_traffic.md").get("traffic_bytes_per_launch")


def issue_ceiling(scan_bytes, blockrows, achieved):
    """Instruction-issue ceiling of the candidate pass from its committed
    rocprofv3 --pmc counts (per launch), no-overlap model: every VALU
    instruction other than an MFMA holds its SIMD VALU_CYCLES cycles (a wave64
    instruction on 16 lanes), each MFMA its measured busy cycles
    (SQ_VALU_MFMA_BUSY_CYCLES), and the two do not overlap; spread evenly over
    the chip's SIMDs at the peak clock, their sum is the shortest time the
    launch could take, and algorithmic bytes / that time the highest rate it
    could reach.  The overlapped bound (the larger of the two alone) is
    reported beside it."""
    c = _profile_lines("scan_c3_candidate_counters.md")
    if not {"SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_VALU_MFMA_BUSY_CYCLES"} <= set(c):
        return None
    valu, mfma = c["SQ_INSTS_VALU"], c["SQ_INSTS_MFMA"]
    valu_s = VALU_CYCLES * (valu - mfma) / (SIMDS * CLOCK_HZ)
    mfma_s = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMDS * CLOCK_HZ)
    t = valu_s + mfma_s
    ceil = scan_bytes / t / 1e9
    ceil_ov = scan_bytes / max(valu_s, mfma_s) / 1e9
    return {"model": "no overlap: non-MFMA VALU x 4 cycles + measured MFMA busy cycles, per SIMD at 2.4 GHz",
            "valu_per_block_row": valu / blockrows, "mfma_per_block_row": mfma / blockrows,
            "non_mfma_valu_per_block_row": (valu - mfma) / blockrows,
            "salu_per_block_row": c.get("SQ_INSTS_SALU", 0.0) / blockrows,
            "valu_issue_us": valu_s * 1e6, "mfma_busy_us": mfma_s * 1e6, "issue_us": t * 1e6,
            "ceiling_GBps": ceil, "frac_of_ceiling": achieved / ceil,
            "overlapped_ceiling_GBps": ceil_ov,
            "source": "profiles/scan_c3_candidate_counters.md (per-launch counts, C3 shape)"}


def cpu_baseline(W, x3):
    """The reference's torch CPU path (scripts/sketch.py:110-131 planes branch:
    water-filling plan + per-level qblock contraction; then the exact sink/local
    top-k with torch.topk), restated in oracle/sketch_torch.py, timed on the GPU
    run's own bytes: KV head 0 of the C3 inputs (keys, queries, variances copied
    back from the device) at all threads and, bounded, its first quarter at 1
    thread; C1 (not a GPU leg) generated on the CPU, at both."""
    import torch
    from oracle import sketch_torch as S

    threads_all = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        threads_all = min(threads_all, int(env))  # the box's CPU share
    saved = torch.get_num_threads()

    def timed(x, threads, reps=5, n=None):
        torch.set_num_threads(threads)
        K, q, var = x["K"][0].float(), x["q"][0].float(), x["var"][0].float()
        if n is not None:
            K = K[:n].contiguous()
        ts = []
        for _ in range(reps + 1):
            t0 = time.perf_counter()
            S.scan_topk(q, K, var, x["budget"], x["k"], x["sink"], x["local"])
            ts.append(time.perf_counter() - t0)
        med = statistics.median(ts[1:])
        return {"tokens_per_s": K.shape[0] / med, "s": med, "n": K.shape[0], "G": q.shape[0], "threads": threads}

    try:
        xc = {"K": x3["K"][:1].cpu(), "q": x3["q"][:1].cpu(), "var": x3["var"][:1].cpu(),
              "budget": x3["budget"], "k": x3["k"], "sink": x3["sink"], "local": x3["local"]}
        c3_all = timed(xc, threads_all)
        c3_one = timed(xc, 1, n=1 << 18)
        del xc
        x1 = W.config_inputs(1, device="cpu")
        c1_all, c1_one = timed(x1, threads_all), timed(x1, 1)
    finally:
        torch.set_num_threads(saved)
    return {"value": c3_all["tokens_per_s"], "unit": "token*heads/s", "cores": threads_all, "kind": "port",
            "sample": f"torch restatement of scripts/sketch.py:110-131 + torch.topk sink/local top-k on the GPU "
                      f"run's own bytes: KV head 0 of the C3 inputs (G={c3_all['G']} query heads x {c3_all['n']} "
                      f"tokens, copied back from the device), B=48, k=512, torch.set_num_threads({threads_all}) "
                      f"(os.cpu_count()={os.cpu_count()}), median of 5 after 1 warm-up: {c3_all['s']:.3f} s",
            "single_thread": dict(c3_one, sample="the same row's first 262144 tokens (a quarter), 1 thread"),
            "config1": {"all_threads": c1_all, "single_thread": c1_one,
                        "sample": "C1 generated on the CPU (C1 is not a GPU leg of this run)"}}


def calib_copy(torch, dev, mib):
    """torch's elementwise copy kernel, 3 launches that each read and write mib
    MiB: the known-size kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE."""
    if mib <= 0:
        return
    src = torch.ones(mib << 18, device=dev, dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log(f"[bench] calibration copy: 3 x {mib} MiB read + written")


def host_scan_only(torch, bp, off, x, store, steps, warmup):
    """The zero-copy fused scan + top-k alone, over a HOST_SUB-superblock store
    in mapped pinned host memory: the command profiled for the bytes the scan
    pulls over PCIe (FETCH_SIZE) against bytes_planes."""
    plan = bp.make_plan(x["g"], x["budget"])
    args = (x["q"], plan, x["k"], x["sink"], x["local"])
    ref = store.scan_topk(*args)
    bp.SUB = HOST_SUB
    try:
        hsrc = bp.PlaneStore(x["K"], keep_code=False)
    finally:
        bp.SUB = 16
    hps = []
    try:
        _, pl_dev, h = off.host_mapped(hsrc.planes_k)
        hps.append(h)
        _, sc_dev, h = off.host_mapped(hsrc.scales_k)
        hps.append(h)
        hstore = bp.PlaneStore.__new__(bp.PlaneStore)
        hstore.BH, hstore.n, hstore.nsb, hstore.sub = hsrc.BH, hsrc.n, hsrc.nsb, hsrc.sub
        hstore.planes32, hstore.scales_k = pl_dev, sc_dev
        del hsrc
        for _ in range(warmup):
            idx = hstore.scan_topk(*args)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            idx = hstore.scan_topk(*args)
        e1.record()
        torch.cuda.synchronize()
        if not bool(torch.equal(idx, ref)):
            raise RuntimeError("host-resident (zero-copy) index sets differ from the HBM path's")
        ms = e0.elapsed_time(e1) / steps
        by = bp.bytes_planes(plan["t"], x["n"])
        log(f"[bench] host-scan-only: {steps} fused calls, {ms:.4f} ms each, bytes_planes {by}, "
            f"{by / (ms * 1e-3) / 1e9:.1f} GB/s")
    finally:
        for h in hps:
            off.free_host(h)


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {a.gpus} is not supported in this build "
              "(the path shards by (batch, KV head) with no exchange; see the design notes)", file=sys.stderr)
        sys.exit(2)
    import torch

    from fathom_amd import bitplane as bp
    from fathom_amd import offload as off
    from fathom_amd import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.decode_only:
        decode = run_decode_step(torch, bp, off, W, dev, max(3, a.steps // 2), 2, a.decode_form)
        log(f"[bench] decode step (config 5): {json.dumps(decode)}")
        return
    t0 = time.perf_counter()
    x = W.config_inputs(a.config, device=dev, n=a.n)
    V = W.synth_values(x["BH"], x["n"], device=dev)
    bp.SUB = -(-x["n"] // bp.BLK)  # the whole-sequence layout (above)
    try:
        store = bp.PlaneStore(x["K"], keep_code=False)
    finally:
        bp.SUB = 16
    torch.cuda.synchronize()
    log(f"[bench] inputs + store built in {time.perf_counter() - t0:.1f} s: {W.CONFIGS[a.config]['name']}"
        f" n={x['n']}")

    if a.host_scan_only:
        host_scan_only(torch, bp, off, x, store, a.steps, a.warmup)
        calib_copy(torch, dev, a.calib_copy_mib)
        return
    hbm = run_regime(torch, bp, off, x, store, x["K"], V, a.steps, a.warmup, a.stages_only)
    st = hbm["stage_ms"]
    n, BH = x["n"], x["BH"]
    # the fused call's GPU time: 20 calls captured in one HIP graph (the stage
    # times above include the host's launch latency between stages); the
    # replayed result must equal the eager one
    scan_topk_ms, idx_graph = _graph_run(
        torch, lambda: store.scan_topk(x["q"], hbm["plan"], x["k"], x["sink"], x["local"]))
    if not bool(torch.equal(idx_graph, hbm["idx"])):
        raise RuntimeError("graph-replayed fused scan+top-k disagrees with the eager call")
    value = n * BH / (scan_topk_ms * 1e-3)
    scores = torch.empty(BH, x["G"], n, device=dev)
    scan_ms = _graph_ms(torch, lambda: store.scan(x["q"], hbm["plan"], out=scores))
    del scores
    fused_stage_ms = run_stages(torch, bp, store, x, hbm["plan"], hbm["idx"])
    cand_ms = fused_stage_ms["candidates"]
    achieved = hbm["scan_bytes"] / (cand_ms * 1e-3) / 1e9
    step_ms = None if a.stages_only else run_step_graph(torch, bp, off, x, store, x["K"], V, hbm["idx"])
    log(f"[bench] HBM: stages {json.dumps({k: round(v, 4) for k, v in st.items()})} ms, "
        f"{hbm['bits_per_token']:.2f} bits/token, fused (graph) {scan_topk_ms:.4f} ms, "
        f"fused stages {json.dumps({k: round(v, 4) for k, v in fused_stage_ms.items()})} ms, "
        f"candidate pass {achieved:.1f} GB/s, step (graph) {step_ms} ms")

    host = None
    if not a.no_host and not a.stages_only:
        hps = []
        try:
            # the host store in 64-block superblocks: the candidate pass then
            # stages four wave-tiles per workgroup, each unit one 512-byte run
            # in 16-byte pieces, the request size zero-copy reads need to
            # reach the link's rate
            bp.SUB = HOST_SUB
            try:
                hsrc = bp.PlaneStore(x["K"], keep_code=False)
            finally:
                bp.SUB = 16
            _, pl_dev, h = off.host_mapped(hsrc.planes_k)
            hps.append(h)
            _, sc_dev, h = off.host_mapped(hsrc.scales_k)
            hps.append(h)
            _, K_dev, h = off.host_mapped(x["K"])
            hps.append(h)
            _, V_dev, h = off.host_mapped(V)
            hps.append(h)
            hstore = bp.PlaneStore.__new__(bp.PlaneStore)
            hstore.BH, hstore.n, hstore.nsb, hstore.sub = hsrc.BH, hsrc.n, hsrc.nsb, hsrc.sub
            hstore.planes32, hstore.scales_k = pl_dev, sc_dev
            del hsrc
            hr = run_regime(torch, bp, off, x, hstore, K_dev, V_dev, max(3, a.steps // 2), 2)
            same = bool(torch.equal(hr["idx"], hbm["idx"]))
            if not same:
                raise RuntimeError("host-resident (zero-copy) index sets differ from the HBM path's")
            hs = hr["stage_ms"]
            tot = hs["plan"] + hs["scan_topk"] + hs["attn"]
            pcie_bytes = hr["scan_bytes"] + hr["row_bytes"]
            # measured pinned H2D copy rate, the reference's memcpy comparison
            src = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
            dst = torch.empty_like(src, device=dev)
            dst.copy_(src, non_blocking=True)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(4):
                dst.copy_(src, non_blocking=True)
            e1.record()
            torch.cuda.synchronize()
            h2d = 4 * src.numel() / (e0.elapsed_time(e1) * 1e-3) / 1e9
            # the reference's mixed regime (--index-hbm, scripts/B_e2e_offload_v2.py:25): the
            # plane index in HBM, only the selected K/V rows read over PCIe
            mx = run_regime(torch, bp, off, x, store, K_dev, V_dev, max(3, a.steps // 2), 2)
            if not bool(torch.equal(mx["idx"], hbm["idx"])):
                raise RuntimeError("index-in-HBM index sets differ from the HBM path's")
            ms_ = mx["stage_ms"]
            mx_tot = ms_["plan"] + ms_["scan_topk"] + ms_["attn"]
            index_hbm = {"what": "plane index in HBM, K/V rows in mapped pinned host memory read zero-copy "
                                 "(the reference's --index-hbm regime)",
                         "stage_ms": {k: round(v, 4) for k, v in ms_.items()}, "step_ms": mx_tot,
                         "pcie_bytes_per_step": mx["row_bytes"], "unique_rows": mx["unique_rows"],
                         "attn_pcie_GBps": mx["row_bytes"] / (ms_["attn"] * 1e-3) / 1e9,
                         "index_sets_equal_hbm": True}
            ci = run_copy_index(torch, bp, off, x, K_dev, V_dev, max(3, a.steps // 2), 2)
            if not bool(torch.equal(ci["idx"], hbm["idx"])):
                raise RuntimeError("copy-index index sets differ from the HBM path's")
            if not bool(torch.equal(ci["pipelined_idx"], hbm["idx"])):
                raise RuntimeError("pipelined (4-chunk) index sets differ from the HBM path's")
            cs = ci["stage_ms"]
            ci_tot = cs["plan"] + cs["copy"] + cs["scan_topk"] + cs["attn"]
            ci_bytes = ci["scan_bytes"] + ci["row_bytes"]
            copy_index = {"stage_ms": {k: round(v, 4) for k, v in cs.items()}, "step_ms": ci_tot,
                          "pcie_bytes_per_step": ci_bytes, "pcie_GBps_step": ci_bytes / (ci_tot * 1e-3) / 1e9,
                          "copy_GBps": ci["scan_bytes"] / (cs["copy"] * 1e-3) / 1e9,
                          "scanned_tokens_per_s": n * BH / ((cs["copy"] + cs["scan_topk"]) * 1e-3),
                          "roofline_pcie": {"peak": PCIE_PEAK_GBPS,
                                            "frac_step": ci_bytes / (ci_tot * 1e-3) / 1e9 / PCIE_PEAK_GBPS},
                          "index_sets_equal_hbm": bool(torch.equal(ci["idx"], hbm["idx"]))}
            if not (torch.equal(ci["idx"], hbm["idx"]) and torch.equal(ci["pipelined_idx"], hbm["idx"])):
                raise RuntimeError("copy-index (whole or pipelined) index sets differ from the HBM path's")
            ps = ci["pipelined_stage_ms"]
            p_tot = sum(ps.values())
            copy_index["pipelined_4_chunks"] = {
                "stage_ms": {k: round(v, 4) for k, v in ps.items()}, "step_ms": p_tot,
                "pcie_GBps_step": ci_bytes / (p_tot * 1e-3) / 1e9,
                "roofline_pcie": {"peak": PCIE_PEAK_GBPS, "frac_step": ci_bytes / (p_tot * 1e-3) / 1e9 / PCIE_PEAK_GBPS},
                "index_sets_equal_hbm": bool(torch.equal(ci["pipelined_idx"], hbm["idx"]))}
            host = {"stage_ms": {k: round(v, 4) for k, v in hs.items()}, "superblock_blocks": HOST_SUB,
                    "scanned_tokens_per_s": n * BH / (hs["scan_topk"] * 1e-3),
                    "step_ms": tot, "pcie_bytes_per_step": pcie_bytes,
                    "pcie_GBps_step": pcie_bytes / (tot * 1e-3) / 1e9,
                    "scan_pcie_GBps": hr["scan_bytes"] / (hs["scan"] * 1e-3) / 1e9,
                    "roofline_pcie": {"peak": PCIE_PEAK_GBPS, "frac_step": pcie_bytes / (tot * 1e-3) / 1e9 / PCIE_PEAK_GBPS,
                                      "frac_scan": hr["scan_bytes"] / (hs["scan"] * 1e-3) / 1e9 / PCIE_PEAK_GBPS},
                    "measured_h2d_memcpy_GBps": h2d, "unique_rows": hr["unique_rows"],
                    "index_sets_equal_hbm": same, "copy_index": copy_index, "index_hbm": index_hbm}
            log(f"[bench] host-resident: {json.dumps(host)}")
        finally:
            for h in hps:
                off.free_host(h)

    calib_copy(torch, dev, a.calib_copy_mib)

    wide = None
    if not a.no_decode and not a.stages_only and a.n is None:
        wide = run_wide_topk(torch, bp, store, x, hbm["plan"])
        log(f"[bench] wide top-k (C3, k = 4096): {json.dumps(wide)}")

    ktab = None
    if not a.no_decode and not a.stages_only and a.n is None:
        ktab = run_kernel_table(torch, bp, W, dev)
        log(f"[bench] kernel table: {json.dumps(ktab)}")

    cfg4 = None
    if not a.no_decode and not a.stages_only and a.n is None:
        cfg4 = run_config4(torch, bp, W, dev)
        log(f"[bench] config 4: {json.dumps(cfg4)}")

    decode = None
    if not a.no_decode and not a.stages_only and a.n is None:
        del store
        torch.cuda.empty_cache()
        decode = run_decode_step(torch, bp, off, W, dev, max(3, a.steps // 2), 2, a.decode_form)
        log(f"[bench] decode step (config 5): {json.dumps(decode)}")

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(W, x)
        log(f"[bench] cpu baseline: {json.dumps(cpu)}")

    rec = {
        "metric": "scanned tokens/s/GPU (scan+top-k) at 1M ctx",
        "value": value, "unit": "token*heads/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": st["plan"] + st["scan_topk"] + st.get("attn", 0.0), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 accumulate (f16 hi + lo split query weights, 21 significant bits, times exact f16 block scales)",
        "data": "synthetic (seeded lognormal-scaled keys, planted keys; no model weights)",
        "config": {"workload": W.CONFIGS[a.config]["name"] + ", index + rows in HBM", "BH": BH, "G": x["G"],
                   "n": n, "budget_bits": x["budget"], "k": x["k"], "sink": x["sink"], "local": x["local"],
                   "bits_per_token": round(hbm["bits_per_token"], 3), "parallelism": "single GPU",
                   "store_layout": "whole-sequence superblock (SUB = n/64), as the reference's 1M scan benchmark"},
        "stage_ms": {k: round(v, 4) for k, v in st.items()},
        "scan_topk_ms": scan_topk_ms,
        "scan_topk_timing": "20 fused calls captured in one HIP graph, 10 replays after 30 ms of warm-up replays (eager per-stage time: stage_ms)",
        "unfused_scan_plus_topk_ms": st["scan"] + st["topk"],
        "roofline": {"bound": "hbm",
                     "kernel": cand_kernel(hbm["plan"].get("units_max", 0)) + " (candidate pass of the fused scan + top-k)",
                     "achieved": achieved, "launch_ms": cand_ms, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": read_traffic(),
                     "algorithmic_bytes_per_launch": hbm["scan_bytes"],
                     "timing": "stage entry point, candidate pass alone, 20 launches in one HIP graph, 10 replays after 30 ms of warm-up replays",
                     "issue_ceiling": issue_ceiling(hbm["scan_bytes"], BH * -(-n // 64), achieved),
                     "whole_call": {"ms": scan_topk_ms, "GBps": hbm["scan_bytes"] / (scan_topk_ms * 1e-3) / 1e9,
                                    "frac": hbm["scan_bytes"] / (scan_topk_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                                    "stage_ms": {k: round(v, 5) for k, v in fused_stage_ms.items()}},
                     "step": None if step_ms is None else {
                         "ms": step_ms, "bytes": hbm["scan_bytes"] + hbm["row_bytes"],
                         "GBps": (hbm["scan_bytes"] + hbm["row_bytes"]) / (step_ms * 1e-3) / 1e9,
                         "frac": (hbm["scan_bytes"] + hbm["row_bytes"]) / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                         "what": "make_plan + fused scan/top-k + attention over the union-gathered rows, one HIP "
                                 "graph; bytes = plane/scale bytes + distinct K/V rows"},
                     "scores_mode_scan_ms": scan_ms},
        "roofline_pcie": None if host is None else {
            "what": "config 3 as written: plane index and K/V rows in mapped pinned host memory, the scan and "
                    "the row gather reading them zero-copy over PCIe",
            "bound": "pcie", "achieved": host["pcie_GBps_step"], "peak": PCIE_PEAK_GBPS, "unit": "GB/s",
            "frac": host["roofline_pcie"]["frac_step"], "frac_scan": host["roofline_pcie"]["frac_scan"],
            "step_ms": host["step_ms"], "scan_topk_ms": host["stage_ms"]["scan_topk"],
            "measured_h2d_memcpy_GBps": host["measured_h2d_memcpy_GBps"],
            "index_sets_equal_hbm": host["index_sets_equal_hbm"]},
        "host_resident": host,
        "decode_step": decode,
        "kernel_table": ktab,
        "config4": cfg4,
        "wide_topk": wide,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
