"""Torch restatement of the reference's CPU scorer, for the CPU baseline timing.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``fathom_amd``) imports it.
``bench.py``'s ``cpu_baseline`` leg times it on the host cores; ``tests/``
pin it against the numpy oracle (``oracle.fathom_oracle.sketch_planes_scores``,
itself pinned against the plane-store scan).

It follows scripts/sketch.py:110-131 (the ``planes:u4:B`` branch of
approx_scores): the per-query reverse water-filling plan by 30 bisection steps
of the water line on [-60, 60] (lines 116-121), then per depth level lvl the
keys re-quantised at lvl bits with the fp32 block absmax and the level's
channels contracted with one matrix product, ``out += (q * [t == lvl]) @
plane.T`` (lines 122-130); and the exact sink/local top-k of
kernels/bitplane.py:372-378 with torch.topk.  The reference runs the same
torch operations on its tensors' device; here they run on the CPU.
"""
import math

import torch

BLK = 64


def plan_depths(g, budget, bmax=4, iters=30):
    """t [D] int64: read depth per channel for the group-summed gain g [D]
    (scripts/sketch.py:116-121; torch.log2 / torch.round as the reference)."""
    lg = torch.log2(g.clamp_min(1e-30))
    bf = torch.full_like(g, float(bmax))
    lo = torch.tensor(-60.0)
    hi = torch.tensor(60.0)
    for _ in range(iters):
        mid = (lo + hi) / 2
        t = ((lg - mid) / 2).round().clamp(min=0).minimum(bf)
        over = t.sum() > budget
        lo = torch.where(over, mid, lo)
        hi = torch.where(over, hi, mid)
    return ((lg - hi) / 2).round().clamp(min=0).minimum(bf).to(torch.int64)


def planes_scores(q, k, var, budget, bmax=4, iters=30):
    """Approximate scores [G, n] float32 of one KV head at one decode position:
    q [G, D] group queries, k [n, D] float32 keys, var [D] calibration variance.
    Returns (scores, t)."""
    g = ((q ** 2) * var).sum(0)
    t = plan_depths(g, budget, bmax, iters)
    n, r = k.shape
    nb = math.ceil(n / BLK)
    cb = torch.cat([k, k.new_zeros(nb * BLK - n, r)]).view(nb, BLK, r)
    amax = cb.abs().amax(1, keepdim=True).clamp_min(1e-8)
    out = torch.zeros(q.shape[0], n)
    for lvl in range(1, bmax + 1):
        m = (t == lvl).to(q.dtype)
        if m.sum() == 0:
            continue
        half = 2.0 ** (lvl - 1)
        sc = amax / half
        plane = (((cb / sc).floor().clamp(-half, half - 1) + 0.5) * sc).view(-1, r)[:n]
        out += (q * m[None]) @ plane.T
    return out, t


def sink_local_topk(scores, k, sink=4, local=32):
    """Exact top-k with sinks and recent tokens forced in (kernels/bitplane.py:372-378):
    scores [..., n] -> int64 [..., k]; ties in torch.topk's order."""
    n = scores.shape[-1]
    s = scores.clone()
    s[..., :sink] = -math.inf
    s[..., max(n - local, 0):] = -math.inf
    top = s.topk(k - sink - local, -1).indices
    fixed = torch.cat([torch.arange(sink), torch.arange(n - local, n)]).expand(*top.shape[:-1], -1)
    return torch.cat([top, fixed], -1)


def scan_topk(q, k, var, budget, topk, sink=4, local=32):
    """The timed CPU path: planes_scores then sink_local_topk."""
    s, _ = planes_scores(q, k, var, budget)
    return sink_local_topk(s, topk, sink, local)
