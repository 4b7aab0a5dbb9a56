"""Helpers of the full-size GPU tests: float64 oracle scores of whole rows and
the end-to-end index-set criterion.

The oracle scores every token of a row from the keys themselves
(oracle.quantise_u4 + oracle.scan_planes), in chunks of whole 64-token blocks,
so the CPU memory stays small at n = 2^20.  A fused GPU selection is then
compared with the oracle's own top-kk of those float64 scores
(scripts/topk_bench.py:9-16 compares with torch.topk of the same scores; the
GPU's scores differ from the oracle's in their last bits, so equality is
asked for everywhere except at the selection boundary):

* every token of the symmetric difference lies at the boundary: its oracle
  score is within 2 * err of the oracle's kk-th largest score, where err is
  the row's largest |GPU score - oracle score| over all of its tokens;
* err itself is within the score tolerance (1e-3 relative + 1e-4 of the row's
  largest |score|);
* the sink and local positions follow in the reference's order.
"""
import numpy as np
import torch

from oracle import fathom_oracle as O

CHUNK = 1 << 16  # tokens per oracle chunk (a multiple of the 64-token block)


def oracle_row_scores(K, q, t, r, n, chunk=CHUNK):
    """float64 scores [G, n] of row r: K [BH, n, D] (any device, any float
    dtype), q [BH, G, D], t [BH, D] numpy."""
    # the quantiser and the scan treat channels independently, and channels
    # with t = 0 contribute nothing: only the plan's channels are quantised
    act = np.nonzero(np.asarray(t[r]) > 0)[0]
    qr = np.asarray(q[r:r + 1], np.float64)[:, :, act]
    tr = np.asarray(t[r:r + 1])[:, act]
    ai = torch.as_tensor(act, device=K.device)
    out = np.empty((qr.shape[1], n))
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        Kc = K[r, s:e].index_select(-1, ai).float().cpu().numpy()[None]
        code, sc = O.quantise_u4(Kc)
        out[:, s:e] = O.scan_planes(qr, code, sc, tr)[0]
    return out


def assert_row_set_parity(idx, s64, sgpu, k, sink, local, who=""):
    """idx [G, k] int64 (GPU selection of one row), s64 [G, n] float64 oracle
    scores, sgpu [G, n] the GPU's scores of the same row."""
    G, n = s64.shape
    kk = k - sink - local
    lo, hi = sink, max(n - local, 0)
    fixed = np.concatenate([np.arange(sink), np.arange(n - local, n)])
    ndiff = 0
    for g in range(G):
        s = s64[g]
        err = float(np.abs(sgpu[g].astype(np.float64) - s).max())
        amax = float(np.abs(s).max())
        tol = 1e-3 * np.abs(s) + 1e-4 * amax
        bad = np.abs(sgpu[g].astype(np.float64) - s) > tol
        assert not bad.any(), f"{who} head {g}: {int(bad.sum())} scores off the oracle (max err {err:.3e})"
        body = s[lo:hi]
        top = np.argpartition(-body, kk - 1)[:kk]
        kth = float(body[top].min())
        ref = set((top + lo).tolist())
        got = idx[g, :kk].tolist()
        assert len(set(got)) == kk, f"{who} head {g}: repeated indices"
        assert all(lo <= x < hi for x in got), f"{who} head {g}: selected a sink/local position"
        got = set(got)
        slack = 2.0 * err + 1e-12 * amax
        for x in got - ref:
            assert s[x] >= kth - slack, f"{who} head {g}: token {x} selected {s[x]:.9g} << kth {kth:.9g}"
        for x in ref - got:
            assert s[x] <= kth + slack, f"{who} head {g}: token {x} dropped {s[x]:.9g} >> kth {kth:.9g}"
        ndiff += len(got ^ ref)
        # the selection is sorted by (GPU score descending, index ascending)
        sel = idx[g, :kk]
        sv = sgpu[g][sel].astype(np.float64)
        assert (np.diff(sv) <= 0).all(), f"{who} head {g}: selection not in descending score order"
        np.testing.assert_array_equal(idx[g, kk:], fixed)
    return ndiff


def check_rows(K, q, t, idx, scores, k, sink, local, rows=None, label=""):
    """Runs the set criterion over rows (all by default); returns the total
    symmetric-difference size.  idx [BH, G, k], scores [BH, G, n] (torch)."""
    BH, G, n = scores.shape
    qn = q.cpu().numpy() if isinstance(q, torch.Tensor) else q
    tn = t.cpu().numpy() if isinstance(t, torch.Tensor) else t
    total = 0
    for r in (range(BH) if rows is None else rows):
        s64 = oracle_row_scores(K, qn, tn, r, n)
        d = assert_row_set_parity(idx[r].cpu().numpy(), s64, scores[r].cpu().numpy(), k, sink, local,
                                  who=f"{label} row {r}")
        total += d
        print(f"[e2e] {label} row {r}: set differences at the boundary: {d}", flush=True)
    return total
