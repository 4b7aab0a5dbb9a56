"""KLT-rotated bit-plane store and per-layer budget allocation, on MI355X.

For models without QK-norm (config 4's Qwen2.5) the reference scans bit planes
of the keys in a per-(layer, KV head) principal basis instead of the raw
channels ("planesK", scripts/R_ruler.py:63-64, 82-84):

* calibration (scripts/sketch.py:44-50): mu = mean of the calibration keys past
  the first SINK * 4 tokens, the principal directions of K - mu with variances
  lam, ordered by their calibration score variance mean((Q @ v)^2) * lam;
* store: bit planes of (K - mu) @ Vt, built once per layer;
* per decode step: qr = q @ Vt, plan gains sum_g qr^2 * lam, scores qr . keys.
  Scores differ from q . K by the per-query constant q . mu, so every top-k
  selection is unchanged by the centring.

The store is a PlaneStore of the rotated keys: the key rotation is a plain fp32
batched GEMM (rocBLAS through torch.matmul, store build only); the query
rotation and gains of each decode step are one gfx950 kernel
(fathom_klt_query); plan, scan and fused scan + top-k are the plane-store
kernels.  The calibration itself (an eigendecomposition per row, offline and
once per layer) runs in float64 on the CPU.

`allocate` is the reference's greedy per-layer budget allocation
(scripts/l4_final_alloc.py:143-154).
"""
import torch

from . import _lib
from .bitplane import D, PlaneStore, make_plan, _need_gpu, _ptr, _stream

SINK = 4  # scripts/sketch.py: calibration statistics skip the first SINK * 4 tokens


def klt_params(Kcal, Qcal, sink=SINK):
    """Per-row KLT basis from calibration keys Kcal [BH, n, D] and queries Qcal
    [BH, m, D] (the G heads' calibration queries of each KV head, flattened):
    returns dict(mu [BH, D], Vt [BH, D, D] (column e = basis vector e), lam [BH, D],
    w [BH, D]) float32 on Kcal's device, components ordered by descending
    calibration score variance w = mean((Qcal @ v)^2) * lam -- scripts/sketch.py:44-50.
    Eigenvectors are defined up to sign; scores do not depend on it."""
    dev = Kcal.device
    K = Kcal.detach().to("cpu", torch.float64)[:, sink * 4:]
    Q = Qcal.detach().to("cpu", torch.float64)
    mu = K.mean(1)
    Kc = K - mu[:, None]
    cov = Kc.transpose(1, 2) @ Kc / K.shape[1]
    lam, V = torch.linalg.eigh(cov)                      # ascending
    lam = lam.clamp_min(0.0)
    w = ((Q @ V) ** 2).mean(1) * lam
    order = w.argsort(-1, descending=True)
    V = torch.gather(V, 2, order[:, None, :].expand_as(V))
    lam = torch.gather(lam, 1, order)
    w = torch.gather(w, 1, order)
    f = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
    return {"mu": f(mu), "Vt": f(V), "lam": f(lam), "w": f(w)}


def klt_query(q, Vt, lam):
    """qr = q @ Vt [BH, G, D] and plan gains sum_g qr^2 * lam [BH, D] in one kernel
    (scripts/R_ruler.py:83)."""
    _need_gpu(q, Vt, lam)
    BH, G, d = q.shape
    qc = q.contiguous().float()
    Vc = Vt.contiguous().float()
    lc = lam.contiguous().float()
    qr = torch.empty(BH, G, d, device=q.device, dtype=torch.float32)
    gain = torch.empty(BH, d, device=q.device, dtype=torch.float32)
    _lib.call("fathom_klt_query", _ptr(qc), _ptr(Vc), _ptr(lc), BH, G, d, _ptr(qr), _ptr(gain), _stream(q.device))
    return qr, gain


class KLTPlaneStore(PlaneStore):
    """Bit-plane store of the KLT-rotated keys (K - mu) @ Vt (scripts/R_ruler.py:63-64).

    params: klt_params(...) output (mu, Vt, lam).  Methods take the unrotated
    query: plan(q, budget) plans from the rotated gains, scan / scan_topk rotate
    q before scanning (scores = qr . dequantised rotated keys, R_ruler.py:84)."""

    def __init__(self, K, params, scale_dtype=torch.float16, keep_code=True):
        _need_gpu(K)
        self.mu = params["mu"].to(K.device, torch.float32).contiguous()
        self.Vt = params["Vt"].to(K.device, torch.float32).contiguous()
        self.lam = params["lam"].to(K.device, torch.float32).contiguous()
        Kr = torch.matmul(K.float() - self.mu[:, None, :], self.Vt)
        super().__init__(Kr, scale_dtype, keep_code)

    def query(self, q):
        """(qr, gains) of query heads q [BH, G, D]."""
        return klt_query(q, self.Vt, self.lam)

    def plan(self, q, budget, bmax=4, iters=30):
        """make_plan over the rotated gains (R_ruler.py:83, waterfill_t)."""
        return make_plan(self.query(q)[1], budget, bmax, iters)

    def scan(self, q, plan, out=None, blocks=None):
        return super().scan(self.query(q)[0], plan, out, blocks)

    def scan_topk(self, q, plan, k, sink=4, local=32, m=None):
        return super().scan_topk(self.query(q)[0], plan, k, sink, local, m)


def allocate(err, budgets, mean_target):
    """Greedy per-layer budget allocation (scripts/l4_final_alloc.py:143-154): every
    layer starts at budgets[0]; while the mean budget is below mean_target, the layer
    whose next step buys the largest error drop per bit, (e_i - e_{i+1}) / (B_{i+1} -
    B_i), moves up one budget (the first such layer on ties); layers at the top
    budget stay.  err[B][L] (dict of dicts or of lists) is the calibration error of
    layer L at budget B.  Returns {L: budget}."""
    budgets = list(budgets)
    layers = list(err[budgets[0]].keys()) if isinstance(err[budgets[0]], dict) else list(range(len(err[budgets[0]])))
    idx = {L: 0 for L in layers}
    while sum(budgets[i] for i in idx.values()) / len(layers) < mean_target:
        best, best_l = -1.0, None
        for L in layers:
            i = idx[L]
            if i + 1 >= len(budgets):
                continue
            d = (err[budgets[i]][L] - err[budgets[i + 1]][L]) / (budgets[i + 1] - budgets[i])
            if d > best:
                best, best_l = d, L
        if best_l is None:
            break
        idx[best_l] += 1
    return {L: budgets[i] for L, i in idx.items()}


__all__ = ["klt_params", "klt_query", "KLTPlaneStore", "allocate", "D"]
