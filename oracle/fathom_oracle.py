"""CPU oracle for the Fathom bit-plane key-scan path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``fathom_amd``) imports,
calls or links this module.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or,
for ``cpu_baseline``, as the timed CPU port of the reference's CPU scorer).

Every function restates one piece of the reference and cites the file:line
(relative to the reference repository root) whose behaviour it follows.  The
restatement is written from the reference's documented semantics; it is not a
translation of its Triton kernels.

Arithmetic conventions (the same ones the HIP kernels use, so that packed
planes, plans and index sets are bit-exact):

* quantiser: fp32 ``x / s`` correctly rounded, ``floor``, clamp to [-8, 7];
  block absmax rounded to the scale dtype with round-to-nearest-even.
* plan: ``lg = flog2(max(g, 1e-30))`` with the build's own log2 (``flog2``
  below: correctly rounded float32 log2 computed in float64 from exact IEEE
  add/mul/div only, so CPU and GPU agree bit for bit), then the reference's
  float32 bisection with round-half-even.
* top-k: order is (score descending, token index ascending); NaN ranks above
  +inf, -0.0 equals +0.0 (torch.topk's comparison semantics).

Parity status per function (how each is pinned; the tests hold the checks):

* quantise_u4 / dequant_planes: paper worked-example codes; prefix theorem
  (depth-t dequantisation == sketch.qblock t-bit quantiser, bit-exact).
* pack_planes / unpack_planes / to_superblocks: pure-Python bit brute force,
  round trip, permutation identity.
* flog2: float64 numpy log2 rounded to float32 (textbook), special values.
* make_plan: paper worked example (t, theta at B=8 and B=6); greedy reverse
  water-filling (sketch.waterfill) on tie-free inputs; invariants.
  The reference itself takes log2 from Triton ``tl.log2`` (GPU) or
  ``torch.log2`` (CPU); at rounding edges of ``(lg - mid)/2`` those may pick a
  different ``t`` than flog2 does: parity unpinned for that edge only.
* scan_planes: worked-example scores; per-bit (plane-word) formulation vs the
  dequantise-then-dot formulation; quantisation-error bound at depth 4.
* sink_local_topk: pure-Python sort by (-score, index) incl. ties/NaN/-0.0.
  The reference (torch.topk) leaves tie order unspecified: parity unpinned
  for ties, the build defines lowest index first.
* gather_rows / gather_union: pure-Python loops; dedup changes traffic only.
* pack_chan4: pure-Python nibble brute force, round trip through the words.
* channel_list: a stable argsort of ~active (numpy, the reference's own formula).
* scan_chan4: equals scan_planes with t = 4 on the listed channels and 0 elsewhere
  (the chan4 store reads every listed channel at full depth); the worked
  example's full-depth scores.
* gather_attention: closed forms (weights fixed by construction, duplicates,
  zero rows, recent-buffer rows), shift invariance, the one-hot limit.
* klt_params: orthonormal basis, lam = variance of the rotated calibration keys,
  score invariance q.(k - mu) = (q Vt).((k - mu) Vt), ordering by w.
* klt_query: score invariance under a random non-symmetric orthonormal basis
  (a transposed rotation fails it) and an explicit per-channel gain loop.
* qblock: equals the plane-prefix dequantisation at fp32 scales (bit-exact), and
  sketch_planes_scores equals the sum of per-level qblock contractions.
* allocate: hand-worked example; brute-force optimum on convex equal-step tables
  (where greedy marginal allocation is optimal).
* gather_runs / copy_index_runs: pure-Python word loops; the copy-index run
  list equals, slot by slot, the reference's offp/lenp/offs/lens formulas
  (hand-computed example in the tests), and scanning the staged copy equals
  scanning the full store (the reference's own PLANES_CHECK criterion).
* sketch_planes_scores (CPU baseline): equals scan_planes on fp32-scaled codes;
  oracle/sketch_torch.py (the torch restatement bench.py times) equals it.
"""
import math

import numpy as np

BLK = 64          # tokens per block (kernels/bitplane.py:19)
NEG_INF = np.float32(-np.inf)


# ----------------------------------------------------------------------------- quantiser
def _round_scale(amax, scale_dtype):
    """Round fp32 absmax to the scale dtype (RNE) and back to fp32."""
    if scale_dtype == "f16":
        with np.errstate(over="ignore"):
            return amax.astype(np.float16).astype(np.float32)
    if scale_dtype == "f32":
        return amax.astype(np.float32)
    if scale_dtype == "bf16":
        return _to_bf16_f32(amax)
    raise ValueError(scale_dtype)


def _to_bf16_f32(x):
    """float32 -> bfloat16 (round to nearest even) -> float32, NaN kept quiet."""
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    bias = np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    r = ((u + bias) >> np.uint64(16)) << np.uint64(16)
    r = np.where(np.isnan(x), (u | np.uint64(0x400000)) & np.uint64(0xFFFF0000), r)
    return r.astype(np.uint32).view(np.float32)


def quantise_u4(K, scale_dtype="f16"):
    """K [..., n, D] float -> (codes uint8 [..., n, D] in [0, 16),
    scales [..., nblk, D] float32 holding the scale-dtype-rounded block absmax).

    Follows kernels/bitplane.py:23-32: pad n to a multiple of 64 with zeros,
    amax = max |x| per (block, channel), clamp_min(1e-8), round to the scale
    dtype, s = amax / 8, code = clamp(floor(x / s), -8, 7) + 8.  NaN codes
    (0/0, NaN input) become 0, as torch's float->uint8 cast gives on x86 and
    CUDA.  NaN inputs propagate into amax as torch.amax does.
    """
    K = np.asarray(K, np.float32)
    *lead, n, d = K.shape
    nb = -(-n // BLK)
    pad = nb * BLK - n
    cb = np.concatenate([K, np.zeros((*lead, pad, d), np.float32)], -2).reshape(*lead, nb, BLK, d)
    with np.errstate(invalid="ignore", divide="ignore"):
        amax = np.abs(cb).max(-2, keepdims=True)          # NaN-propagating like torch.amax
        amax = np.where(np.isnan(amax), amax, np.maximum(amax, np.float32(1e-8)))
        amax = _round_scale(amax, scale_dtype)
        s = amax / np.float32(8)
        v = np.floor(cb / s)
        code = np.clip(v, -8, 7) + 8
        code = np.where(np.isnan(code), 0, code).astype(np.uint8)
    return code.reshape(*lead, nb * BLK, d)[..., :n, :], amax[..., 0, :].astype(np.float32)


def dequant_planes(code, scales, t):
    """Value of the top-t planes: [..., n, D] float32 (kernels/bitplane.py:34-42).

    val = ((code >> (4 - t)) + 0.5 - 2^(t-1)) * a / 2^(t-1), 0 where t == 0.
    ``t`` is a scalar or an int array [D] broadcast over tokens."""
    code = np.asarray(code)
    scales = np.asarray(scales, np.float32)
    n = code.shape[-2]
    nb = -(-n // BLK)
    pad = nb * BLK - n
    cb = np.concatenate([code, np.zeros((*code.shape[:-2], pad, code.shape[-1]), code.dtype)], -2)
    cb = cb.reshape(*code.shape[:-2], nb, BLK, -1).astype(np.int64)
    t = np.asarray(t, np.int64)
    half = np.float32(2.0) ** (t.astype(np.float32) - np.float32(1))
    ct = (cb >> (4 - t)).astype(np.float32)
    val = (ct + np.float32(0.5) - half) * scales[..., :, None, :] / half
    val = np.where(t > 0, val, np.float32(0)).astype(np.float32)
    return val.reshape(*code.shape[:-2], nb * BLK, -1)[..., :n, :]


# ----------------------------------------------------------------------------- bit planes
def pack_planes(code):
    """codes uint8 [..., n, D] -> logical planes uint64 [..., nblk, D, 4]
    (kernels/bitplane.py:44-50): bit i of planes[..., b, j, p] is bit p
    (0 = MSB of the 4-bit code) of token 64 b + i.  Tokens past n (the tail
    of the last block) are packed as code 0, i.e. all four bits clear; the
    codes quantise_u4 computed for its own zero padding are cropped before
    packing, so they never reach the planes."""
    code = np.asarray(code, np.uint8)
    *lead, n, d = code.shape
    nb = -(-n // BLK)
    pad = nb * BLK - n
    cb = np.concatenate([code, np.zeros((*lead, pad, d), np.uint8)], -2).reshape(*lead, nb, BLK, d)
    cb = cb.astype(np.uint64)
    lane = np.arange(BLK, dtype=np.uint64).reshape(BLK, 1)
    planes = []
    for p in range(4):
        bits = (cb >> np.uint64(3 - p)) & np.uint64(1)
        planes.append(np.bitwise_or.reduce(bits << lane, axis=-2))
    return np.stack(planes, -1)


def unpack_planes(planes, n):
    """Inverse of pack_planes: uint64 [..., nblk, D, 4] -> codes uint8 [..., n, D]
    (kernels/bitplane.py:52-58)."""
    planes = np.asarray(planes).view(np.uint64) if np.asarray(planes).dtype == np.int64 else np.asarray(planes, np.uint64)
    *lead, nb, d, _ = planes.shape
    lane = np.arange(BLK, dtype=np.uint64).reshape(BLK, 1, 1)
    bits = (planes[..., None, :, :] >> lane) & np.uint64(1)       # [..., nb, 64, d, 4]
    code = sum(bits[..., p] << np.uint64(3 - p) for p in range(4))
    return code.reshape(*lead, nb * BLK, d)[..., :n, :].astype(np.uint8)


def to_superblocks(planes, scales, sub):
    """Logical [..., nblk, D, 4] / [..., nblk, D] -> kernel order
    [..., nsb, D, 4, sub] / [..., nsb, D, sub], zero padded to whole
    superblocks (kernels/bitplane.py:60-65)."""
    planes = np.asarray(planes)
    scales = np.asarray(scales)
    *lead, nb, d, _ = planes.shape
    nsb = -(-nb // sub)
    pad = nsb * sub - nb
    pl = np.concatenate([planes, np.zeros((*lead, pad, d, 4), planes.dtype)], -3)
    pl = pl.reshape(*lead, nsb, sub, d, 4)
    L = len(lead)
    pl = np.ascontiguousarray(np.transpose(pl, (*range(L), L, L + 2, L + 3, L + 1)))
    sc = np.concatenate([scales, np.zeros((*lead, pad, d), scales.dtype)], -2).reshape(*lead, nsb, sub, d)
    sc = np.ascontiguousarray(np.swapaxes(sc, -1, -2))
    return pl, sc


def bytes_planes(t, n):
    """Bytes a scan moves for plans t [BH, D] over n tokens: per 64-token block
    8 bytes per plane read + 2 bytes per active channel's fp16 scale
    (kernels/bitplane.py:76-78)."""
    t = np.asarray(t, np.float64)
    nb = -(-n // BLK)
    return float(((t.sum(-1) * 8 + (t > 0).sum(-1) * 2) * nb).sum())


# ----------------------------------------------------------------------------- chan4 baseline store
def pack_chan4(code, sub):
    """codes uint8 [..., n, D] -> channel-major 4-bit store uint32 [..., nsb, D, sub, 8]
    (kernels/bitplane.py:67-74): word m of (channel j, block b) holds the codes of
    tokens 8m..8m+7 of the block, nibble k (bits 4k..4k+3) = token 8m + k; tokens
    past n and blocks past nblk are code 0."""
    code = np.asarray(code, np.uint8)
    *lead, n, d = code.shape
    nb = -(-n // BLK)
    nsb = -(-nb // sub)
    pad = nsb * sub * BLK - n
    cb = np.concatenate([code, np.zeros((*lead, pad, d), np.uint8)], -2)
    cb = cb.reshape(*lead, nsb, sub, 8, 8, d).astype(np.uint64)       # [.., nsb, sub, m, k, d]
    shift = (4 * np.arange(8, dtype=np.uint64)).reshape(8, 1)
    words = np.bitwise_or.reduce(cb << shift, axis=-2).astype(np.uint32)   # [.., nsb, sub, m, d]
    nl = len(lead)
    return np.ascontiguousarray(np.moveaxis(words, -1, nl + 1))       # [.., nsb, d, sub, m]


def channel_list(active):
    """active bool [BH, D] -> (act [BH, D] int32: listed channels first, ascending,
    then the others, ascending; nact [BH]) (kernels/bitplane.py:128-132)."""
    active = np.asarray(active, bool)
    act = np.stack([np.concatenate([np.flatnonzero(r), np.flatnonzero(~r)]) for r in active]).astype(np.int32)
    return act, active.sum(-1).astype(np.int32)


def scan_chan4(q, code, scales, act, nact):
    """Scores of the chan4 scan (kernels/bitplane.py:175-198, 348-353; reference
    semantics scan_chan4_reference :365-370): sum over the first nact listed channels
    of q_j * a_bj * (c - 7.5) / 8, i.e. the full-depth dequantised code.  float64,
    [BH, G, n]."""
    q = np.asarray(q, np.float64)
    BH, G, D = q.shape
    out = []
    for b in range(BH):
        mask = np.zeros(D)
        mask[np.asarray(act[b][: int(nact[b])], np.int64)] = 1.0
        val = dequant_planes(code[b], scales[b], 4).astype(np.float64) * mask[None]
        out.append(q[b] @ val.T)
    return np.stack(out)


def bytes_chan4(nact, n):
    """(32 + 2) bytes per listed channel and 64-token block (kernels/bitplane.py:79-80)."""
    nb = -(-n // BLK)
    return float(np.sum(np.asarray(nact, np.float64) * 34 * nb))


# ----------------------------------------------------------------------------- KLT store, budget allocation
def klt_params(Kcal, Qcal, sink=4):
    """Per-row KLT basis (scripts/sketch.py:44-50): mu = mean of Kcal[:, sink*4:],
    SVD of the centred keys, lam = S^2 / N, Vt = V (columns = components), ordered by
    descending w = mean((Qcal @ Vt)^2) * lam.  float64.  Returns dict(mu, Vt, lam, w)."""
    K = np.asarray(Kcal, np.float64)[:, sink * 4:]
    Q = np.asarray(Qcal, np.float64)
    out = {"mu": [], "Vt": [], "lam": [], "w": []}
    for b in range(K.shape[0]):
        mu = K[b].mean(0)
        _, S, Vh = np.linalg.svd(K[b] - mu, full_matrices=False)
        lam = S ** 2 / K.shape[1]
        Vt = Vh.T
        w = ((Q[b] @ Vt) ** 2).mean(0) * lam
        order = np.argsort(-w, kind="stable")
        out["mu"].append(mu)
        out["Vt"].append(Vt[:, order])
        out["lam"].append(lam[order])
        out["w"].append(w[order])
    return {k: np.stack(v) for k, v in out.items()}


def klt_query(q, Vt, lam):
    """qr = q @ Vt and plan gains sum_g qr^2 * lam (scripts/R_ruler.py:83), float64."""
    qr = np.einsum("bgd,bde->bge", np.asarray(q, np.float64), np.asarray(Vt, np.float64))
    return qr, ((qr ** 2) * np.asarray(lam, np.float64)[:, None, :]).sum(1)


def allocate(err, budgets, mean_target):
    """Greedy per-layer allocation (scripts/l4_final_alloc.py:143-154): from budgets[0]
    everywhere, repeatedly move up the layer with the largest (e_i - e_{i+1}) /
    (B_{i+1} - B_i) (first on ties) until the mean budget reaches mean_target or no
    layer can move.  err: {budget: [error per layer]}.  Returns [budget per layer]."""
    budgets = list(budgets)
    nl = len(err[budgets[0]])
    idx = [0] * nl
    while sum(budgets[i] for i in idx) / nl < mean_target:
        slopes = [((err[budgets[idx[L]]][L] - err[budgets[idx[L] + 1]][L]) / (budgets[idx[L] + 1] - budgets[idx[L]]), L)
                  for L in range(nl) if idx[L] + 1 < len(budgets)]
        slopes = [(d, L) for d, L in slopes if d > -1.0]
        if not slopes:
            break
        best = max(d for d, _ in slopes)
        idx[min(L for d, L in slopes if d == best)] += 1
    return [budgets[i] for i in idx]


# ----------------------------------------------------------------------------- log2
_INV_ODD = [1.0 / (2 * k + 1) for k in range(12)]     # correctly rounded doubles
_SQRT2 = 1.4142135623730951                            # nearest double to sqrt(2)
_LOG2E = 1.4426950408889634                            # nearest double to 1/ln(2)


def flog2(x):
    """float32 log2 used by the plan, bit-identical to the HIP kernel's.

    x = m * 2^e with m folded into (1/sqrt2, sqrt2]; ln m = 2 atanh(s),
    s = (m-1)/(m+1), by its odd series to z^11 (z = s^2) in Horner form;
    log2 x = e + ln m * log2(e), all in float64 with separate (unfused)
    IEEE operations, then rounded to float32.  Domain: positive normal
    floats, +inf and NaN (the plan clamps g to >= 1e-30 first)."""
    x = np.asarray(x, np.float32)
    bits = x.view(np.uint32).astype(np.int64)
    e = ((bits >> 23) & 0xFF) - 127
    m = ((bits & 0x7FFFFF) | 0x800000).astype(np.float64) / 8388608.0
    big = m > _SQRT2
    m = np.where(big, m * 0.5, m)
    e = np.where(big, e + 1, e)
    s = (m - 1.0) / (m + 1.0)
    z = s * s
    p = np.full_like(z, _INV_ODD[11])
    for k in range(10, -1, -1):
        p = p * z
        p = p + _INV_ODD[k]
    ln_m = (2.0 * s) * p
    r = e.astype(np.float64) + ln_m * _LOG2E
    out = r.astype(np.float32)
    out = np.where(np.isinf(x) & (x > 0), np.float32(np.inf), out)
    out = np.where(np.isnan(x), np.float32(np.nan), out)
    return out.astype(np.float32)


# ----------------------------------------------------------------------------- plan
def make_plan(g, budget, bmax=4, iters=30):
    """Per-(batch, KV head) reverse water-filling plan (kernels/bitplane.py:83-116;
    same bisection as make_plan_torch :118-126 and scripts/sketch.py:116-121).

    t_j = clip(rint((lg_j - mid) / 2), 0, bmax) with lg = log2(max(g, 1e-30));
    bisection of mid on [-60, 60], ``iters`` halvings, keeping sum(t) <= budget
    at ``hi``; final t from ``hi``.  Returns the reference's dict: t int8
    [BH, D]; pairs int32 [BH, D*bmax] (channel*bmax + plane, channel then plane
    ascending, zero padded); npairs; act int32 [BH, D] (active channels
    ascending, zero padded); nact; cls int32 [BH, bmax, D] (channels with
    t == c, ascending, zero padded); clsn int32 [BH, bmax].  Also returns the
    final ``hi`` (log2 of the water line theta) for checking."""
    g = np.asarray(g, np.float32)
    BH, D = g.shape
    Br = np.broadcast_to(np.asarray(budget, np.float32), (BH,)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        gg = np.where(np.isnan(g), np.float32(1e-30), np.maximum(g, np.float32(1e-30)))
    lg = flog2(gg)
    lo = np.full(BH, -60.0, np.float32)
    hi = np.full(BH, 60.0, np.float32)
    half = np.float32(0.5)
    bm = np.float32(bmax)
    zero = np.float32(0)
    for _ in range(iters):
        mid = (lo + hi) * half
        t = np.minimum(np.maximum(np.rint((lg - mid[:, None]) * half), zero), bm)
        tot = t.sum(-1, dtype=np.float32)
        over = tot > Br
        lo = np.where(over, mid, lo).astype(np.float32)
        hi = np.where(over, hi, mid).astype(np.float32)
    t = np.minimum(np.maximum(np.rint((lg - hi[:, None]) * half), zero), bm).astype(np.int32)
    act = np.zeros((BH, D), np.int32)
    nact = np.zeros(BH, np.int32)
    pairs = np.zeros((BH, D * bmax), np.int32)
    npairs = np.zeros(BH, np.int32)
    cls = np.zeros((BH, bmax, D), np.int32)
    clsn = np.zeros((BH, bmax), np.int32)
    for b in range(BH):
        a = np.nonzero(t[b] > 0)[0]
        act[b, :len(a)] = a
        nact[b] = len(a)
        pr = [j * bmax + p for j in range(D) for p in range(t[b, j])]
        pairs[b, :len(pr)] = pr
        npairs[b] = len(pr)
        for c in range(1, bmax + 1):
            cc = np.nonzero(t[b] == c)[0]
            cls[b, c - 1, :len(cc)] = cc
            clsn[b, c - 1] = len(cc)
    return {"t": t.astype(np.int8), "pairs": pairs, "npairs": npairs, "act": act, "nact": nact,
            "cls": cls, "clsn": clsn, "hi": hi}


def waterfill(w, budget, bmax=4):
    """Greedy reverse water-filling (scripts/sketch.py:19-25): repeatedly give a
    bit to the component with the largest w_j 4^-b_j; returns int bits."""
    w = np.asarray(w, np.float64)
    b = np.zeros(len(w), np.int64)
    for _ in range(int(budget)):
        gain = w * 4.0 ** (-b.astype(np.float64))
        gain[b >= bmax] = -1
        b[int(np.argmax(gain))] += 1
    return b


# ----------------------------------------------------------------------------- scan
def scan_planes(q, code, scales, t):
    """scores[bh, g, tok] = sum_j q[bh, g, j] * dequant(code, a, t[bh])[tok, j]
    in float64 (kernels/bitplane.py:357-363 semantics).  q [BH, G, D],
    code [BH, n, D], scales [BH, nblk, D], t [BH, D] -> [BH, G, n] float64."""
    q = np.asarray(q, np.float64)
    out = []
    for b in range(q.shape[0]):
        val = dequant_planes(code[b], scales[b], np.asarray(t[b], np.int64)).astype(np.float64)
        out.append(q[b] @ val.T)
    return np.stack(out)


def scan_planes_bits(q, planes_sb, scales_sb, t, n, sub):
    """Per-bit formulation straight from superblock-ordered plane words
    (kernels/bitplane.py:138-173 semantics): score = sum over (j, p < t_j) of
    q_j a_bj 2^(3-p)/8 * bit + sum over active j of q_j a_bj (2^-t_j - 1).
    float64, [BH, G, n]."""
    q = np.asarray(q, np.float64)
    pl = np.asarray(planes_sb).view(np.uint64)
    sc = np.asarray(scales_sb, np.float64)
    BH, G, D = q.shape
    nb = -(-n // BLK)
    blocks = np.arange(nb)
    sbi, bi = blocks // sub, blocks % sub
    lane = np.arange(BLK, dtype=np.uint64)
    out = np.zeros((BH, G, nb * BLK))
    for b in range(BH):
        acc = np.zeros((G, nb, BLK))
        for j in range(D):
            tj = int(t[b][j])
            if tj == 0:
                continue
            a = sc[b, sbi, j, bi]                                      # [nb]
            for p in range(tj):
                w = pl[b, sbi, j, p, bi]                               # [nb]
                bits = ((w[:, None] >> lane[None, :]) & np.uint64(1)).astype(np.float64)
                acc += (q[b, :, j][:, None, None] * (a * 2.0 ** (3 - p) / 8)[None, :, None]) * bits[None]
            acc += (q[b, :, j][:, None] * (a * (2.0 ** -tj - 1))[None, :])[:, :, None]
        out[b] = acc.reshape(G, -1)
    return out[:, :, :n]


# ----------------------------------------------------------------------------- top-k
def orderable_keys(s):
    """float32 -> uint32 keys whose unsigned order is torch.topk's value order:
    NaN highest, -0.0 == +0.0."""
    s = np.asarray(s, np.float32)
    s = np.where(s == 0, np.float32(0), s)                            # -0.0 -> +0.0
    u = s.view(np.uint32)
    key = np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    return np.where(np.isnan(s), np.uint32(0xFFFFFFFF), key).astype(np.uint32)


def sink_local_topk(scores, k, sink=4, local=32, m=None):
    """[..., n] scores -> int64 [..., k]: top-(k - sink - local) of the scores
    with [0, sink) and [max(m - local, 0), n) masked to -inf, ordered by
    (score descending, index ascending), then arange(sink), then
    arange(m - local, m) (kernels/bitplane.py:372-378;
    scripts/B_e2e_offload_v2.py:224-227 with m = current length)."""
    s = np.array(scores, np.float32, copy=True)
    n = s.shape[-1]
    m = n if m is None else m
    kk = k - sink - local
    s[..., :sink] = NEG_INF
    s[..., max(m - local, 0):] = NEG_INF
    key = orderable_keys(s)
    order = np.argsort(~key, axis=-1, kind="stable")[..., :kk].astype(np.int64)
    fixed = np.concatenate([np.arange(sink), np.arange(m - local, m)]).astype(np.int64)
    return np.concatenate([order, np.broadcast_to(fixed, (*s.shape[:-1], len(fixed)))], -1)


# ----------------------------------------------------------------------------- row gather
def gather_rows(src, idx):
    """dst[bh, r] = src[bh, idx[bh, r]] for 0 <= idx < cap, zeros otherwise
    (scripts/B_e2e_offload_v2.py:73-83; idx < 0 is the reference's masked
    load, idx >= cap is rejected to a zero row instead of an out-of-bounds read)."""
    src = np.asarray(src)
    idx = np.asarray(idx)
    BH, R = idx.shape
    dst = np.zeros((BH, R, src.shape[-1]), src.dtype)
    for b in range(BH):
        ok = (idx[b] >= 0) & (idx[b] < src.shape[1])
        dst[b, ok] = src[b, idx[b, ok]]
    return dst


def gather_union(idx, n, Ksrc, Vsrc, Krec=None, Vrec=None):
    """Rows of the group-union selection (scripts/B_e2e_offload_v2.py:228-241):
    idx [BH, G, k] (tokens < n from the host store, tokens >= n from the recent
    device buffer at row clamp(idx - n, 0, nrec - 1)).  The reference fetches
    each distinct host token once and forward-fills duplicates; values equal a
    plain gather.  Negative tokens give zero rows (the reference's host index
    stays negative and its gather masks the load).
    Returns (Ks [BH, G, k, D], Vs, n_unique_host [BH])."""
    idx = np.asarray(idx, np.int64)
    BH, G, k = idx.shape
    flat = idx.reshape(BH, -1)
    D = Ksrc.shape[-1]
    Ks = np.zeros((BH, G * k, D), Ksrc.dtype)
    Vs = np.zeros((BH, G * k, D), Vsrc.dtype)
    nu = np.zeros(BH, np.int64)
    for b in range(BH):
        host = (flat[b] >= 0) & (flat[b] < n)
        rec = flat[b] >= n
        Ks[b, host] = Ksrc[b, flat[b, host]]
        Vs[b, host] = Vsrc[b, flat[b, host]]
        if rec.any():
            r = np.clip(flat[b, rec] - n, 0, Krec.shape[1] - 1)
            Ks[b, rec] = Krec[b, r]
            Vs[b, rec] = Vrec[b, r]
        nu[b] = len(np.unique(flat[b, host]))
    return Ks.reshape(BH, G, k, D), Vs.reshape(BH, G, k, D), nu


def gather_attention(q, idx, n, Ksrc, Vsrc, Krec=None, Vrec=None, scale=None):
    """Exact attention over the selected rows (scripts/B_kernel_bench.py:22-27
    gather_attn; scripts/B_e2e_offload_v2.py:242-244): for query head g of row
    bh, s_j = scale * q[bh, g] . K[idx[bh, g, j]] over the k positions j (a token
    selected twice counts twice), out = softmax(s) . V.  Rows as gather_union
    (float arrays holding the bf16 row values); scale defaults to the float32
    value of D ** -0.5, as the reference's fp32 multiply uses it.  float64
    arithmetic.  Returns (out [BH, G, D] float64, n_unique_host [BH])."""
    Ks, Vs, nu = gather_union(idx, n, Ksrc, Vsrc, Krec, Vrec)
    q = np.asarray(q, np.float64)
    D = q.shape[-1]
    sc = float(np.float32(D ** -0.5)) if scale is None else float(scale)
    s = np.einsum("bgd,bgkd->bgk", q, Ks.astype(np.float64)) * sc
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(-1, keepdims=True)
    return np.einsum("bgk,bgkd->bgd", p, Vs.astype(np.float64)), nu


def gather_runs(src, dst, off, ln, nrun):
    """Copy run r, words [off[r], off[r] + ln[r]) of src, to the same words of dst
    for r < nrun; runs with ln <= 0 are skipped (scripts/B_e2e_offload_v2.py:62-71).
    src, dst: 1-D word arrays (dst is copied, not modified)."""
    out = np.array(dst, copy=True)
    for r in range(int(nrun)):
        o, l = int(off[r]), int(ln[r])
        for w in range(max(l, 0)):
            out[o + w] = src[o + w]
    return out


def copy_index_runs(t, nblk, D):
    """The copy-index run list of a plan t [BH, D] over whole-sequence stores
    (scripts/B_e2e_offload_v2.py:190-197), in 4-byte words: slot s = bh * D + j
    has the plane run (s * 4 * nblk * 2, min(t, 4) * nblk * 2) and the scale run
    (s * nblk / 2, [t > 0] * nblk / 2) (nblk even)."""
    t = np.asarray(t, np.int64).reshape(-1)
    slot = np.arange(t.size, dtype=np.int64)
    offp = slot * (4 * nblk * 2)
    lenp = np.clip(t, 0, 4) * (nblk * 2)
    offs = slot * (nblk // 2)
    lens = (t > 0).astype(np.int64) * (nblk // 2)
    return offp, lenp, offs, lens


# ----------------------------------------------------------------------------- CPU baseline (sketch path)
def qblock(c, bits, blk=BLK):
    """Per-(block, column) absmax mid-rise quantiser, fp32 absmax
    (scripts/sketch.py:8-17).  c [n, r] float32, bits [r] ints."""
    c = np.asarray(c, np.float32)
    n, r = c.shape
    nb = -(-n // blk)
    cb = np.concatenate([c, np.zeros((nb * blk - n, r), np.float32)]).reshape(nb, blk, r)
    amax = np.maximum(np.abs(cb).max(1, keepdims=True), np.float32(1e-8))
    bits = np.asarray(bits, np.int64)
    half = (np.float32(2.0) ** (np.maximum(bits, 1) - 1)).astype(np.float32)
    s = amax / half
    out = (np.clip(np.floor(cb / s), -half, half - 1) + np.float32(0.5)) * s
    out[..., bits <= 0] = 0
    return out.reshape(-1, r)[:n]


def sketch_planes_scores(q, k, var, budget, bmax=4, iters=30):
    """CPU scorer of scripts/sketch.py:110-131 ("planes:u4:B") for one KV head
    and one decode position: q [G, D] group queries, k [n, D] fp32 keys,
    var [D] calibration variance.  Plan as make_plan (flog2), then for each
    depth level re-quantise K at lvl bits with the fp32 block absmax and
    accumulate (q * [t == lvl]) @ plane.T.  Returns (scores [G, n] float32, t)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    g = ((q ** 2) * np.asarray(var, np.float32)).sum(0, dtype=np.float32)[None]
    t = make_plan(g, budget, bmax, iters)["t"][0].astype(np.int64)
    n, r = k.shape
    nb = -(-n // BLK)
    cb = np.concatenate([k, np.zeros((nb * BLK - n, r), np.float32)]).reshape(nb, BLK, r)
    amax = np.maximum(np.abs(cb).max(1, keepdims=True), np.float32(1e-8))
    out = np.zeros((q.shape[0], n), np.float32)
    for lvl in range(1, bmax + 1):
        msk = (t == lvl)
        if not msk.any():
            continue
        half = np.float32(2.0 ** (lvl - 1))
        sc = amax / half
        plane = ((np.clip(np.floor(cb / sc), -half, half - 1) + np.float32(0.5)) * sc).reshape(-1, r)[:n]
        out += (q * msk[None].astype(np.float32)) @ plane.T
    return out, t
