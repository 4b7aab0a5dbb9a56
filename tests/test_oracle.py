"""CPU checks that pin the numpy oracle (no GPU).

Each check compares the oracle with something independent of its own
formulas: the paper's worked example, a different quantiser formula (the
sketch quantiser), pure-Python bit loops, the greedy water-filling algorithm,
float64 log2, a per-bit scan formulation, or a brute-force sort.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import fathom_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _worked():
    with open(os.path.join(GOLD, "worked_example.json")) as f:
        return json.load(f)


# ----------------------------------------------------------------------------- worked example (paper App. A)
def test_worked_example_variance_and_gain():
    w = _worked()
    K = np.array(w["keys"], np.float32)
    var = K.var(0, ddof=1)
    np.testing.assert_allclose(var, w["var_3dp"], atol=6e-4)
    qa, qb = np.array(w["q_head_A"], np.float32), np.array(w["q_head_B"], np.float32)
    g = (qa ** 2 + qb ** 2) * var
    np.testing.assert_allclose(g, w["g_2dp"], atol=6e-3)


@pytest.mark.parametrize("budget", [8, 6])
def test_worked_example_plan(budget):
    w = _worked()
    K = np.array(w["keys"], np.float32)
    var = K.var(0, ddof=1)
    g = (np.array(w["q_head_A"], np.float32) ** 2 + np.array(w["q_head_B"], np.float32) ** 2) * var
    p = O.make_plan(g[None], budget)
    exp = w["plan"][str(budget)]
    assert p["t"][0].tolist() == exp["t"]
    theta = 2.0 ** float(p["hi"][0])          # t = round(log4(g / theta)) with log2(theta) = hi
    assert exp["theta_lo"] < theta <= exp["theta_hi"]
    assert round(theta, 3) == exp["theta_printed"]


def test_worked_example_codes_and_one_plane():
    w = _worked()
    K = np.array(w["keys"], np.float32)
    code, sc = O.quantise_u4(K)
    assert sc[0, 2] == np.float32(w["channel2_amax"])
    assert code[:, 2].tolist() == w["channel2_codes"]
    one = O.dequant_planes(code, sc, np.array([0, 0, 1, 0]))[:, 2]
    np.testing.assert_array_equal(one, np.array(w["channel2_one_plane_values"], np.float32))


def test_worked_example_scores():
    w = _worked()
    K = np.array(w["keys"], np.float32)
    q = np.stack([np.array(w["q_head_A"], np.float32), np.array(w["q_head_B"], np.float32)])
    code, sc = O.quantise_u4(K)
    t = np.array(w["plan"]["8"]["t"])
    s = O.scan_planes(q[None], code[None], sc[None], t[None])[0]
    np.testing.assert_allclose(s[0], w["scores_B8_head_A_2dp"], atol=5.1e-3)
    np.testing.assert_allclose(s[1], w["scores_B8_head_B_2dp"], atol=5.1e-3)
    np.testing.assert_allclose(q @ K.T, [w["exact_head_A_2dp"], w["exact_head_B_2dp"]], atol=5.1e-3)
    top2 = [list(np.argsort(-row, kind="stable")[:2]) for row in s]
    assert top2 == [w["top2_head_A"], w["top2_head_B"]]


# ----------------------------------------------------------------------------- quantiser: prefix theorem
def _qblock_given_amax(x, amax, t):
    """scripts/sketch.py:8-17 t-bit mid-rise quantiser, absmax supplied per (block, channel)."""
    n, d = x.shape
    nb = -(-n // 64)
    xb = np.concatenate([x, np.zeros((nb * 64 - n, d), np.float32)]).reshape(nb, 64, d)
    half = np.float32(2.0 ** (t - 1))
    s = amax[:, None, :] / half
    out = (np.clip(np.floor(xb / s), -half, half - 1) + np.float32(0.5)) * s
    return out.reshape(-1, d)[:n]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_prefix_theorem(seed):
    """Depth-t dequantisation of the 4-bit store == the t-bit sketch quantiser with
    the same fp16 absmax, bit for bit, for every t (paper Sec. 3 claim)."""
    rng = np.random.default_rng(seed)
    n, d = 200, 16
    x = (rng.standard_normal((n, d)) * np.exp(rng.standard_normal(d))).astype(np.float32)
    # put some values exactly on cell edges of the fp16 absmax grid
    code, sc = O.quantise_u4(x)
    for blk in range(sc.shape[0]):
        for j in range(0, d, 3):
            x[blk * 64 + 5, j] = sc[blk, j] / 8 * 3 if blk * 64 + 5 < n else 0
            x[min(blk * 64 + 7, n - 1), j] = -sc[blk, j] / 4
    code, sc = O.quantise_u4(x)
    for t in range(1, 5):
        got = O.dequant_planes(code, sc, t)
        ref = _qblock_given_amax(x, sc, t)
        np.testing.assert_array_equal(got, ref)


def test_quantise_edge_values():
    x = np.zeros((130, 4), np.float32)
    x[:, 0] = 1e-9                         # amax -> fp16(1e-8) = 0: x / 0 = +inf -> code 15
    x[:64, 1] = 0.0                        # 0 / 0 -> NaN -> code 0
    x[64:, 1] = np.linspace(-3, 3, 66)
    x[5, 2] = np.nan                       # NaN poisons the block's absmax -> every code 0
    x[:, 3] = 70000.0                      # fp16 overflow -> amax inf -> x / inf = 0 -> code 8
    code, sc = O.quantise_u4(x)
    assert (code[:, 0] == 15).all() and sc[0, 0] == 0
    assert (code[:64, 1] == 0).all()
    assert np.isnan(sc[0, 2]) and (code[:64, 2] == 0).all()
    assert np.isinf(sc[0, 3]) and (code[:, 3] == 8).all()


def test_sketch_scores_equal_store_scores_with_fp32_scales():
    """The CPU baseline scorer (sketch re-quantisation per depth, fp32 absmax) equals the
    store scan on codes quantised with fp32 scales: two formulas, one result."""
    rng = np.random.default_rng(3)
    n, d, G = 300, 32, 3
    k = (rng.standard_normal((n, d)) * np.exp(rng.standard_normal(d))).astype(np.float32)
    q = rng.standard_normal((G, d)).astype(np.float32)
    var = k[16:].var(0, ddof=1)
    s1, t = O.sketch_planes_scores(q, k, var, 20)
    code, sc = O.quantise_u4(k, "f32")
    s2 = O.scan_planes(q[None], code[None], sc[None], t[None])[0]
    np.testing.assert_allclose(s1, s2, rtol=1e-5, atol=1e-4 * np.abs(s2).max())


# ----------------------------------------------------------------------------- packing
def test_pack_bruteforce_and_roundtrip():
    rng = np.random.default_rng(0)
    code = rng.integers(0, 16, size=(2, 130, 3), dtype=np.uint8)
    planes = O.pack_planes(code)
    assert planes.shape == (2, 3, 3, 4) and planes.dtype == np.uint64
    for b in range(2):
        for blk in range(3):
            for j in range(3):
                for p in range(4):
                    word = 0
                    for i in range(64):
                        tok = blk * 64 + i
                        c = int(code[b, tok, j]) if tok < 130 else 0
                        word |= ((c >> (3 - p)) & 1) << i
                    assert int(planes[b, blk, j, p]) == word
    np.testing.assert_array_equal(O.unpack_planes(planes, 130), code)


@pytest.mark.parametrize("sub", [1, 3, 16])
def test_to_superblocks_bruteforce(sub):
    rng = np.random.default_rng(sub)
    nb, d = 5, 3
    planes = rng.integers(0, 2 ** 63, size=(2, nb, d, 4), dtype=np.uint64)
    scales = rng.random((2, nb, d)).astype(np.float32)
    pl, sc = O.to_superblocks(planes, scales, sub)
    nsb = -(-nb // sub)
    assert pl.shape == (2, nsb, d, 4, sub) and sc.shape == (2, nsb, d, sub)
    for b in range(2):
        for s in range(nsb):
            for j in range(d):
                for bs in range(sub):
                    blk = s * sub + bs
                    assert sc[b, s, j, bs] == (scales[b, blk, j] if blk < nb else 0)
                    for p in range(4):
                        assert pl[b, s, j, p, bs] == (planes[b, blk, j, p] if blk < nb else 0)


def test_bytes_planes():
    t = np.array([[4, 3, 1, 0], [0, 0, 0, 0]])
    assert O.bytes_planes(t, 130) == ((8 * 8 + 2 * 3) * 3)


# ----------------------------------------------------------------------------- log2
def test_flog2_matches_float64_log2():
    rng = np.random.default_rng(0)
    e = rng.uniform(-99, 127, 400_000)
    x = (2.0 ** e * rng.uniform(1, 2, e.shape)).astype(np.float32)
    x = np.concatenate([x, np.float32(2.0) ** np.arange(-99, 127, dtype=np.float32),
                        np.array([1e-30, 1.0, 3.0, 0.63333338, 12.216667, 65504.0], np.float32)])
    ref = np.log2(x.astype(np.float64)).astype(np.float32)
    got = O.flog2(x)
    assert np.array_equal(got, ref), int((got != ref).sum())
    assert O.flog2(np.float32(np.inf)) == np.inf and np.isnan(O.flog2(np.float32(np.nan)))


# ----------------------------------------------------------------------------- plan
def test_plan_invariants_and_compaction():
    rng = np.random.default_rng(1)
    BH, d = 12, 128
    g = (np.exp(rng.standard_normal((BH, d)) * 3) * rng.random((BH, d))).astype(np.float32)
    g[0, :10] = 0
    budget = rng.integers(0, 300, BH).astype(np.float32)
    p = O.make_plan(g, budget)
    t = p["t"].astype(np.int64)
    assert (t >= 0).all() and (t <= 4).all()
    assert (t.sum(1) <= budget).all()
    for b in range(BH):
        order = np.argsort(g[b])
        assert (np.diff(t[b][order]) >= 0).all()          # larger gain never gets fewer planes
        a = [j for j in range(d) if t[b, j] > 0]
        assert p["act"][b].tolist() == a + [0] * (d - len(a)) and p["nact"][b] == len(a)
        pr = [j * 4 + q for j in range(d) for q in range(t[b, j])]
        assert p["pairs"][b].tolist() == pr + [0] * (4 * d - len(pr)) and p["npairs"][b] == len(pr)
        for c in range(1, 5):
            cc = [j for j in range(d) if t[b, j] == c]
            assert p["cls"][b, c - 1].tolist() == cc + [0] * (d - len(cc)) and p["clsn"][b, c - 1] == len(cc)


def test_plan_equals_greedy_waterfill():
    """Where the bisection spends the whole budget, t equals the greedy reverse
    water-filling allocation (scripts/sketch.py:19-25) at the same budget."""
    rng = np.random.default_rng(7)
    checked = 0
    for trial in range(60):
        d = 128
        g = np.exp(rng.standard_normal(d) * 3).astype(np.float32)
        B = int(rng.integers(1, 400))
        t = O.make_plan(g[None], B)["t"][0].astype(np.int64)
        if t.sum() != B:
            continue
        assert t.tolist() == O.waterfill(g, B).tolist()
        checked += 1
    assert checked > 40


# ----------------------------------------------------------------------------- scan
@pytest.mark.parametrize("sub", [16, 2, 5])
def test_scan_bits_formulation_equals_dequant_formulation(sub):
    rng = np.random.default_rng(sub)
    BH, G, n, d = 2, 3, 500, 16
    K = (rng.standard_normal((BH, n, d)) * np.exp(rng.standard_normal(d))).astype(np.float32)
    q = rng.standard_normal((BH, G, d)).astype(np.float32)
    code, sc = O.quantise_u4(K)
    t = rng.integers(0, 5, size=(BH, d))
    pl, scb = O.to_superblocks(O.pack_planes(code), sc, sub)
    a = O.scan_planes(q, code, sc, t)
    b = O.scan_planes_bits(q, pl, scb, t, n, sub)
    np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-9)


def test_scan_depth4_error_bound():
    """At depth 4 every value is within a/16 of the key, so |score - q.k| <= sum_j |q_j| a_bj / 16."""
    rng = np.random.default_rng(4)
    n, d = 640, 32
    K = (rng.standard_normal((1, n, d)) * np.exp(rng.standard_normal(d))).astype(np.float32)
    q = rng.standard_normal((1, 2, d)).astype(np.float32)
    code, sc = O.quantise_u4(K)
    s = O.scan_planes(q, code, sc, np.full((1, d), 4))[0]
    exact = q[0].astype(np.float64) @ K[0].T.astype(np.float64)
    bound = (np.abs(q[0]).astype(np.float64) @ np.repeat(sc[0], 64, 0)[:n].T.astype(np.float64)) / 16
    assert (np.abs(s - exact) <= bound * (1 + 1e-6) + 1e-9).all()


# ----------------------------------------------------------------------------- top-k
def _brute_topk(row, k, sink, local, m):
    n = len(row)
    s = [float(v) for v in row]
    for i in range(min(sink, n)):
        s[i] = -math.inf
    for i in range(max(m - local, 0), n):
        s[i] = -math.inf

    def key(i):
        v = s[i]
        return (0, 0.0, i) if math.isnan(v) else (1, -v, i)

    kk = k - sink - local
    return sorted(range(n), key=key)[:kk] + list(range(sink)) + list(range(m - local, m))


@pytest.mark.parametrize("seed", range(6))
def test_topk_bruteforce(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(40, 300))
    rows = rng.integers(-5, 6, size=(3, n)).astype(np.float32)       # many ties
    rows[0, rng.integers(0, n, 5)] = np.nan
    rows[1, rng.integers(0, n, 5)] = -np.inf
    rows[2, rng.integers(0, n, 8)] = -0.0
    sink, local = int(rng.integers(0, 5)), int(rng.integers(0, 10))
    m = n + int(rng.integers(0, 3))
    k = sink + local + int(rng.integers(0, n - sink))
    got = O.sink_local_topk(rows, k, sink, local, m=m)
    for r in range(3):
        assert got[r].tolist() == _brute_topk(rows[r], k, sink, local, m)


# ----------------------------------------------------------------------------- gathers
def test_gather_rows_and_union():
    rng = np.random.default_rng(5)
    BH, n, d, G, k, nrec = 2, 50, 8, 3, 7, 4
    Ks = rng.standard_normal((BH, n, d)).astype(np.float32)
    Vs = rng.standard_normal((BH, n, d)).astype(np.float32)
    Kr = rng.standard_normal((BH, nrec, d)).astype(np.float32)
    Vr = rng.standard_normal((BH, nrec, d)).astype(np.float32)
    idx = rng.integers(0, n + nrec + 2, size=(BH, G, k))
    idx[0, 0, 0] = -1
    K, V, nu = O.gather_union(idx, n, Ks, Vs, Kr, Vr)
    for b in range(BH):
        host = set()
        for g in range(G):
            for i in range(k):
                tok = int(idx[b, g, i])
                if 0 <= tok < n:
                    host.add(tok)
                    exp_k, exp_v = Ks[b, tok], Vs[b, tok]
                elif tok >= n:
                    r = min(max(tok - n, 0), nrec - 1)
                    exp_k, exp_v = Kr[b, r], Vr[b, r]
                else:
                    exp_k = exp_v = np.zeros(d, np.float32)
                np.testing.assert_array_equal(K[b, g, i], exp_k)
                np.testing.assert_array_equal(V[b, g, i], exp_v)
        assert nu[b] == len(host)
    r = O.gather_rows(Ks, np.array([[3, -1, 0], [49, 2, -5]]))
    np.testing.assert_array_equal(r[0, 0], Ks[0, 3])
    assert (r[0, 1] == 0).all() and (r[1, 2] == 0).all()
    np.testing.assert_array_equal(r[1, 0], Ks[1, 49])


def test_gather_runs_and_copy_index_runs_known_answer():
    """Hand-computed: runs [2, 5) and [9, 10) of a 12-word store, a skipped run
    (len 0) and a run past nrun; the copy-index run list of a 2x2 plan with
    nblk = 4 written out from the reference's formulas (B_e2e_offload_v2.py:193)."""
    src = np.arange(100, 112, dtype=np.int32)
    dst = np.full(12, -1, np.int32)
    got = O.gather_runs(src, dst, off=[2, 9, 0, 6], ln=[3, 1, 0, 2], nrun=3)
    exp = np.array([-1, -1, 102, 103, 104, -1, -1, -1, -1, 109, -1, -1], np.int32)
    np.testing.assert_array_equal(got, exp)
    t = np.array([[2, 0], [5, 1]])
    offp, lenp, offs, lens = O.copy_index_runs(t, nblk=4, D=2)
    np.testing.assert_array_equal(offp, [0, 32, 64, 96])     # slot * 4 planes * 4 blocks * 2 words
    np.testing.assert_array_equal(lenp, [16, 0, 32, 8])      # min(t, 4) * 4 blocks * 2 words
    np.testing.assert_array_equal(offs, [0, 2, 4, 6])        # slot * 4 halves / 2
    np.testing.assert_array_equal(lens, [2, 0, 2, 2])


def test_copy_index_runs_cover_exactly_the_scanned_words():
    """The runs of a plan are exactly the words a scan of the whole-sequence store
    reads: every plane word of a listed channel at depth < t, every scale of a
    listed channel, nothing else (checked by marking words on a tiny store)."""
    rng = np.random.default_rng(7)
    BH, D, nblk = 2, 6, 4
    t = rng.integers(0, 5, size=(BH, D))
    offp, lenp, offs, lens = O.copy_index_runs(t, nblk, D)
    words = np.zeros(BH * D * 4 * nblk * 2, np.int32)
    src = np.ones_like(words)
    mark = O.gather_runs(src, words, offp, lenp, len(offp)).reshape(BH, D, 4, nblk * 2)
    for b in range(BH):
        for j in range(D):
            for p in range(4):
                assert (mark[b, j, p] == (1 if p < t[b, j] else 0)).all()
    sc = O.gather_runs(np.ones(BH * D * nblk // 2, np.int32), np.zeros(BH * D * nblk // 2, np.int32), offs, lens,
                       len(offs)).reshape(BH, D, nblk // 2)
    for b in range(BH):
        for j in range(D):
            assert (sc[b, j] == (1 if t[b, j] > 0 else 0)).all()


# ----------------------------------------------------------------------------- attention over gathered rows
def test_gather_attention_closed_forms():
    """Weights fixed by construction, so the expected output is a hand-known mix
    of V rows: q along e0 and K rows c_j * e0 give scores scale * c_j; choosing
    c_j = ln(w_j) / scale makes the softmax weights proportional to w_j."""
    d, n = 8, 6
    sc = float(np.float32(d ** -0.5))
    q = np.zeros((1, 2, d))
    q[0, :, 0] = 1.0
    w = [1.0, 2.0, 4.0, 1.0, 1.0, 1.0]                       # target weight of each token
    K = np.zeros((1, n, d))
    K[0, :, 0] = [math.log(x) / sc for x in w]
    V = np.arange(n * d, dtype=np.float64).reshape(1, n, d) % 7 - 3.0
    # head 0: tokens 0, 1, 2 -> weights 1:2:4; head 1: token 1 twice and token 2
    # once (a duplicate counts per position) -> weights 2+2:4 = 1:1
    idx = np.array([[[0, 1, 2], [1, 1, 2]]])
    out, nu = O.gather_attention(q, idx, n, K, V)
    np.testing.assert_allclose(out[0, 0], (1 * V[0, 0] + 2 * V[0, 1] + 4 * V[0, 2]) / 7.0, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out[0, 1], (V[0, 1] + V[0, 2]) / 2.0, rtol=1e-12, atol=1e-12)
    assert nu[0] == 3
    # a negative token is a zero row: score 0 (weight e^0 = 1) and zero value
    idx2 = np.array([[[0, 2, -1], [3, 4, 5]]])
    out2, nu2 = O.gather_attention(q, idx2, n, K, V)
    np.testing.assert_allclose(out2[0, 0], (1 * V[0, 0] + 4 * V[0, 2] + 0.0) / 6.0, rtol=1e-12, atol=1e-12)
    # equal scores: the plain mean of the selected rows
    np.testing.assert_allclose(out2[0, 1], V[0, 3:6].mean(0), rtol=1e-12, atol=1e-12)
    assert nu2[0] == 5
    # tokens >= n come from the recent buffer (clamped to its last row)
    Kr = np.zeros((1, 2, d))
    Vr = np.full((1, 2, d), 5.0)
    Vr[0, 1] = -5.0
    out3, _ = O.gather_attention(q, np.array([[[n, n + 7], [n + 1, n + 1]]]), n, K, V, Kr, Vr)
    np.testing.assert_allclose(out3[0, 0], np.zeros(d), atol=1e-12)
    np.testing.assert_allclose(out3[0, 1], np.full(d, -5.0), atol=1e-12)


def test_gather_attention_shift_and_scale():
    """Adding one offset row u to every key shifts all scores of a head by
    scale * q.u, which softmax ignores; a huge score spread (q x 1e4) puts all
    the weight on the best-scoring token without overflowing."""
    rng = np.random.default_rng(3)
    BH, G, k, n, d = 2, 3, 5, 40, 16
    q = rng.standard_normal((BH, G, d))
    K = rng.standard_normal((BH, n, d))
    V = rng.standard_normal((BH, n, d))
    idx = rng.integers(0, n, size=(BH, G, k))
    a, _ = O.gather_attention(q, idx, n, K, V)
    b, _ = O.gather_attention(q, idx, n, K + rng.standard_normal((BH, 1, d)), V)
    np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)
    c, _ = O.gather_attention(q * 1e4, idx, n, K, V)       # one token dominates per head
    for bb in range(BH):
        for g in range(G):
            s = K[bb, idx[bb, g]] @ q[bb, g]
            np.testing.assert_allclose(c[bb, g], V[bb, idx[bb, g, int(np.argmax(s))]], rtol=1e-9, atol=1e-9)


# ----------------------------------------------------------------------------- chan4 baseline store
def test_pack_chan4_bruteforce():
    rng = np.random.default_rng(8)
    code = rng.integers(0, 16, size=(2, 150, 5)).astype(np.uint8)
    sub = 2
    w = O.pack_chan4(code, sub)
    assert w.shape == (2, 2, 5, 2, 8) and w.dtype == np.uint32
    for b in range(2):
        for i in range(4 * 64):
            blk, sb, bs = i // 64, (i // 64) // sub, (i // 64) % sub
            m, k = (i % 64) // 8, i % 8
            for j in range(5):
                want = int(code[b, i, j]) if i < 150 else 0
                assert (int(w[b, sb, j, bs, m]) >> (4 * k)) & 15 == want, (b, i, j)


def test_channel_list_and_bytes():
    active = np.array([[0, 1, 0, 1, 1, 0], [1, 1, 1, 1, 1, 1], [0, 0, 0, 0, 0, 0]], bool)
    act, nact = O.channel_list(active)
    np.testing.assert_array_equal(act, [[1, 3, 4, 0, 2, 5], [0, 1, 2, 3, 4, 5], [0, 1, 2, 3, 4, 5]])
    np.testing.assert_array_equal(nact, [3, 6, 0])
    assert O.bytes_chan4(nact, 130) == (3 + 6 + 0) * 34 * 3


def test_scan_chan4_is_full_depth_scan():
    """The chan4 score of a token is sum over listed channels of q_j * a * (c - 7.5) / 8:
    checked by scalar loops, and equal to the plane scan with t = 4 on the listed
    channels and t = 0 elsewhere."""
    rng = np.random.default_rng(9)
    BH, G, n, d = 2, 3, 130, 8
    K = rng.standard_normal((BH, n, d)).astype(np.float32)
    code, sc = O.quantise_u4(K)
    q = rng.standard_normal((BH, G, d))
    active = rng.random((BH, d)) < 0.5
    act, nact = O.channel_list(active)
    s = O.scan_chan4(q, code, sc, act, nact)
    for b in range(BH):
        for g in range(G):
            for i in (0, 63, 64, 129):
                want = sum(q[b, g, j] * float(sc[b, i // 64, j]) * (int(code[b, i, j]) - 7.5) / 8
                           for j in range(d) if active[b, j])
                assert abs(s[b, g, i] - want) <= 1e-12 * (1 + abs(want))
    t = np.where(active, 4, 0)
    np.testing.assert_allclose(s, O.scan_planes(q, code, sc, t), rtol=0, atol=1e-12)


# ----------------------------------------------------------------------------- KLT store, budget allocation
def test_klt_basis_identities():
    """Orthonormal components; lam is the variance of the rotated calibration keys
    (v' C v = lam); scores are invariant under the rotation; components ordered by w."""
    rng = np.random.default_rng(12)
    BH, n, d, m = 2, 400, 16, 24
    A = rng.standard_normal((BH, d, d))
    K = rng.standard_normal((BH, n, d)) @ A + rng.standard_normal((BH, 1, d)) * 3
    Q = rng.standard_normal((BH, m, d))
    p = O.klt_params(K, Q)
    for b in range(BH):
        V = p["Vt"][b]
        np.testing.assert_allclose(V.T @ V, np.eye(d), atol=1e-10)
        Kc = K[b, 16:] - p["mu"][b]
        np.testing.assert_allclose((Kc @ V).var(0), p["lam"][b], rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(p["w"][b], ((Q[b] @ V) ** 2).mean(0) * p["lam"][b], rtol=1e-12)
        assert (np.diff(p["w"][b]) <= 0).all()
        q = rng.standard_normal((3, d))
        np.testing.assert_allclose((q @ V) @ (Kc @ V).T, q @ Kc.T, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("seed", [0, 1])
def test_klt_query_invariance_and_gain_loop(seed):
    """klt_query against what the rotation fixes (scripts/R_ruler.py:82-84):
    with any orthonormal, non-symmetric basis Vt, the rotated query scores the
    rotated centred keys exactly as q scores the centred keys, and the gains are
    sum_g qr^2 lam by an explicit loop.  A transposed rotation breaks the first."""
    rng = np.random.default_rng(seed)
    BH, G, d, n = 2, 3, 12, 50
    Vt = np.stack([np.linalg.qr(rng.standard_normal((d, d)))[0] for _ in range(BH)])
    assert not np.allclose(Vt[0], Vt[0].T)
    lam = rng.random((BH, d)) + 0.1
    q = rng.standard_normal((BH, G, d))
    k = rng.standard_normal((BH, n, d)) * 3
    mu = rng.standard_normal((BH, d))
    qr, gain = O.klt_query(q, Vt, lam)
    for b in range(BH):
        kr = (k[b] - mu[b]) @ Vt[b]                      # the store's rotation of the keys
        np.testing.assert_allclose(qr[b] @ kr.T, q[b] @ (k[b] - mu[b]).T, rtol=1e-10, atol=1e-10)
        bad = (q[b] @ Vt[b].T) @ kr.T                    # the query rotated the other way
        assert not np.allclose(bad, q[b] @ (k[b] - mu[b]).T, atol=1e-3)
        for e in range(d):
            acc = 0.0
            for g in range(G):
                qe = sum(q[b, g, j] * Vt[b, j, e] for j in range(d))
                acc += qe * qe * lam[b, e]
            assert abs(gain[b, e] - acc) <= 1e-12 * max(1.0, abs(acc))


# ----------------------------------------------------------------------------- CPU scorer (sketch)
def test_qblock_is_the_quantiser_at_fp32_scales():
    """sketch.qblock (scripts/sketch.py:8-17) at t bits equals the depth-t
    dequantisation of the 4-bit codes quantised with fp32 block scales (the
    prefix theorem with fp32 absmax), and a 0-bit column is dropped."""
    rng = np.random.default_rng(7)
    n, d = 150, 10
    x = (rng.standard_normal((n, d)) * np.exp(rng.standard_normal(d))).astype(np.float32)
    code, sc = O.quantise_u4(x, "f32")
    for t in range(1, 5):
        np.testing.assert_array_equal(O.qblock(x, np.full(d, t)), O.dequant_planes(code, sc, t))
    bits = np.array([4, 0, 2, 1, 0, 3, 4, 4, 1, 2])
    out = O.qblock(x, bits)
    assert (out[:, bits == 0] == 0).all()
    for j in range(d):
        if bits[j]:
            np.testing.assert_array_equal(out[:, j], O.dequant_planes(code, sc, bits[j])[:, j])


def test_sketch_scores_are_qblock_level_sums():
    """The CPU scorer is the sum over depth levels of the level's channels of q
    times the qblock quantisation at that level (scripts/sketch.py:122-130)."""
    rng = np.random.default_rng(8)
    n, d, G = 260, 24, 2
    k = (rng.standard_normal((n, d)) * np.exp(rng.standard_normal(d))).astype(np.float32)
    q = rng.standard_normal((G, d)).astype(np.float32)
    var = k[16:].var(0, ddof=1)
    s, t = O.sketch_planes_scores(q, k, var, 30)
    ref = np.zeros((G, n))
    for lvl in range(1, 5):
        m = (t == lvl)
        if m.any():
            ref += (q * m[None]).astype(np.float64) @ O.qblock(k, np.full(d, lvl)).T.astype(np.float64)
    np.testing.assert_allclose(s, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_torch_cpu_scorer_matches_oracle():
    """The torch restatement timed as the CPU baseline (oracle/sketch_torch.py)
    against the numpy oracle: same depths, scores within fp32 summation noise,
    same top-k on tie-free scores."""
    import torch
    from oracle import sketch_torch as ST
    from fathom_amd import workloads as W
    x = W.config_inputs(1, n=4096)
    k = x["K"][0].float()
    q = x["q"][0]
    var = x["var"][0]
    s_np, t_np = O.sketch_planes_scores(q.numpy(), k.numpy(), var.numpy(), x["budget"])
    s_t, t_t = ST.planes_scores(q, k, var, x["budget"])
    np.testing.assert_array_equal(t_t.numpy(), t_np)
    np.testing.assert_allclose(s_t.numpy(), s_np, rtol=1e-5, atol=1e-5 * np.abs(s_np).max())
    idx_t = ST.sink_local_topk(s_t, 128, 4, 64)
    idx_o = O.sink_local_topk(s_t.numpy()[None], 128, 4, 64)[0]
    np.testing.assert_array_equal(np.sort(idx_t.numpy(), -1), np.sort(idx_o, -1))


def test_allocate_worked_example():
    """Three layers, budgets 24/32/48: slopes per bit at each step decide by hand.
    Step 1: slopes (24->32) = 0.8/8, 0.4/8, 1.6/8 -> layer 2 to 32 (mean 26.67).
    Step 2: layer 2 (32->48) 0.8/16 = 0.05; layer 0 0.1; layer 1 0.05 -> layer 0 (mean 29.33).
    Step 3: layer 0 (32->48) 0.32/16 = 0.02; layer 1 0.05; layer 2 0.05 -> layer 1 (first of
    the tie) to 32 (mean 32) -> stop at target 32."""
    err = {24: [1.0, 0.9, 2.0], 32: [0.2, 0.5, 0.4], 48: [-0.12, 0.0, -0.4]}
    assert O.allocate(err, (24, 32, 48), 32) == [32, 32, 32]
    assert O.allocate(err, (24, 32, 48), 26) == [24, 24, 32]
    assert O.allocate(err, (24, 32, 48), 100) == [48, 48, 48]        # every layer at the top budget


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_allocate_greedy_optimal_on_convex_equal_steps(seed):
    """Equal budget steps and convex decreasing errors: greedy marginal allocation
    reaches the minimum total error among all allocations of the same total budget."""
    import itertools
    rng = np.random.default_rng(seed)
    budgets = (16, 24, 32, 40, 48)
    nl = 4
    drops = np.sort(rng.random((nl, len(budgets) - 1)), axis=1)[:, ::-1]   # decreasing drops -> convex
    base = rng.random(nl) + 5
    errs = np.concatenate([base[:, None], base[:, None] - np.cumsum(drops, 1)], 1)
    err = {B: list(errs[:, i]) for i, B in enumerate(budgets)}
    for target in (20, 28, 36):
        got = O.allocate(err, budgets, target)
        total = sum(got)
        best = min(sum(errs[L, budgets.index(B)] for L, B in enumerate(c))
                   for c in itertools.product(budgets, repeat=nl) if sum(c) == total)
        assert abs(sum(errs[L, budgets.index(B)] for L, B in enumerate(got)) - best) < 1e-12
