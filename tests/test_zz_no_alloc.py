"""fathom_scan_topk_noalloc (the fused scan + top-k on the library's static
scratch array) against fathom_scan_topk on a caller workspace: the same index
sets, bit for bit, on consecutive calls whose shapes shrink (the array keeps
the previous call's state), on the candidate-chain, row-select and wide
(k - sink - local above 2048) paths; shapes past the array are refused before any launch; the calls after
the first change no device memory."""
import ctypes

import pytest
import torch

from fathom_amd import _lib
from fathom_amd import bitplane as bp
from fathom_amd import workloads as W

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
SCRATCH = 64 << 20  # FATHOM_NOALLOC_SCRATCH_BYTES


def _case(BH, G, n, seed):
    x = W.synth_layer(BH, n, G, seed=seed)
    g = ((x["q"] ** 2) * x["var"][:, None, :]).sum(1)
    st = bp.PlaneStore(x["K"].to(DEV))
    plan = bp.make_plan(g.to(DEV), 56.0)
    return st, plan, x["q"].to(DEV).float().contiguous()


def _noalloc(st, plan, q, k, sink, local, m, idx):
    BH, G, d = q.shape
    cls, clsn = bp._plan_classes(plan, BH, d)
    rc = _lib.lib().fathom_scan_topk_noalloc(
        bp._ptr(q), BH, G, d, bp._ptr(cls), bp._ptr(clsn), cls.shape[1], bp._units_max(plan),
        ctypes.c_void_p(st.planes32.data_ptr()),
        ctypes.c_void_p(st.scales_k.data_ptr()), st.n, int(st.nsb), int(getattr(st, "sub", bp.SUB)), m, k, sink, local, bp._ptr(idx),
        bp._stream(q.device))
    _lib.check(rc, "fathom_scan_topk_noalloc")
    return idx


def test_noalloc_equals_workspace_entry_on_shrinking_calls():
    # (BH, G, n, k, sink, local, m): the chain path twice, the second call
    # smaller, then the row-select path (n <= 32768), then k - sink - local
    # above 2048 (the scores and the wide selection) on the same array
    cases = [(2, 4, 200_000, 512, 4, 32, None), (1, 3, 70_001, 256, 4, 64, 70_010), (2, 7, 20_000, 300, 4, 32, None),
             (1, 4, 12_000, 3000, 4, 32, None)]
    prepared = []
    for i, (BH, G, n, k, sink, local, m) in enumerate(cases):
        print(f"[noalloc] prepare BH={BH} G={G} n={n} k={k}", flush=True)
        st, plan, q = _case(BH, G, n, seed=31 + i)
        m = n if m is None else m
        ref = st.scan_topk(q, plan, k, sink, local, m=m)
        assert _lib.lib().fathom_scan_topk_workspace_bytes(BH, G, n, k, sink, local) <= SCRATCH
        prepared.append((st, plan, q, k, sink, local, m, ref, torch.full_like(ref, -1)))
    torch.cuda.synchronize()
    for st, plan, q, k, sink, local, m, ref, idx in prepared:
        print(f"[noalloc] call BH={q.shape[0]} G={q.shape[1]} n={st.n} k={k}", flush=True)
        _noalloc(st, plan, q, k, sink, local, m, idx)
        torch.cuda.synchronize()
        torch.testing.assert_close(idx, ref, rtol=0, atol=0)
    # once the array is resident, calls take no device memory
    free0 = torch.cuda.mem_get_info()[0]
    for st, plan, q, k, sink, local, m, ref, idx in prepared:
        idx.fill_(-1)
        _noalloc(st, plan, q, k, sink, local, m, idx)
        torch.cuda.synchronize()
        torch.testing.assert_close(idx, ref, rtol=0, atol=0)
    assert torch.cuda.mem_get_info()[0] == free0


def test_noalloc_fallback_rescan():
    """A falling row (its top kk in the first sampled tile: the sample's
    threshold misleads and the row's finalize workgroup rescans it) on the
    static array equals the workspace entry point."""
    print("[noalloc] fallback rescan", flush=True)
    BH, d, n = 2, 128, 90_000
    K = torch.zeros(BH, n, d)
    K[:, :, 0] = torch.linspace(3, -3, n)[None]
    K[:, :, 1] = torch.randn(BH, n, generator=torch.Generator().manual_seed(11)) * 0.01
    st = bp.PlaneStore(K.to(DEV))
    q = torch.zeros(BH, 4, d)
    q[:, :, 0] = 1.0
    q[:, 1::2, 1] = 1.0
    g = torch.ones(BH, d)
    g[:, 0], g[:, 1] = 1000.0, 10.0
    q, plan = q.to(DEV), bp.make_plan(g.to(DEV), 6.0)
    ref = st.scan_topk(q, plan, 512, 4, 32)
    idx = torch.full_like(ref, -1)
    _noalloc(st, plan, q, 512, 4, 32, n, idx)
    torch.cuda.synchronize()
    torch.testing.assert_close(idx, ref, rtol=0, atol=0)


def test_noalloc_fixed_positions_only_on_long_rows():
    """k == sink + local needs no workspace: accepted even where the selection's
    workspace would not fit the static array (rows of 2^20 tokens)."""
    print("[noalloc] k == sink + local at n = 2^20", flush=True)
    BH, G, n = 8, 4, 1 << 20
    assert _lib.lib().fathom_scan_topk_workspace_bytes(BH, G, n, 36, 4, 32) > SCRATCH
    st, plan, q = _case(BH, G, n, seed=5)
    ref = st.scan_topk(q, plan, 36, 4, 32)
    idx = torch.full_like(ref, -1)
    _noalloc(st, plan, q, 36, 4, 32, n, idx)
    torch.cuda.synchronize()
    torch.testing.assert_close(idx, ref, rtol=0, atol=0)


def test_noalloc_graph_replays_equal_eager():
    """One eager call (the array's address is looked up on a device's first
    call), then the call captured in a HIP graph and replayed with eager work
    and synchronisations between replays: every replay equals the workspace
    entry point."""
    print("[noalloc] graph capture", flush=True)
    st, plan, q = _case(2, 4, 100_000, seed=9)
    ref = st.scan_topk(q, plan, 512, 4, 32)
    idx = torch.full_like(ref, -1)
    _noalloc(st, plan, q, 512, 4, 32, st.n, idx)
    torch.cuda.synchronize()
    torch.testing.assert_close(idx, ref, rtol=0, atol=0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            _noalloc(st, plan, q, 512, 4, 32, st.n, idx)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        idx.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(idx, ref, rtol=0, atol=0)
        other = st.scan_topk(q, plan, 256, 4, 32)  # eager work between replays
        torch.cuda.synchronize()
        assert other.shape[-1] == 256


def test_noalloc_refuses_shapes_past_the_array():
    L = _lib.lib()
    need = L.fathom_scan_topk_workspace_bytes(8, 4, 1 << 20, 512, 4, 32)
    assert need > SCRATCH
    null = ctypes.c_void_p(0)
    rc = L.fathom_scan_topk_noalloc(null, 8, 4, 128, null, null, 4, 0, null, null, 1 << 20, (1 << 20) // 1024, 16,
                                    1 << 20, 512, 4, 32, null, null)
    assert rc == _lib.ERR_WORKSPACE
    assert b"static array holds" in L.fathom_last_error()
    rc = L.fathom_scan_topk_noalloc(null, 8, 9, 128, null, null, 4, 0, null, null, 4096, 4, 16, 4096, 64, 4, 32, null,
                                    null)
    assert rc == _lib.ERR_INVALID
