"""Host-resident store support and the top-k row gather of the decode step
(scripts/B_e2e_offload_v2.py:29-39, 73-83, 224-244), on MI355X.

* host_mapped / free_host: pinned, GPU-mapped host memory (hipHostMalloc
  mapped|portable) holding a copy of a tensor; kernels read it zero-copy over
  PCIe through the returned DevPtr.
* gather_rows: the reference's row gather (idx < 0 -> zero row, no traffic).
* gather_union: the decode step's union of the G query heads' selections --
  every distinct host row is read once, duplicates are filled on the device,
  recent tokens (index >= n) come from a device buffer.
* select_and_gather: plan -> fused scan + sink/local top-k -> union gather, the
  selection half of offload_attn (scripts/B_e2e_offload_v2.py:163-242).
* chunk_bounds / stream_planes / stream_chan4: the chunked two-stream pipeline
  (scripts/B_e2e_offload_v2.py:103-144): chunk c + 1's runs cross PCIe on a copy
  stream while chunk c is scanned on a scan stream.
* gather_runs / host_store / copy_index: the copy-index path
  (scripts/B_e2e_offload_v2.py:62-71, 190-197, 267): a store in the
  whole-sequence layout (SUB = nblk) in mapped host memory, whose plan-selected
  runs (first t planes and the scales of every listed channel) are copied into
  an HBM staging store of the same layout and scanned there.
"""
import ctypes
import math

import torch

from . import _lib
from .bitplane import D, make_plan, sink_local_topk, _need_gpu, _ptr, _stream


class DevPtr:
    """Device-visible pointer duck-typed as a tensor for data_ptr() users
    (scripts/B_e2e_offload_v2.py:30-32)."""

    def __init__(self, ptr, dtype):
        self.ptr, self.dtype = ptr, dtype

    def data_ptr(self):
        return self.ptr


def host_mapped(t, coherent=True):
    """Copy tensor t into pinned, GPU-mapped host memory.  Returns (cpu view tensor,
    DevPtr for kernels, host pointer) -- scripts/B_e2e_offload_v2.py:33-38.
    Raises MemoryError when the pinned allocation fails."""
    nb = t.numel() * t.element_size()
    hp, dp = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("fathom_host_alloc_mapped", nb, 1 if coherent else 0, ctypes.byref(hp), ctypes.byref(dp))
    view = torch.frombuffer((ctypes.c_byte * nb).from_address(hp.value), dtype=t.dtype).view(t.shape)
    src = t.contiguous()
    if src.device.type == "cuda":
        _lib.call("fathom_memcpy", ctypes.c_void_p(hp.value), _ptr(src), nb, _stream(src.device))
        torch.cuda.current_stream(src.device).synchronize()
    else:
        view.copy_(src)
    return view, DevPtr(dp.value, t.dtype), hp.value


def free_host(hp):
    _lib.call("fathom_host_free", ctypes.c_void_p(hp))


def gather_runs(src, dst, off, ln, nrun, max_len, CH=4096):
    """Copy run r (4-byte words [off[r], off[r] + ln[r]) of src) to the same words of
    dst for r < nrun[0]; off/ln [R] and nrun [1] are device tensors, so no host sync
    -- scripts/B_e2e_offload_v2.py:62-71.  src/dst: tensors or DevPtr; CH is the
    reference's launch parameter (accepted, unused)."""
    _need_gpu(off, ln, nrun)
    off64 = off.contiguous().to(torch.int64)
    ln64 = ln.contiguous().to(torch.int64)
    nr = nrun.contiguous().to(torch.int32)
    _lib.call("fathom_gather_runs", ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), _ptr(off64),
              _ptr(ln64), _ptr(nr), int(off64.shape[0]), int(max_len), _stream(off.device))


def host_store(store):
    """A copy of a whole-sequence-layout PlaneStore or Chan4Store (built with
    bitplane.SUB = nblk) whose store words and scales live in mapped pinned host
    memory: the returned store's planes32 (chan_k) / scales_k are DevPtr objects, as
    the reference's offload does (scripts/B_e2e_offload_v2.py:267, 296-309).
    Returns (store, host pointers to free with free_host)."""
    from .bitplane import Chan4Store, PlaneStore
    if store.nsb != 1:
        raise ValueError("copy-index stores use the whole-sequence layout: build them with bitplane.SUB = nblk")
    c4 = isinstance(store, Chan4Store)
    _, pl, h1 = host_mapped(store.chan_k if c4 else store.planes_k)
    try:
        _, sc, h2 = host_mapped(store.scales_k)
    except Exception:
        free_host(h1)
        raise
    hs = (Chan4Store if c4 else PlaneStore).__new__(Chan4Store if c4 else PlaneStore)
    hs.BH, hs.n, hs.nsb, hs.sub = store.BH, store.n, store.nsb, store.sub
    hs.code, hs.scales_blk = None, None
    if c4:
        hs.chan_k = pl
    else:
        hs.planes32 = pl
    hs.scales_k = sc
    return hs, (h1, h2)


def staging_store(store, device=None):
    """An HBM store (PlaneStore or Chan4Store, as `store`) with store's shape and
    whole-sequence layout, words and scales zeroed: the target of copy_index and of
    the chunked pipeline."""
    from .bitplane import Chan4Store, PlaneStore
    if store.nsb != 1:
        raise ValueError("copy-index stores use the whole-sequence layout: build them with bitplane.SUB = nblk")
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    c4 = isinstance(store, Chan4Store)
    st = (Chan4Store if c4 else PlaneStore).__new__(Chan4Store if c4 else PlaneStore)
    st.BH, st.n, st.nsb, st.sub = store.BH, store.n, 1, store.sub
    st.code, st.scales_blk = None, None
    if c4:
        st.chan_k = torch.zeros(store.BH, 1, D, store.sub, 8, dtype=torch.int32, device=dev)
    else:
        st.planes_k = torch.zeros(store.BH, 1, D, 4, store.sub, dtype=torch.int64, device=dev)
        st.planes32 = st.planes_k.view(torch.int32)
    st.scales_k = torch.zeros(store.BH, 1, D, store.sub, dtype=torch.float16, device=dev)
    return st


def copy_index(src, staging, plan):
    """Stage the plan's runs -- the first t planes of every listed channel and its
    scales -- from src (a host_store) into staging (an HBM PlaneStore of the same
    whole-sequence layout), at the same offsets; no host sync
    (scripts/B_e2e_offload_v2.py:190-197).  Scanning staging afterwards equals
    scanning the full store."""
    t = plan["t"]
    _need_gpu(t)
    tt = t.contiguous().to(torch.int8)
    if src.nsb != 1 or staging.nsb != 1 or (src.BH, src.n, src.sub) != (staging.BH, staging.n, staging.sub):
        raise ValueError("copy_index needs two whole-sequence-layout stores of the same shape")
    BH, d = tt.shape
    _lib.call("fathom_copy_index", _ptr(tt), BH, d, int(staging.sub), ctypes.c_void_p(src.planes32.data_ptr()),
              ctypes.c_void_p(src.scales_k.data_ptr()), ctypes.c_void_p(staging.planes32.data_ptr()),
              ctypes.c_void_p(staging.scales_k.data_ptr()), _stream(tt.device))


def chunk_bounds(nblk, parts, align=64):
    """Block ranges [(b0, b1)] splitting nblk blocks into `parts` chunks whose interior
    boundaries are multiples of align (scripts/B_e2e_offload_v2.py:105-108)."""
    cuts = {0, nblk} | {min(nblk, (nblk * i // parts) // align * align) for i in range(1, parts)}
    edges = sorted(cuts)
    return list(zip(edges[:-1], edges[1:]))


_PIPE_STREAMS = {}


def _pipe_streams(dev):
    """The copy and scan streams of the pipeline on device dev (default priority)."""
    key = torch.device(dev).index
    if key not in _PIPE_STREAMS:
        _PIPE_STREAMS[key] = (torch.cuda.Stream(dev), torch.cuda.Stream(dev))
    return _PIPE_STREAMS[key]


def _stream_chunks(src, staging, t8, planes, block_bytes, data_attr, scan_chunk, n_out, q, parts):
    """Shared body of stream_planes / stream_chan4: per chunk of blocks, its runs are
    copied on the copy stream and the chunk is scanned on the scan stream after the
    copy's event, so chunk c + 1 crosses PCIe while chunk c is scanned."""
    dev = q.device
    BH, d = t8.shape
    nblk = int(staging.sub)
    s_copy, s_scan = _pipe_streams(dev)
    cur = torch.cuda.current_stream(dev)
    scores = torch.empty(BH, q.shape[1], n_out, device=dev, dtype=torch.float32)
    ev0 = torch.cuda.Event()
    ev0.record(cur)
    s_copy.wait_event(ev0)
    s_scan.wait_event(ev0)
    t8.record_stream(s_copy)
    scores.record_stream(s_scan)
    for b0, b1 in chunk_bounds(nblk, parts):
        with torch.cuda.stream(s_copy):
            _lib.call("fathom_copy_index_range", _ptr(t8), BH, d, nblk, b0, b1, block_bytes, planes,
                      ctypes.c_void_p(getattr(src, data_attr).data_ptr()), ctypes.c_void_p(src.scales_k.data_ptr()),
                      ctypes.c_void_p(getattr(staging, data_attr).data_ptr()),
                      ctypes.c_void_p(staging.scales_k.data_ptr()), _stream(dev))
            ev = torch.cuda.Event()
            ev.record(s_copy)
        with torch.cuda.stream(s_scan):
            s_scan.wait_event(ev)
            scan_chunk(scores, b0, b1)
    ev1 = torch.cuda.Event()
    ev1.record(s_scan)
    cur.wait_event(ev1)
    return scores


def stream_planes(src, staging, q, plan, parts=4):
    """Chunked copy-index scan (scripts/B_e2e_offload_v2.py:116-130 stream_planes):
    blocks are split by chunk_bounds; each chunk's plan-selected plane runs and
    scales go from src (host_store) into staging (staging_store) on a copy stream
    while the previous chunk is scanned on a scan stream.  Returns scores
    [BH, G, n], bit-identical to staging.scan after a whole copy_index."""
    t8 = plan["t"].contiguous().to(torch.int8)
    _need_gpu(q, t8)
    if src.nsb != 1 or staging.nsb != 1 or (src.BH, src.n, src.sub) != (staging.BH, staging.n, staging.sub):
        raise ValueError("stream_planes needs two whole-sequence-layout stores of the same shape")
    return _stream_chunks(src, staging, t8, 4, 8, "planes32",
                          lambda out, b0, b1: staging.scan(q, plan, out=out, blocks=(b0, b1)), staging.n, q, parts)


def stream_chan4(src, staging, q, active, act, nact, parts=4):
    """The chan4 store's chunked copy-index scan (scripts/B_e2e_offload_v2.py:132-144
    stream_chan4): the active channels' nibble runs and scales of each chunk are
    copied while the previous chunk is scanned.  Returns scores [BH, G, n]."""
    a8 = active.contiguous().to(torch.int8)
    _need_gpu(q, a8)
    if src.nsb != 1 or staging.nsb != 1 or (src.BH, src.n, src.sub) != (staging.BH, staging.n, staging.sub):
        raise ValueError("stream_chan4 needs two whole-sequence-layout stores of the same shape")
    return _stream_chunks(src, staging, a8, 1, 32, "chan_k",
                          lambda out, b0, b1: staging.scan(q, act, nact, out=out, blocks=(b0, b1)), staging.n, q,
                          parts)


def gather_rows(src, cap, idx, BH, dtype=torch.bfloat16, d=D):
    """dst[bh, r, :] = src[bh, idx[bh, r], :] for rows of d elements of dtype; src may
    live in mapped host memory (zero-copy); idx < 0 (or >= cap) gives a zero row --
    scripts/B_e2e_offload_v2.py:73-83."""
    _need_gpu(idx)
    idx32 = idx.contiguous().to(torch.int32)
    R = idx32.shape[1]
    dst = torch.empty(BH, R, d, device=idx.device, dtype=dtype)
    row_bytes = d * dst.element_size()
    _lib.call("fathom_gather_rows", ctypes.c_void_p(src.data_ptr()), int(cap), _ptr(idx32), BH, R, row_bytes,
              _ptr(dst), _stream(idx.device))
    return dst


def gather_union(idx, n, Ksrc, Vsrc, cap, Krec=None, Vrec=None, dtype=torch.bfloat16, d=D):
    """idx [BH, G, k] selected tokens -> (Ks, Vs) [BH, G, k, d] of dtype and the number
    of distinct host rows fetched per row [BH] int32.  Tokens < n are read from
    Ksrc/Vsrc [BH, cap, d] (tensor or DevPtr, usually mapped host memory), each
    distinct token once; tokens >= n from Krec/Vrec [BH, nrec, d] (device) at row
    clamp(idx - n, 0, nrec - 1); negative tokens give zero rows
    (scripts/B_e2e_offload_v2.py:228-241)."""
    _need_gpu(idx)
    BH, G, k = idx.shape
    GK = G * k
    flat = idx.reshape(BH, GK).contiguous().to(torch.int64)
    dev = idx.device
    Ks = torch.empty(BH, G, k, d, device=dev, dtype=dtype)
    Vs = torch.empty(BH, G, k, d, device=dev, dtype=dtype)
    nu = torch.empty(BH, device=dev, dtype=torch.int32)
    nbytes = _lib.lib().fathom_gather_union_workspace_bytes(BH, GK)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    row_bytes = d * Ks.element_size()
    nrec = 0
    if Krec is not None:
        Krec = Krec.reshape(BH, -1, d).contiguous()
        Vrec = Vrec.reshape(BH, -1, d).contiguous()
        nrec = Krec.shape[1]
    _lib.call("fathom_gather_union", _ptr(flat), BH, GK, int(n), ctypes.c_void_p(Ksrc.data_ptr()),
              ctypes.c_void_p(Vsrc.data_ptr()), int(cap), _ptr(Krec), _ptr(Vrec), nrec, row_bytes, _ptr(Ks), _ptr(Vs),
              _ptr(nu), _ptr(ws), nbytes, _stream(dev))
    return Ks, Vs, nu


def gather_attention(q, idx, n, Ksrc, Vsrc, cap, Krec=None, Vrec=None, scale=None, unique=None):
    """Exact attention over the selected rows, fused with their gather:
    out[bh, g] = softmax(scale * q[bh, g] . K[idx[bh, g]]) . V[idx[bh, g]] in fp32
    over bf16 rows of D = 128 (scripts/B_kernel_bench.py:22-27;
    scripts/B_e2e_offload_v2.py:228-244).  Row sources as in gather_union: tokens
    < n from Ksrc/Vsrc [BH, cap, D] (tensor or DevPtr, HBM or mapped host), tokens
    >= n from Krec/Vrec, negative tokens as zero rows.  unique=True forms each row's
    union first, so each distinct token is read once, and returns its size;
    unique=False reads the rows per selected position with one launch fewer (for
    rows in device memory) and returns n_unique None; the default is True for
    mapped host rows (DevPtr) and False for tensors, and False beyond G <= 8
    and G * k <= 16384 positions per row (there unique=True only adds the
    counts, from a hash table in global memory; the rows are read per
    position either way).  scale defaults to D ** -0.5.
    Returns (out [BH, G, D] fp32, n_unique [BH] int32 or None)."""
    _need_gpu(q, idx)
    BH, G, k = idx.shape
    if q.shape != (BH, G, D):
        raise ValueError(f"gather_attention: q {tuple(q.shape)} must be [BH, G, {D}] = [{BH}, {G}, {D}]")
    for name, t in (("Ksrc", Ksrc), ("Vsrc", Vsrc), ("Krec", Krec), ("Vrec", Vrec)):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"gather_attention: {name} must hold bf16 rows, got {t.dtype}")
    dev = q.device
    qf = q.float().contiguous()
    flat = idx.contiguous().to(torch.int64)
    out = torch.empty(BH, G, D, device=dev, dtype=torch.float32)
    if unique is None:
        unique = isinstance(Ksrc, DevPtr) and G <= 8 and G * k <= 16384
    nu = torch.empty(BH, device=dev, dtype=torch.int32) if unique else None
    nbytes = _lib.lib().fathom_gather_attention_workspace_bytes(BH, G, k)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    nrec = 0
    if Krec is not None:
        Krec = Krec.reshape(BH, -1, D).contiguous()
        Vrec = Vrec.reshape(BH, -1, D).contiguous()
        nrec = Krec.shape[1]
    sc = float(D) ** -0.5 if scale is None else float(scale)
    _lib.call("fathom_gather_attention", _ptr(qf), _ptr(flat), BH, G, k, int(n), ctypes.c_void_p(Ksrc.data_ptr()),
              ctypes.c_void_p(Vsrc.data_ptr()), int(cap), _ptr(Krec), _ptr(Vrec), nrec, sc, _ptr(out), _ptr(nu),
              _ptr(ws), nbytes, _stream(dev))
    return out, nu


def gather_attn(q, Kc, Vc, idx):
    """Drop-in for scripts/B_kernel_bench.py:22 gather_attn: q [BH, G, D] fp32,
    Kc/Vc [BH, n, D] bf16 (device), idx [BH, G, k] -> [BH, G, D] fp32."""
    n = Kc.shape[1]
    out, _ = gather_attention(q, idx, n, Kc.contiguous(), Vc.contiguous(), n)
    return out


def select_and_gather(store, q, var, budget, k, Ksrc, Vsrc, sink=4, local=32, m=None, Krec=None, Vrec=None,
                      dtype=torch.bfloat16, scores=False):
    """One decode step's selection for all (batch, KV head) rows: g = sum_g q^2 var,
    plan, scan over `store` (HBM or host-resident), sink/local top-k, union row
    gather.  q [BH, G, D] fp32, var [BH, D].  Returns dict(plan, scores, idx, K, V,
    n_unique) -- scripts/B_e2e_offload_v2.py:181, 203, 224-241.

    The selection is the fused scan + top-k (store.scan_topk: no score tensor,
    "scores" is None); scores=True runs the reference's two steps instead (the
    score rows, then sink_local_topk of them) and returns the scores too.  Both
    select the same indices."""
    g = ((q.float() ** 2) * var[:, None, :]).sum(1)
    plan = make_plan(g, budget)
    n = store.n
    m = n if m is None else m
    if scores:
        scores = store.scan(q, plan)
        idx = sink_local_topk(scores, k, sink, local, m=m)
    else:
        scores = None
        idx = store.scan_topk(q, plan, k, sink, local, m=m)
    Ks, Vs, nu = gather_union(idx, n, Ksrc, Vsrc, n, Krec, Vrec, dtype=dtype, d=q.shape[-1])
    return {"plan": plan, "scores": scores, "idx": idx, "K": Ks, "V": Vs, "n_unique": nu}
