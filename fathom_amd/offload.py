"""Host-resident store support and the top-k row gather of the decode step
(scripts/B_e2e_offload_v2.py:29-39, 73-83, 224-244), on MI355X.

* host_mapped / free_host: pinned, GPU-mapped host memory (hipHostMalloc
  mapped|portable) holding a copy of a tensor; kernels read it zero-copy over
  PCIe through the returned DevPtr.
* gather_rows: the reference's row gather (idx < 0 -> zero row, no traffic).
* gather_union: the decode step's union of the G query heads' selections --
  every distinct host row is read once, duplicates are filled on the device,
  recent tokens (index >= n) come from a device buffer.
* select_and_gather: plan -> scan -> sink/local top-k -> union gather, the
  selection half of offload_attn (scripts/B_e2e_offload_v2.py:163-242).
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


def select_and_gather(store, q, var, budget, k, Ksrc, Vsrc, sink=4, local=32, m=None, Krec=None, Vrec=None,
                      dtype=torch.bfloat16):
    """One decode step's selection for all (batch, KV head) rows: g = sum_g q^2 var,
    plan, scan over `store` (HBM or host-resident), sink/local top-k, union row
    gather.  q [BH, G, D] fp32, var [BH, D].  Returns dict(plan, scores, idx, K, V,
    n_unique) -- scripts/B_e2e_offload_v2.py:181, 203, 224-241."""
    g = ((q.float() ** 2) * var[:, None, :]).sum(1)
    plan = make_plan(g, budget)
    scores = store.scan(q, plan)
    n = store.n
    m = n if m is None else m
    idx = sink_local_topk(scores, k, sink, local, m=m)
    Ks, Vs, nu = gather_union(idx, n, Ksrc, Vsrc, n, Krec, Vrec, dtype=dtype, d=q.shape[-1])
    return {"plan": plan, "scores": scores, "idx": idx, "K": Ks, "V": Vs, "n_unique": nu}
