"""Drop-in replacement of the reference module kernels/bitplane.py on MI355X.

Same names, arguments, defaults, return shapes and dtypes as the reference
(import it the same way: ``from fathom_amd.bitplane import *``); every tensor
operation runs in the hand-written gfx950 kernels of libfathom_hip.so through
its C ABI, asynchronously on the current torch stream.  Inputs must live on the
GPU (or, for store/row buffers, in mapped pinned host memory): there is no CPU
path, and a missing library raises ImportError.

Store semantics (per 64-token block and channel j): 4-bit mid-rise code c in
[0, 16) with block absmax a: value = (c + 0.5 - 8) * a / 8.  Bit p (0 = MSB) of
the block's 64 codes is one 64-bit plane word; reading the top t planes gives
c_t = c >> (4 - t) and value_t = (c_t + 0.5 - 2^(t-1)) * a / 2^(t-1), the t-bit
mid-rise quantiser with the same scale.  The kernel order is the reference's
superblock layout planes_k [BH, nsb, D, 4, SUB] / scales_k [BH, nsb, D, SUB],
so each (channel, plane) unit of a superblock is SUB*8 contiguous bytes.

Module globals BLK, SUB, D, SBT, and the class attributes PlaneStore.kernel /
cls_cfg / fma_cfg, exist for compatibility with callers that set them
(kernels/bitplane.py:19-20, 317-339).  SUB selects the superblock size of stores
built afterwards (SUB = nblk gives the whole-sequence layout); the launch
configuration attributes are accepted and ignored (one exact kernel serves
every setting).
"""
import ctypes
import math

import torch

from . import _lib

BLK, SUB, D = 64, 16, 128
SBT = BLK * SUB
# stages of PlaneStore.scan_topk_stages (FATHOM_STAGE_* of include/fathom_hip.h)
STAGE_SAMPLE, STAGE_SELECT, STAGE_CANDIDATES, STAGE_FINALIZE, STAGE_ALL = 1, 2, 4, 8, 15

__all__ = ["BLK", "SUB", "D", "SBT", "quantise_u4", "dequant_planes", "pack_planes", "unpack_planes",
           "to_superblocks", "pack_chan4", "bytes_planes", "bytes_chan4", "make_plan", "make_plan_torch",
           "channel_list", "scan_planes_reference", "scan_chan4_reference", "PlaneStore", "Chan4Store",
           "sink_local_topk"]


# ----------------------------------------------------------------------------- helpers
def _stream(dev=None):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ptr(x):
    return ctypes.c_void_p(x.data_ptr()) if x is not None else ctypes.c_void_p(0)


def _need_gpu(*tensors):
    for t in tensors:
        if torch.is_tensor(t) and t.device.type != "cuda":
            raise ValueError(f"fathom_amd runs on the GPU; got a tensor on {t.device} "
                             "(move inputs to the device, there is no CPU path)")


_KDT = {torch.float32: _lib.DT_F32, torch.float16: _lib.DT_F16, torch.bfloat16: _lib.DT_BF16}


def _key_input(K):
    """Keys as a contiguous fp32/fp16/bf16 tensor (other dtypes go through float32)."""
    if K.dtype not in _KDT:
        K = K.float()
    return K.contiguous()


def _lead(shape):
    return int(math.prod(shape)) if len(shape) else 1


# ----------------------------------------------------------------------------- quantiser + packing
def quantise_u4(K, scale_dtype=torch.float16):
    """K [..., n, D] -> codes uint8 [..., n, D] in [0, 16) and scales [..., nblk, D]
    (block absmax in scale_dtype) -- kernels/bitplane.py:23-32.

    code = clamp(floor(x / (amax / 8)), -8, 7) + 8 with amax the block's absmax
    clamped to 1e-8 and rounded to scale_dtype (round to nearest even)."""
    _need_gpu(K)
    if scale_dtype not in _KDT:
        raise ValueError(f"scale_dtype {scale_dtype} unsupported (float16, bfloat16, float32)")
    Kc = _key_input(K)
    *lead, n, d = Kc.shape
    nb = math.ceil(n / BLK)
    code = torch.empty(*lead, n, d, dtype=torch.uint8, device=K.device)
    scales = torch.empty(*lead, nb, d, dtype=scale_dtype, device=K.device)
    _lib.call("fathom_quantise_pack", _ptr(Kc), _KDT[Kc.dtype], _lead(lead), n, d, _KDT[scale_dtype], 0,
              _ptr(code), _ptr(scales), None, None, None, _stream(K.device))
    return code, scales


def dequant_planes(code, scales, t):
    """Reference dequantisation of the top-t planes (t int tensor [D] or scalar):
    [..., n, D] fp32 -- kernels/bitplane.py:34-42."""
    _need_gpu(code, scales)
    if scales.dtype not in _KDT:
        raise ValueError(f"scale dtype {scales.dtype} unsupported")
    code = code.contiguous()
    scales = scales.contiguous()
    *lead, n, d = code.shape
    tt = torch.as_tensor(t, device=code.device).to(torch.int32)
    tt = (tt.expand(d) if tt.dim() == 0 else tt).contiguous()
    if tt.shape != (d,):
        raise ValueError(f"t must be a scalar or [{d}], got {tuple(tt.shape)}")
    out = torch.empty(*lead, n, d, dtype=torch.float32, device=code.device)
    _lib.call("fathom_dequant_planes", _ptr(code), _ptr(scales), _KDT[scales.dtype], _ptr(tt), _lead(lead), n, d,
              _ptr(out), _stream(code.device))
    return out


def pack_planes(code):
    """codes uint8 [..., n, D] -> logical planes int64 [..., nblk, D, 4] (bit i of
    planes[b, j, p] = bit p (0 = MSB) of token 64b+i's code) -- kernels/bitplane.py:44-50."""
    _need_gpu(code)
    code = code.contiguous().to(torch.uint8)
    *lead, n, d = code.shape
    nb = math.ceil(n / BLK)
    planes = torch.empty(*lead, nb, d, 4, dtype=torch.int64, device=code.device)
    _lib.call("fathom_pack_planes", _ptr(code), _lead(lead), n, d, _ptr(planes), _stream(code.device))
    return planes


def unpack_planes(planes, n):
    """Inverse of pack_planes: int64 [..., nblk, D, 4] -> codes uint8 [..., n, D] -- kernels/bitplane.py:52-58."""
    _need_gpu(planes)
    planes = planes.contiguous()
    *lead, nb, d, four = planes.shape
    if four != 4:
        raise ValueError("planes must have a trailing dimension of 4")
    code = torch.empty(*lead, n, d, dtype=torch.uint8, device=planes.device)
    _lib.call("fathom_unpack_planes", _ptr(planes), _lead(lead), nb, d, n, _ptr(code), _stream(planes.device))
    return code


def to_superblocks(planes, scales):
    """Logical [..., nblk, D, 4] / [..., nblk, D] -> kernel order [..., nsb, D, 4, SUB] int64 /
    [..., nsb, D, SUB] (scales' dtype), zero padded to whole superblocks, SUB = the module
    global at call time -- kernels/bitplane.py:60-65."""
    _need_gpu(planes, scales)
    planes = planes.contiguous()
    scales = scales.contiguous()
    *lead, nb, d, _ = planes.shape
    sub = int(SUB)
    nsb = math.ceil(nb / sub)
    pl = torch.empty(*lead, nsb, d, 4, sub, dtype=torch.int64, device=planes.device)
    sc = torch.empty(*lead, nsb, d, sub, dtype=scales.dtype, device=planes.device)
    _lib.call("fathom_to_superblocks", _ptr(planes), _ptr(scales), scales.element_size(), _lead(lead), nb, d, sub,
              _ptr(pl), _ptr(sc), _stream(planes.device))
    return pl, sc


def pack_chan4(code):
    """codes uint8 [..., n, D] -> the channel-major 4-bit store int32 [..., nsb, D, SUB, 8]
    (word m of a (channel, block) holds tokens 8m..8m+7, nibble k = token 8m + k;
    zero padded to whole superblocks of SUB blocks) -- kernels/bitplane.py:67-74."""
    _need_gpu(code)
    code = code.contiguous().to(torch.uint8)
    *lead, n, d = code.shape
    sub = int(SUB)
    nsb = math.ceil(math.ceil(n / BLK) / sub)
    words = torch.empty(*lead, nsb, d, sub, 8, dtype=torch.int32, device=code.device)
    _lib.call("fathom_pack_chan4", _ptr(code), _lead(lead), n, d, sub, _ptr(words), _stream(code.device))
    return words


def bytes_chan4(nact, n):
    """Bytes a chan4 scan moves: (32 + 2) per listed channel and 64-token block --
    kernels/bitplane.py:79-80."""
    nb = math.ceil(n / BLK)
    return float((nact.float() * (32 + 2) * nb).sum())


def channel_list(active):
    """active bool [BH, D] -> (act int32 [BH, D]: listed channels first, ascending,
    then the others; nact int32 [BH]) -- kernels/bitplane.py:128-132."""
    _need_gpu(active)
    BH, d = active.shape
    a8 = active.contiguous().to(torch.uint8)
    act = torch.empty(BH, d, dtype=torch.int32, device=active.device)
    nact = torch.empty(BH, dtype=torch.int32, device=active.device)
    _lib.call("fathom_channel_list", _ptr(a8), BH, d, _ptr(act), _ptr(nact), _stream(active.device))
    return act, nact


def bytes_planes(t, n):
    """Bytes a scan moves for plans t [BH, D] (planes per channel) over n tokens:
    sum_j 8*t_j + 2*#active per 64-token block -- kernels/bitplane.py:76-78."""
    nb = math.ceil(n / BLK)
    return float(((t.float().sum(-1) * 8 + (t > 0).float().sum(-1) * 2) * nb).sum())


# ----------------------------------------------------------------------------- plan
def make_plan(g, budget, bmax=4, iters=30):
    """g [BH, D] fp32 group-summed gain q_j^2 Var(k_j); budget scalar or [BH] (code
    bits per token).  Returns the reference's dict of device tensors: t int8
    [BH, D], pairs int32 [BH, D*bmax], npairs [BH], act [BH, D], nact [BH], cls
    [BH, bmax, D], clsn [BH, bmax] -- kernels/bitplane.py:83-116."""
    _need_gpu(g)
    BH, d = g.shape
    dev = g.device
    gf = g.contiguous().float()
    t = torch.empty(BH, d, dtype=torch.int8, device=dev)
    pairs = torch.empty(BH, d * bmax, dtype=torch.int32, device=dev)
    npairs = torch.empty(BH, dtype=torch.int32, device=dev)
    act = torch.empty(BH, d, dtype=torch.int32, device=dev)
    nact = torch.empty(BH, dtype=torch.int32, device=dev)
    cls = torch.empty(BH, bmax, d, dtype=torch.int32, device=dev)
    clsn = torch.empty(BH, bmax, dtype=torch.int32, device=dev)
    outs = (_ptr(t), _ptr(pairs), _ptr(npairs), _ptr(act), _ptr(nact), _ptr(cls), _ptr(clsn), _stream(dev))
    # a host-side bound on sum(t) (the bisection keeps it within the budget),
    # known without a device sync for float budgets and host tensors; the scan
    # uses it only to pick its register layout
    units_max = 0
    if torch.is_tensor(budget):
        if budget.device.type == "cpu" and budget.numel() > 0:
            bmx = float(budget.float().max())
            units_max = int(math.floor(bmx)) if math.isfinite(bmx) else 0
        budget = budget.to(device=dev, dtype=torch.float32).expand(BH).contiguous()
        _lib.call("fathom_make_plan", _ptr(gf), _ptr(budget), BH, d, int(bmax), int(iters), *outs)
    else:  # one float for every row: a kernel argument
        bf = float(budget)
        units_max = int(math.floor(bf)) if math.isfinite(bf) else 0
        _lib.call("fathom_make_plan_uniform", _ptr(gf), bf, BH, d, int(bmax), int(iters), *outs)
    units_max = max(0, min(units_max, int(bmax) * d)) if units_max > 0 else 0
    return {"t": t, "pairs": pairs, "npairs": npairs, "act": act, "nact": nact, "cls": cls, "clsn": clsn,
            "units_max": units_max}


def make_plan_torch(g, budget, bmax=4, iters=30):
    """The plan's depths as a float tensor [BH, D] (the reference's torch form,
    kernels/bitplane.py:118-126), computed by the same gfx950 plan kernel."""
    return make_plan(g, budget, bmax, iters)["t"].float()


# ----------------------------------------------------------------------------- store + scan
def _units_max(plan):
    """The plan's host-side bound on sum(t) per row (0: unknown)."""
    return int(plan.get("units_max", 0)) if isinstance(plan, dict) else 0


def _plan_classes(plan, BH, d):
    """The plan's depth-class lists as the scan kernels read them: cls int32
    [BH, bmax, D] and clsn int32 [BH, bmax], contiguous, on the GPU."""
    cls, clsn = plan["cls"], plan["clsn"]
    _need_gpu(cls, clsn)
    if cls.dim() != 3 or cls.shape[0] != BH or cls.shape[2] != d or tuple(clsn.shape) != tuple(cls.shape[:2]):
        raise ValueError(f"plan cls/clsn of shapes {tuple(cls.shape)}/{tuple(clsn.shape)} do not match BH={BH}, D={d}")
    return cls.to(torch.int32).contiguous(), clsn.to(torch.int32).contiguous()


# Query heads per scan launch: a matrix row tile of the scan kernels holds 8
# heads x {hi, lo} weights.  The store methods run more heads (G > 8) as groups
# of at most 8 over the same store, one launch each.
G_CALL = 8


def _head_groups(G):
    return [(g0, min(g0 + G_CALL, G)) for g0 in range(0, G, G_CALL)]


class PlaneStore:
    """K [BH, n, D] (any float dtype, on the GPU) -> superblock-ordered bit-plane
    store on the same device (kernels/bitplane.py:310-340).

    Attributes as in the reference: BH, n, code [BH, n, D] uint8 (dropped with
    keep_code=False), scales_blk [BH, nblk, D], planes_k [BH, nsb, D, 4, SUB]
    int64, scales_k [BH, nsb, D, SUB] fp16, nsb, planes32 (int32 view).  The
    planes/scales attributes may be replaced by objects with a data_ptr() into
    mapped host memory (the reference's DevPtr idiom); scan then reads the store
    zero-copy over PCIe."""

    kernel = "cls"
    fma_cfg = {"NB": 2, "KK": 8, "num_warps": 1, "num_stages": 1}
    cls_cfg = {"NB": 4, "KK": 4, "num_warps": 1, "num_stages": 1}

    def __init__(self, K, scale_dtype=torch.float16, keep_code=True):
        _need_gpu(K)
        self.BH, self.n, d = K.shape
        if d != D:
            raise AssertionError(f"PlaneStore needs D == {D}, got {d}")
        if scale_dtype not in _KDT:
            raise ValueError(f"scale_dtype {scale_dtype} unsupported")
        Kc = _key_input(K)
        dev = K.device
        nb = math.ceil(self.n / BLK)
        self.sub = int(SUB)
        self.nsb = math.ceil(nb / self.sub)
        self.code = torch.empty(self.BH, self.n, d, dtype=torch.uint8, device=dev) if keep_code else None
        self.scales_blk = torch.empty(self.BH, nb, d, dtype=scale_dtype, device=dev)
        self.planes_k = torch.empty(self.BH, self.nsb, d, 4, self.sub, dtype=torch.int64, device=dev)
        self.scales_k = torch.empty(self.BH, self.nsb, d, self.sub, dtype=torch.float16, device=dev)
        _lib.call("fathom_quantise_pack", _ptr(Kc), _KDT[Kc.dtype], self.BH, self.n, d, _KDT[scale_dtype], self.sub,
                  _ptr(self.code), _ptr(self.scales_blk), None, _ptr(self.planes_k), _ptr(self.scales_k),
                  _stream(dev))
        self.planes32 = self.planes_k.view(torch.int32)

    def scan(self, q, plan, out=None, blocks=None):
        """q [BH, G, D] fp32, plan from make_plan -> scores fp32 [BH, G, n];
        blocks=(b0, b1) scans only 64-token blocks [b0, b1) into `out`."""
        _need_gpu(q)
        BH, G, d = q.shape
        if BH != self.BH:
            raise AssertionError(f"q has BH={BH}, store has {self.BH}")
        if plan["cls"].shape[1] > 4:
            raise ValueError("the store holds 4 planes: plan with bmax <= 4")
        out = torch.empty(BH, G, self.n, device=q.device, dtype=torch.float32) if out is None else out
        if out.dtype != torch.float32 or not out.is_contiguous() or tuple(out.shape) != (BH, G, self.n):
            raise ValueError(f"out must be a contiguous float32 [{BH}, {G}, {self.n}] tensor")
        if G > G_CALL:
            for g0, g1 in _head_groups(G):
                part = out[:, g0:g1].contiguous()
                PlaneStore.scan(self, q[:, g0:g1], plan, out=part, blocks=blocks)
                out[:, g0:g1].copy_(part)
            return out
        nb = math.ceil(self.n / BLK)
        b0, b1 = (0, nb) if blocks is None else (int(blocks[0]), int(blocks[1]))
        sub = int(getattr(self, "sub", SUB))
        qc = q.contiguous().float()
        cls, clsn = _plan_classes(plan, BH, d)
        _lib.call("fathom_scan_planes", _ptr(qc), BH, G, d, _ptr(cls), _ptr(clsn), cls.shape[1], _units_max(plan),
                  ctypes.c_void_p(self.planes32.data_ptr()), ctypes.c_void_p(self.scales_k.data_ptr()), self.n,
                  int(self.nsb), sub, b0, b1, _ptr(out), _stream(q.device))
        return out

    def scan_topk(self, q, plan, k, sink=4, local=32, m=None):
        """Fused scan + sink/local top-k: the same int64 indices [BH, G, k] as
        sink_local_topk(self.scan(q, plan), k, sink, local, m), without writing the
        score tensor (the scan keeps only candidates above a sampled threshold)."""
        _need_gpu(q)
        BH, G, d = q.shape
        if BH != self.BH:
            raise AssertionError(f"q has BH={BH}, store has {self.BH}")
        if plan["cls"].shape[1] > 4:
            raise ValueError("the store holds 4 planes: plan with bmax <= 4")
        if G > G_CALL:
            return torch.cat([PlaneStore.scan_topk(self, q[:, g0:g1], plan, k, sink, local, m) for g0, g1 in _head_groups(G)], 1)
        n = self.n
        m = n if m is None else int(m)
        sub = int(getattr(self, "sub", SUB))
        qc = q.contiguous().float()
        idx = torch.empty(BH, G, int(k), dtype=torch.int64, device=q.device)
        L = _lib.lib()
        nbytes = L.fathom_scan_topk_workspace_bytes(BH, G, n, int(k), int(sink), int(local))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        cls, clsn = _plan_classes(plan, BH, d)
        _lib.call("fathom_scan_topk", _ptr(qc), BH, G, d, _ptr(cls), _ptr(clsn), cls.shape[1], _units_max(plan),
                  ctypes.c_void_p(self.planes32.data_ptr()), ctypes.c_void_p(self.scales_k.data_ptr()), n,
                  int(self.nsb), sub, m, int(k), int(sink), int(local), _ptr(idx), _ptr(ws), nbytes,
                  _stream(q.device))
        return idx

    def _plan_call_args(self, q, g, budget, bmax):
        """Shared argument checks of the plan_scan_topk calls: (qc, gf, budget
        pointer tensor or None, budget value, units bound)."""
        _need_gpu(q, g)
        BH, G, d = q.shape
        if BH != self.BH:
            raise AssertionError(f"q has BH={BH}, store has {self.BH}")
        if tuple(g.shape) != (BH, d):
            raise ValueError(f"plan_scan_topk: g {tuple(g.shape)} must be [BH, D] = [{BH}, {d}]")
        if bmax > 4:
            raise ValueError("the store holds 4 planes: plan with bmax <= 4")
        units_max, bptr, bval = 0, None, 0.0
        if torch.is_tensor(budget):
            if budget.device.type == "cpu" and budget.numel() > 0:
                bmx = float(budget.float().max())
                units_max = int(math.floor(bmx)) if math.isfinite(bmx) else 0
            bptr = budget.to(device=q.device, dtype=torch.float32).expand(BH).contiguous()
        else:
            bval = float(budget)
            units_max = int(math.floor(bval)) if math.isfinite(bval) else 0
        units_max = max(0, min(units_max, int(bmax) * d)) if units_max > 0 else 0
        return q.contiguous().float(), g.contiguous().float(), bptr, bval, units_max

    def plan_scan_topk_attention(self, q, g, budget, k, Ksrc, Vsrc, sink=4, local=32, m=None, bmax=4, iters=30,
                                 scale=None):
        """plan_scan_topk(q, g, budget, k, ...) then offload.gather_attention over its
        indices with K/V bf16 rows [BH, cap, 128] in device memory: the decode
        step's plan -> scan -> top-k -> gather + attention chain
        (scripts/B_kernel_bench.py:64-101) in one call.  Rows of at most 32768
        tokens with k <= 512 select and attend in the same workgroups.  Returns
        (idx [BH, G, k] int64, out [BH, G, 128] fp32), equal to the separate
        calls'."""
        _need_gpu(q, g, Ksrc, Vsrc)
        BH, G, d = q.shape
        for name, t in (("Ksrc", Ksrc), ("Vsrc", Vsrc)):
            if t.dtype != torch.bfloat16 or t.dim() != 3 or t.shape[0] != BH or t.shape[2] != d or not t.is_contiguous():
                raise ValueError(f"plan_scan_topk_attention: {name} must be contiguous bf16 [BH, cap, {d}]")
        if Ksrc.shape != Vsrc.shape:
            raise ValueError("plan_scan_topk_attention: Ksrc and Vsrc shapes differ")
        if G > G_CALL:
            parts = [PlaneStore.plan_scan_topk_attention(self, q[:, g0:g1], g, budget, k, Ksrc, Vsrc, sink, local, m,
                                                         bmax, iters, scale) for g0, g1 in _head_groups(G)]
            return torch.cat([r[0] for r in parts], 1), torch.cat([r[1] for r in parts], 1)
        qc, gf, bptr, bval, units_max = self._plan_call_args(q, g, budget, bmax)
        n = self.n
        m = n if m is None else int(m)
        sub = int(getattr(self, "sub", SUB))
        idx = torch.empty(BH, G, int(k), dtype=torch.int64, device=q.device)
        out = torch.empty(BH, G, d, dtype=torch.float32, device=q.device)
        sc = float(d) ** -0.5 if scale is None else float(scale)
        L = _lib.lib()
        nbytes = L.fathom_plan_scan_topk_attention_workspace_bytes(BH, G, d, int(bmax), n, int(k), int(sink), int(local))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        _lib.call("fathom_plan_scan_topk_attention", _ptr(qc), _ptr(gf), _ptr(bptr), bval, BH, G, d, int(bmax),
                  int(iters), units_max, ctypes.c_void_p(self.planes32.data_ptr()),
                  ctypes.c_void_p(self.scales_k.data_ptr()), n, int(self.nsb), sub, m, int(k), int(sink), int(local),
                  _ptr(idx), None, ctypes.c_void_p(Ksrc.data_ptr()), ctypes.c_void_p(Vsrc.data_ptr()), int(Ksrc.shape[1]),
                  sc, _ptr(out), _ptr(ws), nbytes, _stream(q.device))
        return idx, out

    def plan_scan_topk(self, q, g, budget, k, sink=4, local=32, m=None, bmax=4, iters=30, return_t=False):
        """make_plan(g, budget, bmax, iters) then scan_topk(q, plan, k, sink, local, m)
        in one call (kernels/bitplane.py:83-116, then the scan and top-k): the same
        indices [BH, G, k].  Rows of at most 32768 tokens are planned inside the
        scan's prologue, so no plan launch precedes it (the decode chain of
        scripts/B_kernel_bench.py:74).  return_t=True also returns the plan's
        depths t [BH, D] int8."""
        BH, G, d = q.shape
        if G > G_CALL:
            parts = [PlaneStore.plan_scan_topk(self, q[:, g0:g1], g, budget, k, sink, local, m, bmax, iters, True)
                     for g0, g1 in _head_groups(G)]
            idx = torch.cat([r[0] for r in parts], 1)
            return (idx, parts[0][1]) if return_t else idx
        qc, gf, bptr, bval, units_max = self._plan_call_args(q, g, budget, bmax)
        n = self.n
        m = n if m is None else int(m)
        sub = int(getattr(self, "sub", SUB))
        idx = torch.empty(BH, G, int(k), dtype=torch.int64, device=q.device)
        t = torch.empty(BH, d, dtype=torch.int8, device=q.device) if return_t else None
        L = _lib.lib()
        nbytes = L.fathom_plan_scan_topk_workspace_bytes(BH, G, d, int(bmax), n, int(k), int(sink), int(local))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        _lib.call("fathom_plan_scan_topk", _ptr(qc), _ptr(gf), _ptr(bptr), bval, BH, G, d, int(bmax), int(iters),
                  units_max, ctypes.c_void_p(self.planes32.data_ptr()), ctypes.c_void_p(self.scales_k.data_ptr()), n,
                  int(self.nsb), sub, m, int(k), int(sink), int(local), _ptr(idx), _ptr(t), _ptr(ws), nbytes,
                  _stream(q.device))
        return (idx, t) if return_t else idx

    def scan_topk_stages(self, q, plan, k, stages, ws=None, idx=None, sink=4, local=32, m=None):
        """Stages of scan_topk (bit mask of STAGE_*) on a caller-kept workspace
        (bench.py times the candidate pass alone this way; the reference has no
        counterpart).  Returns (idx, ws); pass both back to run later stages
        over the state the earlier ones left."""
        _need_gpu(q)
        BH, G, d = q.shape
        n = self.n
        m = n if m is None else int(m)
        sub = int(getattr(self, "sub", SUB))
        qc = q.contiguous().float()
        L = _lib.lib()
        nbytes = L.fathom_scan_topk_workspace_bytes(BH, G, n, int(k), int(sink), int(local))
        if idx is None:
            idx = torch.empty(BH, G, int(k), dtype=torch.int64, device=q.device)
        if ws is None:
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        if ws.numel() < nbytes:
            raise ValueError(f"workspace of {ws.numel()} bytes, need {nbytes}")
        cls, clsn = _plan_classes(plan, BH, d)
        _lib.call("fathom_scan_topk_stages", _ptr(qc), BH, G, d, _ptr(cls), _ptr(clsn), cls.shape[1], _units_max(plan),
                  ctypes.c_void_p(self.planes32.data_ptr()), ctypes.c_void_p(self.scales_k.data_ptr()), n,
                  int(self.nsb), sub, m, int(k), int(sink), int(local), _ptr(idx), _ptr(ws), nbytes, int(stages),
                  _stream(q.device))
        return idx, ws

    def nbytes(self):
        return self.BH * self.nsb * D * 4 * int(getattr(self, "sub", SUB)) * 8 + \
            self.BH * self.nsb * D * int(getattr(self, "sub", SUB)) * 2


class Chan4Store:
    """K [BH, n, D] -> the chan4 baseline store (kernels/bitplane.py:342-355): codes,
    block scales, chan_k int32 [BH, nsb, D, SUB, 8] and scales_k fp16 [BH, nsb, D, SUB],
    built in one pass on the GPU.  scan(q, act, nact) reads the nact listed channels
    of each row at full depth; like PlaneStore, chan_k / scales_k may be replaced by
    DevPtr objects into mapped host memory."""

    cfg = {"NB": 2, "KK": 1, "num_warps": 1, "num_stages": 1}

    def __init__(self, K, scale_dtype=torch.float16, keep_code=True):
        _need_gpu(K)
        self.BH, self.n, d = K.shape
        if d != D:
            raise AssertionError(f"Chan4Store needs D == {D}, got {d}")
        if scale_dtype not in _KDT:
            raise ValueError(f"scale_dtype {scale_dtype} unsupported")
        Kc = _key_input(K)
        dev = K.device
        nb = math.ceil(self.n / BLK)
        self.sub = int(SUB)
        self.nsb = math.ceil(nb / self.sub)
        self.code = torch.empty(self.BH, self.n, d, dtype=torch.uint8, device=dev) if keep_code else None
        self.scales_blk = torch.empty(self.BH, nb, d, dtype=scale_dtype, device=dev)
        self.chan_k = torch.empty(self.BH, self.nsb, d, self.sub, 8, dtype=torch.int32, device=dev)
        self.scales_k = torch.empty(self.BH, self.nsb, d, self.sub, dtype=torch.float16, device=dev)
        _lib.call("fathom_quantise_chan4", _ptr(Kc), _KDT[Kc.dtype], self.BH, self.n, d, _KDT[scale_dtype], self.sub,
                  _ptr(self.code), _ptr(self.scales_blk), _ptr(self.chan_k), _ptr(self.scales_k), _stream(dev))

    def scan(self, q, act, nact, out=None, blocks=None):
        """q [BH, G, D] fp32, act/nact from channel_list -> scores fp32 [BH, G, n];
        blocks=(b0, b1) scans only 64-token blocks [b0, b1) into `out`."""
        _need_gpu(q, act, nact)
        BH, G, d = q.shape
        if BH != self.BH:
            raise AssertionError(f"q has BH={BH}, store has {self.BH}")
        out = torch.empty(BH, G, self.n, device=q.device, dtype=torch.float32) if out is None else out
        if out.dtype != torch.float32 or not out.is_contiguous() or tuple(out.shape) != (BH, G, self.n):
            raise ValueError(f"out must be a contiguous float32 [{BH}, {G}, {self.n}] tensor")
        if G > G_CALL:
            for g0, g1 in _head_groups(G):
                part = out[:, g0:g1].contiguous()
                Chan4Store.scan(self, q[:, g0:g1], act, nact, out=part, blocks=blocks)
                out[:, g0:g1].copy_(part)
            return out
        nb = math.ceil(self.n / BLK)
        b0, b1 = (0, nb) if blocks is None else (int(blocks[0]), int(blocks[1]))
        qc = q.contiguous().float()
        a32 = act.to(torch.int32).contiguous()
        n32 = nact.to(torch.int32).contiguous()
        _lib.call("fathom_scan_chan4", _ptr(qc), BH, G, d, _ptr(a32), _ptr(n32),
                  ctypes.c_void_p(self.chan_k.data_ptr()), ctypes.c_void_p(self.scales_k.data_ptr()), self.n,
                  int(self.nsb), int(self.sub), b0, b1, _ptr(out), _stream(q.device))
        return out

    def nbytes(self):
        return self.BH * self.nsb * D * self.sub * (32 + 2)


def scan_planes_reference(q, code, scales, t):
    """q [BH, G, D], code uint8 [BH, n, D], scales [BH, nblk, D], t [BH, D] ->
    [BH, G, n]: q @ dequant_planes(...)^T per row (kernels/bitplane.py:357-363);
    dequantisation in the gfx950 kernel, the product a library GEMM."""
    out = []
    for b in range(q.shape[0]):
        val = dequant_planes(code[b], scales[b], t[b].long())
        out.append(q[b].float() @ val.T)
    return torch.stack(out)


def scan_chan4_reference(q, code, scales, active):
    """[BH, G, n] = q @ (full-depth dequantised codes masked to the active channels)^T
    (kernels/bitplane.py:365-370); dequantisation in the gfx950 kernel, the product a
    library GEMM."""
    out = []
    for b in range(q.shape[0]):
        val = dequant_planes(code[b], scales[b], torch.full((code.shape[-1],), 4, device=code.device))
        out.append(q[b].float() @ (val * active[b].float()[None]).T)
    return torch.stack(out)


# ----------------------------------------------------------------------------- top-k
def sink_local_topk(scores, k, sink=4, local=32, m=None):
    """scores [..., n] -> selected indices int64 [..., k] = top-(k - sink - local) among
    non-sink/non-local tokens (score descending, lowest index first on ties), then
    the sinks, then the last `local` positions -- kernels/bitplane.py:372-378.
    m (default n) is the current sequence length: the local window is
    [m - local, m) as in scripts/B_e2e_offload_v2.py:224-227."""
    _need_gpu(scores)
    *lead, n = scores.shape
    m = n if m is None else int(m)
    s = scores.contiguous().float()
    rows = _lead(lead)
    idx = torch.empty(*lead, k, dtype=torch.int64, device=scores.device)
    nbytes = _lib.lib().fathom_topk_workspace_bytes(rows, n, k)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=scores.device)
    _lib.call("fathom_sink_local_topk", _ptr(s), rows, n, m, int(k), int(sink), int(local), _ptr(idx), _ptr(ws),
              nbytes, _stream(scores.device))
    return idx
