"""Lazy safetensors reader for captured activations (scripts/capsio.py's role).

Reads only the requested leading-dimension rows of a tensor with one
``os.pread`` per slice, without mapping the whole file -- the capture files of
the reference (post-RoPE q/k/v per layer, tens of GB) do not fit the host's
memory at once.  Subset of the ``safetensors.safe_open`` API the reference's
scripts use: ``keys()``, ``get_slice(name)[a:b, ...]`` / ``.get_shape()``,
``get_tensor(name)``, ``name in f``, iteration.  dtypes: F16, BF16, F32 (and
F64, I64, I32, U8).  Only the JSON header and raw little-endian bytes are read:
nothing in the file is executed.
"""
import json
import os
import struct

import numpy as np
import torch

_DT = {"F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32, "F64": torch.float64,
       "I64": torch.int64, "I32": torch.int32, "U8": torch.uint8}


class _Slice:
    def __init__(self, f, base, meta):
        self.f, self.base, self.meta = f, base, meta

    def get_shape(self):
        return list(self.meta["shape"])

    def get_dtype(self):
        return self.meta["dtype"]

    def __getitem__(self, idx):
        shape = self.meta["shape"]
        idx = idx if isinstance(idx, tuple) else (idx,)
        lead, rest = idx[0], idx[1:]
        if not shape:
            raise IndexError("scalar tensor")
        n0 = shape[0]
        if isinstance(lead, int):
            r0 = lead % n0
            r1, squeeze = r0 + 1, True
        else:
            r0, r1, step = lead.indices(n0)
            if step != 1:
                raise IndexError("only unit-step slices of the leading dimension")
            r1, squeeze = max(r1, r0), False
        dt = _DT[self.meta["dtype"]]
        esize = torch.empty(0, dtype=dt).element_size()
        row = int(np.prod(shape[1:], dtype=np.int64)) * esize
        start = self.meta["data_offsets"][0] + r0 * row
        nbytes = (r1 - r0) * row
        buf = os.pread(self.f.fileno(), nbytes, self.base + start) if nbytes else b""
        if len(buf) != nbytes:
            raise IOError(f"short read: {len(buf)} of {nbytes} bytes")
        t = torch.frombuffer(bytearray(buf), dtype=dt) if nbytes else torch.empty(0, dtype=dt)
        t = t.reshape(r1 - r0, *shape[1:])
        if squeeze:
            t = t[0]
            return t[rest] if rest else t
        return t[(slice(None),) + rest] if rest else t


class CapsFile:
    """An open safetensors file: header parsed, tensors read on access."""

    def __init__(self, path):
        self.f = open(path, "rb")
        (n,) = struct.unpack("<Q", self.f.read(8))
        self.hdr = json.loads(self.f.read(n))
        self.metadata = self.hdr.pop("__metadata__", None)
        self.base = 8 + n

    def keys(self):
        return list(self.hdr)

    def get_slice(self, name):
        return _Slice(self.f, self.base, self.hdr[name])

    def get_tensor(self, name):
        return self.get_slice(name)[:]

    def __getitem__(self, name):
        return self.get_tensor(name)

    def __contains__(self, name):
        return name in self.hdr

    def __iter__(self):
        return iter(self.hdr)

    def __len__(self):
        return len(self.hdr)

    def close(self):
        self.f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def safe_open(path, framework="pt", device="cpu"):
    """safetensors.safe_open stand-in (framework / device accepted, tensors on the CPU)."""
    return CapsFile(path)


def load_file(path):
    """Lazy stand-in for safetensors.torch.load_file: tensors load on access."""
    return CapsFile(path)
