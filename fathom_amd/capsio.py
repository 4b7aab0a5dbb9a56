"""Row-range reader for safetensors capture files (the role of scripts/capsio.py).

The reference calibrates the KLT basis and the per-layer budgets from captured
activations (post-RoPE q/k per layer and KV head) stored as safetensors files
far larger than host memory, so only the rows a caller asks for may be read.
This module is built in three layers:

* ``index_file``: parses the safetensors header (an 8-byte little-endian length
  and a JSON table of name -> dtype, shape, [begin, end) byte offsets into the
  data section) into ``TensorEntry`` records, checking that every byte range
  lies inside the file and matches its dtype and shape;
* ``read_rows``: the one I/O primitive -- rows [r0, r1) of a tensor's leading
  dimension, read with ``os.preadv`` straight into the memory of the returned
  tensor (no intermediate buffer, no memory map);
* ``CapsReader`` and the ``safe_open`` / ``load_file`` adapters that give the
  subset of the safetensors API the reference's scripts use: ``keys()``,
  ``get_slice(name)`` (``.get_shape()``, ``[i]``, ``[a:b]``, ``[a:b, ...]``),
  ``get_tensor(name)``, ``name in f``, iteration.

Only the header JSON and raw little-endian bytes are interpreted: nothing in a
file is executed.
"""
import json
import os
import struct
from dataclasses import dataclass

import torch

_DTYPES = {"F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
           "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8, "U8": torch.uint8,
           "BOOL": torch.bool}
_MAX_HEADER = 100 << 20  # safetensors caps the header at 100 MB


@dataclass(frozen=True)
class TensorEntry:
    """Where one tensor lives in the file: absolute byte range [begin, end)."""
    name: str
    dtype: torch.dtype
    shape: tuple
    begin: int
    end: int

    @property
    def rows(self):
        return self.shape[0] if self.shape else 1

    @property
    def row_bytes(self):
        """Bytes of one index of the leading dimension (the whole tensor for a scalar)."""
        size = torch.empty((), dtype=self.dtype).element_size()
        for s in self.shape[1:]:
            size *= s
        return size


def index_file(fd):
    """Parses the header of the safetensors file open as fd.  Returns
    ({name: TensorEntry}, metadata dict or None); raises ValueError on a
    malformed header or a byte range outside the file."""
    size = os.fstat(fd).st_size
    head = os.pread(fd, 8, 0)
    if len(head) != 8:
        raise ValueError("not a safetensors file: shorter than 8 bytes")
    (hlen,) = struct.unpack("<Q", head)
    if hlen > _MAX_HEADER or 8 + hlen > size:
        raise ValueError(f"safetensors header of {hlen} bytes does not fit a {size}-byte file")
    table = json.loads(os.pread(fd, hlen, 8))
    meta = table.pop("__metadata__", None)
    data0 = 8 + hlen
    entries = {}
    for name, rec in table.items():
        dt = _DTYPES.get(rec.get("dtype"))
        if dt is None:
            raise ValueError(f"{name}: unsupported dtype {rec.get('dtype')!r}")
        shape = tuple(int(s) for s in rec["shape"])
        b, e = (int(v) for v in rec["data_offsets"])
        ent = TensorEntry(name, dt, shape, data0 + b, data0 + e)
        if not (0 <= b <= e and ent.end <= size):
            raise ValueError(f"{name}: byte range [{b}, {e}) lies outside the data section")
        if ent.end - ent.begin != ent.rows * ent.row_bytes:
            raise ValueError(f"{name}: {ent.end - ent.begin} bytes for shape {shape} of {rec['dtype']}")
        entries[name] = ent
    return entries, meta


def read_rows(fd, ent, r0, r1):
    """Rows [r0, r1) of ent's leading dimension as a new CPU tensor
    [r1 - r0, *shape[1:]] (a scalar tensor: r0 = 0, r1 = 1)."""
    if not (0 <= r0 <= r1 <= ent.rows):
        raise IndexError(f"{ent.name}: rows [{r0}, {r1}) of {ent.rows}")
    out = torch.empty((r1 - r0,) + ent.shape[1:], dtype=ent.dtype)
    want = (r1 - r0) * ent.row_bytes
    if want:
        view = memoryview(out.view(torch.uint8).reshape(-1).numpy())
        got = 0
        while got < want:  # preadv may return short counts
            n = os.preadv(fd, [view[got:]], ent.begin + r0 * ent.row_bytes + got)
            if n <= 0:
                raise IOError(f"{ent.name}: file ended after {got} of {want} bytes")
            got += n
    return out


class _RowView:
    """get_slice's result: indexing reads only the leading-dimension rows it
    selects; further indices apply to the rows read."""

    def __init__(self, reader, ent):
        self._reader, self._ent = reader, ent

    def get_shape(self):
        return list(self._ent.shape)

    def get_dtype(self):
        return next(k for k, v in _DTYPES.items() if v == self._ent.dtype)

    def __getitem__(self, key):
        key = key if isinstance(key, tuple) else (key,)
        if not self._ent.shape:
            if key not in ((), (Ellipsis,)):
                raise IndexError("a scalar tensor takes no index")
            return read_rows(self._reader.fd, self._ent, 0, 1).reshape(())
        first, rest = key[0], key[1:]
        if first is Ellipsis:
            rows, rest = slice(None), key
        else:
            rows = first
        n = self._ent.rows
        if isinstance(rows, slice):
            r0, r1, step = rows.indices(n)
            t = read_rows(self._reader.fd, self._ent, r0, max(r0, r1) if step > 0 else r0)
            if step != 1:
                if step < 0:
                    raise IndexError("negative steps over the leading dimension")
                t = t[::step]
            return t[(slice(None),) + rest] if rest else t
        i = int(rows)
        if i < 0:
            i += n
        t = read_rows(self._reader.fd, self._ent, i, i + 1)[0]
        return t[rest] if rest else t


class CapsReader:
    """An open capture file: the header index, tensors read on access."""

    def __init__(self, path):
        self.fd = os.open(path, os.O_RDONLY)
        try:
            self.entries, self.metadata = index_file(self.fd)
        except Exception:
            os.close(self.fd)
            raise

    # safetensors.safe_open interface
    def keys(self):
        return list(self.entries)

    def get_slice(self, name):
        return _RowView(self, self.entries[name])

    def get_tensor(self, name):
        ent = self.entries[name]
        t = read_rows(self.fd, ent, 0, ent.rows)
        return t if ent.shape else t.reshape(())

    def metadata_dict(self):
        return self.metadata

    # dict-like access of load_file's result
    def __getitem__(self, name):
        return self.get_tensor(name)

    def __contains__(self, name):
        return name in self.entries

    def __iter__(self):
        return iter(self.entries)

    def __len__(self):
        return len(self.entries)

    def close(self):
        if self.fd >= 0:
            os.close(self.fd)
            self.fd = -1

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def safe_open(path, framework="pt", device="cpu"):
    """The safetensors.safe_open call of the reference's scripts; tensors are
    read to the CPU (framework and device are accepted as given)."""
    return CapsReader(path)


def load_file(path):
    """Stand-in for safetensors.torch.load_file that reads each tensor on access."""
    return CapsReader(path)
