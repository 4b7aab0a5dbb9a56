"""CPU checks of the C ABI boundary: the built library loads, exports every
entry point include/fathom_hip.h declares, and the Python binding declares a
prototype for each; the Python API refuses host tensors (no CPU fallback)."""
import ctypes
import os
import re

import pytest
import torch

from fathom_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fathom_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fathom_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "fathom_scan_planes" in names and "fathom_sink_local_topk" in names
    assert len(names) == len(_lib.PROTOTYPES)
    assert set(names) == set(_lib.PROTOTYPES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    assert _lib.lib().fathom_version().decode().startswith("fathom-hip")


def test_workspace_queries_and_argument_errors_without_gpu():
    L = _lib.lib()
    assert L.fathom_topk_workspace_bytes(32, 1 << 20, 512) >= 32 * (1 << 20) * 8
    e = 8 * 2048  # per position: chain link, chain start, head counts, distinct-token entry
    assert L.fathom_gather_union_workspace_bytes(8, 2048) == e * (4 + 4 + 16 + 8) + 256
    nsplit = 2048 // 64  # partial softmax triples of 64 tokens (or positions) each
    assert (L.fathom_gather_attention_workspace_bytes(8, 4, 512)
            == e * (4 + 4 + 16 + 8) + 256 + 8 * nsplit * 4 * 130 * 4)
    rc = L.fathom_gather_attention(None, None, 1, 4, 512, 10, None, None, 10, None, None, 0, 1.0, None, None,
                                   None, 0, None)
    assert rc == _lib.ERR_INVALID
    assert L.fathom_gather_attention_workspace_bytes(8, 9, 512) > 0  # G > 8 is rejected by the call itself
    # argument validation happens before any HIP call
    rc = L.fathom_make_plan(None, None, 1, 128, 4, 30, None, None, None, None, None, None, None, None)
    assert rc == _lib.ERR_INVALID and b"null" in L.fathom_last_error()
    with pytest.raises(ValueError):
        _lib.check(rc, "fathom_make_plan")
    rc = L.fathom_make_plan_uniform(None, 48.0, 1, 128, 4, 30, None, None, None, None, None, None, None, None)
    assert rc == _lib.ERR_INVALID and b"null" in L.fathom_last_error()


def test_python_api_rejects_host_tensors():
    from fathom_amd import bitplane as bp
    with pytest.raises(ValueError, match="GPU"):
        bp.quantise_u4(torch.zeros(2, 64, 128))
    with pytest.raises(ValueError, match="GPU"):
        bp.make_plan(torch.ones(2, 128), 48)


def test_host_mapped_allocation_failure_raises_memory_error():
    """A pinned mapped allocation that cannot be satisfied (here 4 PiB) becomes
    MemoryError with the library's message, and nothing is leaked or mapped."""
    from fathom_amd import offload as off

    class Huge:  # stands in for a tensor too large to pin; host_mapped reads only these
        dtype = torch.float32

        def numel(self):
            return 1 << 50

        def element_size(self):
            return 4

    with pytest.raises(MemoryError, match="hipHostMalloc"):
        off.host_mapped(Huge())
    hp, dp = ctypes.c_void_p(), ctypes.c_void_p()
    rc = _lib.lib().fathom_host_alloc_mapped(1 << 52, 1, ctypes.byref(hp), ctypes.byref(dp))
    assert rc == _lib.ERR_ALLOC and hp.value is None and dp.value is None
    with pytest.raises(MemoryError):
        _lib.check(rc, "fathom_host_alloc_mapped")
