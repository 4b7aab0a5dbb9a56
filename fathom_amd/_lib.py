"""ctypes binding of libfathom_hip.so (the C ABI declared in include/fathom_hip.h).

The library is loaded once, from this package directory.  A missing library is
an ImportError at first use: there is no CPU fallback for any entry point.
"""
import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfathom_hip.so")

OK, ERR_INVALID, ERR_HIP, ERR_ALLOC, ERR_WORKSPACE = 0, 1, 2, 3, 4
DT_F32, DT_F16, DT_BF16 = 0, 1, 2

_vp, _i32, _i64, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t

# name -> (restype, argtypes); one entry per declaration of include/fathom_hip.h
PROTOTYPES = {
    "fathom_version": (ctypes.c_char_p, []),
    "fathom_last_error": (ctypes.c_char_p, []),
    "fathom_quantise_pack": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "fathom_pack_planes": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "fathom_unpack_planes": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "fathom_to_superblocks": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "fathom_dequant_planes": (_i32, [_vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp, _vp]),
    "fathom_make_plan": (_i32, [_vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "fathom_make_plan_uniform": (_i32, [_vp, ctypes.c_float, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _vp, _vp]),
    "fathom_scan_planes": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                  _vp, _vp]),
    "fathom_pack_chan4": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "fathom_quantise_chan4": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _vp]),
    "fathom_channel_list": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "fathom_scan_chan4": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "fathom_klt_query": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp]),
    "fathom_scan_topk_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "fathom_scan_topk": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                _i64, _vp, _vp, _sz, _vp]),
    "fathom_scan_topk_stages": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                       _i64, _i64, _vp, _vp, _sz, _i32, _vp]),
    "fathom_plan_scan_topk_workspace_bytes": (_sz, [_i64, _i64, _i64, _i32, _i64, _i64, _i64, _i64]),
    "fathom_plan_scan_topk": (_i32, [_vp, _vp, _vp, ctypes.c_float, _i64, _i64, _i64, _i32, _i32, _i64, _vp, _vp, _i64,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "fathom_plan_scan_topk_attention_workspace_bytes": (_sz, [_i64, _i64, _i64, _i32, _i64, _i64, _i64, _i64]),
    "fathom_plan_scan_topk_attention": (_i32, [_vp, _vp, _vp, ctypes.c_float, _i64, _i64, _i64, _i32, _i32, _i64, _vp,
                                               _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64,
                                               ctypes.c_float, _vp, _vp, _sz, _vp]),
    "fathom_scan_topk_noalloc": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                        _i64, _i64, _vp, _vp]),
    "fathom_topk_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fathom_sink_local_topk": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "fathom_gather_rows": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp]),
    "fathom_gather_union_workspace_bytes": (_sz, [_i64, _i64]),
    "fathom_gather_union": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp,
                                   _vp, _sz, _vp]),
    "fathom_gather_attention_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fathom_gather_attention": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64,
                                       ctypes.c_float, _vp, _vp, _vp, _sz, _vp]),
    "fathom_gather_runs": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fathom_copy_index": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "fathom_copy_index_range": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp]),
    "fathom_host_alloc_mapped": (_i32, [_sz, _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "fathom_host_free": (_i32, [_vp]),
    "fathom_memcpy": (_i32, [_vp, _vp, _sz, _vp]),
}

_lib = None
_lock = threading.Lock()


class FathomError(RuntimeError):
    """A HIP-side failure reported by the library (status FATHOM_ERR_HIP)."""


def lib():
    """The loaded library with prototypes set; raises ImportError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(f"{LIB_PATH} is not built; run `python -m fathom_amd.build` "
                                  "(fathom_amd has no CPU fallback)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in PROTOTYPES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(rc, what):
    """Raise the Python error matching a library status."""
    if rc == OK:
        return
    msg = f"{what}: {lib().fathom_last_error().decode(errors='replace')}"
    if rc == ERR_INVALID:
        raise ValueError(msg)
    if rc == ERR_ALLOC:
        raise MemoryError(msg)
    if rc == ERR_WORKSPACE:
        raise ValueError(msg)
    raise FathomError(msg)


def call(name, *args):
    """Call entry point `name` and raise on a non-zero status."""
    check(getattr(lib(), name)(*args), name)
