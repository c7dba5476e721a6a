"""ctypes binding of libpdscope_moe.so (the C-ABI in include/pdscope_moe.h).

There is no fallback: if the library is missing or fails to load, every
operation raises.  Build it with ``python -m pdscope_amd.build``.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpdscope_moe.so"

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# name -> (argtypes, restype)
SIGNATURES = {
    "pdscope_last_error": ([], ctypes.c_char_p),
    "pdscope_version": ([], ctypes.c_char_p),
    "pdscope_route_workspace_bytes": ([], _sz),
    "pdscope_route_workspace_size": ([_i32, _i32, _i32], _sz),
    "pdscope_route_topk": ([_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pdscope_route_hist": ([_vp, _i32, _i32, _vp, _vp], _i32),
    "pdscope_pack": ([_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pdscope_pack_workspace_size": ([_i32, _i32, _i32], _sz),
    "pdscope_pack_static": ([_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pdscope_pack_static_max_ids": ([], _sz),
    "pdscope_schedule": ([_vp, _i32, _vp, _i32, _i32, _vp, _vp], _i32),
    "pdscope_schedule_balanced": ([_vp, _i32, _vp, _i32, _i32, _vp, _vp, _vp], _i32),
    "pdscope_schedule_balanced_pair": ([_vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "pdscope_pack_schedule_balanced": ([_vp, _i32, _i32, _i32] + [_vp] * 6 + [_vp, _i32, _i32, _i32] + [_vp] * 4,
                                       _i32),
    "pdscope_grouped_block_m": ([_i32], _i32),
    "pdscope_grouped_block_m_max": ([_i32, _i32], _i32),
    "pdscope_swiglu_grouped": ([_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _i32, _vp, _vp, _vp], _i32),
    "pdscope_swiglu_grouped_gateup": ([_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _i32, _vp, _vp], _i32),
    "pdscope_swiglu_grouped_down": ([_vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _i32, _vp, _vp], _i32),
    "pdscope_merge": ([_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp], _i32),
    "pdscope_merge_ordered": ([_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp], _i32),
    "pdscope_swiglu_decode": ([_vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _vp, _i32, _vp], _i32),
    "pdscope_decode_workspace_bytes": ([], _sz),
    "pdscope_decode_layer_supported": ([_i32, _i32, _i32, _i32], _i32),
    "pdscope_decode_layer_chained_supported": ([_i32, _i32, _i32, _i32, _i32], _i32),
    "pdscope_decode_layer": ([_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                              _vp, _vp], _i32),
    "pdscope_decode_layer_chained": ([_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp,
                                      _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pdscope_decode_bind": ([_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             _vp, ctypes.POINTER(_vp)], _i32),
    "pdscope_decode_run": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp], _i32),
    "pdscope_decode_unbind": ([_vp], None),
    "pdscope_stage_expert": ([_vp, _vp, _sz, _vp, _vp], _i32),
    "pdscope_stage_merge": ([_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _vp], _i32),
    "pdscope_dispatch_pack": ([_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp], _i32),
}

_LIB = None


class PDScopeError(RuntimeError):
    """A C-ABI call returned non-zero (message from pdscope_last_error)."""


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m pdscope_amd.build` "
                               "(the gfx950 HIP library is required, there is no CPU path)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = lib
    return _LIB


def call(name: str, *args) -> int:
    """Invoke a C-ABI entry point; raise PDScopeError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if isinstance(rc, int) and rc != 0:
        raise_for(name, rc)
    return rc


def raise_for(name: str, rc: int):
    """Raise for the non-zero status `rc` of entry point `name`: ValueError for
    an invalid argument, PDScopeError for a HIP error."""
    msg = load().pdscope_last_error().decode(errors="replace")
    if rc == 1:
        raise ValueError(f"{name}: {msg}")
    raise PDScopeError(f"{name} failed ({rc}): {msg}")


def version() -> str:
    return load().pdscope_version().decode()
