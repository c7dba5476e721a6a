"""numpy front end of the C oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the reference restatement that tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg check against.  The product package never imports
this module.

bf16 tensors are numpy ``uint16`` arrays of raw bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)


def build(force: bool = False) -> Path:
    """Compile oracle/liboracle.so with gcc (oracle/Makefile)."""
    target = HERE / "liboracle.so"
    if force or not target.exists():
        subprocess.run(["make", "-C", str(HERE), "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return target


def lib():
    global _LIB
    if _LIB is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f64_to_bf16.restype = ctypes.c_uint16
        L.orc_f64_to_bf16.argtypes = [ctypes.c_double]
        L.orc_expf.restype = ctypes.c_float
        L.orc_expf.argtypes = [ctypes.c_float]
        L.orc_route_logits.restype = None
        L.orc_route_logits.argtypes = [_u16p, _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _u16p]
        L.orc_route_from_logits.restype = ctypes.c_int
        L.orc_route_from_logits.argtypes = [_u16p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _i32p, _u16p, _f32p]
        L.orc_route_hist.restype = None
        L.orc_route_hist.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, _i32p]
        L.orc_pack.restype = ctypes.c_int
        L.orc_pack.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p, _i32p,
                               _i32p, _i32p, _i32p]
        L.orc_expert_forward.restype = None
        L.orc_expert_forward.argtypes = [_u16p, ctypes.c_int, _u16p, _u16p, _u16p, ctypes.c_int,
                                         ctypes.c_int, _u16p, _u16p]
        L.orc_expert_forward_fp.restype = None
        L.orc_expert_forward_fp.argtypes = [_u16p, ctypes.c_int, _u16p, _u16p, _u16p, ctypes.c_int,
                                            ctypes.c_int, _f32p]
        L.orc_merge.restype = None
        L.orc_merge.argtypes = [_u16p, _i32p, _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                _u16p, _u16p]
        L.orc_index_add_bf16.restype = None
        L.orc_index_add_bf16.argtypes = [_u16p, ctypes.c_int, _i64p, _u16p, _u16p, ctypes.c_int64]
        L.orc_merge_ordered.restype = None
        L.orc_merge_ordered.argtypes = [_u16p, _i32p, _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        _u16p, _u16p]
        L.orc_moe_layer.restype = ctypes.c_int
        L.orc_moe_layer.argtypes = [_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, _u16p, _f32p,
                                    ctypes.POINTER(_u16p), _u16p, _u16p, _i32p, _u16p]
        L.cpu_moe_forward_rows.restype = ctypes.c_int
        L.cpu_moe_forward_rows.argtypes = [_u16p, ctypes.c_int, _i64p, _f32p,
                                           ctypes.POINTER(_u16p), ctypes.c_int, ctypes.c_int,
                                           _u16p, ctypes.c_int]
        L.cpu_moe_decode.restype = ctypes.c_int
        L.cpu_moe_decode.argtypes = [_u16p, _i32p, _u16p, ctypes.c_int, ctypes.POINTER(_u16p),
                                     ctypes.c_int, ctypes.c_int, _u16p, ctypes.c_int]
        _LIB = L
    return _LIB


def _p(a, typ):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(typ)


def _u16(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


# ---------------------------------------------------------------- bf16 codec

def f32_to_bf16(a) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (vectorised, same rule as C)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return (a.astype(np.uint32) << 16).view(np.float32)


def expf(x: float) -> float:
    return lib().orc_expf(float(x))


def f64_to_bf16_scalar(d: float) -> int:
    return int(lib().orc_f64_to_bf16(float(d)))


# ---------------------------------------------------------------- A1 / A2

def route_logits(x, gate):
    x, gate = _u16(x), _u16(gate)
    T, H = x.shape
    E = gate.shape[0]
    out = np.empty((T, E), np.uint16)
    lib().orc_route_logits(_p(x, _u16p), _p(gate, _u16p), T, H, E, _p(out, _u16p))
    return out


def route_from_logits(logits, k, normalize=True, bias=None, want_probs=False):
    logits = _u16(logits)
    T, E = logits.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.uint16)
    probs = np.empty((T, E), np.float32) if want_probs else None
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_route_from_logits(_p(logits, _u16p), _p(b, _f32p), T, E, k, int(bool(normalize)),
                                     _p(ids, _i32p), _p(w, _u16p), _p(probs, _f32p))
    if rc:
        raise ValueError("oracle route: invalid arguments")
    return (ids, w, probs) if want_probs else (ids, w)


def route(x, gate, k, normalize=True, bias=None):
    logits = route_logits(x, gate)
    ids, w = route_from_logits(logits, k, normalize, bias)
    return logits, ids, w


def route_hist(ids, E):
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    hist = np.empty(E, np.int32)
    lib().orc_route_hist(_p(ids, _i32p), ids.size, E, _p(hist, _i32p))
    return hist


# ---------------------------------------------------------------- A3

def pack(ids, E):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    n = T * k
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    ptok = np.empty(n, np.int32)
    ppos = np.empty(n, np.int32)
    row_of = np.empty(n, np.int32)
    rc = lib().orc_pack(_p(ids, _i32p), T, k, E, _p(counts, _i32p), _p(offsets, _i32p),
                        _p(ptok, _i32p), _p(ppos, _i32p), _p(row_of, _i32p))
    if rc:
        raise ValueError("oracle pack: expert id outside [0, E)")
    return dict(counts=counts, offsets=offsets, perm_token=ptok, perm_pos=ppos, row_of=row_of)


# ---------------------------------------------------------------- A4 / A8

def expert_forward(x, wg, wu, wd, want_h=False):
    x, wg, wu, wd = _u16(x), _u16(wg), _u16(wu), _u16(wd)
    m, H = x.shape
    I = wg.shape[0]
    y = np.empty((m, H), np.uint16)
    h = np.empty((m, I), np.uint16) if want_h else None
    lib().orc_expert_forward(_p(x, _u16p), m, _p(wg, _u16p), _p(wu, _u16p), _p(wd, _u16p), H, I,
                             _p(y, _u16p), _p(h, _u16p))
    return (y, h) if want_h else y


def expert_forward_fp(x, wg, wu, wd):
    x, wg, wu, wd = _u16(x), _u16(wg), _u16(wu), _u16(wd)
    m, H = x.shape
    I = wg.shape[0]
    y = np.empty((m, H), np.float32)
    lib().orc_expert_forward_fp(_p(x, _u16p), m, _p(wg, _u16p), _p(wu, _u16p), _p(wd, _u16p), H, I,
                                _p(y, _f32p))
    return y


def merge(y, row_of, w, add_in=None):
    y, w = _u16(y), _u16(w)
    row_of = np.ascontiguousarray(row_of, dtype=np.int32)
    T, k = w.shape
    H = y.shape[1]
    out = np.empty((T, H), np.uint16)
    a = None if add_in is None else _u16(add_in)
    lib().orc_merge(_p(y, _u16p), _p(row_of, _i32p), _p(w, _u16p), T, k, H, _p(a, _u16p),
                    _p(out, _u16p))
    return out


def merge_ordered(y, row_of, w, add_in=None):
    """The reference's default merge (pdscope_runtime.py:466-468): per token,
    its k weighted rows added in bf16 in ascending expert id; add_in last."""
    y, w = _u16(y), _u16(w)
    row_of = np.ascontiguousarray(row_of, dtype=np.int32)
    T, k = w.shape
    H = y.shape[1]
    if k > 64:
        raise ValueError("merge_ordered: k <= 64")
    out = np.empty((T, H), np.uint16)
    a = None if add_in is None else _u16(add_in)
    lib().orc_merge_ordered(_p(y, _u16p), _p(row_of, _i32p), _p(w, _u16p), T, k, H, _p(a, _u16p),
                            _p(out, _u16p))
    return out


def index_add_bf16(out, tokens, rows, w):
    """torch's bf16 index_add_ of rows * w into out, row by row (returns a new array)."""
    out = np.array(_u16(out), copy=True)
    rows, w = _u16(rows), _u16(w).reshape(-1)
    tokens = np.ascontiguousarray(tokens, dtype=np.int64).reshape(-1)
    n, H = rows.shape
    if out.ndim != 2 or out.shape[1] != H or tokens.size != n or w.size != n:
        raise ValueError("index_add_bf16: shapes")
    if n and (tokens.min() < 0 or tokens.max() >= out.shape[0]):
        raise ValueError("index_add_bf16: token index out of range")
    lib().orc_index_add_bf16(_p(out, _u16p), H, _p(tokens, _i64p), _p(rows, _u16p), _p(w, _u16p), n)
    return out


def moe_layer(x, gate, slots, k, normalize=True, bias=None):
    """slots: list of E uint16 arrays, each the flat gate|up|down block."""
    x, gate = _u16(x), _u16(gate)
    T, H = x.shape
    E = gate.shape[0]
    I = slots[0].size // (3 * H)
    arr = (_u16p * E)(*[_p(_u16(s), _u16p) for s in slots])
    out = np.empty((T, H), np.uint16)
    logits = np.empty((T, E), np.uint16)
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_moe_layer(_p(x, _u16p), T, H, I, E, k, int(bool(normalize)), _p(gate, _u16p),
                             _p(b, _f32p), arr, _p(out, _u16p), _p(logits, _u16p), _p(ids, _i32p),
                             _p(w, _u16p))
    if rc:
        raise ValueError("oracle moe_layer failed")
    return dict(out=out, logits=logits, ids=ids, weights=w)


# ---------------------------------------------------------------- CPU baseline

def cpu_moe_rows(x, selected, coeff, slots_ptrs, H, I, nthreads):
    """slots_ptrs: sequence of integer host addresses (bf16 gate|up|down blocks)."""
    x = _u16(x)
    rows = x.shape[0]
    sel = np.ascontiguousarray(selected, dtype=np.int64)
    c = np.ascontiguousarray(coeff, dtype=np.float32)
    arr = (_u16p * len(slots_ptrs))(*[ctypes.cast(p, _u16p) for p in slots_ptrs])
    out = np.empty_like(x)
    rc = lib().cpu_moe_forward_rows(_p(x, _u16p), rows, _p(sel, _i64p), _p(c, _f32p), arr, H, I,
                                    _p(out, _u16p), int(nthreads))
    if rc:
        raise RuntimeError("cpu_moe_forward_rows unavailable (needs AVX2+FMA)")
    return out


def cpu_moe_decode(x, ids, w, slots_ptrs, H, I, nthreads, out=None):
    x = _u16(x).reshape(-1)
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    w = _u16(w).reshape(-1)
    arr = (_u16p * len(slots_ptrs))(*[ctypes.cast(p, _u16p) for p in slots_ptrs])
    if out is None:
        out = np.empty(H, np.uint16)
    rc = lib().cpu_moe_decode(_p(x, _u16p), _p(ids, _i32p), _p(w, _u16p), ids.size, arr, H, I,
                              _p(out, _u16p), int(nthreads))
    if rc:
        raise RuntimeError("cpu_moe_decode unavailable (needs AVX2+FMA)")
    return out
