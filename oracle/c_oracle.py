"""ctypes binding of the C oracle (test infrastructure only; see
``oracle/mxfp4_oracle.c``).  Builds the library on first use when it is
missing and a compiler is available."""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build as _build

_lib = None
_DT = {"f32": 0, "bf16": 1, "f16": 2}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_build.LIB):
            _build.build()
        l = ctypes.CDLL(_build.LIB)
        l.oracle_dequant.restype = ctypes.c_int
        l.oracle_dequant.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
        l.oracle_quant.restype = ctypes.c_int
        l.oracle_quant.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        l.oracle_make_routing.restype = ctypes.c_int64
        l.oracle_make_routing.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        for name, ret in (("oracle_dequant_elem_f32", ctypes.c_uint32),
                          ("oracle_dequant_elem_bf16", ctypes.c_uint16),
                          ("oracle_dequant_elem_f16", ctypes.c_uint16)):
            fn = getattr(l, name)
            fn.restype = ret
            fn.argtypes = [ctypes.c_uint, ctypes.c_uint]
        _lib = l
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant_bits(packed: np.ndarray, scales: np.ndarray, dtype: str) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    k = p.shape[-1] * 2
    rows = int(np.prod(p.shape[:-1])) if p.ndim > 1 else 1
    out = np.empty(p.shape[:-1] + (k,), dtype=np.uint32 if dtype == "f32" else np.uint16)
    rc = lib().oracle_dequant(_ptr(p), _ptr(s), rows, k, _DT[dtype], _ptr(out))
    if rc:
        raise ValueError(f"oracle_dequant failed ({rc})")
    return out


def quant(x: np.ndarray, mode: str):
    """mode "ties_away" (test:28-60) or "rne" (OCP MX)."""
    xf = np.ascontiguousarray(x, dtype=np.float32)
    k = xf.shape[-1]
    rows = int(np.prod(xf.shape[:-1])) if xf.ndim > 1 else 1
    packed = np.empty(xf.shape[:-1] + (k // 2,), dtype=np.uint8)
    scales = np.empty(xf.shape[:-1] + (k // 32,), dtype=np.uint8)
    rc = lib().oracle_quant(_ptr(xf), rows, k, 0 if mode == "ties_away" else 1,
                            _ptr(packed), _ptr(scales))
    if rc:
        raise ValueError(f"oracle_quant failed ({rc})")
    return packed, scales


def make_routing(topk_ids: np.ndarray, num_experts: int, block_m: int):
    ids = np.ascontiguousarray(np.asarray(topk_ids).reshape(-1), dtype=np.int64)
    n = ids.size
    sorted_ids = np.empty(n + num_experts * block_m, dtype=np.int32)
    expert_ids = np.empty(n + num_experts, dtype=np.int32)
    blocks = lib().oracle_make_routing(_ptr(ids), n, num_experts, block_m,
                                       _ptr(sorted_ids), _ptr(expert_ids))
    return (sorted_ids[: blocks * block_m].copy(), expert_ids[:blocks].copy(),
            np.array([blocks * block_m], dtype=np.int32))
