"""ctypes loader for libmxfp4_gfx950.so and the glue every operator shares.

The library is the only compute path: if it is missing or fails to load, the
operators raise ``RuntimeError`` -- there is no CPU or eager-PyTorch fallback.
``MXFP4_GFX950_LIB`` may point at another build of the library.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MXFP4_GFX950_LIB", os.path.join(_HERE, "libmxfp4_gfx950.so"))

# include/mxfp4_gfx950.h
OK, ERR_TYPE, ERR_VALUE, ERR_NOT_IMPLEMENTED, ERR_RUNTIME, ERR_HIP = range(6)
DT_F32, DT_BF16, DT_F16, DT_U8, DT_I32, DT_I64, DT_F8E4M3, DT_F8E5M2 = range(8)
QUANT_TIES_AWAY, QUANT_RNE = 0, 1
ABI_VERSION = 1

_DTYPE_CODES = {
    torch.float32: DT_F32,
    torch.bfloat16: DT_BF16,
    torch.float16: DT_F16,
    torch.uint8: DT_U8,
    torch.int32: DT_I32,
    torch.int64: DT_I64,
    torch.float8_e4m3fn: DT_F8E4M3,
    torch.float8_e5m2: DT_F8E5M2,
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

# name -> argtypes (restype is int for all but mxfp4_last_error)
SIGNATURES = {
    "mxfp4_abi_version": [],
    "mxfp4_dequant": [_P, _I64, _P, _I64, _I64, _I64, _P, _I, _P],
    "mxfp4_linear_w4a16": [_P, _I, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P],
    "mxfp4_linear_w4a16_workspace_size": [_I64, _I64, _I64, _P],
    "mxfp4_linear_w4a16_ws": [_P, _I, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P, _I64, _P],
    "mxfp4_linear_w4a4": [_P, _P, _I64, _I64, _P, _P, _I64, _P, _I, _P],
    "mxfp4_moe_align_sizes": [_I64, _I, _I, _P, _P, _P],
    "mxfp4_moe_align": [_P, _I, _I64, _I, _I, _P, _P, _P, _P, _I64, _P],
    "mxfp4_moe_route": [_P, _I64, _I, _I64, _I, _I, _P, _P, _I, _P],
    "mxfp4_moe_gemm": [_P, _I, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _I, _I64, _P, _P,
                       _P, _I, _P, _P, _P, _I64, _I, _I64, _I, _P],
    "mxfp4_moe_gemm_pre": [_P, _I, _I64, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I,
                           _I64, _P, _P, _P, _I, _P, _P, _P, _I64, _I, _I64, _I, _P],
    "mxfp4_fused_moe_workspace_size": [_I64, _I, _I64, _I, _I, _P],
    "mxfp4_fused_moe": [_P, _I, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _I, _P, _P, _P, _I,
                        _P, _I, _I64, _I, _P, _I64, _P],
    "mxfp4_fused_moe_pre": [_P, _I, _I64, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I,
                            _P, _P, _P, _I, _P, _I, _I64, _I, _P, _I64, _P],
    "mxfp4_moe_layer_workspace_size": [_I64, _I, _I, _I64, _I64, _P],
    "mxfp4_moe_layer": [_P, _I, _I64, _I64, _P, _P, _P, _P, _I, _I64, _P, _P, _I, _I, _P, _P,
                        _I64, _P],
    "mxfp4_moe_layer_noalloc": [_P, _I, _I64, _I64, _P, _P, _P, _P, _I, _I64, _P, _P, _I, _I,
                                _P, _P],
    "mxfp4_quant": [_P, _I, _I64, _I64, _I64, _I, _P, _P, _P],
    "mxfp4_prepack_w4a16_size": [_I64, _I64, _I64, _P, _P],
    "mxfp4_prepack_w4a16": [_P, _P, _I64, _I64, _I64, _P, _P, _P],
    "mxfp4_linear_w4a16_pre": [_P, _I, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _I64,
                               _P],
    "mxfp4_moe_layer_pre": [_P, _I, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I64, _P, _P,
                            _I, _I, _P, _P, _I64, _P],
}

_lib = None
_lock = threading.Lock()


def load():
    """Load (once) and return the library; raise RuntimeError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"mxfp4_amd: HIP library not found at {LIB_PATH}; build it with "
                "`python mxfp4-gfx936_amd/build.py` (there is no fallback path)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        lib.mxfp4_last_error.argtypes = []
        lib.mxfp4_last_error.restype = ctypes.c_char_p
        if lib.mxfp4_abi_version() != ABI_VERSION:
            raise RuntimeError("mxfp4_amd: libmxfp4_gfx950.so ABI version mismatch; rebuild it")
        _lib = lib
    return _lib


_ERRORS = {
    ERR_TYPE: TypeError,
    ERR_VALUE: ValueError,
    ERR_NOT_IMPLEMENTED: NotImplementedError,
    ERR_RUNTIME: RuntimeError,
    ERR_HIP: RuntimeError,
}


def check(rc: int) -> None:
    """Raise the exception class of a non-zero status with the library message."""
    if rc != OK:
        msg = load().mxfp4_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, RuntimeError)(msg)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; returns it.  CPU tensors are refused:
    this backend has no host path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"mxfp4_amd runs on ROCm devices only; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


# torch's current-stream lookup without building a Stream object (~0.1 us
# instead of ~2 us per call); the public API where it is absent
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device):
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def on_device(device: torch.device):
    """Context making ``device`` current for the library's HIP calls (a no-op
    when it already is)."""
    if device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def aligned(t: torch.Tensor, nbytes: int = 16) -> torch.Tensor:
    """Row-contiguous copy unless ``t`` is already contiguous and aligned."""
    if not t.is_contiguous() or t.data_ptr() % nbytes:
        t = t.contiguous()
        if t.data_ptr() % nbytes:
            t = t.clone()
    return t
