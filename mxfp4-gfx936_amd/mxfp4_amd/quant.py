# SPDX-License-Identifier: MIT
"""MXFP4 activation quantizer and the dense W4A4 linear on MI355X.

``dynamic_mxfp4_quant(x, mode)`` turns [..., K] bf16/fp16/fp32 activations
into packed E2M1 [..., K/2] + E8M0 [..., K/32] on the device:

* ``mode="ties_away"`` reproduces the reference test quantizer
  ``torch_dynamic_mxfp4_quant`` (tests/test_moe_mxfp4_soft.py:28-60 of
  lutianshu824/mxfp4-gfx936) bit for bit;
* ``mode="rne"`` is the OCP MX rule used for the W4A4 benchmark
  configuration: E = floor(log2(amax)) - 2, E2M1 round-to-nearest-even,
  saturation at +-6.

``linear_mxfp4_w4a4`` multiplies packed activations by packed weights on
gfx950's block-scaled FP4 MFMA (the packed-A semantics of
integration/aiter/moe_op_mxfp4.py:206-214, 329-338 with a single expert).
"""

from __future__ import annotations

import torch

from . import _lib

_MODES = {"ties_away": _lib.QUANT_TIES_AWAY, "rne": _lib.QUANT_RNE}


def dynamic_mxfp4_quant(x: torch.Tensor, mode: str = "ties_away"):
    """Quantize the last dimension of ``x`` in blocks of 32; returns
    (packed uint8 [..., K/2], scales uint8 [..., K/32])."""
    if mode not in _MODES:
        raise ValueError(f"unknown quantizer mode {mode!r}")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"x must be bf16, fp16 or fp32, got {x.dtype}")
    k = x.shape[-1]
    if k % 32:
        raise ValueError("test quantizer requires K divisible by 32")
    device = _lib.require_device(x)
    lib = _lib.load()
    rows = x.numel() // k if k else 0
    packed = torch.empty((*x.shape[:-1], k // 2), dtype=torch.uint8, device=device)
    scales = torch.empty((*x.shape[:-1], k // 32), dtype=torch.uint8, device=device)
    if rows and k:
        x2 = x.reshape(rows, k)
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        with _lib.on_device(device):
            _lib.check(lib.mxfp4_quant(
                _lib.ptr(x2), _lib.dtype_code(x.dtype), rows, k, x2.stride(0), _MODES[mode],
                _lib.ptr(packed), _lib.ptr(scales), _lib.stream_of(device)))
    return packed, scales


def linear_mxfp4_w4a4(a_packed: torch.Tensor, a_scales: torch.Tensor, w_packed: torch.Tensor,
                      w_scales: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """out [M, N] = dequant(a) . dequant(w)^T with FP32 accumulation, rounded
    once to ``out_dtype`` (bf16, fp16 or fp32)."""
    for t, name in ((a_packed, "a_packed"), (a_scales, "a_scales"), (w_packed, "w_packed"),
                    (w_scales, "w_scales")):
        if t.dtype != torch.uint8:
            raise TypeError(f"{name} must be uint8, got {t.dtype}")
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"unsupported output dtype {out_dtype}")
    if a_packed.ndim != 2 or w_packed.ndim != 2:
        raise ValueError("packed operands must be 2D")
    m, n, k = a_packed.shape[0], w_packed.shape[0], a_packed.shape[1] * 2
    if w_packed.shape[1] * 2 != k:
        raise ValueError(f"activation K {k} does not match weight K {w_packed.shape[1] * 2}")
    if k % 32:
        raise ValueError(f"logical K must be divisible by 32, got {k}")
    if a_scales.shape != (m, k // 32) or w_scales.shape != (n, k // 32):
        raise ValueError("one E8M0 scale is required for every 32 MXFP4 values")
    device = _lib.require_device(a_packed, a_scales, w_packed, w_scales)
    lib = _lib.load()
    out = torch.empty((m, n), dtype=out_dtype, device=device)
    if m and n:
        a = _lib.aligned(a_packed)
        w = _lib.aligned(w_packed)
        with _lib.on_device(device):
            _lib.check(lib.mxfp4_linear_w4a4(
                _lib.ptr(a), _lib.ptr(a_scales.contiguous()), m, k, _lib.ptr(w),
                _lib.ptr(w_scales.contiguous()), n, _lib.ptr(out), _lib.dtype_code(out_dtype),
                _lib.stream_of(device)))
    return out
