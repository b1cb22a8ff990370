# SPDX-License-Identifier: MIT
"""MI355X (gfx950) implementation of the ``moe_op_mxfp4_soft`` operator surface.

Same names, signatures, argument meaning and exception behaviour as the
reference module ``src/aiter/ops/triton/moe_op_mxfp4_soft.py`` of
lutianshu824/mxfp4-gfx936 ("soft" below), so callers and tests written for
it run unchanged; every function computes through hand-written HIP kernels in
``libmxfp4_gfx950.so`` on the tensor's device and stream.  There is one
backend: the reference's env switch ``MXFP4_GFX936_BACKEND`` is still
validated (soft:45-49) but both of its values run the HIP kernels.

This file can be imported as ``mxfp4_amd.moe_op_mxfp4_soft`` or loaded by
path with importlib, as the reference tests load their module (test:10-19).
"""

from __future__ import annotations

import ctypes
import functools
import os
import sys

import torch

try:
    from . import _lib
    from .prepack import PrepackedWeights, check_prepacked, lookup_prepacked
except ImportError:  # loaded by file path, outside its package
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    from mxfp4_amd import _lib  # type: ignore[no-redef]
    from mxfp4_amd.prepack import (  # type: ignore[no-redef]
        PrepackedWeights, check_prepacked, lookup_prepacked)

# soft:12-29 (OCP E2M1 code -> value; bit 3 is the sign)
_MXFP4_E2M1_VALUES = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)

_KERNEL_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


@functools.lru_cache(maxsize=1)
def _has_compatible_triton_compiler() -> bool:
    """soft:34-42 (policy name kept).  The reference probes for the DTK clang
    its Triton kernels need; this backend's kernels are compiled ahead of
    time, so what ``MXFP4_GFX936_BACKEND=triton`` needs is the built HIP
    library.  True when that file exists."""
    return os.path.isfile(_lib.LIB_PATH)


def _backend() -> str:
    """soft:45-49: ``MXFP4_GFX936_BACKEND`` in {safe, triton}, default safe;
    anything else fails loudly.  Both values select the HIP kernels here."""
    backend = os.getenv("MXFP4_GFX936_BACKEND", "safe")
    if backend not in ("safe", "triton"):
        raise ValueError(f"unknown gfx936 MXFP4 backend: {backend}")
    return backend


def _reference_rounding() -> bool:
    """``MXFP4_GFX950_ROUNDING``: ``once`` (default) scales the FP32 sum by
    a_scale * b_scale[e] (* route weight) and rounds once to C's dtype, as
    the reference's Triton kernel does (soft:167-173); ``reference`` makes
    the safe value follow the reference safe path's sequence instead
    (soft:487-494: the GEMM result rounded to C's dtype, times a_scale and
    rounded, times b_scale[e] and rounded, times the route weight in FP32
    and rounded).  Anything else fails loudly."""
    mode = os.getenv("MXFP4_GFX950_ROUNDING", "once")
    if mode not in ("once", "reference"):
        raise ValueError(f"unknown MXFP4_GFX950_ROUNDING: {mode}")
    return mode == "reference"


def _require_triton_compiler() -> None:
    """soft:52-57: the ``triton`` backend value fails loudly, with the
    reference's message, when ``_has_compatible_triton_compiler`` says no
    (looked up at call time, so a monkeypatched probe is honoured)."""
    if not _has_compatible_triton_compiler():
        raise RuntimeError(
            "MXFP4_GFX936_BACKEND=triton requires a compatible compiler; "
            "set TRITON_HIP_CLANG_PATH explicitly"
        )


def _is_validated_triton_linear_shape(m: int, n: int) -> bool:
    """soft:60-62: the reference's fused-kernel shape guard (M >= 370 and
    N >= 2048).  Kept as policy: every shape runs the HIP kernels here, and
    the kernel is chosen from the shape by the library itself."""
    return m >= 370 and n >= 2048


def dequant_mxfp4(
    packed: torch.Tensor,
    block_scales: torch.Tensor,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Dequantize packed OCP MXFP4 E2M1 values with E8M0 block scales.

    soft:277-307.  out[..., k] = E2M1[nibble(k)] * 2**(s[..., k//32] - 127),
    evaluated exactly in FP32 and rounded once to ``dtype`` (RNE), with the
    low nibble as the even k; s = 255 gives NaN.  Bit-exact with the
    reference for float32 / bfloat16 / float16 outputs; other float dtypes
    are converted from the exact FP32 result, as the reference's ``.to``.
    """
    if packed.dtype != torch.uint8:
        raise TypeError(f"packed must be uint8, got {packed.dtype}")
    if block_scales.dtype != torch.uint8:
        raise TypeError(f"block_scales must be uint8, got {block_scales.dtype}")

    logical_k = packed.shape[-1] * 2
    if logical_k % 32 != 0:
        raise ValueError(f"logical K must be divisible by 32, got {logical_k}")
    if block_scales.shape[:-1] != packed.shape[:-1]:
        raise ValueError("packed and block_scales leading dimensions must match")
    if block_scales.shape[-1] * 32 != logical_k:
        raise ValueError("one E8M0 scale is required for every 32 MXFP4 values")

    device = _lib.require_device(packed, block_scales)
    lib = _lib.load()
    kernel_dtype = dtype if dtype in _KERNEL_DTYPES else torch.float32
    out_shape = (*packed.shape[:-1], logical_k)
    out = torch.empty(out_shape, dtype=kernel_dtype, device=device)
    rows = out.numel() // logical_k if logical_k else 0
    if rows and logical_k:
        p = _lib.aligned(packed.reshape(rows, logical_k // 2))
        s = block_scales.reshape(rows, logical_k // 32).contiguous()
        with _lib.on_device(device):
            _lib.check(lib.mxfp4_dequant(
                _lib.ptr(p), p.stride(0), _lib.ptr(s), s.stride(0), rows, logical_k,
                _lib.ptr(out), _lib.dtype_code(kernel_dtype), _lib.stream_of(device)))
    return out if kernel_dtype == dtype else out.to(dtype)


_LINEAR_WS: dict = {}


def _linear_workspace_bytes(lib, m: int, k: int, n: int) -> int:
    """Split-K workspace bytes of the dense linear (a pure function of the
    sizes, cached)."""
    key = (m, k, n)
    v = _LINEAR_WS.get(key)
    if v is None:
        out = ctypes.c_int64(0)
        _lib.check(lib.mxfp4_linear_w4a16_workspace_size(m, k, n, ctypes.byref(out)))
        if len(_LINEAR_WS) >= 4096:
            _LINEAR_WS.clear()
        v = _LINEAR_WS[key] = out.value
    return v


def linear_mxfp4_soft(
    x: torch.Tensor,
    packed: torch.Tensor,
    block_scales: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    prepacked: PrepackedWeights | None = None,
) -> torch.Tensor:
    """Weight-only OCP MXFP4 linear: ``x @ dequant(packed, block_scales).T (+ bias)``.

    soft:310-376.  BF16/FP16 activations, FP32 accumulation, one rounding to
    x.dtype.  A bias of x's dtype and shape [N] is fused into the epilogue;
    any other bias is added afterwards with torch's promotion, as the
    reference does (soft:374-375).  ``prepacked`` (keyword only; from
    ``prepack_w4a16(packed, block_scales)``) lets the prefill kernels read
    the fragment-ordered copy; the result is bitwise the same.  Without it,
    a current copy recorded with ``prepack.register_prepacked(packed,
    block_scales)`` is used.
    """
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"x must be fp16 or bf16, got {x.dtype}")
    if packed.dtype != torch.uint8 or block_scales.dtype != torch.uint8:
        raise TypeError("packed weights and E8M0 scales must be uint8")
    if packed.ndim != 2 or block_scales.ndim != 2:
        raise ValueError("linear weights and scales must be 2D")
    logical_k = packed.shape[1] * 2
    if x.shape[-1] != logical_k:
        raise ValueError(f"input K {x.shape[-1]} does not match weight K {logical_k}")
    if logical_k % 128 != 0:
        raise ValueError(f"logical K must be divisible by 128, got {logical_k}")
    if block_scales.shape != (packed.shape[0], logical_k // 32):
        raise ValueError("one E8M0 scale is required for every 32 MXFP4 values")

    input_shape = x.shape
    if _backend() == "triton":
        _require_triton_compiler()  # soft:333-334
    device = _lib.require_device(x, packed, block_scales, bias)
    lib = _lib.load()
    n = packed.shape[0]
    pre = check_prepacked(prepacked, 1, n, logical_k, device, "linear_mxfp4_soft", packed,
                          block_scales)
    if prepacked is None:
        pre = lookup_prepacked(packed, block_scales)
    x_2d = _lib.aligned(x.reshape(-1, logical_k))
    w = _lib.aligned(packed)
    s = block_scales.contiguous()
    fuse_bias = (bias is not None and bias.dtype == x.dtype and bias.ndim == 1
                 and bias.shape[0] == n)
    b = bias.contiguous() if fuse_bias else None
    output = torch.empty((x_2d.shape[0], n), dtype=x.dtype, device=device)
    if x_2d.shape[0] and n:
        # GEMMs too small to fill the GPU split K through a workspace
        ws_bytes = _linear_workspace_bytes(lib, x_2d.shape[0], logical_k, n)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
        with _lib.on_device(device):
            _lib.check(lib.mxfp4_linear_w4a16_pre(
                _lib.ptr(x_2d), _lib.dtype_code(x.dtype), x_2d.shape[0], logical_k,
                x_2d.stride(0), _lib.ptr(w), _lib.ptr(s),
                _lib.ptr(pre.nibbles if pre else None), _lib.ptr(pre.scales if pre else None),
                n, _lib.ptr(b), _lib.ptr(output), _lib.ptr(ws), ws_bytes,
                _lib.stream_of(device)))
    if bias is not None and not fuse_bias:
        output = output + bias
    return output.reshape(*input_shape[:-1], n)


def make_routing_device(topk_ids: torch.Tensor, num_experts: int, block_m: int):
    """Device-side routing metadata (the vllm:119-146 format) without a host
    sync.  Returns (sorted_ids, expert_ids, num_tokens_post_padded), the first
    two sized to their capacity; entries at or beyond
    ``num_tokens_post_padded[0]`` (resp. its block count) are unused."""
    device = _lib.require_device(topk_ids)
    lib = _lib.load()
    ids = topk_ids.reshape(-1)
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    ids = ids.contiguous()
    n = ids.numel()
    import ctypes
    ms, mb, wsb = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _lib.check(lib.mxfp4_moe_align_sizes(n, num_experts, block_m, ctypes.byref(ms),
                                         ctypes.byref(mb), ctypes.byref(wsb)))
    sorted_ids = torch.empty(ms.value, dtype=torch.int32, device=device)
    expert_ids = torch.empty(mb.value, dtype=torch.int32, device=device)
    npp = torch.empty(1, dtype=torch.int32, device=device)
    ws = torch.empty(max(wsb.value // 4, 1), dtype=torch.int32, device=device)
    with _lib.on_device(device):
        _lib.check(lib.mxfp4_moe_align(
            _lib.ptr(ids), _lib.dtype_code(ids.dtype), n, num_experts, block_m,
            _lib.ptr(sorted_ids), _lib.ptr(expert_ids), _lib.ptr(npp), _lib.ptr(ws),
            wsb.value, _lib.stream_of(device)))
    return sorted_ids, expert_ids, npp


def _moe_gemm_launch(A, A_mx_scale, B, B_mx_scale, C2d, A_scale, B_scale, topk_weights,
                     mul_routed_weight, sorted_ids, expert_ids, npp, block_m, num_valid,
                     top_k, device, pre=None):
    """Launch the routed grouped GEMM writing rows of the contiguous 2-D view
    ``C2d`` [routes, N] (``pre``: a current prepacked copy of B, or None)."""
    lib = _lib.load()
    num_experts, n, k = B.shape[0], B.shape[1], B.shape[2] * 2
    a_code = _lib.dtype_code(A.dtype)
    a_row_stride = A.stride(0)
    pre_b, pre_s = (None, None) if pre is None else (pre.nibbles, pre.scales)
    with _lib.on_device(device):
        _lib.check(lib.mxfp4_moe_gemm_pre(
            _lib.ptr(A), a_code, A.shape[0], a_row_stride, _lib.ptr(A_mx_scale), _lib.ptr(B),
            _lib.ptr(B_mx_scale), _lib.ptr(pre_b), _lib.ptr(pre_s), num_experts, n, k,
            _lib.ptr(C2d), _lib.dtype_code(C2d.dtype),
            C2d.stride(0), _lib.ptr(A_scale), _lib.ptr(B_scale), _lib.ptr(topk_weights),
            1 if mul_routed_weight else 0, _lib.ptr(sorted_ids), _lib.ptr(expert_ids),
            _lib.ptr(npp), sorted_ids.numel(), block_m, num_valid, top_k,
            _lib.stream_of(device)))


_FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)


def _prepare_moe_operands(A, B, C, A_scale, B_scale, A_mx_scale, B_mx_scale, topk_weights,
                          topk_ids, top_k, fp8_activations=False):
    """Shared shape checks and layout normalisation for the routed GEMM.
    ``fp8_activations`` (AITER's entry): OCP FP8 A (e4m3 / e5m2) stays in
    its format, with optional E8M0 A_mx_scale [M, K/32], for the
    block-scaled MFMA; otherwise non-packed A is converted to C.dtype."""
    matmul_dtype = C.dtype
    if B.ndim != 3 or B_mx_scale.shape != (B.shape[0], B.shape[1], B.shape[2] * 2 // 32):
        raise ValueError("B must be [E, N, K/2] with B_mx_scale [E, N, K/32]")
    logical_k = B.shape[2] * 2
    if logical_k % 32 != 0:
        raise ValueError(f"logical K must be divisible by 32, got {logical_k}")
    if A.dtype == torch.uint8:
        if A_mx_scale is None:
            raise ValueError("packed MXFP4 activations require A_mx_scale")
        # the reference dequantizes packed A with dequant_mxfp4 (soft:471),
        # whose checks (soft:283-294) give these exception types
        if A_mx_scale.dtype != torch.uint8:
            raise TypeError(f"block_scales must be uint8, got {A_mx_scale.dtype}")
        a_k = A.shape[-1] * 2
        if a_k % 32 != 0:
            raise ValueError(f"logical K must be divisible by 32, got {a_k}")
        if A_mx_scale.shape[:-1] != A.shape[:-1]:
            raise ValueError("packed and block_scales leading dimensions must match")
        if A_mx_scale.shape[-1] * 32 != a_k:
            raise ValueError("one E8M0 scale is required for every 32 MXFP4 values")
        # a K or rank the expert GEMM cannot take fails in the reference's
        # matmul (soft:487-490), a RuntimeError
        if A.ndim != 2 or a_k != logical_k:
            raise RuntimeError("packed activations must be [M, K/2] with A_mx_scale [M, K/32]")
        act = _lib.aligned(A)
        act_mx = A_mx_scale.contiguous()
    elif fp8_activations and A.dtype in _FP8_DTYPES:
        if A.ndim != 2 or A.shape[1] != logical_k:
            raise RuntimeError(f"activations must be [M, {logical_k}], got {tuple(A.shape)}")
        if A_mx_scale is not None:
            if A_mx_scale.dtype != torch.uint8:
                raise TypeError(f"A_mx_scale must be uint8, got {A_mx_scale.dtype}")
            if A_mx_scale.shape != (A.shape[0], logical_k // 32):
                raise ValueError("one E8M0 scale is required for every 32 FP8 values")
            act_mx = A_mx_scale.contiguous()
        else:
            act_mx = None
        act = _lib.aligned(A)
    else:
        if A_mx_scale is not None:
            raise ValueError("unpacked activations must not provide A_mx_scale")
        if A.ndim != 2 or A.shape[1] != logical_k:
            raise RuntimeError(f"activations must be [M, {logical_k}], got {tuple(A.shape)}")
        # soft:475 converts A to the compute dtype; with C in FP32, bf16 and
        # fp16 A go in as they are, and the kernels widen them exactly
        # (bf16 A: the W4A16 prefill tiles storing FP32; fp16: the FP32 MFMA)
        keep = A.dtype == matmul_dtype or (matmul_dtype == torch.float32
                                           and A.dtype in (torch.bfloat16, torch.float16))
        act = A if keep else A.to(matmul_dtype)
        act = _lib.aligned(act)
        act_mx = None
    m = topk_ids.shape[0]
    if C.shape != (m, top_k, B.shape[1]):
        raise RuntimeError(
            f"C must be [M, top_k, N] = {(m, top_k, B.shape[1])}, got {tuple(C.shape)}")
    if act.shape[0] < m:
        raise RuntimeError("fewer activation rows than top-k rows")
    if A_scale.numel() == 0:
        # the reference reads A_scale.reshape(-1)[0] (soft:477)
        raise IndexError("index 0 is out of bounds for dimension 0 with size 0")
    a_scale = A_scale.reshape(-1)[:1].to(torch.float32).contiguous()
    if B_scale.numel() < B.shape[0]:
        raise RuntimeError("B_scale must hold one scale per expert")
    b_scale = B_scale.reshape(-1).to(torch.float32).contiguous()
    weights = topk_weights.to(torch.float32).contiguous()
    ids = topk_ids if topk_ids.dtype in (torch.int32, torch.int64) else topk_ids.to(torch.int64)
    ids = ids.contiguous()
    return act, act_mx, _lib.aligned(B), B_mx_scale.contiguous(), a_scale, b_scale, weights, ids


def fused_moe_mxfp4_soft(
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    A_scale: torch.Tensor,
    B_scale: torch.Tensor,
    A_mx_scale: torch.Tensor | None,
    B_mx_scale: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    mul_routed_weight: bool,
    top_k: int,
    swizzle_mx_a: bool,
    swizzle_mx_b: bool,
) -> None:
    """Routed MXFP4 MoE GEMM writing ``C`` [M, top_k, N] in place.

    soft:379-494 (safe semantics): C is zero-filled, then for every (token t,
    slot s) whose expert e = topk_ids[t, s] is in [0, E):
    C[t, s] = A[t] . dequant(B[e])^T * A_scale[0] * B_scale[e]
    (* topk_weights[t, s] when ``mul_routed_weight``), FP32 accumulation, one
    rounding to C.dtype (with ``MXFP4_GFX950_ROUNDING=reference`` the safe
    path's own rounding sequence, soft:487-494; see ``_reference_rounding``).
    A is bf16/fp16/fp32 (converted to C.dtype, soft:475)
    or packed MXFP4 with ``A_mx_scale`` (W4A4 on the block-scaled MFMA).
    Like the reference's safe path, the routing metadata arguments are not
    consulted (soft:466): one library call builds the routing on the device
    from ``topk_ids`` (no host synchronisation) and runs the grouped GEMM;
    rows of out-of-range ids get zeros, so C needs no separate fill.  With
    ``MXFP4_GFX936_BACKEND=triton`` the reference's checks of that backend
    run (soft:410-427: compiler, unpacked activations, non-empty metadata of
    a supported block size, K a multiple of 128; RuntimeError otherwise) and,
    as its Triton kernel does (soft:428-464, 100-115), C is zero-filled and
    the grouped GEMM runs over the caller's ``sorted_token_ids`` /
    ``expert_ids`` / ``num_tokens_post_padded`` (expert -1 blocks give
    zeros; routes the metadata does not name stay zero).  A prepacked copy
    of B recorded with ``prepack.register_prepacked`` is read instead of B
    while it is current (bitwise the same C).
    """
    if swizzle_mx_a or swizzle_mx_b:
        raise NotImplementedError("the gfx936 software fallback does not support swizzled scales")
    if topk_ids.shape != topk_weights.shape or topk_ids.shape[1] != top_k:
        raise ValueError("top-k ids and weights must have matching (M, top_k) shapes")
    if B.dtype != torch.uint8 or B_mx_scale is None:
        raise TypeError("the gfx936 software fallback requires packed MXFP4 weights")

    matmul_dtype = C.dtype
    if matmul_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported software fallback compute dtype: {matmul_dtype}")

    if _backend() == "triton":
        _require_triton_compiler()
        routing_ready = (
            A.dtype != torch.uint8
            and sorted_token_ids.numel() > 0
            and expert_ids.numel() > 0
            and num_tokens_post_padded.numel() == 1
            and B.shape[-1] * 2 % 128 == 0
            and sorted_token_ids.numel() % expert_ids.numel() == 0
        )
        if not routing_ready:
            raise RuntimeError(
                "the experimental Triton MoE backend requires unpacked "
                "activations and valid padded routing metadata"
            )
        block_m = sorted_token_ids.numel() // expert_ids.numel()
        if block_m not in (16, 32, 64, 128):
            raise RuntimeError(f"unsupported Triton routing block size: {block_m}")
        _fused_moe_caller_metadata(A, B, C, A_scale, B_scale, B_mx_scale, topk_weights, topk_ids,
                                   sorted_token_ids, expert_ids, num_tokens_post_padded,
                                   mul_routed_weight, top_k, block_m)
        return
    del sorted_token_ids, expert_ids, num_tokens_post_padded
    # bit 0: route weights; bit 1: the safe path's rounding sequence
    flags = (1 if mul_routed_weight else 0) | (2 if _reference_rounding() else 0)
    # operand checks first (soft:468-477), then the device
    act, act_mx, b, b_mx, a_scale, b_scale, weights, ids = _prepare_moe_operands(
        A, B, C, A_scale, B_scale, A_mx_scale, B_mx_scale, topk_weights, topk_ids, top_k)
    device = _lib.require_device(A, B, C, A_scale, B_scale, A_mx_scale, B_mx_scale,
                                 topk_weights, topk_ids)
    m = ids.shape[0]
    num_routes = ids.numel()
    if num_routes == 0 or C.numel() == 0:
        return
    lib = _lib.load()
    num_experts, n, k = b.shape[0], b.shape[1], b.shape[2] * 2
    a_code, c_code = _lib.dtype_code(act.dtype), _lib.dtype_code(C.dtype)
    ws_bytes = _fused_workspace_bytes(lib, m, top_k, num_experts, a_code, c_code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    out = C if C.is_contiguous() and C.data_ptr() % 16 == 0 else torch.empty(
        C.shape, dtype=C.dtype, device=device)
    pre = lookup_prepacked(B, B_mx_scale)
    pre_b, pre_s = (None, None) if pre is None else (pre.nibbles, pre.scales)
    with _lib.on_device(device):
        _lib.check(lib.mxfp4_fused_moe_pre(
            _lib.ptr(act), a_code, act.shape[0], act.stride(0), _lib.ptr(act_mx), _lib.ptr(b),
            _lib.ptr(b_mx), _lib.ptr(pre_b), _lib.ptr(pre_s), num_experts, n, k, _lib.ptr(out),
            c_code, _lib.ptr(a_scale),
            _lib.ptr(b_scale), _lib.ptr(weights), flags, _lib.ptr(ids),
            _lib.dtype_code(ids.dtype), m, top_k, _lib.ptr(ws), ws_bytes,
            _lib.stream_of(device)))
    if out is not C:
        C.copy_(out)


_FUSED_WS: dict = {}


def _fused_workspace_bytes(lib, m: int, top_k: int, num_experts: int, a_code: int,
                           c_code: int) -> int:
    """Workspace bytes of mxfp4_fused_moe (a pure function of the sizes, cached)."""
    key = (m, top_k, num_experts, a_code, c_code)
    v = _FUSED_WS.get(key)
    if v is None:
        out = ctypes.c_int64(0)
        _lib.check(lib.mxfp4_fused_moe_workspace_size(m, top_k, num_experts, a_code, c_code,
                                                      ctypes.byref(out)))
        if len(_FUSED_WS) >= 4096:
            _FUSED_WS.clear()
        v = _FUSED_WS[key] = out.value
    return v


def _fused_moe_caller_metadata(A, B, C, A_scale, B_scale, B_mx_scale, topk_weights, topk_ids,
                               sorted_token_ids, expert_ids, num_tokens_post_padded,
                               mul_routed_weight, top_k, block_m):
    """The ``triton`` backend value (soft:428-464): C zero-filled, then the
    grouped GEMM over the caller's routing metadata (its kernel takes no
    A_mx_scale: the activations are unpacked)."""
    act, act_mx, b, b_mx, a_scale, b_scale, weights, ids = _prepare_moe_operands(
        A, B, C, A_scale, B_scale, None, B_mx_scale, topk_weights, topk_ids, top_k)
    device = _lib.require_device(A, B, C, A_scale, B_scale, B_mx_scale, topk_weights, topk_ids,
                                 sorted_token_ids, expert_ids, num_tokens_post_padded)
    C.zero_()
    num_routes = ids.numel()
    if num_routes == 0 or C.numel() == 0:
        return
    sorted_ids = sorted_token_ids.to(torch.int32).contiguous()
    experts = expert_ids.to(torch.int32).contiguous()
    npp = num_tokens_post_padded.reshape(1).to(torch.int32).contiguous()
    out = C if C.is_contiguous() and C.data_ptr() % 16 == 0 else torch.zeros(
        C.shape, dtype=C.dtype, device=device)
    _moe_gemm_launch(act, act_mx, b, b_mx, out.view(num_routes, B.shape[1]), a_scale, b_scale,
                     weights, mul_routed_weight, sorted_ids, experts, npp, block_m, num_routes,
                     top_k, device, lookup_prepacked(B, B_mx_scale))
    if out is not C:
        C.copy_(out)
