# SPDX-License-Identifier: MIT
"""AITER entry point ``fused_moe_mxfp4`` on MI355X.

Mirrors ``integration/aiter/moe_op_mxfp4.py`` ("aiter") of
lutianshu824/mxfp4-gfx936: the 18-parameter signature of aiter:367-386 and
the semantics of its native kernel (aiter:28-364) -- the caller's routing
metadata is used (``sorted_token_ids`` padded with ids >= topk_ids.numel(),
one expert per ``config["BLOCK_SIZE_M"]`` block, expert -1 writes zeros,
``num_tokens_post_padded`` bounds the work) and C is *not* zero-filled
(rows the metadata never names keep their contents).  Where the reference
dispatches gfx936 to the soft op (aiter:390-410), this module is the gfx950
branch: it runs the HIP kernels of libmxfp4_gfx950.so.

Activations: bf16 / fp16 / fp32 (converted to C.dtype), packed MXFP4
(uint8 with ``A_mx_scale``), or OCP FP8 -- ``torch.float8_e4m3fn`` /
``torch.float8_e5m2``, the "e4m3" / "e5m2" formats aiter:11-20 hands to
``tl.dot_scaled`` -- which run on gfx950's block-scaled f8f6f4 MFMA with the
FP8 operand format, each product exact, FP32 accumulation.  FP8 A may come
without ``A_mx_scale`` (the reference's host path, aiter:413-418: every
scale 1) or with E8M0 scales [M, K/32] (the kernel's micro-scaled A,
aiter:182-214, 329-338, which the reference's host assert does not let
through).

Differences, all explicit: swizzled MX scales raise NotImplementedError
(the reference kernel marks them TODO, aiter:69-70, 189-205); ``config``
contributes only BLOCK_SIZE_M (tile shapes are chosen by the library);
``compute_type`` must name C's dtype; FP8 A with ``A_mx_scale`` is accepted.
A prepacked copy of B recorded with ``prepack.register_prepacked`` is read
by the W4A16 prefill kernels while it is current (bitwise the same C).
"""

from __future__ import annotations

from typing import Any, Dict

import torch

from . import _lib
from .moe_op_mxfp4_soft import _FP8_DTYPES, _moe_gemm_launch, _prepare_moe_operands
from .prepack import lookup_prepacked

_COMPUTE_NAMES = {
    torch.bfloat16: ("bfloat16", "bf16"),
    torch.float16: ("float16", "fp16"),
    torch.float32: ("float32", "fp32"),
}


def _compute_matches(compute_type, dtype: torch.dtype) -> bool:
    if compute_type is None:
        return True
    if isinstance(compute_type, torch.dtype):
        return compute_type == dtype
    text = str(compute_type).lower()
    return any(name in text for name in _COMPUTE_NAMES.get(dtype, ()))


def fused_moe_mxfp4(
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    A_scale: torch.Tensor,
    B_scale: torch.Tensor,
    A_mx_scale: torch.Tensor,
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
    config: Dict[str, Any],
    compute_type,
) -> None:
    """aiter:367-472 semantics on gfx950 (see the module docstring)."""
    if swizzle_mx_a or swizzle_mx_b:
        raise NotImplementedError("swizzled MX scales are not supported by the gfx950 backend")
    # aiter:412-424
    assert topk_weights.stride(1) == 1
    assert sorted_token_ids.stride(0) == 1
    assert A_scale is not None
    assert B_scale is not None
    if A.dtype == torch.uint8:
        assert A_mx_scale is not None, "A_mx_scale should exist when A is mxfp4"
    elif A.dtype not in _FP8_DTYPES:
        assert A_mx_scale is None, "A_mx_scale should not exist when A is not mxfp4"
    assert B_mx_scale is not None
    if B.dtype != torch.uint8:
        raise TypeError("fused_moe_mxfp4 requires packed MXFP4 weights")
    if C.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported compute dtype: {C.dtype}")
    if not _compute_matches(compute_type, C.dtype):
        raise TypeError(f"compute_type {compute_type} does not match C dtype {C.dtype}")
    block_m = int(config["BLOCK_SIZE_M"])
    if block_m % 16 != 0 or block_m <= 0:
        raise RuntimeError(f"unsupported routing block size: {block_m}")
    em = sorted_token_ids.numel()
    if em % block_m != 0 or expert_ids.numel() * block_m < em:
        raise RuntimeError("sorted_token_ids must hold whole BLOCK_SIZE_M blocks")
    if num_tokens_post_padded.numel() != 1:
        raise RuntimeError("num_tokens_post_padded must hold one value")

    act, act_mx, b, b_mx, a_scale, b_scale, weights, ids = _prepare_moe_operands(
        A, B, C, A_scale, B_scale, A_mx_scale, B_mx_scale, topk_weights, topk_ids, top_k,
        fp8_activations=True)
    device = _lib.require_device(A, B, C, sorted_token_ids, expert_ids, num_tokens_post_padded)
    num_routes = ids.numel()
    if em == 0 or C.numel() == 0:
        return
    sorted_ids = sorted_token_ids.to(torch.int32).contiguous()
    experts = expert_ids.to(torch.int32).contiguous()
    npp = num_tokens_post_padded.reshape(1).to(torch.int32).contiguous()
    out = C if C.is_contiguous() and C.data_ptr() % 16 == 0 else C.contiguous().clone()
    _moe_gemm_launch(act, act_mx, b, b_mx, out.view(num_routes, B.shape[1]), a_scale, b_scale,
                     weights, mul_routed_weight, sorted_ids, experts, npp, block_m, num_routes,
                     top_k, device, lookup_prepacked(B, B_mx_scale))
    if out is not C:
        C.copy_(out)
