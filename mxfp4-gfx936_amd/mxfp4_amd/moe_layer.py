# SPDX-License-Identifier: MIT
"""The routed MoE layer of the vLLM adapter, on MI355X.

``moe_layer`` is the composition of ``_moe_apply`` in
``integration/vllm/vllm_mxfp4_gfx936.py`` ("vllm") of lutianshu824/mxfp4-gfx936
(vllm:233-265, with the soft op as vllm:149-185):

    gate_up = moe(x, w13)                      [M, top_k, 2I], x.dtype
    h       = silu(gate_up[..., :I]) * gate_up[..., I:]
    down    = moe(h, w2) * topk_weights        [M * top_k, H]
    out     = down.reshape(M, top_k, H).sum(1)

It runs as one C-ABI call: device routing (no host sync, unlike the host loop
of vllm:119-146), the gate_up grouped GEMM with SiLU*mul fused into its
epilogue (rounding g, u, silu(g) and the product to x.dtype as the reference
does), the down grouped GEMM with the route weight fused into its epilogue,
and a deterministic FP32 top-k combine.  ``make_routing`` exposes the routing
metadata in the reference format; ``route_topk`` computes the layer's
``topk_weights`` / ``topk_ids`` from router logits on the device.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .moe_op_mxfp4_soft import make_routing_device
from .prepack import PrepackedWeights, check_prepacked


def moe_layer(
    x: torch.Tensor,
    w13: torch.Tensor,
    w13_scale: torch.Tensor,
    w2: torch.Tensor,
    w2_scale: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    activation: str = "silu",
    *,
    prepacked13: PrepackedWeights | None = None,
    prepacked2: PrepackedWeights | None = None,
) -> torch.Tensor:
    """vllm:233-265 for MXFP4 expert weights; returns [M, H] in x.dtype.

    x [M, H] (bf16/fp16); w13 u8 [E, 2I, H/2], w13_scale u8 [E, 2I, H/32];
    w2 u8 [E, H, I/2], w2_scale u8 [E, H, I/32]; topk_weights [M, top_k];
    topk_ids [M, top_k] int.  Slots whose id is outside [0, E) contribute 0.
    prepacked13 / prepacked2 (keyword only; ``prepack_w4a16`` of w13 / w2)
    let the prefill GEMMs read the fragment-ordered copies; the result is
    bitwise the same.
    """
    if activation != "silu":
        raise NotImplementedError(f"the gfx936 MXFP4 adapter supports silu, got {activation}")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"x must be fp16 or bf16, got {x.dtype}")
    for t, name in ((w13, "w13"), (w13_scale, "w13_scale"), (w2, "w2"), (w2_scale, "w2_scale")):
        if t.dtype != torch.uint8:
            raise TypeError(f"{name} must be uint8, got {t.dtype}")
    if x.ndim != 2:
        raise ValueError("x must be [M, H]")
    m, hidden = x.shape
    if w13.ndim != 3 or w2.ndim != 3:
        raise ValueError("expert weights must be [E, N, K/2]")
    num_experts = w13.shape[0]
    inter = w13.shape[1] // 2
    if (w13.shape != (num_experts, 2 * inter, hidden // 2)
            or w13_scale.shape != (num_experts, 2 * inter, hidden // 32)
            or w2.shape != (num_experts, hidden, inter // 2)
            or w2_scale.shape != (num_experts, hidden, inter // 32)):
        raise ValueError("inconsistent MoE weight shapes")
    if hidden % 32 or inter % 32:
        raise ValueError("hidden and intermediate sizes must be multiples of 32")
    if topk_ids.shape != topk_weights.shape or topk_ids.ndim != 2 or topk_ids.shape[0] != m:
        raise ValueError("top-k ids and weights must have matching (M, top_k) shapes")
    top_k = topk_ids.shape[1]
    device = _lib.require_device(x, w13, w13_scale, w2, w2_scale, topk_weights, topk_ids)
    lib = _lib.load()
    pre13 = check_prepacked(prepacked13, num_experts, 2 * inter, hidden, device,
                            "moe_layer w13", w13, w13_scale)
    pre2 = check_prepacked(prepacked2, num_experts, hidden, inter, device, "moe_layer w2", w2,
                           w2_scale)

    xc = _lib.aligned(x)
    ids = topk_ids if topk_ids.dtype in (torch.int32, torch.int64) else topk_ids.to(torch.int64)
    ids = ids.contiguous()
    weights = topk_weights.to(torch.float32).contiguous()
    out = torch.empty((m, hidden), dtype=x.dtype, device=device)
    if m == 0:
        return out
    nbytes = ctypes.c_int64()
    _lib.check(lib.mxfp4_moe_layer_workspace_size(m, top_k, num_experts, hidden, inter,
                                                  ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=device)
    with _lib.on_device(device):
        _lib.check(lib.mxfp4_moe_layer_pre(
            _lib.ptr(xc), _lib.dtype_code(x.dtype), m, hidden, _lib.ptr(_lib.aligned(w13)),
            _lib.ptr(w13_scale.contiguous()), _lib.ptr(pre13.nibbles if pre13 else None),
            _lib.ptr(pre13.scales if pre13 else None), _lib.ptr(_lib.aligned(w2)),
            _lib.ptr(w2_scale.contiguous()), _lib.ptr(pre2.nibbles if pre2 else None),
            _lib.ptr(pre2.scales if pre2 else None), num_experts, inter, _lib.ptr(weights),
            _lib.ptr(ids), _lib.dtype_code(ids.dtype), top_k, _lib.ptr(out), _lib.ptr(ws),
            nbytes.value, _lib.stream_of(device)))
    return out


def make_routing(topk_ids: torch.Tensor, block_m: int = 64, num_experts: int | None = None):
    """vllm:119-146 on the device: (sorted_ids, expert_ids, num_tokens_post_padded).

    Unlike the reference this does not synchronise the host; the first two
    tensors are sized to their capacity and only the first
    ``num_tokens_post_padded[0]`` entries (and as many blocks) are defined.
    ``num_experts`` defaults to ``topk_ids.max() + 1`` (which synchronises);
    ids outside [0, num_experts) are dropped.
    """
    if num_experts is None:
        num_experts = int(topk_ids.max().item()) + 1 if topk_ids.numel() else 1
    return make_routing_device(topk_ids, num_experts, block_m)


def route_topk(router_logits: torch.Tensor, top_k: int, renormalize: bool = True,
               ids_dtype: torch.dtype = torch.int64):
    """Router logits -> (topk_weights, topk_ids) on the device, the inputs of
    ``moe_layer`` (vllm:233-265): softmax over the experts, top-k (as the
    reference tests build them, test:242-244), then, with ``renormalize``,
    weights divided by their sum.  ``router_logits`` [..., E] (converted to
    float32) -> float32 and ``ids_dtype`` (int64 as ``torch.topk``, or int32)
    tensors [..., top_k]; slot r holds the r-th most probable expert, ties
    to the lower expert id.  Logits must be finite; E <= 1024,
    top_k <= min(E, 64)."""
    if ids_dtype not in (torch.int32, torch.int64):
        raise TypeError(f"topk_ids dtype must be int32 or int64, got {ids_dtype}")
    if router_logits.dim() < 1:
        raise ValueError("router_logits needs an expert dimension")
    num_experts = router_logits.shape[-1]
    if not 1 <= top_k <= min(num_experts, 64) or num_experts > 1024:
        raise ValueError(f"unsupported top_k {top_k} for {num_experts} experts")
    device = _lib.require_device(router_logits)
    lead = router_logits.shape[:-1]
    logits = router_logits.reshape(-1, num_experts).to(torch.float32)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    m = logits.shape[0]
    weights = torch.empty((*lead, top_k), dtype=torch.float32, device=device)
    ids = torch.empty((*lead, top_k), dtype=ids_dtype, device=device)
    if m == 0:
        return weights, ids
    lib = _lib.load()
    with _lib.on_device(device):
        _lib.check(lib.mxfp4_moe_route(
            _lib.ptr(logits), m, num_experts, logits.stride(0), top_k, int(bool(renormalize)),
            _lib.ptr(weights), _lib.ptr(ids), _lib.dtype_code(ids_dtype), _lib.stream_of(device)))
    return weights, ids
