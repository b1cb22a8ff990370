"""vLLM hooks: the compressed-tensors MXFP4 schemes on the gfx950 backend.

Mirrors the reference adapter ``integration/vllm/vllm_mxfp4_gfx936.py``
(vllm:1-275): the same two schemes are patched with functions of the same
names and meaning,

* ``CompressedTensorsW4A16Mxfp4`` (dense W4A16 layers):
  ``process_weights_after_loading`` (vllm:68-70) and ``apply_weights``
  (vllm:105-116) -> ``linear_mxfp4_soft``;
* ``CompressedTensorsW4A4Mxfp4MoEMethod`` (the MoE layers):
  ``process_weights_after_loading`` (vllm:215-230) and ``apply``
  (vllm:233-265) -> ``moe_layer`` (device routing, gate_up with SiLU*mul,
  down with the route weight, top-k sum; no host synchronisation).

After loading, each layer also gets a prepacked copy of its weights
(``prepack_w4a16``: the fragment-ordered layout its prefill GEMMs read;
bitwise-equal results) as ``layer.mxfp4_prepacked`` (dense) or
``layer.mxfp4_prepacked13`` / ``layer.mxfp4_prepacked2`` (MoE), unless
``MXFP4_GFX950_PREPACK=0`` or the weights are not on a GPU.  The apply hooks
prepack again when a parameter was replaced or written in place since
(its version counter moved); after writes through ``param.data``, which
PyTorch does not version, call ``refresh_prepacked(layer)``.

Call ``install()`` before constructing ``vllm.LLM``.  ``install(dense_cls,
moe_cls)`` patches the given classes instead of importing vLLM's (how the
tests exercise it without vLLM).  ``MXFP4_IMPLEMENTATION`` is read as the
reference reads it (vllm:28-36): ``safe`` (default) and ``triton`` run the
HIP kernels; ``reference`` (alias ``bf16``) is the reference's debug path,
a library GEMM in the activation dtype on weights dequantized by the
bit-exact dequant kernel (vllm:73-102, 188-212); any other value raises
ValueError.
"""

from __future__ import annotations

import os

import torch
import torch.nn.functional as F
from torch.nn.parameter import Parameter

from .moe_layer import moe_layer
from .moe_op_mxfp4_soft import dequant_mxfp4, linear_mxfp4_soft
from .prepack import prepack_w4a16

MIN_VLLM = (0, 15, 0)  # vllm:24-27

# the implementation install() selected (None: read the environment per call)
_IMPL = None


def _implementation() -> str:
    """vllm:28-33: ``MXFP4_IMPLEMENTATION`` in {safe, triton, reference}, with
    ``bf16`` an alias of ``reference``; anything else is a ValueError."""
    impl = os.getenv("MXFP4_IMPLEMENTATION", "safe")
    if impl == "bf16":
        impl = "reference"
    if impl not in ("reference", "safe", "triton"):
        raise ValueError(f"unknown MXFP4 implementation: {impl}")
    return impl


def _active() -> str:
    return _IMPL if _IMPL is not None else _implementation()


# ---------------------------------------------------------------- debug path
# MXFP4_IMPLEMENTATION=reference: the reference's independent bf16 path, a
# library GEMM in the activation dtype on dequantized weights.  The
# reference dequantizes with compressed-tensors' unpack and torch.ldexp
# (vllm:73-91); here the dequant kernel does it, which gives the same
# values (every E2M1 x 2^(s-127) is exact in FP32; s = 255 -> NaN; one
# rounding to the dtype).  Like the reference's, the MoE loop synchronises
# the host once per expert: it is for checking, not for speed.

def _bf16_linear(x, packed, block_scales, bias=None):
    """vllm:94-102: x @ dequant(W).T (+ bias), in x.dtype."""
    k = packed.shape[-1] * 2
    weight = dequant_mxfp4(packed, block_scales, x.dtype)
    out = x.reshape(-1, k) @ weight.T
    if bias is not None:
        out = out + bias
    return out.reshape(*x.shape[:-1], packed.shape[0])


def _bf16_moe_gemm(act, packed, scales, topk_ids, topk_weights, routed):
    """vllm:188-212: for each expert present, its (token, slot) pairs'
    rows times the dequantized expert weights (times the route weight when
    ``routed``, in FP32), rounded to the activation dtype; other slots 0."""
    out = torch.zeros((topk_ids.shape[0], topk_ids.shape[1], packed.shape[1]),
                      dtype=act.dtype, device=act.device)
    for e in torch.unique(topk_ids, sorted=True).tolist():
        tok, slot = torch.nonzero(topk_ids == e, as_tuple=True)
        vals = act[tok] @ dequant_mxfp4(packed[e], scales[e], act.dtype).T
        if routed:
            vals = vals * topk_weights[tok, slot, None]
        out[tok, slot] = vals.to(act.dtype)
    return out


def _bf16_moe_layer(x, w13, s13, w2, s2, topk_weights, topk_ids):
    """vllm:233-265 over _bf16_moe_gemm: gate_up, silu(gate) * up, down with
    the route weights, sum over the top-k slots."""
    gate_up = _bf16_moe_gemm(x, w13, s13, topk_ids, topk_weights, False)
    inter = gate_up.shape[-1] // 2
    h = (F.silu(gate_up[..., :inter]) * gate_up[..., inter:]).reshape(topk_ids.numel(), inter)
    down = _bf16_moe_gemm(h, w2, s2, topk_ids.reshape(-1, 1), topk_weights.reshape(-1, 1), True)
    return down[:, 0].reshape(topk_ids.shape[0], topk_ids.shape[1], x.shape[-1]).sum(dim=1)


def _prepacked(packed, scales):
    """The prepacked copy of loaded weights, or None where it does not apply.
    Made from the parameters the apply hooks pass (not their ``.data``,
    whose version counter is a separate one), so an in-place update of a
    parameter shows as a stale copy."""
    if os.getenv("MXFP4_GFX950_PREPACK", "1") == "0" or not packed.is_cuda:
        return None
    if (packed.shape[-1] * 2) % 64 != 0:
        return None
    return prepack_w4a16(packed, scales)


def _current(layer, attr, packed, scales):
    """The layer's prepacked copy ``attr``, made again first if the weights
    were replaced or written in place since it was made."""
    pre = getattr(layer, attr, None)
    if pre is not None and not pre.is_current(packed, scales):
        pre = _prepacked(packed, scales)
        setattr(layer, attr, pre)
    return pre


def refresh_prepacked(layer) -> None:
    """Prepack a layer's weights again, e.g. after a weight update written
    through ``param.data`` (which PyTorch does not version)."""
    if hasattr(layer, "mxfp4_prepacked"):
        layer.mxfp4_prepacked = _prepacked(layer.weight_packed, layer.weight_scale)
    if hasattr(layer, "mxfp4_prepacked13"):
        layer.mxfp4_prepacked13 = _prepacked(layer.w13_weight, layer.w13_weight_scale)
    if hasattr(layer, "mxfp4_prepacked2"):
        layer.mxfp4_prepacked2 = _prepacked(layer.w2_weight, layer.w2_weight_scale)


def _dense_process_weights_after_loading(self, layer):
    """vllm:68-70: plain frozen parameters for the packed weight and scales,
    plus their prepacked copy."""
    del self
    layer.weight_packed = Parameter(layer.weight_packed.data, requires_grad=False)
    layer.weight_scale = Parameter(layer.weight_scale.data, requires_grad=False)
    layer.mxfp4_prepacked = _prepacked(layer.weight_packed, layer.weight_scale)


def _dense_apply_weights(self, layer, x, bias=None, input_quant_args=None,
                         silu_quant_args=None):
    """vllm:105-116: x @ dequant(weight).T (+ bias) on the W4A16 kernels."""
    del self, input_quant_args, silu_quant_args
    if _active() == "reference":
        return _bf16_linear(x, layer.weight_packed, layer.weight_scale, bias)
    pre = _current(layer, "mxfp4_prepacked", layer.weight_packed, layer.weight_scale)
    return linear_mxfp4_soft(x, layer.weight_packed, layer.weight_scale, bias, prepacked=pre)


def _moe_process_weights_after_loading(self, layer):
    """vllm:215-230: the packed expert weights become ``w13_weight`` /
    ``w2_weight`` (frozen); the ``*_packed`` attributes are removed."""
    del self
    layer.w13_weight = Parameter(layer.w13_weight_packed.data, requires_grad=False)
    layer.w13_weight_scale = Parameter(layer.w13_weight_scale.data, requires_grad=False)
    layer.w2_weight = Parameter(layer.w2_weight_packed.data, requires_grad=False)
    layer.w2_weight_scale = Parameter(layer.w2_weight_scale.data, requires_grad=False)
    delattr(layer, "w13_weight_packed")
    delattr(layer, "w2_weight_packed")
    layer.mxfp4_prepacked13 = _prepacked(layer.w13_weight, layer.w13_weight_scale)
    layer.mxfp4_prepacked2 = _prepacked(layer.w2_weight, layer.w2_weight_scale)


def _moe_apply(self, layer, x, topk_weights, topk_ids, use_nn_moe=False):
    """vllm:233-265: the routed MoE layer for [tokens, hidden] activations."""
    del self, use_nn_moe
    if layer.activation != "silu":
        raise NotImplementedError(
            f"the gfx936 MXFP4 adapter supports silu, got {layer.activation}")
    if _active() == "reference":
        return _bf16_moe_layer(x, layer.w13_weight, layer.w13_weight_scale, layer.w2_weight,
                               layer.w2_weight_scale, topk_weights, topk_ids)
    pre13 = _current(layer, "mxfp4_prepacked13", layer.w13_weight, layer.w13_weight_scale)
    pre2 = _current(layer, "mxfp4_prepacked2", layer.w2_weight, layer.w2_weight_scale)
    return moe_layer(x, layer.w13_weight, layer.w13_weight_scale, layer.w2_weight,
                     layer.w2_weight_scale, topk_weights, topk_ids, activation=layer.activation,
                     prepacked13=pre13, prepacked2=pre2)


def _vllm_classes():
    try:
        import vllm
        from vllm.model_executor.layers.quantization.compressed_tensors.compressed_tensors_moe import (  # noqa: E501
            CompressedTensorsW4A4Mxfp4MoEMethod,
        )
        from vllm.model_executor.layers.quantization.compressed_tensors.schemes.compressed_tensors_w4a16_mxfp4 import (  # noqa: E501
            CompressedTensorsW4A16Mxfp4,
        )
    except ImportError as e:
        raise ImportError(f"the gfx950 MXFP4 adapter needs vLLM >= 0.15: {e}") from e
    version = tuple(int(p) for p in vllm.__version__.split("+")[0].split(".")[:3] if p.isdigit())
    if version < MIN_VLLM:
        raise RuntimeError(f"the gfx950 MXFP4 adapter requires vLLM >= 0.15, got {vllm.__version__}")
    return CompressedTensorsW4A16Mxfp4, CompressedTensorsW4A4Mxfp4MoEMethod


def install(dense_cls=None, moe_cls=None) -> str:
    """Patch the dense and MoE scheme classes (vllm:268-275); returns the
    implementation name.  With no arguments the classes come from vLLM."""
    global _IMPL
    impl = _implementation()
    if dense_cls is None or moe_cls is None:
        d, m = _vllm_classes()
        dense_cls = d if dense_cls is None else dense_cls
        moe_cls = m if moe_cls is None else moe_cls
    _IMPL = impl
    # the operators read this switch too (vllm:34-36, soft:45-49)
    os.environ["MXFP4_GFX936_BACKEND"] = "triton" if impl == "triton" else "safe"
    dense_cls.process_weights_after_loading = _dense_process_weights_after_loading
    dense_cls.apply_weights = _dense_apply_weights
    moe_cls.process_weights_after_loading = _moe_process_weights_after_loading
    moe_cls.apply = _moe_apply
    print(f"MXFP4_GFX950_ADAPTER_ACTIVE torch={torch.__version__} implementation={impl}")
    return impl
