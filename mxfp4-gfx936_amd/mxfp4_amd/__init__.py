# SPDX-License-Identifier: MIT
"""mxfp4_amd -- MI355X (gfx950) MXFP4 backend behind the ``moe_op_mxfp4_soft``
operator surface of lutianshu824/mxfp4-gfx936.

Operators (all compute in libmxfp4_gfx950.so, on the tensors' device and
current stream; no host synchronisation, no fallback path):

* ``dequant_mxfp4``, ``linear_mxfp4_soft``, ``fused_moe_mxfp4_soft`` --
  drop-in for src/aiter/ops/triton/moe_op_mxfp4_soft.py;
* ``fused_moe_mxfp4`` -- AITER's entry (integration/aiter/moe_op_mxfp4.py);
* ``moe_layer`` / ``make_routing`` -- the vLLM MoE layer and routing
  metadata (integration/vllm/vllm_mxfp4_gfx936.py:119-146, 233-265);
  ``route_topk`` -- router logits -> the layer's top-k weights and ids;
* ``dynamic_mxfp4_quant`` / ``linear_mxfp4_w4a4`` -- activation quantizer
  and dense W4A4 on the block-scaled FP4 MFMA;
* ``prepack_w4a16`` -- the fragment-ordered weight copy the prefill GEMMs
  read when given one (``prepacked=`` / ``prepacked13=``, ``prepacked2=``);
  ``register_prepacked`` records one for expert weights, which
  ``fused_moe_mxfp4_soft`` / ``fused_moe_mxfp4`` then find by address.

``mxfp4_amd.vllm_adapter.install()`` points vLLM's compressed-tensors MXFP4
schemes at these operators (integration/vllm/vllm_mxfp4_gfx936.py).
"""

from .moe_op_mxfp4_soft import (  # noqa: F401
    _MXFP4_E2M1_VALUES,
    dequant_mxfp4,
    fused_moe_mxfp4_soft,
    linear_mxfp4_soft,
    make_routing_device,
)
from .moe_op_mxfp4 import fused_moe_mxfp4  # noqa: F401
from .moe_layer import make_routing, moe_layer, route_topk  # noqa: F401
from .quant import dynamic_mxfp4_quant, linear_mxfp4_w4a4  # noqa: F401
from .prepack import (  # noqa: F401
    PrepackedWeights,
    lookup_prepacked,
    prepack_w4a16,
    register_prepacked,
    unregister_prepacked,
)
from . import _lib  # noqa: F401

__all__ = [
    "dequant_mxfp4",
    "linear_mxfp4_soft",
    "fused_moe_mxfp4_soft",
    "fused_moe_mxfp4",
    "moe_layer",
    "make_routing",
    "route_topk",
    "make_routing_device",
    "dynamic_mxfp4_quant",
    "linear_mxfp4_w4a4",
    "prepack_w4a16",
    "PrepackedWeights",
    "register_prepacked",
    "unregister_prepacked",
    "lookup_prepacked",
]
