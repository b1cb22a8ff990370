# SPDX-License-Identifier: MIT
"""Prepacked MXFP4 weights for the prefill GEMMs.

The reference accepts only the checkpoint layout (row-major nibbles and
E8M0 bytes) and leaves kernel-friendly swizzled layouts to AITER's own
kernels (aiter:189-205, 229-248; soft:398-399 rejects them).  Here the
offline repack is explicit: ``prepack_w4a16`` turns (packed, block_scales)
into a fragment-ordered copy (per 16-row group and 64-deep K step, the
nibbles in the order the MFMA fragments are read, and the E8M0 bytes as the
high halves of the conversion instruction's FP32 scale operands), made once
when the weights are loaded (the vLLM adapter does it in process_weights_after_loading,
vllm:68-70).  ``linear_mxfp4_soft(..., prepacked=...)`` and
``moe_layer(..., prepacked13=..., prepacked2=...)`` then read the copy in
their prefill kernels; the results are bitwise equal to the checkpoint-layout
calls.  Decode-sized calls keep using the checkpoint layout, which must stay
allocated.

A copy belongs to the weights it was made from.  It records their storage
address and version counter (``Tensor._version``, which in-place writes to
the tensor or its views bump); a call given the copy with other tensors, or
with the same tensors after such a write (``with torch.no_grad():
param.copy_(...)``), raises ``ValueError`` instead of reading stale
weights, and the vLLM hooks prepack such weights again before the call.
Writes through ``param.data`` are not versioned by PyTorch (``.data`` is a
new tensor with its own counter) and are not seen: prepack again after them
(``vllm_adapter.refresh_prepacked(layer)`` for a vLLM layer).

The reference's signatures (soft:310-313, 379-396, aiter:367-386) have no
place for a copy.  ``register_prepacked(weights, scales)`` prepacks dense
[N, K/2] or expert [E, N, K/2] weights once and records the copy against
those tensors; ``linear_mxfp4_soft`` (without ``prepacked=``),
``fused_moe_mxfp4_soft`` and ``fused_moe_mxfp4`` then look it up by the
weights' address and use it while it is current (same tensors, same shapes,
no in-place write since), with bitwise the same result.  A stale entry is
dropped at lookup and the call reads the checkpoint layout; an entry also
goes when the registered weight tensor is freed.
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class PrepackedWeights:
    """Fragment-ordered copy of ``experts`` MXFP4 matrices of ``rows`` x ``k``.

    nibbles: uint8 [experts * ceil(rows/16) * k/64 * 512]
    scales:  int16 [experts * ceil(rows/16) * k/64 * 32] (operand high halves)
    """

    nibbles: torch.Tensor
    scales: torch.Tensor
    experts: int
    rows: int
    k: int
    # (data_ptr, _version) of the packed weights and of the scales it was
    # made from; None when unknown (a copy built by hand)
    source: tuple | None = None

    def matches(self, experts: int, rows: int, k: int, device: torch.device) -> bool:
        return (self.experts, self.rows, self.k) == (experts, rows, k) and \
            self.nibbles.device == device and self.scales.device == device

    def is_current(self, packed: torch.Tensor, block_scales: torch.Tensor) -> bool:
        """True when (packed, block_scales) are the tensors this copy was made
        from and neither was written in place since."""
        if self.source is None:
            return True
        return self.source == (_source_of(packed), _source_of(block_scales))


def _source_of(t: torch.Tensor):
    """(storage address, version counter) of a tensor; inference-mode tensors
    keep no version counter, and then only the address is compared."""
    try:
        version = t._version
    except RuntimeError:
        version = None
    return (t.data_ptr(), version)


def prepack_w4a16(packed: torch.Tensor, block_scales: torch.Tensor) -> PrepackedWeights:
    """Prepack [rows, K/2] / [rows, K/32] (dense) or [E, rows, K/2] /
    [E, rows, K/32] (experts) uint8 weights on their GPU.  K % 64 == 0."""
    if packed.dtype != torch.uint8 or block_scales.dtype != torch.uint8:
        raise TypeError("packed weights and E8M0 scales must be uint8")
    if packed.ndim not in (2, 3) or block_scales.ndim != packed.ndim:
        raise ValueError("prepack takes [rows, K/2] or [E, rows, K/2] weights")
    p3 = packed if packed.ndim == 3 else packed.unsqueeze(0)
    s3 = block_scales if block_scales.ndim == 3 else block_scales.unsqueeze(0)
    experts, rows, half_k = p3.shape
    k = half_k * 2
    if s3.shape != (experts, rows, k // 32):
        raise ValueError("one E8M0 scale is required for every 32 MXFP4 values")
    if k % 64 != 0:
        raise ValueError(f"prepack needs K divisible by 64, got {k}")
    if experts < 1 or rows < 1:
        raise ValueError("prepack needs at least one row")
    device = _lib.require_device(packed, block_scales)
    lib = _lib.load()
    nb, sb = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(lib.mxfp4_prepack_w4a16_size(experts, rows, k, ctypes.byref(nb), ctypes.byref(sb)))
    nibbles = torch.empty(nb.value, dtype=torch.uint8, device=device)
    scales = torch.empty(sb.value // 2, dtype=torch.int16, device=device)
    w = _lib.aligned(p3)
    s = s3.contiguous()
    with _lib.on_device(device):
        _lib.check(lib.mxfp4_prepack_w4a16(
            _lib.ptr(w), _lib.ptr(s), experts, rows, k, _lib.ptr(nibbles), _lib.ptr(scales),
            _lib.stream_of(device)))
    return PrepackedWeights(nibbles, scales, experts, rows, k,
                            (_source_of(packed), _source_of(block_scales)))


def check_prepacked(pre: PrepackedWeights | None, experts: int, rows: int, k: int,
                    device: torch.device, what: str, packed: torch.Tensor | None = None,
                    block_scales: torch.Tensor | None = None) -> PrepackedWeights | None:
    """Validate a caller's prepacked copy against the weights of the call
    (shapes and device; with ``packed`` / ``block_scales``, also that the copy
    was made from those tensors and they have not been written since)."""
    if pre is None:
        return None
    if not isinstance(pre, PrepackedWeights):
        raise TypeError(f"{what}: prepacked weights must come from prepack_w4a16")
    if not pre.matches(experts, rows, k, device):
        raise ValueError(
            f"{what}: prepacked copy is for {pre.experts} x {pre.rows} x {pre.k} on "
            f"{pre.nibbles.device}, the call has {experts} x {rows} x {k} on {device}")
    if packed is not None and block_scales is not None and not pre.is_current(packed,
                                                                              block_scales):
        raise ValueError(
            f"{what}: prepacked copy is stale: it was made from other weight tensors, or "
            f"they were written in place since; call prepack_w4a16 again")
    return pre


# data_ptr of the registered packed weights -> (copy, weak reference to that
# tensor); the reference's callback removes the entry when the tensor is
# freed, so a later tensor at the same address never meets the old copy
_REGISTRY: dict = {}
_REGISTRY_LOCK = threading.Lock()


def register_prepacked(packed: torch.Tensor, block_scales: torch.Tensor,
                       prepacked: PrepackedWeights | None = None) -> PrepackedWeights:
    """Record a prepacked copy of dense weights ``packed`` [N, K/2] /
    ``block_scales`` [N, K/32] or expert weights [E, N, K/2] / [E, N, K/32]
    for the operators that take no copy argument (made here with
    ``prepack_w4a16`` unless ``prepacked`` is given, which must have been made
    from these tensors).  Registering the same tensor again replaces the
    copy.  Returns the registered copy."""
    if packed.ndim not in (2, 3) or block_scales.ndim != packed.ndim:
        raise ValueError("register_prepacked takes weights [N, K/2] / [N, K/32] or "
                         "[E, N, K/2] / [E, N, K/32]")
    experts, rows, k = _dims(packed)
    if prepacked is None:
        prepacked = prepack_w4a16(packed, block_scales)
    check_prepacked(prepacked, experts, rows, k, packed.device, "register_prepacked", packed,
                    block_scales)
    key = packed.data_ptr()

    def _drop(ref, key=key):
        with _REGISTRY_LOCK:
            entry = _REGISTRY.get(key)
            if entry is not None and entry[1] is ref:
                del _REGISTRY[key]

    with _REGISTRY_LOCK:
        _REGISTRY[key] = (prepacked, weakref.ref(packed, _drop))
    return prepacked


def unregister_prepacked(packed: torch.Tensor) -> None:
    """Forget the copy registered for ``packed`` (no error if there is none)."""
    with _REGISTRY_LOCK:
        _REGISTRY.pop(packed.data_ptr(), None)


def _dims(packed: torch.Tensor):
    """(experts, rows, K) of dense [N, K/2] or expert [E, N, K/2] weights."""
    if packed.ndim == 2:
        return 1, packed.shape[0], packed.shape[1] * 2
    return packed.shape[0], packed.shape[1], packed.shape[2] * 2


def lookup_prepacked(packed: torch.Tensor, block_scales: torch.Tensor) -> PrepackedWeights | None:
    """The registered copy of (packed, block_scales) when it is current, else
    None.  An entry whose registered weight tensor was written in place since
    is removed (version counters only grow, so it cannot become current)."""
    if not _REGISTRY or packed.ndim not in (2, 3):
        return None
    key = packed.data_ptr()
    with _REGISTRY_LOCK:
        entry = _REGISTRY.get(key)
    registered = None if entry is None else entry[1]()
    if registered is None:
        return None
    pre = entry[0]
    experts, rows, k = _dims(packed)
    if not pre.matches(experts, rows, k, packed.device):
        return None
    if pre.is_current(packed, block_scales):
        return pre
    if _source_of(registered) != pre.source[0]:
        # judged on the registered tensor's own counter: another tensor over
        # the same memory (param.data) counts writes separately
        with _REGISTRY_LOCK:
            if _REGISTRY.get(key) is entry:
                del _REGISTRY[key]
    return None
