"""The vLLM adapter (mxfp4_amd.vllm_adapter) on the CPU with fake scheme
classes and layers: what it patches (vllm:268-275), the weight renames of
process_weights_after_loading (vllm:68-70, 215-230), the implementation switch
(vllm:28-36), and that apply / apply_weights hand the layer's tensors to
linear_mxfp4_soft / moe_layer (recorded here; the operators themselves are
covered by the GPU tests), or under MXFP4_IMPLEMENTATION=reference compose
the debug path (vllm:94-102, 188-265; here with the oracle's dequant in place
of the device kernel).  vLLM is not installed in this image."""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from _helpers import rand_act, rand_mxfp4
from mxfp4_amd import vllm_adapter as va
from oracle import mxfp4_oracle as O


@pytest.fixture(autouse=True)
def _restore_backend_switch(monkeypatch):
    # install() sets MXFP4_GFX936_BACKEND for the operators and records the
    # implementation; monkeypatch restores both after each test
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "safe")
    monkeypatch.setattr(va, "_IMPL", None)


class _Dense:
    pass


class _MoE:
    pass


def test_install_patches_both_schemes(monkeypatch, capsys):
    monkeypatch.delenv("MXFP4_IMPLEMENTATION", raising=False)
    assert va.install(_Dense, _MoE) == "safe"
    assert _Dense.process_weights_after_loading is va._dense_process_weights_after_loading
    assert _Dense.apply_weights is va._dense_apply_weights
    assert _MoE.process_weights_after_loading is va._moe_process_weights_after_loading
    assert _MoE.apply is va._moe_apply
    assert "MXFP4_GFX950_ADAPTER_ACTIVE" in capsys.readouterr().out


@pytest.mark.parametrize("impl,expect", [("safe", "safe"), ("triton", "triton"),
                                         ("reference", "reference"), ("bf16", "reference"),
                                         ("cuda", None)])
def test_implementation_switch(monkeypatch, impl, expect):
    # vllm:28-36: bf16 is an alias of reference, the operators' backend
    # switch is triton only for triton
    monkeypatch.setenv("MXFP4_IMPLEMENTATION", impl)
    if expect is None:
        with pytest.raises(ValueError, match="unknown MXFP4 implementation"):
            va.install(_Dense, _MoE)
    else:
        assert va.install(_Dense, _MoE) == expect
        assert va._IMPL == expect
        import os
        assert os.environ["MXFP4_GFX936_BACKEND"] == ("triton" if expect == "triton" else "safe")


def test_install_without_vllm_says_so(monkeypatch):
    monkeypatch.delenv("MXFP4_IMPLEMENTATION", raising=False)
    with pytest.raises(ImportError, match="vLLM"):
        va.install()


def test_dense_weights_become_frozen_parameters():
    layer = types.SimpleNamespace(weight_packed=torch.zeros(4, 16, dtype=torch.uint8),
                                  weight_scale=torch.full((4, 1), 127, dtype=torch.uint8))
    va._dense_process_weights_after_loading(object(), layer)
    for t in (layer.weight_packed, layer.weight_scale):
        assert isinstance(t, torch.nn.Parameter) and not t.requires_grad
    assert layer.weight_packed.dtype == torch.uint8
    assert layer.mxfp4_prepacked is None  # CPU weights: no prepacked copy


def test_prepacked_copy_made_for_gpu_weights_unless_disabled(monkeypatch):
    made = []
    monkeypatch.setattr(va, "prepack_w4a16", lambda p, s: made.append((p, s)) or "copy")
    gpu_w = types.SimpleNamespace(is_cuda=True, shape=(64, 1024))
    assert va._prepacked(gpu_w, "S") == "copy" and made == [(gpu_w, "S")]
    # K = 2 * 48 = 96 is not a multiple of 64: the kernels keep the checkpoint layout
    assert va._prepacked(types.SimpleNamespace(is_cuda=True, shape=(64, 48)), "S") is None
    monkeypatch.setenv("MXFP4_GFX950_PREPACK", "0")
    assert va._prepacked(gpu_w, "S") is None and len(made) == 1


def test_moe_weights_renamed_like_the_reference():
    layer = types.SimpleNamespace(
        w13_weight_packed=torch.zeros(2, 64, 16, dtype=torch.uint8),
        w13_weight_scale=torch.zeros(2, 64, 1, dtype=torch.uint8),
        w2_weight_packed=torch.zeros(2, 32, 16, dtype=torch.uint8),
        w2_weight_scale=torch.zeros(2, 32, 1, dtype=torch.uint8))
    va._moe_process_weights_after_loading(object(), layer)
    assert not hasattr(layer, "w13_weight_packed") and not hasattr(layer, "w2_weight_packed")
    for name in ("w13_weight", "w13_weight_scale", "w2_weight", "w2_weight_scale"):
        t = getattr(layer, name)
        assert isinstance(t, torch.nn.Parameter) and not t.requires_grad
    assert layer.w13_weight.shape == (2, 64, 16) and layer.w2_weight.shape == (2, 32, 16)
    assert layer.mxfp4_prepacked13 is None and layer.mxfp4_prepacked2 is None


def test_apply_paths_call_the_operators(monkeypatch):
    calls = []
    monkeypatch.setattr(va, "linear_mxfp4_soft",
                        lambda *a, **k: calls.append(("linear", a, k)) or "y")
    monkeypatch.setattr(va, "moe_layer",
                        lambda *a, **k: calls.append(("moe", a, k)) or "z")
    dense = types.SimpleNamespace(weight_packed="W", weight_scale="S")
    assert va._dense_apply_weights(object(), dense, "x", "b", input_quant_args=1,
                                   silu_quant_args=2) == "y"
    assert calls[-1] == ("linear", ("x", "W", "S", "b"), {"prepacked": None})
    class Copy:  # stands in for the copy process_weights_after_loading made
        def is_current(self, packed, scales):
            return True
    P, P13, P2 = Copy(), Copy(), Copy()
    dense.mxfp4_prepacked = P
    va._dense_apply_weights(object(), dense, "x")
    assert calls[-1] == ("linear", ("x", "W", "S", None), {"prepacked": P})
    moe = types.SimpleNamespace(activation="silu", w13_weight="A", w13_weight_scale="As",
                                w2_weight="B", w2_weight_scale="Bs")
    assert va._moe_apply(object(), moe, "x", "tw", "ti", use_nn_moe=True) == "z"
    assert calls[-1] == ("moe", ("x", "A", "As", "B", "Bs", "tw", "ti"),
                         {"activation": "silu", "prepacked13": None, "prepacked2": None})
    moe.mxfp4_prepacked13, moe.mxfp4_prepacked2 = P13, P2
    va._moe_apply(object(), moe, "x", "tw", "ti")
    assert calls[-1][2] == {"activation": "silu", "prepacked13": P13, "prepacked2": P2}
    moe.activation = "gelu"
    with pytest.raises(NotImplementedError, match="silu"):
        va._moe_apply(object(), moe, "x", "tw", "ti")


def test_reference_debug_path_composition(monkeypatch):
    # MXFP4_IMPLEMENTATION=reference on CPU tensors, with the oracle's
    # dequant (soft:277-307 in torch) standing in for the device kernel:
    # the dense path is x @ dequant(W).T + bias and the MoE path the layer
    # composed over the per-expert loop -- the oracle's own restatements of
    # the same reference functions give the same bits
    monkeypatch.setattr(va, "dequant_mxfp4", lambda p, s, dt: O.dequant_safe(p, s, dt))
    monkeypatch.setattr(va, "_IMPL", "reference")
    rng = np.random.default_rng(91)
    w, ws = rand_mxfp4(rng, (48,), 128)
    x = rand_act(92, (3, 5, 128))
    bias = rand_act(93, (48,))
    dense = types.SimpleNamespace(weight_packed=torch.from_numpy(w),
                                  weight_scale=torch.from_numpy(ws))
    y = va._dense_apply_weights(object(), dense, x, bias)
    assert y.shape == (3, 5, 48) and y.dtype == torch.bfloat16
    assert torch.equal(y, O.linear_safe(x, w, ws, bias))
    e, hidden, inter, m, top_k = 6, 64, 32, 7, 3
    w13, s13 = (torch.from_numpy(a) for a in rand_mxfp4(rng, (e, 2 * inter), hidden))
    w2, s2 = (torch.from_numpy(a) for a in rand_mxfp4(rng, (e, hidden), inter))
    xm = rand_act(94, (m, hidden))
    tw, ti = torch.topk(torch.softmax(torch.randn(m, e, generator=torch.Generator().manual_seed(95)),
                                      -1), top_k, dim=-1)
    moe = types.SimpleNamespace(activation="silu", w13_weight=w13, w13_weight_scale=s13,
                                w2_weight=w2, w2_weight_scale=s2)
    z = va._moe_apply(object(), moe, xm, tw, ti)
    assert z.shape == (m, hidden) and z.dtype == torch.bfloat16
    assert torch.equal(z, O.moe_layer_safe(xm, w13, s13, w2, s2, tw, ti))
