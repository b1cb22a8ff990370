"""The prepacked weight layout: its numpy statement pinned on the CPU, and
validation of prepacked copies against the call they are passed to."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import prepack_layout_np
from mxfp4_amd.prepack import PrepackedWeights, check_prepacked


def test_prepack_layout_known_positions():
    # every byte distinct enough to locate: row r, byte b -> (r * 7 + b) % 256
    e, rows, k = 2, 20, 128
    packed = ((np.arange(rows)[:, None] * 7 + np.arange(k // 2)[None, :]) % 256).astype(np.uint8)
    packed = np.stack([packed, packed ^ 0xFF])
    scales = (np.arange(rows)[:, None] + 10 * np.arange(k // 32)[None, :]).astype(np.uint8)
    scales = np.stack([scales, scales + 1])
    nib, sc = prepack_layout_np(packed, scales)
    assert nib.shape == (2, 2, 2, 64, 8) and sc.shape == (2, 2, 2, 16, 2)
    # lane 37 = quad 2, row 5 of group 1 (row 21: padding) and group 0 (row 5)
    for ex in range(2):
        for st in range(2):
            got = nib[ex, 0, st, 37]
            for j in range(2):
                off = st * 32 + j * 16 + 2 * 4
                assert (got[j * 4:(j + 1) * 4] == packed[ex, 5, off:off + 4]).all()
            assert (nib[ex, 1, st, 37] == 0).all()
            for j in range(2):
                assert sc[ex, 0, st, 5, j] == (int(scales[ex, 5, 2 * st + j]) << 7) | 0x40
                assert sc[ex, 1, st, 5, j] == (127 << 7) | 0x40
            # group 1, row 3 = weight row 19 (live)
            assert sc[ex, 1, st, 3, 1] == (int(scales[ex, 19, 2 * st + 1]) << 7) | 0x40


def test_prepack_layout_is_a_permutation():
    # rows a multiple of 16: the nibble blocks hold every weight byte once
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, size=(3, 48, 128), dtype=np.uint8)
    scales = rng.integers(0, 256, size=(3, 48, 8), dtype=np.uint8)
    nib, sc = prepack_layout_np(packed, scales)
    assert np.array_equal(np.sort(nib.reshape(3, -1), axis=1), np.sort(packed.reshape(3, -1), axis=1))
    # the scale operand (the stored half shifted up) has the E8M0 byte as its
    # exponent field and mantissa 0x400000
    op = sc.astype(np.uint32) << 16
    assert np.array_equal(np.sort((op >> 23).reshape(3, -1), axis=1),
                          np.sort(scales.reshape(3, -1).astype(np.uint32), axis=1))
    assert ((op & 0x7FFFFF) == 0x400000).all()
    # the scale operand as a float is 1.5 * 2^(s - 127) for normal bytes,
    # byte 255 gives NaN
    v = op.view(np.float32)
    b = (op >> 23).astype(np.int64)
    normal = (b > 0) & (b < 255)
    assert np.allclose(v[normal], 1.5 * np.exp2(b[normal] - 127.0), rtol=0)
    assert np.isnan(v[b == 255]).all()


def test_check_prepacked_rejects_mismatches():
    pre = PrepackedWeights(torch.zeros(512, dtype=torch.uint8), torch.zeros(32), 1, 16, 64)
    cpu = torch.device("cpu")
    assert check_prepacked(None, 1, 16, 64, cpu, "t") is None
    assert check_prepacked(pre, 1, 16, 64, cpu, "t") is pre
    with pytest.raises(ValueError, match="prepacked copy is for 1 x 16 x 64"):
        check_prepacked(pre, 1, 32, 64, cpu, "t")
    with pytest.raises(ValueError):
        check_prepacked(pre, 2, 16, 64, cpu, "t")
    with pytest.raises(TypeError, match="prepack_w4a16"):
        check_prepacked((pre.nibbles, pre.scales), 1, 16, 64, cpu, "t")


def test_check_prepacked_rejects_stale_copies():
    from mxfp4_amd.prepack import _source_of
    cpu = torch.device("cpu")
    w = torch.zeros((16, 32), dtype=torch.uint8)
    s = torch.zeros((16, 2), dtype=torch.uint8)
    pre = PrepackedWeights(torch.zeros(512, dtype=torch.uint8), torch.zeros(32), 1, 16, 64,
                           (_source_of(w), _source_of(s)))
    assert check_prepacked(pre, 1, 16, 64, cpu, "t", w, s) is pre
    # a view of the same storage at the same address and version is the same weights
    assert check_prepacked(pre, 1, 16, 64, cpu, "t", w.view(16, 32), s) is pre
    # other tensors of the same shape
    with pytest.raises(ValueError, match="stale"):
        check_prepacked(pre, 1, 16, 64, cpu, "t", w.clone(), s)
    # an in-place write bumps the version counter (also through a view)
    w[0, 0] = 1
    with pytest.raises(ValueError, match="stale"):
        check_prepacked(pre, 1, 16, 64, cpu, "t", w, s)
    pre2 = PrepackedWeights(pre.nibbles, pre.scales, 1, 16, 64, (_source_of(w), _source_of(s)))
    s[:, 1:].fill_(3)
    with pytest.raises(ValueError, match="stale"):
        check_prepacked(pre2, 1, 16, 64, cpu, "t", w, s)
    # inference-mode tensors keep no version: the address is still compared
    with torch.inference_mode():
        wi = torch.zeros((16, 32), dtype=torch.uint8)
    pre3 = PrepackedWeights(pre.nibbles, pre.scales, 1, 16, 64, (_source_of(wi), _source_of(s)))
    assert check_prepacked(pre3, 1, 16, 64, cpu, "t", wi, s) is pre3
    with pytest.raises(ValueError, match="stale"):
        check_prepacked(pre3, 1, 16, 64, cpu, "t", w, s)


def test_vllm_hooks_prepack_again_after_an_update(monkeypatch):
    # the apply hooks' freshness rule with a stand-in for the device prepack
    from torch.nn import Parameter

    from mxfp4_amd import vllm_adapter as V
    from mxfp4_amd.prepack import _source_of
    made = []

    def fake_prepacked(packed, scales):
        made.append(1)
        return PrepackedWeights(torch.zeros(1), torch.zeros(1), 1, packed.shape[0],
                                packed.shape[1] * 2, (_source_of(packed), _source_of(scales)))

    monkeypatch.setattr(V, "_prepacked", fake_prepacked)

    class Layer:
        pass
    layer = Layer()
    layer.weight_packed = Parameter(torch.zeros((16, 32), dtype=torch.uint8), requires_grad=False)
    layer.weight_scale = Parameter(torch.zeros((16, 2), dtype=torch.uint8), requires_grad=False)
    layer.mxfp4_prepacked = V._prepacked(layer.weight_packed, layer.weight_scale)
    first = layer.mxfp4_prepacked
    assert V._current(layer, "mxfp4_prepacked", layer.weight_packed, layer.weight_scale) is first
    with torch.no_grad():
        layer.weight_packed.copy_(torch.ones((16, 32), dtype=torch.uint8))
    second = V._current(layer, "mxfp4_prepacked", layer.weight_packed, layer.weight_scale)
    assert second is not first and layer.mxfp4_prepacked is second and len(made) == 2
    # current again: no further prepack
    assert V._current(layer, "mxfp4_prepacked", layer.weight_packed, layer.weight_scale) is second
    # a replaced parameter is other weights
    layer.weight_scale = Parameter(torch.ones((16, 2), dtype=torch.uint8), requires_grad=False)
    V._current(layer, "mxfp4_prepacked", layer.weight_packed, layer.weight_scale)
    assert len(made) == 3
    V.refresh_prepacked(layer)
    assert len(made) == 4


def test_registry_serves_current_copies_only():
    # register / lookup / unregister with a hand-built copy of CPU tensors
    # (the rule is host logic; the GPU tests run the operators through it)
    import gc

    from mxfp4_amd.prepack import (_REGISTRY, _source_of, lookup_prepacked, register_prepacked,
                                   unregister_prepacked)
    w = torch.zeros((2, 16, 32), dtype=torch.uint8)
    s = torch.zeros((2, 16, 2), dtype=torch.uint8)

    def copy_of(w, s):
        return PrepackedWeights(torch.zeros(1), torch.zeros(1), 2, 16, 64,
                                (_source_of(w), _source_of(s)))
    pre = register_prepacked(w, s, copy_of(w, s))
    assert lookup_prepacked(w, s) is pre
    assert lookup_prepacked(w.view(2, 16, 32), s) is pre
    assert lookup_prepacked(w.clone(), s) is None           # other weights
    assert lookup_prepacked(w, s.clone()) is None           # other scales: not served ...
    assert lookup_prepacked(w, s) is pre                    # ... but not dropped either
    assert lookup_prepacked(w[:1], s[:1]) is None           # another shape at the address
    with pytest.raises(ValueError, match="stale"):
        register_prepacked(w.clone(), s, pre)                # a copy of other tensors
    with pytest.raises(ValueError, match="prepacked copy is for"):
        register_prepacked(w[:, :8], s[:, :8], pre)
    w[1, 3, 0] = 7                                          # in-place write: stale for good
    assert lookup_prepacked(w, s) is None
    assert w.data_ptr() not in _REGISTRY
    pre2 = register_prepacked(w, s, copy_of(w, s))
    assert lookup_prepacked(w, s) is pre2
    unregister_prepacked(w)
    assert lookup_prepacked(w, s) is None
    unregister_prepacked(w)                                 # no error when absent
    # the entry goes with the registered tensor, so memory reused at that
    # address never meets the old copy
    w3 = torch.zeros((2, 16, 32), dtype=torch.uint8)
    register_prepacked(w3, s, copy_of(w3, s))
    key = w3.data_ptr()
    del w3
    gc.collect()
    assert key not in _REGISTRY
    with pytest.raises(ValueError, match=r"\[N, K/2\]"):
        register_prepacked(w[0, 0], s[0, 0], pre)
    # dense weights [N, K/2]: one expert of N rows
    wd = torch.zeros((16, 32), dtype=torch.uint8)
    sd = torch.zeros((16, 2), dtype=torch.uint8)
    pd = PrepackedWeights(torch.zeros(1), torch.zeros(1), 1, 16, 64, (_source_of(wd), _source_of(sd)))
    assert register_prepacked(wd, sd, pd) is pd
    assert lookup_prepacked(wd, sd) is pd
    with pytest.raises(ValueError, match="prepacked copy is for 1 x 16 x 64"):
        register_prepacked(wd[:8], sd[:8], pd)
    unregister_prepacked(wd)
    assert lookup_prepacked(wd, sd) is None


def test_prepacked_entry_points_refuse_half_a_copy():
    # the C-ABI _pre entry points need both halves of the copy; the check
    # runs before anything touches the device
    import ctypes

    from mxfp4_amd import _lib
    lib = _lib.load()
    null, fake = ctypes.c_void_p(), ctypes.c_void_p(4096)
    rc = lib.mxfp4_moe_gemm_pre(null, _lib.DT_BF16, 1, 128, null, null, null, fake, null, 4, 64,
                                128, null, _lib.DT_BF16, 64, null, null, null, 0, null, null, null,
                                16, 16, 2, 2, null)
    assert rc == _lib.ERR_VALUE and "come together" in lib.mxfp4_last_error().decode()
    rc = lib.mxfp4_fused_moe_pre(null, _lib.DT_BF16, 1, 128, null, null, null, null, fake, 4, 64,
                                 128, null, _lib.DT_BF16, null, null, null, 0, null, _lib.DT_I32,
                                 1, 2, null, 0, null)
    assert rc == _lib.ERR_VALUE and "come together" in lib.mxfp4_last_error().decode()
    # the workspace covers either layout's routing blocks
    a, b = ctypes.c_int64(), ctypes.c_int64()
    assert lib.mxfp4_fused_moe_workspace_size(512, 4, 16, _lib.DT_BF16, _lib.DT_BF16,
                                              ctypes.byref(a)) == 0
    assert lib.mxfp4_fused_moe_workspace_size(512, 4, 16, _lib.DT_F32, _lib.DT_F32,
                                              ctypes.byref(b)) == 0
    assert a.value > 0 and b.value > 0
