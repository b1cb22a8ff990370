"""The drop-in boundary, on the CPU: the C-ABI library loads and exports
every declared entry point, its argument checks return the documented error
classes before anything is enqueued, and the Python surface raises the
reference's exception types (soft:283-294, 317-329, 398-407) in the
reference's order."""

from __future__ import annotations

import ctypes
import importlib.util
import os
import re

import pytest
import torch

from mxfp4_amd import _lib
import mxfp4_amd as mx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mxfp4_gfx950.h")
SOFT = os.path.join(ROOT, "mxfp4-gfx936_amd", "mxfp4_amd", "moe_op_mxfp4_soft.py")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(mxfp4_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES or name == "mxfp4_last_error"
    assert lib.mxfp4_abi_version() == _lib.ABI_VERSION


def _split_ws(m, k, n):
    out = ctypes.c_int64(-1)
    assert _lib.load().mxfp4_linear_w4a16_workspace_size(m, k, n, ctypes.byref(out)) == _lib.OK
    return out.value


def test_linear_split_k_workspace_plan():
    # the dense linear splits K (FP32 slices in a caller workspace) only for
    # grids that would leave CUs idle; decode sizes and full grids need none
    assert _split_ws(1, 4096, 2048) == 0          # skinny decode kernel
    assert _split_ws(48, 4096, 2048) == 0         # 32-row skinny blocks
    assert _split_ws(4096, 2048, 5120) == 0       # the headline fills the GPU
    assert _split_ws(370, 2048, 5120) == 0        # 480 tiles of 32 rows
    assert _split_ws(128, 2048, 5120) == 0        # short K: slices do not pay
    assert _split_ws(370, 4096, 2048) == 4 * 370 * 2048 * 4
    assert _split_ws(128, 4096, 2048) == 4 * 128 * 2048 * 4
    assert _split_ws(200, 4096, 2048) == 4 * 200 * 2048 * 4
    assert _split_ws(130, 8192, 640) == 8 * 130 * 640 * 4
    assert _split_ws(64, 2048, 1536) == 4 * 64 * 1536 * 4
    assert _split_ws(64, 8192, 1024) > 0          # long K: split beats skinny
    out = ctypes.c_int64(0)
    assert _lib.load().mxfp4_linear_w4a16_workspace_size(-1, 128, 8, ctypes.byref(out)) \
        == _lib.ERR_VALUE


def test_c_abi_argument_errors_without_launch():
    lib = _lib.load()
    null = ctypes.c_void_p()
    rc = lib.mxfp4_dequant(null, 16, null, 1, 1, 32, null, 9, null)
    assert rc == _lib.ERR_TYPE
    rc = lib.mxfp4_dequant(null, 16, null, 1, 1, 48, null, _lib.DT_BF16, null)
    assert rc == _lib.ERR_VALUE
    assert "divisible by 32" in lib.mxfp4_last_error().decode()
    rc = lib.mxfp4_linear_w4a16(null, _lib.DT_F32, 1, 128, 128, null, null, 8, null, null, null)
    assert rc == _lib.ERR_TYPE
    rc = lib.mxfp4_linear_w4a16(null, _lib.DT_BF16, 1, 96, 96, null, null, 8, null, null, null)
    assert rc == _lib.ERR_VALUE
    assert "divisible by 128" in lib.mxfp4_last_error().decode()
    rc = lib.mxfp4_moe_gemm(null, _lib.DT_BF16, 1, 128, null, null, null, 4, 64, 128, null,
                            _lib.DT_I32, 64, null, null, null, 0, null, null, null, 16, 16, 2,
                            2, null)
    assert rc == _lib.ERR_TYPE
    rc = lib.mxfp4_moe_gemm(null, _lib.DT_U8, 1, 64, null, null, null, 4, 64, 128, null,
                            _lib.DT_BF16, 64, null, null, null, 0, null, null, null, 16, 16, 2,
                            2, null)
    assert rc == _lib.ERR_VALUE and "A_mx_scale" in lib.mxfp4_last_error().decode()
    rc = lib.mxfp4_quant(null, _lib.DT_BF16, 1, 40, 40, 0, null, null, null)
    assert rc == _lib.ERR_VALUE
    rc = lib.mxfp4_quant(null, _lib.DT_BF16, 1, 64, 64, 7, null, null, null)
    assert rc == _lib.ERR_VALUE


def test_c_abi_size_queries():
    lib = _lib.load()
    ms, mb, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert lib.mxfp4_moe_align_sizes(8, 128, 16, ctypes.byref(ms), ctypes.byref(mb),
                                     ctypes.byref(ws)) == 0
    # 8 routes can touch at most 8 experts: 8 + 8 * 15 padded rows
    assert ms.value == 128 and mb.value == 8 and ws.value == 128 * 4
    assert lib.mxfp4_moe_align_sizes(4096 * 8, 128, 128, ctypes.byref(ms), ctypes.byref(mb),
                                     ctypes.byref(ws)) == 0
    assert ms.value >= 4096 * 8 and ms.value % 128 == 0 and mb.value == ms.value // 128
    assert lib.mxfp4_moe_align_sizes(8, 2000, 16, ctypes.byref(ms), ctypes.byref(mb),
                                     ctypes.byref(ws)) == _lib.ERR_VALUE
    nb = ctypes.c_int64()
    assert lib.mxfp4_moe_layer_workspace_size(512, 8, 128, 2048, 768, ctypes.byref(nb)) == 0
    assert nb.value >= 512 * 8 * (2048 + 768) * 2


def test_backend_env(monkeypatch):
    monkeypatch.delenv("MXFP4_GFX936_BACKEND", raising=False)
    from mxfp4_amd import moe_op_mxfp4_soft as soft
    assert soft._backend() == "safe"
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "unknown")
    with pytest.raises(ValueError, match="unknown gfx936 MXFP4 backend"):
        soft._backend()
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "triton")
    assert soft._backend() == "triton"


def test_rounding_env(monkeypatch):
    from mxfp4_amd import moe_op_mxfp4_soft as soft
    monkeypatch.delenv("MXFP4_GFX950_ROUNDING", raising=False)
    assert soft._reference_rounding() is False
    monkeypatch.setenv("MXFP4_GFX950_ROUNDING", "reference")
    assert soft._reference_rounding() is True
    monkeypatch.setenv("MXFP4_GFX950_ROUNDING", "twice")
    with pytest.raises(ValueError, match="MXFP4_GFX950_ROUNDING"):
        soft._reference_rounding()


def test_soft_module_loads_by_path_like_the_reference_tests():
    spec = importlib.util.spec_from_file_location("moe_op_mxfp4_soft", SOFT)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    assert module._MXFP4_E2M1_VALUES[8] == 0.0 and str(module._MXFP4_E2M1_VALUES[8]) == "-0.0"
    for name in ("dequant_mxfp4", "linear_mxfp4_soft", "fused_moe_mxfp4_soft"):
        assert callable(getattr(module, name))


def test_dequant_validation():
    u8 = torch.zeros((2, 16), dtype=torch.uint8)
    s8 = torch.zeros((2, 1), dtype=torch.uint8)
    with pytest.raises(TypeError, match="packed must be uint8"):
        mx.dequant_mxfp4(u8.to(torch.int8), s8)
    with pytest.raises(TypeError, match="block_scales must be uint8"):
        mx.dequant_mxfp4(u8, s8.to(torch.int8))
    with pytest.raises(ValueError, match="divisible by 32"):
        mx.dequant_mxfp4(torch.zeros((2, 8), dtype=torch.uint8), s8)
    with pytest.raises(ValueError, match="leading dimensions"):
        mx.dequant_mxfp4(u8, torch.zeros((3, 1), dtype=torch.uint8))
    with pytest.raises(ValueError, match="every 32"):
        mx.dequant_mxfp4(u8, torch.zeros((2, 2), dtype=torch.uint8))
    # valid arguments on the CPU: no host path, fails loudly
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        mx.dequant_mxfp4(u8, s8)


def test_linear_validation():
    x = torch.zeros((2, 128), dtype=torch.bfloat16)
    w = torch.zeros((8, 64), dtype=torch.uint8)
    s = torch.zeros((8, 4), dtype=torch.uint8)
    with pytest.raises(TypeError, match="fp16 or bf16"):
        mx.linear_mxfp4_soft(x.float(), w, s)
    with pytest.raises(TypeError, match="must be uint8"):
        mx.linear_mxfp4_soft(x, w.to(torch.int8), s)
    with pytest.raises(ValueError, match="must be 2D"):
        mx.linear_mxfp4_soft(x, w[None], s)
    with pytest.raises(ValueError, match="does not match weight K"):
        mx.linear_mxfp4_soft(x[:, :64], w, s)
    with pytest.raises(ValueError, match="divisible by 128"):
        mx.linear_mxfp4_soft(torch.zeros((2, 96), dtype=torch.bfloat16),
                             torch.zeros((8, 48), dtype=torch.uint8),
                             torch.zeros((8, 3), dtype=torch.uint8))
    with pytest.raises(ValueError, match="every 32"):
        mx.linear_mxfp4_soft(x, w, s[:, :3])
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        mx.linear_mxfp4_soft(x, w, s)


def _moe_args(**kw):
    m, k, n, e, top_k = 4, 128, 64, 4, 2
    args = dict(
        A=torch.zeros((m, k), dtype=torch.bfloat16),
        B=torch.zeros((e, n, k // 2), dtype=torch.uint8),
        C=torch.zeros((m, top_k, n), dtype=torch.bfloat16),
        A_scale=torch.ones(1), B_scale=torch.ones(e), A_mx_scale=None,
        B_mx_scale=torch.zeros((e, n, k // 32), dtype=torch.uint8),
        topk_weights=torch.ones((m, top_k)), topk_ids=torch.zeros((m, top_k), dtype=torch.int64),
        sorted_token_ids=torch.empty(0), expert_ids=torch.empty(0),
        num_tokens_post_padded=torch.empty(0), mul_routed_weight=False, top_k=top_k,
        swizzle_mx_a=False, swizzle_mx_b=False)
    args.update(kw)
    return args


def test_fused_moe_validation_order():
    with pytest.raises(NotImplementedError, match="swizzled"):
        mx.fused_moe_mxfp4_soft(**_moe_args(swizzle_mx_b=True, B=torch.zeros(1)))
    with pytest.raises(ValueError, match="matching"):
        mx.fused_moe_mxfp4_soft(**_moe_args(topk_weights=torch.ones((4, 3))))
    with pytest.raises(ValueError, match="matching"):
        mx.fused_moe_mxfp4_soft(**_moe_args(top_k=3))
    with pytest.raises(TypeError, match="packed MXFP4 weights"):
        mx.fused_moe_mxfp4_soft(**_moe_args(B=torch.zeros((4, 64, 64), dtype=torch.int8)))
    with pytest.raises(TypeError, match="packed MXFP4 weights"):
        mx.fused_moe_mxfp4_soft(**_moe_args(B_mx_scale=None))
    with pytest.raises(TypeError, match="compute dtype"):
        mx.fused_moe_mxfp4_soft(**_moe_args(C=torch.zeros((4, 2, 64), dtype=torch.float64)))
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        mx.fused_moe_mxfp4_soft(**_moe_args())


def test_aiter_entry_validation():
    base = _moe_args()
    for k in ("sorted_token_ids", "expert_ids", "num_tokens_post_padded"):
        base.pop(k)
    meta = dict(sorted_token_ids=torch.zeros(16, dtype=torch.int32),
                expert_ids=torch.zeros(1, dtype=torch.int32),
                num_tokens_post_padded=torch.tensor([16], dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        mx.fused_moe_mxfp4(**{**base, **meta, "swizzle_mx_a": True},
                           config={"BLOCK_SIZE_M": 16}, compute_type=torch.bfloat16)
    with pytest.raises(TypeError, match="compute_type"):
        mx.fused_moe_mxfp4(**base, **meta, config={"BLOCK_SIZE_M": 16},
                           compute_type=torch.float16)
    with pytest.raises(RuntimeError, match="block size"):
        mx.fused_moe_mxfp4(**base, **meta, config={"BLOCK_SIZE_M": 24},
                           compute_type="tl.bfloat16")
    with pytest.raises(AssertionError):
        mx.fused_moe_mxfp4(**{**base, **meta, "A_mx_scale": torch.zeros(1)},
                           config={"BLOCK_SIZE_M": 16}, compute_type=torch.bfloat16)


def test_moe_layer_and_quant_validation():
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    w13 = torch.zeros((4, 64, 32), dtype=torch.uint8)
    s13 = torch.zeros((4, 64, 2), dtype=torch.uint8)
    w2 = torch.zeros((4, 64, 16), dtype=torch.uint8)
    s2 = torch.zeros((4, 64, 1), dtype=torch.uint8)
    ids = torch.zeros((2, 2), dtype=torch.int64)
    w = torch.ones((2, 2))
    with pytest.raises(NotImplementedError, match="silu"):
        mx.moe_layer(x, w13, s13, w2, s2, w, ids, activation="gelu")
    with pytest.raises(ValueError, match="inconsistent"):
        mx.moe_layer(x, w13, s13, w2[:, :32], s2, w, ids)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        mx.moe_layer(x, w13, s13, w2, s2, w, ids)
    with pytest.raises(ValueError, match="unknown quantizer mode"):
        mx.dynamic_mxfp4_quant(x, mode="floor")
    with pytest.raises(ValueError, match="divisible by 32"):
        mx.dynamic_mxfp4_quant(x[:, :40])


def test_route_topk_argument_errors():
    # the router's argument checks run before anything touches a device
    x = torch.zeros(4, 8)
    with pytest.raises(TypeError):
        mx.route_topk(x, 2, ids_dtype=torch.int16)
    with pytest.raises(ValueError):
        mx.route_topk(x, 9)
    with pytest.raises(ValueError):
        mx.route_topk(torch.zeros(4, 2000), 2)
    lib = _lib.load()
    i64, f32 = _lib.dtype_code(torch.int64), _lib.dtype_code(torch.float32)
    # C ABI: ids must be int32/int64, row stride >= experts, top_k <= experts
    assert lib.mxfp4_moe_route(None, 4, 8, 8, 2, 1, None, None, f32, None) == _lib.ERR_TYPE
    assert lib.mxfp4_moe_route(None, 4, 8, 4, 2, 1, None, None, i64, None) == _lib.ERR_VALUE
    assert lib.mxfp4_moe_route(None, 4, 8, 8, 9, 1, None, None, i64, None) == _lib.ERR_VALUE
    assert lib.mxfp4_moe_route(None, 4, 2048, 2048, 2, 1, None, None, i64, None) == _lib.ERR_VALUE
    assert lib.mxfp4_moe_route(None, 0, 8, 8, 2, 1, None, None, i64, None) == _lib.OK


def test_reference_policy_names(monkeypatch):
    # soft:34-62, with the behaviour the reference tests check (test:63-78,
    # 136-141): the shape guard, and the triton value failing loudly when the
    # compiler probe says no (the probe is looked up at call time)
    from mxfp4_amd import moe_op_mxfp4_soft as soft
    assert soft._is_validated_triton_linear_shape(369, 2048) is False
    assert soft._is_validated_triton_linear_shape(370, 2047) is False
    assert soft._is_validated_triton_linear_shape(370, 2048) is True
    assert soft._has_compatible_triton_compiler() is True  # the HIP library is built
    soft._require_triton_compiler()
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "triton")
    monkeypatch.setattr(soft, "_has_compatible_triton_compiler", lambda: False)
    with pytest.raises(RuntimeError, match="TRITON_HIP_CLANG_PATH"):
        soft._require_triton_compiler()
    x = torch.zeros((2, 128), dtype=torch.bfloat16)
    w = torch.zeros((8, 64), dtype=torch.uint8)
    s = torch.zeros((8, 4), dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="TRITON_HIP_CLANG_PATH"):
        soft.linear_mxfp4_soft(x, w, s)
    with pytest.raises(RuntimeError, match="TRITON_HIP_CLANG_PATH"):
        soft.fused_moe_mxfp4_soft(**_moe_args())


def test_fused_moe_triton_value_checks_metadata(monkeypatch):
    # soft:410-427: the triton value needs unpacked activations and padded
    # metadata of block size 16/32/64/128 (RuntimeError otherwise); the safe
    # value ignores the metadata
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "triton")
    with pytest.raises(RuntimeError, match="valid padded routing metadata"):
        mx.fused_moe_mxfp4_soft(**_moe_args())
    meta = dict(sorted_token_ids=torch.zeros(48, dtype=torch.int32),
                expert_ids=torch.zeros(2, dtype=torch.int32),
                num_tokens_post_padded=torch.tensor([48], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="block size: 24"):
        mx.fused_moe_mxfp4_soft(**_moe_args(**meta))
    meta["expert_ids"] = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm devices only"):  # valid: reaches the device
        mx.fused_moe_mxfp4_soft(**_moe_args(**meta))
    packed = _moe_args(A=torch.zeros((4, 64), dtype=torch.uint8),
                       A_mx_scale=torch.zeros((4, 4), dtype=torch.uint8), **meta)
    with pytest.raises(RuntimeError, match="unpacked activations"):
        mx.fused_moe_mxfp4_soft(**packed)
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "safe")
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        mx.fused_moe_mxfp4_soft(**packed)


def test_fused_moe_operand_exceptions_follow_the_reference():
    # packed A goes through the reference's dequant_mxfp4 checks (soft:471,
    # 283-294); a K the expert GEMM cannot take fails in its matmul
    # (RuntimeError); an empty A_scale fails its [0] read (soft:477)
    a = torch.zeros((4, 64), dtype=torch.uint8)
    with pytest.raises(ValueError, match="require A_mx_scale"):
        mx.fused_moe_mxfp4_soft(**_moe_args(A=a))
    with pytest.raises(TypeError, match="block_scales must be uint8"):
        mx.fused_moe_mxfp4_soft(**_moe_args(A=a, A_mx_scale=torch.zeros((4, 4))))
    with pytest.raises(ValueError, match="leading dimensions"):
        mx.fused_moe_mxfp4_soft(**_moe_args(A=a, A_mx_scale=torch.zeros((3, 4), dtype=torch.uint8)))
    with pytest.raises(ValueError, match="every 32"):
        mx.fused_moe_mxfp4_soft(**_moe_args(A=a, A_mx_scale=torch.zeros((4, 2), dtype=torch.uint8)))
    with pytest.raises(RuntimeError, match=r"\[M, K/2\]"):
        mx.fused_moe_mxfp4_soft(**_moe_args(A=a[:, :32],
                                            A_mx_scale=torch.zeros((4, 2), dtype=torch.uint8)))
    with pytest.raises(ValueError, match="must not provide A_mx_scale"):
        mx.fused_moe_mxfp4_soft(**_moe_args(A_mx_scale=torch.zeros((4, 4), dtype=torch.uint8)))
    with pytest.raises(IndexError):
        mx.fused_moe_mxfp4_soft(**_moe_args(A_scale=torch.ones(0)))
