"""The gate_up epilogue's SiLU on every finite, normal bf16 / fp16 input,
through the MoE layer's C-ABI path: gate weights an identity, up weights
picking a constant-1 input column, down weights an identity, one expert,
top_k = 1, route weight 1.  Every product and sum is then exact, so output
column j is silu(x_j) rounded to the activation type (a -0 comes out as
+0 from the down GEMM's accumulation) -- the value the
build-time table (``mxfp4-gfx936_amd/silu_table.py``: torch's FP32 steps,
vllm:249-252) holds for x_j.  64 tokens take the decode kernels (direct
routing, fused down + combine), 1024 tokens the prefill GEMMs."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import mxfp4_oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "mxfp4-gfx936_amd"))
import silu_table as S  # noqa: E402

pytestmark = pytest.mark.gpu

I, H = 1024, 1152  # inter, hidden: test columns 0..1023, constant 1 at H - 1


def _weights():
    gate = np.zeros((I, H), np.float32)
    gate[np.arange(I), np.arange(I)] = 1.0
    up = np.zeros((I, H), np.float32)
    up[:, H - 1] = 1.0
    w13, s13 = O.quant_mxfp4_rne(np.concatenate([gate, up]))
    down = np.zeros((H, I), np.float32)
    down[np.arange(I), np.arange(I)] = 1.0
    w2, s2 = O.quant_mxfp4_rne(down)
    # identity blocks are exact in MXFP4 (1.0 and 0)
    assert np.array_equal(O.dequant_values(w13, s13, "f32"), np.concatenate([gate, up]))
    assert np.array_equal(O.dequant_values(w2, s2, "f32"), down)
    return [torch.from_numpy(t[None]).cuda() for t in (w13, s13, w2, s2)]


def _inputs(kind):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp = (bits >> 7) & 0xFF if kind == "bf16" else (bits >> 10) & 0x1F
    top = 0xFF if kind == "bf16" else 0x1F
    vals = bits[(exp != 0) & (exp != top)]  # finite and normal
    grid = np.zeros(64 * I, np.uint16)
    grid[:vals.size] = vals
    return grid.reshape(64, I)


@pytest.mark.parametrize("reps", [1, 16], ids=["decode_64_tokens", "prefill_1024_tokens"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_silu_epilogue_every_input(dtype, reps):
    kind = "bf16" if dtype == torch.bfloat16 else "f16"
    grid = _inputs(kind)
    x = torch.zeros((64, H), dtype=dtype)
    x[:, :I] = torch.from_numpy(grid.view(np.int16)).view(dtype)
    x[:, H - 1] = 1.0
    x = x.repeat(reps, 1).cuda()
    m = x.shape[0]
    w13, s13, w2, s2 = _weights()
    w = torch.ones((m, 1), dtype=torch.float32, device="cuda")
    ids = torch.zeros((m, 1), dtype=torch.int64, device="cuda")
    y = mx.moe_layer(x, w13, s13, w2, s2, w, ids)
    got = y[:, :I].cpu().view(torch.int16).numpy().view(np.uint16).reshape(reps, 64, I)
    want = S.silu_table(kind)[grid]
    # silu = -0 (x < -88.7: exp overflows FP32) comes out of the identity
    # down GEMM as -0 + 0 = +0; compare zeros without their sign
    sign0 = np.uint16(0x8000)
    got = np.where(got == sign0, np.uint16(0), got)
    want = np.where(want == sign0, np.uint16(0), want)
    for r in range(reps):
        bad = np.argwhere(got[r] != want)
        assert bad.size == 0, (
            f"{kind} rep {r}: {len(bad)} outputs differ, first input bits "
            f"0x{grid[tuple(bad[0])]:04x}: got 0x{got[r][tuple(bad[0])]:04x}, "
            f"want 0x{want[tuple(bad[0])]:04x}")
