"""GPU parity over randomized shapes (fixed seeds): the dense W4A16 linear
(soft:310-376) and the MoE layer (vllm:233-265) at shapes the targeted tests
do not pin -- odd M and N, K from 128 to 8192, bias, fp16, prepacked
weights, 4 to 256 experts, top-1 to top-8 -- so the tile configurations,
split-K plans, decode kernels and routing paths the dispatch picks all meet
the same bar.  Whole outputs are held to FP32-accumulated device GEMMs of
the exact operands (themselves pinned against the FP64 oracle on sampled
rows) and must be no worse than the reference safe path on the same inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import mxfp4_oracle as O

from _helpers import (assert_layer_blocks, assert_rows_parity, cuda, dequant_device, fp32_gemm,
                      moe_layer_device, rand_act, rand_mxfp4, safe_linear_device)

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]
TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _linear_cases(count=36):
    rng = np.random.default_rng(20261202)
    ms = [1, 2, 3, 5, 8, 9, 15, 16, 17, 31, 32, 33, 47, 64, 65, 96, 127, 128, 129, 200, 255,
          256, 257, 370, 511, 777, 1024, 1500, 2100, 4097]
    ks = [128, 256, 384, 640, 768, 1024, 1536, 2048, 3072, 4096, 8192]
    ns = [16, 48, 80, 112, 144, 200, 256, 272, 320, 500, 640, 1000, 1024, 1536, 2048, 2560, 5120]
    cases = []
    while len(cases) < count:
        m, k, n = int(rng.choice(ms)), int(rng.choice(ks)), int(rng.choice(ns))
        if m * k > 1 << 24 or n * k > 1 << 24 or m * n > 1 << 23:
            continue
        cases.append((m, k, n, "f16" if rng.random() < 0.3 else "bf16", bool(rng.random() < 0.3),
                      bool(rng.random() < 0.5)))
    return cases


@pytest.mark.parametrize("m,k,n,dt,bias,pre", _linear_cases(),
                         ids=lambda v: str(v) if not isinstance(v, bool) else ("y" if v else "n"))
def test_linear_shape_fuzz(m, k, n, dt, bias, pre):
    seed = m * 7919 + k * 31 + n
    rng = np.random.default_rng(seed)
    # fp16: smaller scales keep every product and sum finite
    lo, hi = (116, 121) if dt == "f16" else (120, 128)
    packed, scales = rand_mxfp4(rng, (n,), k, lo=lo, hi=hi)
    x = rand_act(seed + 1, (m, k), TDT[dt])
    b = rand_act(seed + 2, (n,), TDT[dt]) if bias else None
    xd, pd, sd = cuda(x), cuda(packed), cuda(scales)
    bd = cuda(b) if bias else None
    pw = mx.prepack_w4a16(pd, sd) if pre else None
    y = mx.linear_mxfp4_soft(xd, pd, sd, bd, prepacked=pw)
    assert y.shape == (m, n) and y.dtype == TDT[dt]
    # whole-output oracle: the exact operands in an FP32 GEMM (+ bias);
    # the reference safe path rounds the GEMM, then adds the bias (soft:372-376)
    o32 = fp32_gemm(xd, dequant_device(packed, scales, dt))
    ref = safe_linear_device(xd, packed, scales)
    if bias:
        o32 = o32 + bd.float()
        ref = ref + bd
    rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, min(m, 6), replace=False)]))
    o64 = O.linear_fp64(x.float().numpy()[rows], packed, scales,
                        b.float().numpy() if bias else None, w_dtype=dt)
    pin = O.parity_errors(o32[torch.from_numpy(rows).cuda()].cpu().numpy(), o64)
    assert pin["norm_rel"] <= 1e-5, pin
    assert_rows_parity(y, o32, ref, what=f"linear {m}x{k}x{n} {dt} bias={bias} pre={pre}",
                       row_block=max(1, 4096 // n), fmt=TDT[dt])


def _moe_cases(count=14):
    rng = np.random.default_rng(20261203)
    cases = []
    while len(cases) < count:
        m = int(rng.choice([1, 2, 3, 5, 8, 13, 24, 40, 64, 100, 300, 700, 1500]))
        e = int(rng.choice([4, 8, 16, 64, 128, 256]))
        top_k = int(rng.choice([1, 2, 4, 6, 8]))
        hidden = int(rng.choice([128, 256, 512, 1024, 2048, 4096]))
        inter = int(rng.choice([64, 96, 128, 256, 384, 768, 1536]))
        if top_k > e or e * inter * hidden > 1 << 27:
            continue
        pre = bool(rng.random() < 0.5) and hidden % 64 == 0 and inter % 64 == 0
        cases.append((m, e, top_k, hidden, inter, pre))
    return cases


@pytest.mark.parametrize("m,e,top_k,hidden,inter,pre", _moe_cases(),
                         ids=lambda v: str(v) if not isinstance(v, bool) else ("y" if v else "n"))
def test_moe_layer_shape_fuzz(m, e, top_k, hidden, inter, pre):
    seed = m * 131 + e * 17 + top_k * 5 + hidden + inter
    rng = np.random.default_rng(seed)
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter)
    x = rand_act(seed + 1, (m, hidden))
    g = torch.Generator().manual_seed(seed + 2)
    p = torch.softmax(torch.randn((m, e), generator=g), dim=-1)
    w, ids = torch.topk(p, k=top_k, dim=-1)
    w = (w / w.sum(-1, keepdim=True)).float()
    xd, wd, idd = cuda(x), cuda(w), cuda(ids)
    d13w, d13s, d2w, d2s = cuda(w13), cuda(s13), cuda(w2), cuda(s2)
    kw = {}
    if pre:
        kw = {"prepacked13": mx.prepack_w4a16(d13w, d13s), "prepacked2": mx.prepack_w4a16(d2w, d2s)}
    y = mx.moe_layer(xd, d13w, d13s, d2w, d2s, wd, idd, **kw)
    assert y.shape == (m, hidden) and y.dtype == torch.bfloat16
    d13, d2 = mx.dequant_mxfp4(d13w, d13s, torch.bfloat16), mx.dequant_mxfp4(d2w, d2s, torch.bfloat16)
    o32, routes = moe_layer_device(xd, d13, d2, wd, idd, "f32", return_routes=True)
    ref = moe_layer_device(xd, d13, d2, wd, idd, "ref")
    rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, min(m, 6), replace=False)]))
    oracle = O.moe_layer_fp64(x.float().numpy()[rows], w13, s13, w2, s2, w.numpy()[rows],
                              ids.numpy()[rows])
    pin = O.parity_errors(o32[torch.from_numpy(rows).cuda()].cpu().numpy(), oracle)
    assert pin["norm_rel"] <= 2e-4, pin
    assert_layer_blocks(y, o32, ref, routes, row_block=min(128, m),
                        what=f"moe layer m={m} e={e} top_k={top_k} {hidden}/{inter} pre={pre}")
