"""GPU parity over randomized shapes (fixed seeds): the dense W4A16 linear
(soft:310-376), the MoE layer (vllm:233-265), the W4A4 linear (aiter:329-338)
and the soft fused operator (soft:379-494) at shapes the targeted tests do
not pin -- odd M and N, K from 32 to 8192, bias, fp16 / fp32 compute,
packed activations, prepacked weights, 2 to 256 experts, top-1 to top-8 --
so the tile configurations, split-K plans, decode kernels and routing paths
the dispatch picks all meet the same bar.  Whole outputs are held to FP32-accumulated device GEMMs of
the exact operands (themselves pinned against the FP64 oracle on sampled
rows) and must be no worse than the reference safe path on the same inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import mxfp4_oracle as O

from _helpers import (assert_layer_blocks, assert_parity, assert_rows_parity, cuda, dequant_device,
                      fp32_gemm, moe_layer_device, rand_act, rand_mxfp4, safe_linear_device)

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


def _w4a4_cases(count=12):
    rng = np.random.default_rng(20261204)
    cases = []
    while len(cases) < count:
        m = int(rng.choice([1, 2, 7, 16, 33, 100, 255, 256, 700, 1000, 2100, 3000]))
        k = int(rng.choice([32, 64, 96, 128, 160, 256, 384, 1024, 2080, 4096]))
        n = int(rng.choice([16, 48, 64, 100, 256, 300, 512, 1024, 2048, 4100]))
        if m * k > 1 << 23 or n * k > 1 << 23:
            continue
        cases.append((m, k, n, str(rng.choice(["bf16", "f16", "f32"]))))
    return cases


@pytest.mark.parametrize("m,k,n,out", _w4a4_cases(), ids=str)
def test_w4a4_linear_shape_fuzz(m, k, n, out):
    # packed activations x packed weights (aiter:329-338): every product of
    # two E2M1 values and their scales is exact, so an FP32 GEMM of the
    # exactly dequantized operands is the whole-output oracle
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[out]
    a = rand_act(m + 3 * k, (m, k)).float().numpy()
    w = (rand_act(n + 5 * k, (n, k)).float() * 0.02).numpy()
    ap, asc = O.quant_mxfp4_rne(a)
    wp, wsc = O.quant_mxfp4_rne(w)
    y = mx.linear_mxfp4_w4a4(cuda(ap), cuda(asc), cuda(wp), cuda(wsc), tdt)
    assert y.shape == (m, n) and y.dtype == tdt
    o32 = fp32_gemm(dequant_device(ap, asc, "f32"), dequant_device(wp, wsc, "f32"))
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).choice(m, min(m, 4), False)]))
    o64 = O.dequant_values(ap[rows], asc[rows], "f32") @ O.dequant_values(wp, wsc, "f32").T
    pin = O.parity_errors(o32[torch.from_numpy(rows).cuda()].cpu().numpy(), o64)
    assert pin["norm_rel"] <= 1e-5, pin
    assert_rows_parity(y, o32, what=f"w4a4 {m}x{k}x{n} {out}", row_block=max(1, 4096 // n),
                       fmt=None if out == "f32" else tdt)


def _fused_cases(count=12):
    rng = np.random.default_rng(20261205)
    cases = []
    while len(cases) < count:
        m = int(rng.choice([1, 3, 8, 20, 64, 150, 400, 600]))
        e = int(rng.choice([2, 5, 16, 64]))
        top_k = int(rng.choice([1, 2, 3, 8]))
        k = int(rng.choice([128, 256, 768, 1024, 2048]))
        n = int(rng.choice([32, 96, 200, 512, 1024]))
        c = str(rng.choice(["bf16", "f16", "f32"]))
        a = str(rng.choice(["act", "act", "packed"]))
        if top_k > e or e * n * k > 1 << 26 or (a == "packed" and c == "f16"):
            continue
        cases.append((m, e, top_k, k, n, c, a, bool(rng.random() < 0.5)))
    return cases


@pytest.mark.parametrize("m,e,top_k,k,n,c,a,routed", _fused_cases(),
                         ids=lambda v: str(v) if not isinstance(v, bool) else ("rw" if v else "norw"))
def test_fused_moe_shape_fuzz(m, e, top_k, k, n, c, a, routed):
    # the soft operator (soft:379-494) over random shapes, compute dtypes
    # (C in bf16 / fp16 / fp32: the FP32-MFMA path), packed or unpacked
    # activations, A_scale / B_scale and route weights on or off
    seed = m * 7 + e * 11 + top_k * 13 + k + n
    rng = np.random.default_rng(seed)
    lo, hi = (116, 121) if c == "f16" else (120, 128)
    wp, ws = rand_mxfp4(rng, (e, n), k, lo=lo, hi=hi)
    cdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[c]
    g = torch.Generator().manual_seed(seed)
    tw, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
    b_scale = rng.uniform(0.5, 2.0, size=e).astype(np.float32)
    if a == "packed":
        ap, asc = O.quant_mxfp4_ties_away(rand_act(seed + 1, (m, k)).float().numpy())
        A, A_mx = cuda(ap), cuda(asc)
        a_vals = O.dequant_values(ap, asc, c)
    else:
        x = rand_act(seed + 1, (m, k), torch.float16 if c == "f16" else torch.bfloat16)
        A, A_mx = cuda(x), None
        a_vals = x.float().numpy()
    C = torch.full((m, top_k, n), 7.0, dtype=cdt, device="cuda")  # zero-filled by the op
    mx.fused_moe_mxfp4_soft(A, cuda(wp), C, torch.full((1,), 0.75, device="cuda"),
                            cuda(torch.from_numpy(b_scale)), A_mx, cuda(ws), cuda(tw), cuda(ids),
                            torch.empty(0, device="cuda"), torch.empty(0, device="cuda"),
                            torch.empty(0, device="cuda"), routed, top_k, False, False)
    oracle = O.fused_moe_fp64(a_vals, wp, ws, 0.75, b_scale, tw.numpy(), ids.numpy(), routed,
                              compute_dtype=c)
    assert_parity(C, oracle, fmt=None if c == "f32" else c,
                  what=f"fused moe m={m} e={e} top_k={top_k} {k}x{n} C={c} A={a} rw={routed}")
