"""GPU parity at BASELINE.json's own configurations.

* Config 1: the dense W4A16 linear at its exact workload (M=64, K=2048,
  N=2048, seeded codes/scales/activations).
* Config 5's edge sweep through the routed decode kernels: every E2M1 code
  at E8M0 1 (subnormal weights) and 254 (+-inf weights) in the experts of
  the BASELINE MoE shape (E=128, top-8, H=2048, I=768; the down GEMM's K=768
  is not a multiple of a 256/512 tile), through ``moe_layer`` (w13 or w2
  carrying the edge codes) and ``fused_moe_mxfp4_soft``, at M in {1, 8, 32},
  route weights on and off.  A quarter of the experts carry the edge
  weights; the routing puts 8, 1, 0 or 2 of them in each token's top-8, so
  every output mixes ordinary and edge routes.  Where +-inf meets the data,
  the NaN / +-inf pattern is independent of summation order and is asserted
  exactly; everything finite is held to the parity bars.
* Whole outputs at the full sizes of configs 2-4 (linear M=4096, MoE layer
  M=512 / 4096 and its gate_up GEMM, W4A4 8192x4096x4096): every output
  row, in blocks finer than any kernel tile, against an FP32-accumulated GEMM
  of the exact dequantized operands on the device (itself pinned against
  the FP64 oracle on sampled rows), and no worse than the reference safe
  path run on the device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import mxfp4_oracle as O

from _helpers import (assert_layer_blocks, assert_layer_parity, assert_parity, assert_rows_parity,
                      cuda, fp32_gemm, moe_layer_device, rand_act, rand_mxfp4,
                      safe_linear_device)

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]

E, H, I, TOPK = 128, 2048, 768, 8
SPECIAL = np.arange(1, E, 4)  # the experts that carry the edge weights


# ---------------------------------------------------------------- config 1

def test_config1_dense_linear():
    # x bf16 [64, 2048] ~ N(0, 1); W u8 [2048, 1024], codes uniform 0..15;
    # S u8 [2048, 64] uniform 120..128; bf16 out, FP32 accumulation
    rng = np.random.default_rng(20260810)
    m, k, n = 64, 2048, 2048
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(20260810, (m, k))
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    ref = safe_linear_device(cuda(x), packed, scales)
    oracle = O.linear_fp64(x.float().numpy(), packed, scales)
    assert_parity(y, oracle, ref=ref, what="config 1")
    assert torch.equal(y, mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales)))


# ---------------------------------------------------------------- config 5 edge sweep

def _rolled(rows: int, k: int, scale: int):
    """Every E2M1 code in every row (rolled by the row index), one E8M0 byte."""
    codes = np.tile(np.arange(16, dtype=np.uint8), (rows, k // 16))
    for r in range(rows):
        codes[r] = np.roll(codes[r], r)
    return O.pack_codes(codes), np.full((rows, k // 32), scale, dtype=np.uint8)


def _single_inf(rng, rows: int, k: int):
    """Ordinary random rows, except that row n holds one +-inf: in 32-block
    n % (k/32), coded E8M0 254, every code is 0 but the one at position
    (7n) % 32, which is +-inf (codes 4-7 / 12-15)."""
    packed, scales = rand_mxfp4(rng, (rows,), k)
    codes = O.unpack_codes(packed)
    for n in range(rows):
        b0 = n % (k // 32)
        codes[n, b0 * 32:(b0 + 1) * 32] = 0
        codes[n, b0 * 32 + (7 * n) % 32] = (4, 5, 6, 7, 12, 13, 14, 15)[n % 8]
        scales[n, b0] = 254
    return O.pack_codes(codes), scales


@pytest.fixture(scope="module")
def edge_base():
    rng = np.random.default_rng(20260850)
    w13, s13 = rand_mxfp4(rng, (E, 2 * I), H)
    w2, s2 = rand_mxfp4(rng, (E, H), I)
    return {"w13": w13, "s13": s13, "w2": w2, "s2": s2, "v13": {}, "v2": {}}


def _values(base, name, special=None):
    """e -> dequantized expert e (the oracle's values), cached for the
    ordinary experts; the edge experts' values come from ``special``
    (an array, or a dict expert -> array)."""
    cache = base["v" + name[1:]]
    packed, scales = base[name], base["s" + name[1:]]

    def get(e):
        if special is not None and e % 4 == 1:
            return special[e] if isinstance(special, dict) else special
        v = cache.get(e)
        if v is None:
            v = cache[e] = O.dequant_values(packed[e], scales[e], "bf16").astype(np.float32)
        return v
    return get


def _edge_routing(m: int, seed: int, route_weights: bool):
    """top-8 ids with 8, 1, 0, 2, 8, 1, ... edge experts per token (in
    shuffled slots) and positive weights summing to 1 (or all ones)."""
    rng = np.random.default_rng(seed)
    normal = np.setdiff1d(np.arange(E), SPECIAL)
    nsp = np.array([(8, 1, 0, 2)[t % 4] for t in range(m)])
    ids = np.empty((m, TOPK), dtype=np.int64)
    for t in range(m):
        row = np.concatenate([rng.choice(SPECIAL, nsp[t], replace=False),
                              rng.choice(normal, TOPK - nsp[t], replace=False)])
        rng.shuffle(row)
        ids[t] = row
    if route_weights:
        w = rng.random((m, TOPK)) + 0.05
        w = w / w.sum(1, keepdims=True)
    else:
        w = np.ones((m, TOPK))
    return w.astype(np.float32), ids, nsp


def _dequant_experts(w, s, dt=torch.bfloat16):
    """All experts dequantized on the device by the bit-exact dequant kernel
    (pinned against the oracle over every code x scale in test_gpu_dequant_linear)."""
    return mx.dequant_mxfp4(cuda(w), cuda(s), dt)


@pytest.mark.parametrize("route_weights", [True, False], ids=["rw_on", "rw_off"])
@pytest.mark.parametrize("scale", [1, 254])
@pytest.mark.parametrize("which", ["w13", "w2"])
@pytest.mark.parametrize("m", [1, 8, 32])
def test_config5_layer_edge_sweep(m, which, scale, route_weights, edge_base):
    b = edge_base
    w13, s13, w2, s2 = b["w13"], b["s13"], b["w2"], b["s2"]
    rows, k = (2 * I, H) if which == "w13" else (H, I)
    sp, ss = _rolled(rows, k, scale)
    spv = O.dequant_values(sp, ss, "bf16").astype(np.float32)
    if which == "w13":
        w13, s13 = w13.copy(), s13.copy()
        w13[SPECIAL], s13[SPECIAL] = sp, ss
        v13, v2 = _values(b, "w13", spv), _values(b, "w2")
    else:
        w2, s2 = w2.copy(), s2.copy()
        w2[SPECIAL], s2[SPECIAL] = sp, ss
        v13, v2 = _values(b, "w13"), _values(b, "w2", spv)
    x = rand_act(20260851 + m, (m, H))
    w, ids, nsp = _edge_routing(m, 20260852 + m, route_weights)
    xd, wd, idd = cuda(x), cuda(w), cuda(ids)
    y = mx.moe_layer(xd, cuda(w13), cuda(s13), cuda(w2), cuda(s2), wd, idd)
    ref = moe_layer_device(xd, _dequant_experts(w13, s13), _dequant_experts(w2, s2), wd, idd,
                           "ref")
    yn = y.float().cpu().numpy()
    oracle, routes = O.moe_layer_fp64(x.float().numpy(), w13, s13, w2, s2, w, ids,
                                      w13_values=v13, w2_values=v2, return_routes=True)
    what = f"layer edge m={m} {which} s={scale} rw={route_weights}"
    if scale == 254:
        # every edge row holds +inf and -inf weights: each route through an
        # edge expert is NaN, and so is its token's top-k sum
        assert np.array_equal(np.isnan(yn), np.isnan(oracle)), what
        assert np.all(np.isnan(yn[nsp > 0])) and not np.isnan(yn[nsp == 0]).any(), what
        groups = [nsp == 0]
    else:
        assert np.all(np.isfinite(yn)), what
        # tokens routed only to subnormal-weight experts are checked on their own scale
        groups = [nsp == 8, nsp < 8]
    for g in groups:
        if g.any():
            assert_layer_parity(yn[g], oracle[g], ref.float().cpu().numpy()[g], what=what,
                                routes=routes[g])


def _fused_ref(a, bd, w, ids, mul_routed_weight):
    """soft:476-494 on the device with unit scales: per expert, the GEMM in
    the compute dtype rounded to it, the route weight applied in FP32, rounded."""
    m, top_k = ids.shape
    out = torch.zeros((m, top_k, bd.shape[1]), dtype=a.dtype, device=a.device)
    for e in torch.unique(ids).tolist():
        t, s = (ids == e).nonzero(as_tuple=True)
        v = torch.matmul(a[t], bd[e].T)
        if mul_routed_weight:
            v = v * w[t, s, None]
        out[t, s] = v.to(a.dtype)
    return out


def _fused_call(a, wp, ws, w, ids, mul_routed_weight):
    m = a.shape[0]
    C = torch.empty((m, TOPK, wp.shape[1]), dtype=torch.bfloat16, device="cuda")
    e = torch.empty(0, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.ones(1, device="cuda"),
                            torch.ones(wp.shape[0], device="cuda"), None, cuda(ws), cuda(w),
                            cuda(ids), e, e, e, mul_routed_weight, TOPK, False, False)
    return C


@pytest.mark.parametrize("mul_routed_weight", [True, False], ids=["rw_on", "rw_off"])
@pytest.mark.parametrize("scale", [1, 254])
@pytest.mark.parametrize("shape", ["gate_up", "down"])
@pytest.mark.parametrize("m", [1, 8, 32])
def test_config5_fused_moe_edge_sweep(m, shape, scale, mul_routed_weight, edge_base):
    b = edge_base
    name = "w13" if shape == "gate_up" else "w2"
    wp, ws = b[name].copy(), b["s" + name[1:]].copy()
    rows, k = wp.shape[1], wp.shape[2] * 2
    sp, ss = _rolled(rows, k, scale)
    wp[SPECIAL], ws[SPECIAL] = sp, ss
    vals = _values(b, name, O.dequant_values(sp, ss, "bf16").astype(np.float32))
    a = rand_act(20260853 + m, (m, k))
    w, ids, nsp = _edge_routing(m, 20260854 + m, True)
    C = _fused_call(a, wp, ws, w, ids, mul_routed_weight)
    ref = _fused_ref(cuda(a), _dequant_experts(wp, ws), cuda(w), cuda(ids), mul_routed_weight)
    Cn, refn = C.float().cpu().numpy(), ref.float().cpu().numpy()
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 1.0, np.ones(E), w, ids,
                              mul_routed_weight, b_values=vals)
    edge = np.isin(ids, SPECIAL)
    what = f"fused edge m={m} {shape} s={scale} rw={mul_routed_weight}"
    if scale == 254:
        assert np.array_equal(np.isnan(Cn), np.isnan(oracle)), what
        assert np.all(np.isnan(Cn[edge])) and not np.isnan(Cn[~edge]).any(), what
        groups = [~edge]
    else:
        assert np.all(np.isfinite(Cn)), what
        groups = [edge, ~edge]
    for g in groups:
        if g.any():
            assert_parity(Cn[g], oracle[g], ref=refn[g], what=what, fmt="bf16")


@pytest.mark.parametrize("m", [8, 32])
def test_config5_single_inf_weights_exact(m, edge_base):
    # one +-inf per edge-expert row, zeros in its block: every edge route's
    # output is sign(x at that K position) * sign(code) * inf, exactly --
    # which pins the nibble order, the K offset of every 32-block and the
    # row of every route through the routed decode GEMM
    b = edge_base
    rng = np.random.default_rng(20260855)
    wp, ws = b["w13"].copy(), b["s13"].copy()
    sp, ss = _single_inf(rng, 2 * I, H)
    wp[SPECIAL], ws[SPECIAL] = sp, ss
    vals = _values(b, "w13", O.dequant_values(sp, ss, "bf16").astype(np.float32))
    a = rand_act(20260856 + m, (m, H))
    w, ids, nsp = _edge_routing(m, 20260857 + m, True)
    C = _fused_call(a, wp, ws, w, ids, True).float().cpu().numpy()
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 1.0, np.ones(E), w, ids, True,
                              b_values=vals)
    edge = np.isin(ids, SPECIAL)
    assert np.all(np.isinf(oracle[edge]) | np.isnan(oracle[edge]))
    assert np.isinf(oracle[edge]).mean() > 0.99
    np.testing.assert_array_equal(C[edge], oracle[edge])  # NaN where NaN, same infinities
    assert_parity(C[~edge], oracle[~edge], what=f"single-inf m={m} ordinary routes")


@pytest.mark.parametrize("m", [8, 32])
def test_config5_layer_infinite_gates(m, edge_base):
    # the fused SiLU*mul epilogue on infinite gates: one gate row per edge
    # expert holds a single +-inf weight, so that gate is +inf or -inf;
    # silu(+inf) * u = +-inf, silu(-inf) = NaN (torch's F.silu, vllm:249-252),
    # and the down GEMM and top-k sum spread them into an exact NaN / +-inf
    # pattern per output column
    b = edge_base
    rng = np.random.default_rng(20260858)
    w13, s13 = b["w13"].copy(), b["s13"].copy()
    special = {}
    gp, gs = _single_inf(rng, 8, H)
    for e in SPECIAL:
        row = (int(e) * 37) % I
        w13[e, row], s13[e, row] = gp[int(e) % 8], gs[int(e) % 8]
        special[int(e)] = O.dequant_values(w13[e], s13[e], "bf16").astype(np.float32)
    v13, v2 = _values(b, "w13", special), _values(b, "w2")
    x = rand_act(20260859 + m, (m, H))
    w, ids, nsp = _edge_routing(m, 20260860 + m, True)
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(b["w2"]), cuda(b["s2"]), cuda(w),
                     cuda(ids)).float().cpu().numpy()
    oracle, routes = O.moe_layer_fp64(x.float().numpy(), w13, s13, b["w2"], b["s2"], w, ids,
                                      w13_values=v13, w2_values=v2, return_routes=True)
    assert np.isnan(oracle).any() and np.isinf(oracle).any()
    np.testing.assert_array_equal(np.isnan(y), np.isnan(oracle))
    inf = np.isinf(oracle)
    np.testing.assert_array_equal(y[inf], oracle[inf])
    fin = nsp == 0
    ref = moe_layer_device(cuda(x), _dequant_experts(w13, s13), _dequant_experts(b["w2"], b["s2"]),
                           cuda(w), cuda(ids), "ref").float().cpu().numpy()
    assert_layer_parity(y[fin], oracle[fin], ref[fin], what=f"infinite gates m={m}",
                        routes=routes[fin])


# ---------------------------------------------------------------- whole outputs at full size

def _pin_f32(ref32: torch.Tensor, rows: np.ndarray, oracle: np.ndarray):
    """The FP32 device GEMM agrees with the FP64 oracle on sampled rows
    (to far below the bf16 rounding the parity bars measure)."""
    e = O.parity_errors(ref32[torch.from_numpy(rows).cuda()].double().cpu().numpy(), oracle)
    assert e["norm_rel"] <= 1e-5 and e["elem_rel"] <= 1e-3, e


@pytest.mark.parametrize("k,n", [(2048, 5120), (4096, 2048)], ids=["qkv", "o_proj"])
def test_linear_whole_output_m4096(k, n):
    m = 4096
    rng = np.random.default_rng(20260810 + m + k)
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(20260810 + m, (m, k))
    xd = cuda(x)
    y = mx.linear_mxfp4_soft(xd, cuda(packed), cuda(scales))
    from _helpers import dequant_device
    wd = dequant_device(packed, scales)
    ref16 = torch.matmul(xd, wd.T)
    ref32 = fp32_gemm(xd, wd)
    rows = np.sort(rng.choice(m, 24, replace=False))
    _pin_f32(ref32, rows, O.linear_fp64(x.float().numpy()[rows], packed, scales))
    assert_rows_parity(y, ref32, ref16, what=f"linear m={m} k={k} n={n}", row_block=16)


@pytest.fixture(scope="module")
def layer_weights_full():
    rng = np.random.default_rng(20260815)
    w13, s13 = rand_mxfp4(rng, (E, 2 * I), H)
    w2, s2 = rand_mxfp4(rng, (E, H), I)
    return w13, s13, w2, s2


def _route(m, seed):
    g = torch.Generator().manual_seed(seed)
    p = torch.softmax(torch.randn((m, E), generator=g), dim=-1)
    w, ids = torch.topk(p, k=TOPK, dim=-1)
    return (w / w.sum(-1, keepdim=True)).float(), ids


@pytest.mark.parametrize("m", [512, 4096])
def test_moe_layer_whole_output(m, layer_weights_full):
    w13, s13, w2, s2 = layer_weights_full
    x = rand_act(20260816 + m, (m, H))
    w, ids = _route(m, 20260817 + m)
    xd, wd, idd = cuda(x), cuda(w), cuda(ids)
    y = mx.moe_layer(xd, cuda(w13), cuda(s13), cuda(w2), cuda(s2), wd, idd)
    d13, d2 = _dequant_experts(w13, s13), _dequant_experts(w2, s2)
    o32, routes = moe_layer_device(xd, d13, d2, wd, idd, "f32", return_routes=True)
    ref = moe_layer_device(xd, d13, d2, wd, idd, "ref")
    rows = np.sort(np.random.default_rng(m).choice(m, 16, replace=False))
    oracle = O.moe_layer_fp64(x.float().numpy()[rows], w13, s13, w2, s2, w.numpy()[rows],
                              ids.numpy()[rows])
    # the FP32 composition against the FP64 oracle on sampled tokens: both
    # round at the reference's points, so they differ only where an FP32
    # sum lands on the other side of a bf16 rounding boundary
    e = O.parity_errors(o32[torch.from_numpy(rows).cuda()].cpu().numpy(), oracle)
    assert e["norm_rel"] <= 2e-4, e
    assert_layer_blocks(y, o32, ref, routes, what=f"moe layer m={m}")


@pytest.mark.parametrize("m,top_k", [(2000, 4), (300, 8)])
def test_moe_layer_skewed_routing_whole_output(m, top_k):
    # skewed routing over 16 experts (several with no route, some with a
    # handful): experts padded to half a tile, odd halves run as
    # half-height tiles, ids int32
    e, hidden, inter = 16, 512, 256
    rng = np.random.default_rng(m + top_k)
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter)
    pr = np.array([40, 10, 8, 6, 5, 4, 3, 2, 1, 1, 0.5, 0.2, 0.05, 0, 0, 0], dtype=np.float64)
    ids = np.stack([rng.choice(e, size=top_k, replace=False, p=pr / pr.sum())
                    for _ in range(m)]).astype(np.int32)
    w = rng.uniform(0.05, 1.0, size=(m, top_k)).astype(np.float32)
    x = rand_act(m, (m, hidden))
    xd, wd, idd = cuda(x), cuda(w), cuda(ids)
    y = mx.moe_layer(xd, cuda(w13), cuda(s13), cuda(w2), cuda(s2), wd, idd)
    d13, d2 = _dequant_experts(w13, s13), _dequant_experts(w2, s2)
    o32, routes = moe_layer_device(xd, d13, d2, wd, idd, "f32", return_routes=True)
    ref = moe_layer_device(xd, d13, d2, wd, idd, "ref")
    assert_layer_blocks(y, o32, ref, routes, what=f"skewed moe layer m={m} top_k={top_k}",
                         row_block=100)


def test_fused_moe_whole_output_m4096(layer_weights_full):
    # the gate_up GEMM of the MoE layer at 4096 tokens (32768 routes over
    # 128-row expert blocks: the persistent routed kernel), every route row
    w13, s13, _, _ = layer_weights_full
    m = 4096
    a = rand_act(20260870, (m, H))
    w, ids = _route(m, 20260871)
    ad = cuda(a)
    C = torch.empty((m, TOPK, 2 * I), dtype=torch.bfloat16, device="cuda")
    e = torch.empty(0, device="cuda")
    mx.fused_moe_mxfp4_soft(ad, cuda(w13), C, torch.ones(1, device="cuda"),
                            torch.ones(E, device="cuda"), None, cuda(s13), cuda(w), cuda(ids),
                            e, e, e, True, TOPK, False, False)
    d13 = _dequant_experts(w13, s13)
    ref = _fused_ref(ad, d13, cuda(w), cuda(ids), True)
    o32 = torch.empty((m, TOPK, 2 * I), dtype=torch.float64, device="cuda")
    idd, wd = cuda(ids), cuda(w)
    for ex in torch.unique(idd).tolist():
        t, s = (idd == ex).nonzero(as_tuple=True)
        o32[t, s] = (fp32_gemm(ad[t], d13[ex]) * wd[t, s, None]).double()
    rows = np.arange(0, m, 512)
    oracle = O.fused_moe_fp64(a.float().numpy()[rows], w13, s13, 1.0, np.ones(E),
                              w.numpy()[rows], ids.numpy()[rows], True)
    eo = O.parity_errors(o32[torch.from_numpy(rows).cuda()].cpu().numpy(), oracle)
    assert eo["norm_rel"] <= 1e-5, eo
    assert_rows_parity(C.reshape(m * TOPK, -1), o32.reshape(m * TOPK, -1),
                       ref.reshape(m * TOPK, -1), what="fused moe m=4096", row_block=16)


def test_w4a4_whole_output():
    # M=8192, K=4096, N=4096, both operands RNE-quantized
    m, k, n = 8192, 4096, 4096
    ad = cuda(rand_act(4, (m, k)))
    wd = cuda(rand_act(5, (n, k)).float() * 0.02)
    ap, asc = mx.dynamic_mxfp4_quant(ad, "rne")
    wp, wsc = mx.dynamic_mxfp4_quant(wd, "rne")
    y = mx.linear_mxfp4_w4a4(ap, asc, wp, wsc)
    # exact operand values (E2M1 x 2^e is exact in bf16 at these scales)
    a_bf = mx.dequant_mxfp4(ap, asc, torch.bfloat16)
    w_bf = mx.dequant_mxfp4(wp, wsc, torch.bfloat16)
    assert torch.equal(a_bf.float(), mx.dequant_mxfp4(ap, asc, torch.float32))
    ref32 = fp32_gemm(a_bf, w_bf)
    ref16 = torch.matmul(a_bf, w_bf.T)  # the safe path: dequant, bf16 GEMM (soft:468-490)
    rows = np.sort(np.random.default_rng(6).choice(m, 16, replace=False))
    apn, ascn = ap.cpu().numpy()[rows], asc.cpu().numpy()[rows]
    oracle = O.dequant_values(apn, ascn, "f32") @ O.dequant_values(
        wp.cpu().numpy(), wsc.cpu().numpy(), "f32").T
    _pin_f32(ref32, rows, oracle)
    assert_rows_parity(y, ref32, ref16, what="w4a4 8192x4096x4096", row_block=16)
