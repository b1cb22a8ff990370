"""GPU parity: routed MoE (soft op, AITER entry, device routing, the vLLM MoE
layer) against the FP64 oracle, the reference's per-(token, slot) GEMV loop
(test:270-285) and the reference safe path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import c_oracle, mxfp4_oracle as O

from _helpers import assert_layer_parity, assert_parity, cuda, rand_act, rand_mxfp4

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]


def _route(m, num_experts, top_k, seed):
    """softmax -> top-k -> renormalize of seeded router logits."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn((m, num_experts), generator=g)
    p = torch.softmax(logits, dim=-1)
    w, ids = torch.topk(p, k=top_k, dim=-1)
    return (w / w.sum(-1, keepdim=True)).float(), ids


def _empty():
    return torch.empty(0, device="cuda")


# ---------------------------------------------------------------- soft op

@pytest.mark.parametrize("m_value", [1, 2, 4, 8, 64])
@pytest.mark.parametrize("quantize_activations", [False, True])
@pytest.mark.parametrize("mul_routed_weight", [False, True])
def test_fused_moe_matrix(m_value, quantize_activations, mul_routed_weight):
    # test:216-285 (the 20-case operator matrix) on the HIP backend
    torch.manual_seed(20260810 + m_value)
    n_value, k_value, experts, top_k = 64, 128, 4, 2
    activations = torch.randn((m_value, k_value), dtype=torch.bfloat16)
    weights = torch.randn((experts, n_value, k_value), dtype=torch.bfloat16)
    wp, ws = O.quant_mxfp4_ties_away(weights.float().numpy())
    if quantize_activations:
        ap, asc = O.quant_mxfp4_ties_away(activations.float().numpy())
        kernel_a, kernel_amx = cuda(ap), cuda(asc)
        ref_a = O.dequant_values(ap, asc, "bf16")
    else:
        kernel_a, kernel_amx = cuda(activations), None
        ref_a = activations.float().numpy().astype(np.float64)
    logits = torch.randn((m_value, experts), dtype=torch.float32)
    topk_weights, topk_ids = torch.topk(torch.softmax(logits, dim=-1), k=top_k, dim=-1)
    actual = torch.empty((m_value, top_k, n_value), device="cuda", dtype=torch.bfloat16)
    scalar_a = torch.tensor([0.75], device="cuda")
    scalar_b = torch.linspace(0.5, 1.25, experts, device="cuda")
    mx.fused_moe_mxfp4_soft(kernel_a, cuda(wp), actual, scalar_a, scalar_b, kernel_amx, cuda(ws),
                            cuda(topk_weights), cuda(topk_ids), _empty(), _empty(), _empty(),
                            mul_routed_weight, top_k, False, False)
    # the reference's own GEMV loop (test:270-281), on the device
    dq = torch.from_numpy(O.dequant_bits(wp, ws, "bf16").view(np.int16)).view(torch.bfloat16).cuda()
    ra = torch.from_numpy(ref_a.astype(np.float32)).to(torch.bfloat16).cuda()
    expected = torch.empty_like(actual)
    for t in range(m_value):
        for s in range(top_k):
            e = int(topk_ids[t, s])
            v = torch.matmul(ra[t], dq[e].transpose(0, 1)) * scalar_a[0] * scalar_b[e]
            if mul_routed_weight:
                v = v * topk_weights[t, s].cuda()
            expected[t, s] = v.to(expected.dtype)
    # The loop rounds to bf16 after the matmul and after each scalar multiply
    # (up to four roundings, test:274-281); the HIP epilogue applies the
    # scales to the FP32 accumulator and rounds once, so the two may differ
    # by a few bf16 steps (at most 4, as the next test derives; on these
    # seeds within 2e-2).  The strict bar is the FP64 parity below, where
    # ours must also be no worse than the loop.
    torch.testing.assert_close(actual, expected, rtol=2e-2, atol=2e-2)
    oracle = O.fused_moe_fp64(ref_a, wp, ws, 0.75, scalar_b.cpu().numpy(), topk_weights.numpy(),
                              topk_ids.numpy(), mul_routed_weight)
    assert_parity(actual, oracle, ref=expected)


def _bf16_ulp_distance(a, b):
    """Distance of two bf16 tensors in units in the last place (the bit
    patterns mapped to ordered integers; +0 and -0 coincide)."""
    def ordered(t):
        i = t.view(torch.int16).int()
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (ordered(a) - ordered(b)).abs()


@pytest.mark.parametrize("m_value", [1, 2, 4, 8, 64])
@pytest.mark.parametrize("quantize_activations", [False, True])
@pytest.mark.parametrize("mul_routed_weight", [False, True])
def test_fused_moe_matrix_reference_rounding(m_value, quantize_activations, mul_routed_weight,
                                             monkeypatch):
    # MXFP4_GFX950_ROUNDING=reference: the safe path's rounding sequence
    # (soft:487-494), which the per-(token, slot) loop shares but for its
    # GEMV's summation order -- so the reference's own bar (test:283-285,
    # rtol=atol=1e-2) holds on the test's own inputs, and results sit within
    # one bf16 step of the loop's (a sum on the other side of a rounding
    # boundary) carried through the scalar multiplies
    monkeypatch.setenv("MXFP4_GFX950_ROUNDING", "reference")
    torch.manual_seed(20260810 + m_value)
    n_value, k_value, experts, top_k = 64, 128, 4, 2
    activations = torch.randn((m_value, k_value), device="cuda", dtype=torch.bfloat16)
    weights = torch.randn((experts, n_value, k_value), device="cuda", dtype=torch.bfloat16)
    wp, ws = (cuda(t) for t in O.quant_mxfp4_ties_away(weights.float().cpu().numpy()))
    dq = mx.dequant_mxfp4(wp, ws, torch.bfloat16)
    if quantize_activations:
        ap, asc = O.quant_mxfp4_ties_away(activations.float().cpu().numpy())
        kernel_a, kernel_amx = cuda(ap), cuda(asc)
        ref_a = mx.dequant_mxfp4(kernel_a, kernel_amx, torch.bfloat16)
    else:
        kernel_a, kernel_amx, ref_a = activations, None, activations
    logits = torch.randn((m_value, experts), device="cuda", dtype=torch.float32)
    topk_weights, topk_ids = torch.topk(torch.softmax(logits, dim=-1), k=top_k, dim=-1)
    actual = torch.empty((m_value, top_k, n_value), device="cuda", dtype=torch.bfloat16)
    scalar_a = torch.tensor([0.75], device="cuda", dtype=torch.float32)
    scalar_b = torch.linspace(0.5, 1.25, experts, device="cuda")
    mx.fused_moe_mxfp4_soft(kernel_a, wp, actual, scalar_a, scalar_b, kernel_amx, ws,
                            topk_weights, topk_ids, _empty(), _empty(), _empty(),
                            mul_routed_weight, top_k, False, False)
    expected = torch.empty_like(actual)
    for t in range(m_value):
        for s in range(top_k):
            e = int(topk_ids[t, s])
            v = torch.matmul(ref_a[t], dq[e].transpose(0, 1)) * scalar_a[0] * scalar_b[e]
            if mul_routed_weight:
                v = v * topk_weights[t, s]
            expected[t, s] = v.to(expected.dtype)
    torch.testing.assert_close(actual, expected, rtol=1e-2, atol=1e-2)
    assert int(_bf16_ulp_distance(actual, expected).max()) <= 2


@pytest.mark.parametrize("m_value", [1, 2, 4, 8, 64])
@pytest.mark.parametrize("quantize_activations", [False, True])
@pytest.mark.parametrize("mul_routed_weight", [False, True])
def test_fused_moe_matrix_reference_inputs(m_value, quantize_activations, mul_routed_weight):
    # The operator matrix on the very inputs the reference's test draws
    # (test:219-243: torch.manual_seed(20260810 + m), then randn on the
    # device for activations, weights and router logits, in that order),
    # weights and activations quantized by the reference's quantizer
    # (test:28-60, restated by the oracle) and the dequantized operands made
    # by this backend's dequant.  The per-(token, slot) loop (test:270-281)
    # rounds to bf16 after the GEMV and after each scalar multiply; this
    # backend, like the reference's own Triton kernel (soft:167-173), scales
    # the FP32 accumulator and rounds once.  A rounding of the loop errs by at
    # most half the bf16 step of the value v it rounds, a step within (v/256,
    # v/128]; the later multiplies scale value and error by f, so the carried
    # error stays below one step of the final value.  Three such roundings,
    # the loop's last half step and this backend's half step put the two
    # results at most 4 bf16 steps apart; the FP64 oracle then decides which
    # is closer.
    torch.manual_seed(20260810 + m_value)
    n_value, k_value, experts, top_k = 64, 128, 4, 2
    activations = torch.randn((m_value, k_value), device="cuda", dtype=torch.bfloat16)
    weights = torch.randn((experts, n_value, k_value), device="cuda", dtype=torch.bfloat16)
    wp, ws = (cuda(t) for t in O.quant_mxfp4_ties_away(weights.float().cpu().numpy()))
    dq = mx.dequant_mxfp4(wp, ws, torch.bfloat16)
    if quantize_activations:
        ap, asc = O.quant_mxfp4_ties_away(activations.float().cpu().numpy())
        kernel_a, kernel_amx = cuda(ap), cuda(asc)
        ref_a = mx.dequant_mxfp4(kernel_a, kernel_amx, torch.bfloat16)
    else:
        kernel_a, kernel_amx, ref_a = activations, None, activations
    logits = torch.randn((m_value, experts), device="cuda", dtype=torch.float32)
    topk_weights, topk_ids = torch.topk(torch.softmax(logits, dim=-1), k=top_k, dim=-1)
    actual = torch.empty((m_value, top_k, n_value), device="cuda", dtype=torch.bfloat16)
    scalar_a = torch.tensor([0.75], device="cuda", dtype=torch.float32)
    scalar_b = torch.linspace(0.5, 1.25, experts, device="cuda")
    mx.fused_moe_mxfp4_soft(kernel_a, wp, actual, scalar_a, scalar_b, kernel_amx, ws,
                            topk_weights, topk_ids, _empty(), _empty(), _empty(),
                            mul_routed_weight, top_k, False, False)
    expected = torch.empty_like(actual)
    for t in range(m_value):
        for s in range(top_k):
            e = int(topk_ids[t, s])
            v = torch.matmul(ref_a[t], dq[e].transpose(0, 1)) * scalar_a[0] * scalar_b[e]
            if mul_routed_weight:
                v = v * topk_weights[t, s]
            expected[t, s] = v.to(expected.dtype)
    dist = _bf16_ulp_distance(actual, expected)
    assert int(dist.max()) <= 4, f"{int(dist.max())} bf16 steps from the reference loop"
    oracle = O.fused_moe_fp64(ref_a.float().cpu().numpy().astype(np.float64), wp.cpu().numpy(),
                              ws.cpu().numpy(), 0.75, scalar_b.cpu().numpy(),
                              topk_weights.cpu().numpy(), topk_ids.cpu().numpy(),
                              mul_routed_weight)
    assert_parity(actual, oracle, ref=expected)


@pytest.mark.parametrize("c_dtype", [torch.float16, torch.float32])
def test_fused_moe_compute_dtypes(c_dtype):
    rng = np.random.default_rng(41)
    m, k, n, e, top_k = 24, 256, 80, 6, 3
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(41, (m, k))  # bf16 activations converted to C.dtype (soft:475)
    w, ids = _route(m, e, top_k, 42)
    C = torch.empty((m, top_k, n), dtype=c_dtype, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.ones(1, device="cuda"),
                            torch.ones(e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                            _empty(), _empty(), _empty(), True, top_k, False, False)
    dt = "f16" if c_dtype == torch.float16 else "f32"
    oracle = O.fused_moe_fp64(O.round_to_dtype(a.float().numpy(), dt), wp, ws, 1.0, np.ones(e),
                              w.numpy(), ids.numpy(), True, compute_dtype=dt)
    assert_parity(C, oracle, what=str(c_dtype))


@pytest.mark.parametrize("a_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale_range", [(116, 130), (1, 3)])
def test_fused_moe_fp32_compute_tiled(a_dtype, scale_range):
    # C in FP32 (soft:405-407): the FP32-MFMA tiled path over several tile
    # rows (block_m 64 at 1200 routes over 16 experts), column tiles with a
    # ragged tail (N = 200), a_scale / b_scale and route weights; scale
    # bytes 1-3 make every weight an FP32 subnormal or near it (the MFMA
    # must keep them)
    rng = np.random.default_rng(51 + scale_range[0])
    m, k, n, e, top_k = 300, 1024, 200, 16, 4
    wp, ws = rand_mxfp4(rng, (e, n), k, lo=scale_range[0], hi=scale_range[1])
    a = rand_act(52, (m, k)).to(a_dtype)
    w, ids = _route(m, e, top_k, 53)
    b_scale = torch.from_numpy(rng.uniform(0.5, 2.0, size=e).astype(np.float32))
    C = torch.empty((m, top_k, n), dtype=torch.float32, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.full((1,), 0.75, device="cuda"),
                            cuda(b_scale), None, cuda(ws), cuda(w), cuda(ids),
                            _empty(), _empty(), _empty(), True, top_k, False, False)
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.75, b_scale.numpy(), w.numpy(),
                              ids.numpy(), True, compute_dtype="f32")
    assert np.abs(oracle).max() > 0
    assert_parity(C, oracle, what=f"{a_dtype} scales {scale_range}")


def test_fused_moe_out_of_range_ids_stay_zero():
    rng = np.random.default_rng(43)
    m, k, n, e, top_k = 5, 128, 48, 4, 2
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(43, (m, k))
    ids = torch.tensor([[0, 1], [4, 2], [-1, 3], [1, 1], [9, 0]])
    w = torch.rand((m, top_k))
    C = torch.full((m, top_k, n), 5.0, dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.ones(1, device="cuda"),
                            torch.ones(e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                            _empty(), _empty(), _empty(), False, top_k, False, False)
    out = C.float().cpu()
    for t, s in ((1, 0), (2, 0), (4, 0)):
        assert torch.all(out[t, s] == 0)
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 1.0, np.ones(e), w.numpy(),
                              ids.numpy(), False)
    assert_parity(C, oracle)


@pytest.mark.parametrize("m", [1, 8, 32])
def test_fused_moe_decode_shapes(m):
    # BASELINE config 5 gate_up shape: E=128, top-8, K=2048 -> N=1536
    rng = np.random.default_rng(20260820 + m)
    e, k, n, top_k = 128, 2048, 1536, 8
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(20260820 + m, (m, k))
    w, ids = _route(m, e, top_k, 20260830 + m)
    C = torch.empty((m, top_k, n), dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.ones(1, device="cuda"),
                            torch.ones(e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                            _empty(), _empty(), _empty(), True, top_k, False, False)
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 1.0, np.ones(e), w.numpy(), ids.numpy(),
                              True)
    assert_parity(C, oracle, what=f"moe decode m={m}")


# ---------------------------------------------------------------- AITER entry

@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
def test_aiter_entry_uses_metadata(block_m):
    rng = np.random.default_rng(block_m)
    m, k, n, e, top_k = 40, 256, 96, 5, 2
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(block_m, (m, k))
    w, ids = _route(m, e, top_k, 100 + block_m)
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    # mark the blocks of expert 2 as not on this device (EP sentinel -1)
    exp_ = exp_.copy()
    exp_[exp_ == 2] = -1
    C = torch.full((m, top_k, n), 3.0, dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4(cuda(a), cuda(wp), C, torch.tensor([0.5], device="cuda"),
                       torch.linspace(1, 2, e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                       cuda(srt), cuda(exp_), cuda(npp), True, top_k, False, False,
                       {"BLOCK_SIZE_M": block_m}, torch.bfloat16)
    out = C.float().cpu().numpy()
    ids_np = ids.numpy()
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.5, np.linspace(1, 2, e), w.numpy(),
                              ids_np, True)
    oracle[ids_np == 2] = 0.0  # expert -1 blocks write zeros
    assert_parity(out, oracle)


@pytest.mark.parametrize("block_m", [64, 128, 256])
@pytest.mark.parametrize("k", [256, 1024])
def test_aiter_entry_w4a4_metadata(block_m, k):
    # packed MXFP4 activations through caller metadata, with an expert -1
    # block and enough routes to fill several row blocks per expert; K = 1024
    # (a multiple of 512) stages four stages of scales per load
    rng = np.random.default_rng(block_m + 1)
    m, n, e, top_k = 300, 320, 4, 2
    wp, ws = rand_mxfp4(rng, (e, n), k)
    ap, asc = O.quant_mxfp4_ties_away(rand_act(block_m + 7, (m, k)).float().numpy())
    w, ids = _route(m, e, top_k, 200 + block_m)
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    exp_ = exp_.copy()
    exp_[exp_ == 1] = -1
    C = torch.full((m, top_k, n), 3.0, dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4(cuda(ap), cuda(wp), C, torch.tensor([0.5], device="cuda"),
                       torch.linspace(1, 2, e, device="cuda"), cuda(asc), cuda(ws), cuda(w),
                       cuda(ids), cuda(srt), cuda(exp_), cuda(npp), True, top_k, False, False,
                       {"BLOCK_SIZE_M": block_m}, torch.bfloat16)
    ids_np = ids.numpy()
    oracle = O.fused_moe_fp64(O.dequant_values(ap, asc, "bf16"), wp, ws, 0.5,
                              np.linspace(1, 2, e), w.numpy(), ids_np, True)
    oracle[ids_np == 1] = 0.0
    assert_parity(C.float().cpu().numpy(), oracle)


def test_aiter_entry_pipelined_decode_grid():
    # 16-row blocks over enough expert blocks x column groups (>= 512
    # two-step workgroups) take the software-pipelined decode kernel; one
    # expert's blocks are marked not on this device (-1)
    rng = np.random.default_rng(77)
    m, k, n, e, top_k, block_m = 48, 512, 8192, 16, 4, 16
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(77, (m, k))
    w, ids = _route(m, e, top_k, 177)
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    exp_ = exp_.copy()
    exp_[exp_ == 3] = -1
    C = torch.full((m, top_k, n), 3.0, dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4(cuda(a), cuda(wp), C, torch.tensor([0.5], device="cuda"),
                       torch.linspace(1, 2, e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                       cuda(srt), cuda(exp_), cuda(npp), True, top_k, False, False,
                       {"BLOCK_SIZE_M": block_m}, torch.bfloat16)
    ids_np = ids.numpy()
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.5, np.linspace(1, 2, e), w.numpy(),
                              ids_np, True)
    oracle[ids_np == 3] = 0.0
    assert_parity(C.float().cpu().numpy(), oracle)


# ---------------------------------------------------------------- routing

@pytest.mark.parametrize("n_tokens,top_k,num_experts,block_m",
                         [(1, 8, 128, 16), (8, 8, 128, 16), (33, 4, 16, 32), (128, 8, 128, 32),
                          (100, 8, 256, 16), (256, 8, 128, 64), (512, 8, 128, 64),
                          (700, 3, 7, 128), (64, 4, 300, 16), (4096, 8, 128, 128),
                          # single-workgroup kernel: a few experts with hundreds of
                          # routes each, and a block size that is not a power of two
                          (512, 8, 3, 48), (128, 8, 5, 16), (96, 8, 256, 32),
                          # per-chunk counts + one scan-and-place launch (<= 64
                          # chunks of 1024 routes), and the three-launch path beyond
                          (2048, 8, 512, 32), (600, 8, 1024, 16), (8192, 8, 128, 64),
                          (513, 8, 256, 16), (9000, 8, 64, 128)])
def test_device_routing_matches_oracle(n_tokens, top_k, num_experts, block_m):
    g = torch.Generator().manual_seed(n_tokens * 7 + top_k)
    ids = torch.randint(-1, num_experts + 1, (n_tokens, top_k), generator=g)
    srt, exp_, npp = mx.make_routing(cuda(ids), block_m=block_m, num_experts=num_experts)
    used = int(npp[0])
    r_srt, r_exp, r_npp = c_oracle.make_routing(ids.numpy(), num_experts, block_m)
    assert used == int(r_npp[0])
    assert np.array_equal(srt[:used].cpu().numpy(), r_srt)
    assert np.array_equal(exp_[:used // block_m].cpu().numpy(), r_exp)
    # int32 ids give the same metadata
    srt32, _, npp32 = mx.make_routing(cuda(ids.to(torch.int32)), block_m=block_m,
                                      num_experts=num_experts)
    assert int(npp32[0]) == used and torch.equal(srt32[:used], srt[:used])


# ---------------------------------------------------------------- MoE layer

def _layer_weights(seed, e=128, hidden=2048, inter=768):
    rng = np.random.default_rng(seed)
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter)
    return w13, s13, w2, s2


@pytest.fixture(scope="module")
def layer_weights():
    return _layer_weights(20260815)


@pytest.mark.parametrize("m", [1, 8, 32, 256, 512, 4096])
def test_moe_layer_vs_oracle(m, layer_weights):
    w13, s13, w2, s2 = layer_weights
    x = rand_act(20260816 + m, (m, 2048))
    w, ids = _route(m, 128, 8, 20260817 + m)
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    assert y.shape == (m, 2048) and y.dtype == torch.bfloat16
    # each token depends only on its own row and routing: check a sample
    rows = np.arange(m) if m <= 32 else np.sort(np.random.default_rng(m).choice(m, 32, False))
    oracle, routes = O.moe_layer_fp64(x.float().numpy()[rows], w13, s13, w2, s2,
                                      w.numpy()[rows], ids.numpy()[rows], return_routes=True)
    t = torch.from_numpy
    safe = O.moe_layer_safe(x[rows], t(w13), t(s13), t(w2), t(s2), w[rows], ids[rows])
    assert_layer_parity(y[t(rows).cuda()], oracle, safe, what=f"moe layer m={m}", routes=routes)


def test_vllm_adapter_moe_and_dense_on_device(layer_weights):
    # the vLLM hooks on real layers: weights renamed as vllm:215-230, then
    # apply / apply_weights equal the operators they wrap, bit for bit
    import types
    from mxfp4_amd import vllm_adapter as va
    w13, s13, w2, s2 = layer_weights
    layer = types.SimpleNamespace(activation="silu", w13_weight_packed=cuda(w13),
                                  w13_weight_scale=cuda(s13), w2_weight_packed=cuda(w2),
                                  w2_weight_scale=cuda(s2))
    va._moe_process_weights_after_loading(None, layer)
    x = cuda(rand_act(71, (8, 2048)))
    w, ids = _route(8, 128, 8, 72)
    y = va._moe_apply(None, layer, x, cuda(w), cuda(ids))
    ref = mx.moe_layer(x, cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    assert torch.equal(y, ref)
    dense = types.SimpleNamespace(weight_packed=cuda(w13[0]), weight_scale=cuda(s13[0]))
    va._dense_process_weights_after_loading(None, dense)
    yd = va._dense_apply_weights(None, dense, x)
    assert torch.equal(yd, mx.linear_mxfp4_soft(x, cuda(w13[0]), cuda(s13[0])))


def test_vllm_reference_debug_path_on_device(layer_weights, monkeypatch):
    # MXFP4_IMPLEMENTATION=reference (vllm:94-102, 188-265): the device
    # dequant kernel + a library GEMM in bf16, against the FP64 oracle and
    # the reference safe path restated on the CPU
    import types
    from mxfp4_amd import vllm_adapter as va
    monkeypatch.setattr(va, "_IMPL", "reference")
    w13, s13, w2, s2 = layer_weights
    layer = types.SimpleNamespace(activation="silu", w13_weight=cuda(w13),
                                  w13_weight_scale=cuda(s13), w2_weight=cuda(w2),
                                  w2_weight_scale=cuda(s2))
    m = 6
    x = rand_act(73, (m, 2048))
    w, ids = _route(m, 128, 8, 74)
    y = va._moe_apply(None, layer, cuda(x), cuda(w), cuda(ids))
    assert y.shape == (m, 2048) and y.dtype == torch.bfloat16
    oracle, routes = O.moe_layer_fp64(x.float().numpy(), w13, s13, w2, s2, w.numpy(),
                                      ids.numpy(), return_routes=True)
    t = torch.from_numpy
    safe = O.moe_layer_safe(x, t(w13), t(s13), t(w2), t(s2), w, ids)
    _same_numerics_as_reference(y, safe, oracle, "vllm reference path, moe")
    dense = types.SimpleNamespace(weight_packed=cuda(w13[5]), weight_scale=cuda(s13[5]))
    bias = rand_act(75, (1536,))
    xd = rand_act(76, (2, 3, 2048))
    yd = va._dense_apply_weights(None, dense, cuda(xd), cuda(bias))
    assert yd.shape == (2, 3, 1536)
    od = O.linear_fp64(xd.reshape(6, 2048).float().numpy(), w13[5], s13[5],
                       bias.float().numpy())
    _same_numerics_as_reference(yd.reshape(6, 1536),
                                O.linear_safe(xd, w13[5], s13[5], bias).reshape(6, 1536), od,
                                "vllm reference path, dense")


def _same_numerics_as_reference(y, safe, oracle, what):
    """The debug path is the reference's own composition (every intermediate
    rounded to bf16), so its bar is the reference's: its error against the
    FP64 oracle no worse than the safe path's restated on the CPU (x1.1), and
    the two within a few bf16 steps of each other (only the BLAS summation
    order differs)."""
    y = y.float().cpu().numpy()
    r = safe.float().cpu().numpy()
    e, er = O.parity_errors(y, oracle), O.parity_errors(r, oracle)
    assert e["norm_rel"] <= 1.1 * er["norm_rel"] + 1e-4, (what, e, er)
    gap = np.linalg.norm(y - r) / np.linalg.norm(r)
    assert gap <= 1e-2, (what, gap)


def test_moe_layer_hidden_not_multiple_of_128():
    # hidden 1056 (K % 128 == 32 for gate_up): routed blocks of 64 go to the
    # register-staged tiled kernel; inter 320 keeps the down GEMM on it too
    rng = np.random.default_rng(1056)
    e, hidden, inter, top_k, m = 8, 1056, 320, 2, 256
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter)
    x = rand_act(1056, (m, hidden))
    w, ids = _route(m, e, top_k, 1057)
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    rows = np.sort(np.random.default_rng(3).choice(m, 24, False))
    oracle, routes = O.moe_layer_fp64(x.float().numpy()[rows], w13, s13, w2, s2,
                                      w.numpy()[rows], ids.numpy()[rows], return_routes=True)
    t = torch.from_numpy
    safe = O.moe_layer_safe(x[rows], t(w13), t(s13), t(w2), t(s2), w[rows], ids[rows])
    assert_layer_parity(y[t(rows).cuda()], oracle, safe, what="moe layer hidden 1056",
                        routes=routes)


def test_moe_layer_small_vs_golden_and_safe():
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "small_cases.npz"))
    y = mx.moe_layer(cuda(torch.from_numpy(g["layer_x"]).to(torch.bfloat16)), cuda(g["layer_w13"]),
                     cuda(g["layer_s13"]), cuda(g["layer_w2"]), cuda(g["layer_s2"]),
                     cuda(g["layer_w"]), cuda(g["layer_ids"]))
    t = lambda k: torch.from_numpy(g[k])  # noqa: E731
    safe = O.moe_layer_safe(t("layer_x").to(torch.bfloat16), t("layer_w13"), t("layer_s13"),
                            t("layer_w2"), t("layer_s2"), t("layer_w"), t("layer_ids"))
    oracle, routes = O.moe_layer_fp64(g["layer_x"], g["layer_w13"], g["layer_s13"],
                                      g["layer_w2"], g["layer_s2"], g["layer_w"], g["layer_ids"],
                                      return_routes=True)
    assert np.array_equal(oracle, g["layer_y"])
    assert_layer_parity(y, g["layer_y"], safe, routes=routes)


def _fp16_layer_oracle(xs, w13, s13, w2, s2, w, ids):
    """The MoE layer in float64 with the fp16 rounding points of the
    reference composition (gate_up, silu, product, down; FP32-exact sum).
    Returns the layer output and the rounded per-route down outputs."""
    m, top_k = ids.shape
    ones = np.ones(w13.shape[0])
    gu = O.round_to_dtype(O.fused_moe_fp64(xs, w13, s13, 1.0, ones, w, ids, False,
                                           compute_dtype="f16"), "f16")
    inter = gu.shape[-1] // 2
    gg, uu = gu[..., :inter], gu[..., inter:]
    h = O.round_to_dtype(O.round_to_dtype(gg / (1 + np.exp(-gg)), "f16") * uu, "f16")
    d = O.fused_moe_fp64(h.reshape(m * top_k, inter), w2, s2, 1.0, ones, w.reshape(-1, 1),
                         ids.reshape(-1, 1), True, compute_dtype="f16")
    routes = O.round_to_dtype(d, "f16")[:, 0].reshape(m, top_k, -1)
    return routes.sum(1), routes


def test_moe_layer_fp16_and_invalid_ids():
    rng = np.random.default_rng(5)
    # small scales keep every fp16 intermediate finite
    w13, s13 = rand_mxfp4(rng, (8, 256), 256, lo=116, hi=121)
    w2, s2 = rand_mxfp4(rng, (8, 256), 128, lo=116, hi=121)
    m = 12
    x = rand_act(6, (m, 256), torch.float16)
    w, ids = _route(m, 8, 2, 7)
    ids[3, 1] = 8   # out of range: contributes nothing
    ids[5, 0] = -1
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    assert y.dtype == torch.float16
    oracle, routes = _fp16_layer_oracle(x.float().numpy(), w13, s13, w2, s2, w.numpy(),
                                        ids.numpy())
    t = torch.from_numpy
    safe = O.moe_layer_safe(x, t(w13), t(s13), t(w2), t(s2), w, ids)
    assert_layer_parity(y, oracle, safe, routes=routes, fmt="f16")


def test_moe_layer_fp16_multi_round_grid():
    # fp16 layer with ~165 routed 64-row blocks: both GEMMs have more tiles
    # than resident workgroups (64 x 384 SiLU tiles, 64 x 256 plain ones);
    # sampled rows against the fp16-rounded oracle
    rng = np.random.default_rng(2600)
    e, hidden, inter, top_k, m = 8, 2048, 768, 4, 2600
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden, lo=116, hi=121)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter, lo=116, hi=121)
    x = rand_act(2601, (m, hidden), torch.float16)
    w, ids = _route(m, e, top_k, 2602)
    ids[17, 2] = -1  # dropped: contributes nothing
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    rows = np.sort(np.concatenate([[17], np.random.default_rng(9).choice(m, 47, False)]))
    rows = np.unique(rows)
    oracle, routes = _fp16_layer_oracle(x.float().numpy()[rows], w13, s13, w2, s2,
                                        w.numpy()[rows], ids.numpy()[rows])
    t = torch.from_numpy
    safe = O.moe_layer_safe(x[rows], t(w13), t(s13), t(w2), t(s2), w[rows], ids[rows])
    assert_layer_parity(y[t(rows).cuda()], oracle, safe, what="fp16 layer, several rounds",
                        routes=routes, fmt="f16")


def test_moe_layer_fp16_wide_routed_tiles():
    # fp16 layer at 480 tokens over 128 experts: 32-row blocks whose 32 x 256
    # grids would spill past one round, so the SiLU GEMM runs 32 x 384 and
    # the plain one 32 x 512 tiles (2 stages); sampled rows against the
    # fp16-rounded oracle
    rng = np.random.default_rng(480)
    e, hidden, inter, top_k, m = 128, 2048, 768, 8, 480
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden, lo=116, hi=121)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter, lo=116, hi=121)
    x = rand_act(481, (m, hidden), torch.float16)
    w, ids = _route(m, e, top_k, 482)
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    rows = np.sort(np.random.default_rng(483).choice(m, 40, False))
    oracle, routes = _fp16_layer_oracle(x.float().numpy()[rows], w13, s13, w2, s2,
                                        w.numpy()[rows], ids.numpy()[rows])
    t = torch.from_numpy
    safe = O.moe_layer_safe(x[rows], t(w13), t(s13), t(w2), t(s2), w[rows], ids[rows])
    assert_layer_parity(y[t(rows).cuda()], oracle, safe, what="fp16 layer, wide routed tiles",
                        routes=routes, fmt="f16")


@pytest.mark.parametrize("m,n,k,dtype,block_m",
                         [(2300, 3072, 256, torch.float16, 128),
                          (2300, 3068, 256, torch.bfloat16, 128),
                          (2048, 2048, 256, torch.bfloat16, 128),
                          (1200, 2048, 256, torch.float16, 64),
                          (1600, 1536, 768, torch.bfloat16, 64)])
def test_routed_gemm_multi_round_grid(m, n, k, dtype, block_m):
    # several rounds of tiles: 68-75 routed 128-row blocks (the persistent
    # kernel; 128 x 256 tiles at N = 3072, whose rounds are 88% full, and at
    # N = 3068, whose rows take 8-byte stores instead of 16-byte ones;
    # 128 x 128 at N = 2048), or 83-108 blocks of 64 rows (64 x 256 tiles,
    # 3 stages).  Expert -1 blocks, ids outside [0, E) (rows left
    # untouched), route weights, per-expert scales
    rng = np.random.default_rng(n + k)
    e, top_k = 8, 4
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(n + 1, (m, k), dtype)
    w, ids = _route(m, e, top_k, n + 2)
    dropped = ((5, 1), (77, 0), (1000, 3))
    ids[5, 1], ids[77, 0], ids[1000, 3] = -1, e, e + 3
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    exp_ = exp_.copy()
    exp_[exp_ == 6] = -1
    C = torch.full((m, top_k, n), 3.0, dtype=dtype, device="cuda")
    mx.fused_moe_mxfp4(cuda(a), cuda(wp), C, torch.tensor([0.5], device="cuda"),
                       torch.linspace(1, 2, e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                       cuda(srt), cuda(exp_), cuda(npp), True, top_k, False, False,
                       {"BLOCK_SIZE_M": block_m}, dtype)
    ids_np = ids.numpy()
    dt = "f16" if dtype == torch.float16 else "bf16"
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.5, np.linspace(1, 2, e), w.numpy(),
                              ids_np, True, compute_dtype=dt)
    oracle[ids_np == 6] = 0.0  # expert -1 blocks write zeros
    out = C.float().cpu().numpy()
    for t_, s_ in dropped:
        assert np.all(out[t_, s_] == 3.0)
        oracle[t_, s_] = 3.0
    assert_parity(out, oracle, what=f"n={n} {dtype}")


# ---------------------------------------------------------------- router

@pytest.mark.parametrize("m,e,top_k,renorm,ids_dtype",
                         [(1, 128, 8, True, torch.int64), (4096, 128, 8, True, torch.int32),
                          (333, 60, 4, False, torch.int64), (17, 1024, 16, True, torch.int64),
                          (8, 7, 7, False, torch.int32), (100, 256, 64, True, torch.int64),
                          (5, 65, 1, True, torch.int32)])
def test_route_topk_matches_oracle(m, e, top_k, renorm, ids_dtype):
    g = torch.Generator().manual_seed(m * 31 + e)
    logits = torch.randn((m, e), generator=g) * 2.0
    w, ids = mx.route_topk(cuda(logits), top_k, renormalize=renorm, ids_dtype=ids_dtype)
    assert w.dtype == torch.float32 and ids.dtype == ids_dtype and w.shape == (m, top_k)
    ow, oids = O.route_topk_fp64(logits.numpy(), top_k, renormalize=renorm)
    assert np.array_equal(ids.cpu().numpy(), oids)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=2e-6, atol=0)


def test_route_topk_strided_3d_and_ties():
    # a [2, 9, E] view with a row stride past E; rows with tied logits pick
    # the lower expert id first
    g = torch.Generator().manual_seed(5)
    base = torch.randn((2, 9, 200), generator=g)
    logits = base[..., 10:138]  # 128 experts, row stride 200
    logits[0, 3, :] = 0.0
    logits[1, 4, [5, 77, 100]] = 9.0
    w, ids = mx.route_topk(cuda(base)[..., 10:138], 4)
    ow, oids = O.route_topk_fp64(logits.numpy(), 4)
    assert w.shape == (2, 9, 4)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert ids[0, 3].tolist() == [0, 1, 2, 3] and ids[1, 4, :3].tolist() == [5, 77, 100]
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=2e-6, atol=0)


def test_route_topk_feeds_the_layer(layer_weights):
    # the device router's output drives the MoE layer like torch's routing
    w13, s13, w2, s2 = layer_weights
    m = 64
    x = rand_act(640, (m, 2048))
    g = torch.Generator().manual_seed(641)
    logits = torch.randn((m, 128), generator=g)
    w, ids = mx.route_topk(cuda(logits), 8)
    p = torch.softmax(logits, -1)
    tw, tids = torch.topk(p, 8, -1)
    tw = tw / tw.sum(-1, keepdim=True)
    assert torch.equal(ids.cpu(), tids)
    assert torch.allclose(w.cpu(), tw, rtol=2e-6, atol=0)
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), w, ids)
    oracle, routes = O.moe_layer_fp64(x.float().numpy(), w13, s13, w2, s2, tw.numpy(),
                                      tids.numpy(), return_routes=True)
    t = torch.from_numpy
    safe = O.moe_layer_safe(x, t(w13), t(s13), t(w2), t(s2), tw, tids)
    assert_layer_parity(y, oracle, safe, what="layer on device routing", routes=routes)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,top_k,hidden,inter,e",
                         [(4, 16, 2048, 768, 32), (3, 6, 1024, 256, 32), (8, 8, 2048, 768, 128)],
                         ids=["k16_two_k_waves", "k6_masked_routes", "k8_four_column_steps"])
def test_moe_layer_fused_decode_top_k(m, top_k, hidden, inter, e, dtype):
    # the fused down + top-k kernel (<= 64 routes): top_k 16 fills four
    # route waves and, at 512 workgroups of 16 waves, takes two K waves of
    # up to two trips; top_k 6 leaves two of a wave's four route slots
    # empty and takes 8-column workgroups (192 workgroups).  8 tokens over
    # 128 experts: the gate_up stream kernel takes four column steps per
    # workgroup (64 row blocks x 12 workgroups)
    rng = np.random.default_rng(600 + top_k)
    # small scales keep every fp16 intermediate finite
    w13, s13 = rand_mxfp4(rng, (e, 2 * inter), hidden, lo=116, hi=121)
    w2, s2 = rand_mxfp4(rng, (e, hidden), inter, lo=116, hi=121)
    x = rand_act(601 + top_k, (m, hidden), dtype)
    w, ids = _route(m, e, top_k, 602 + top_k)
    y = mx.moe_layer(cuda(x), cuda(w13), cuda(s13), cuda(w2), cuda(s2), cuda(w), cuda(ids))
    assert y.dtype == dtype and y.shape == (m, hidden)
    if dtype == torch.float16:
        oracle, routes = _fp16_layer_oracle(x.float().numpy(), w13, s13, w2, s2, w.numpy(),
                                            ids.numpy())
    else:
        oracle, routes = O.moe_layer_fp64(x.float().numpy(), w13, s13, w2, s2, w.numpy(),
                                          ids.numpy(), return_routes=True)
    t = torch.from_numpy
    safe = O.moe_layer_safe(x, t(w13), t(s13), t(w2), t(s2), w, ids)
    assert_layer_parity(y, oracle, safe, what=f"fused decode top_k={top_k} {dtype}",
                        routes=routes, fmt="f16" if dtype == torch.float16 else "bf16")


# ---------------------------------------------------------------- FP8 activations

_FP8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _assert_fp8_parity(y, oracle, a_val, wp, ws, ids, alpha, what, out_fmt="bf16"):
    """Parity bar of the FP8-activation GEMMs.  The block-scaled MFMA adds
    each group of 8 consecutive K products keeping ~12 bits below the
    group's largest product (measured with one MFMA: 448 + 2^-3 -> 448.125,
    448 + 2^-6 -> 448, 448 - 448 + 2^-9 -> 0; sums across groups keep FP32
    precision), which E2M1 x E2M1 products never exceed but FP8's wider
    range can.  So besides norm-wise <= NORM_TOL, each element must be
    within ELEM_TOL (denominator floor 1e-3 * rms) or within
    2^-10 * sum over its K groups of max|a| * max|w| (times the scales and
    route weight) plus one step of the output."""
    y = y.float().cpu().numpy().astype(np.float64) if isinstance(y, torch.Tensor) else y
    e = O.parity_errors(y, oracle)
    assert e["norm_rel"] <= O.NORM_TOL, f"{what} norm-wise {e['norm_rel']:.3e}"
    m, k = a_val.shape
    amax = np.abs(a_val).reshape(m, k // 8, 8).max(-1)                       # [m, G]
    w_val = O.dequant_values(wp, ws, "bf16")                                  # [E, n, k]
    ne, n = w_val.shape[:2]
    wmax = np.abs(w_val).reshape(ne, n, k // 8, 8).max(-1)                    # [E, n, G]
    ids = np.asarray(ids)
    budget = np.zeros(oracle.shape)
    for ex in range(ne):
        t, sl = np.nonzero(ids == ex)
        budget[t, sl] = (amax[t] @ wmax[ex].T) * np.asarray(alpha)[t, sl, None] * 2.0 ** -10
    floor = 1e-3 * np.sqrt(np.mean(oracle * oracle))
    diff = np.abs(y - oracle)
    bad = ((diff / np.maximum(np.abs(oracle), floor) > O.ELEM_TOL)
           & (diff > budget + (O.format_ulp(oracle, out_fmt) if out_fmt else 0.0)))
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond {O.ELEM_TOL} and the "
                           f"MFMA's group-alignment budget (max elementwise {e['elem_rel']:.3e})")


def _mxfp8_quant(a: np.ndarray, fmt: str):
    """MXFP8 test data: per 32 along K, scale byte 127 + floor(log2 amax) - emax
    (emax 7 for e4m3, 14 for e5m2: the block's largest magnitude lands in
    [2^emax, 2^(emax+1)), inside the format), values rounded to the format by
    torch's own conversion."""
    emax = 7 if fmt == "e4m3" else 14
    blocks = a.reshape(a.shape[0], -1, 32)
    amax = np.abs(blocks).max(-1)
    e = np.floor(np.log2(np.maximum(amax, 2.0 ** -100))).astype(np.int64) - emax
    scales = np.clip(127 + e, 1, 254).astype(np.uint8)
    q = blocks / np.exp2(scales.astype(np.float64) - 127)[..., None]
    codes = torch.from_numpy(q.reshape(a.shape).astype(np.float32)).to(_FP8[fmt])
    return codes.view(torch.uint8).numpy(), scales


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
@pytest.mark.parametrize("k", [1024, 384, 160])
def test_aiter_entry_fp8_every_byte_at_every_k(fmt, block_m, k):
    # one-hot weights (row j of each expert is 1.0 at K = j) make every
    # output a single exact product, fp8(A[t, j]) * 2^(sa - 127) * 2^(sb - 127),
    # checked bit for bit in FP32: each activation row holds all finite
    # bytes of the format across K, so every byte value is decoded at
    # every K position, through the MFMA's FP8 operand layout and the A / B
    # scale of each 32-block.  K = 1024 takes the grouped-scale
    # direct-to-LDS kernel on 64- / 128-row blocks, 384 its per-stage-scale
    # variant, 160 (not a multiple of 128) the register-staged kernel, as do
    # 16- / 32-row blocks; an expert -1 block writes zeros
    rng = np.random.default_rng(block_m * 7 + k + (1 if fmt == "e5m2" else 0))
    m, e, top_k = 96, 3, 2
    n = k
    finite = [b for b in range(256) if not ((b & 0x7F) == 0x7F if fmt == "e4m3"
                                            else (b & 0x7C) == 0x7C)]
    ab = np.stack([np.resize(np.roll(finite, 13 * t), k) for t in range(m)]).astype(np.uint8)
    amx = rng.integers(120, 135, size=(m, k // 32), dtype=np.uint8)
    codes = np.zeros((e, n, k), dtype=np.uint8)
    codes[:, np.arange(n), np.arange(n)] = 2  # E2M1 1.0
    wp = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    ws = rng.integers(124, 131, size=(e, n, k // 32), dtype=np.uint8)
    w, ids = _route(m, e, top_k, 300 + block_m)
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    exp_ = exp_.copy()
    exp_[exp_ == 1] = -1
    C = torch.full((m, top_k, n), 3.0, dtype=torch.float32, device="cuda")
    mx.fused_moe_mxfp4(torch.from_numpy(ab).view(_FP8[fmt]).cuda(), cuda(wp), C,
                       torch.ones(1, device="cuda"), torch.ones(e, device="cuda"), cuda(amx),
                       cuda(ws), cuda(w), cuda(ids), cuda(srt), cuda(exp_), cuda(npp), False,
                       top_k, False, False, {"BLOCK_SIZE_M": block_m}, torch.float32)
    ids_np = ids.numpy()
    a_val = O.fp8_scaled_values(ab, amx, fmt)                          # [m, k]
    b_scale = O.e8m0_to_f32(ws).astype(np.float64)                      # [e, n, k/32]
    want = a_val[:, None, :] * np.take_along_axis(
        np.repeat(b_scale, 32, axis=-1), np.arange(n)[None, :, None], axis=-1)[..., 0][ids_np]
    want[ids_np == 1] = 0.0
    got = C.cpu().numpy().astype(np.float64)
    assert np.array_equal(got, want), (
        f"{int((got != want).sum())} of {got.size} outputs differ (fp8 {fmt}, block {block_m}, "
        f"k {k})")


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("block_m", [16, 64, 128])
@pytest.mark.parametrize("scaled", [True, False], ids=["a_mx", "no_a_mx"])
def test_aiter_entry_fp8_activations(fmt, block_m, scaled):
    # MXFP8 activations from N(0, 1) data (with A_mx_scale) or FP8 values of
    # N(0, 1) data without scales (the reference's host path), route
    # weights, an expert -1 block, against the FP64 oracle
    rng = np.random.default_rng(block_m * 3 + (1 if fmt == "e5m2" else 0) + (5 if scaled else 0))
    m, n, e, top_k, k = 300, 320, 4, 2, 1024
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rng.standard_normal((m, k))
    if scaled:
        ab, amx = _mxfp8_quant(a, fmt)
    else:
        ab = torch.from_numpy(a.astype(np.float32)).to(_FP8[fmt]).view(torch.uint8).numpy()
        amx = None
    w, ids = _route(m, e, top_k, 300 + block_m)
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    exp_ = exp_.copy()
    exp_[exp_ == 1] = -1
    C = torch.full((m, top_k, n), 3.0, dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4(torch.from_numpy(ab).view(_FP8[fmt]).cuda(), cuda(wp), C,
                       torch.tensor([0.5], device="cuda"), torch.linspace(1, 2, e, device="cuda"),
                       cuda(amx) if scaled else None, cuda(ws), cuda(w), cuda(ids), cuda(srt),
                       cuda(exp_), cuda(npp), True, top_k, False, False,
                       {"BLOCK_SIZE_M": block_m}, torch.bfloat16)
    ids_np = ids.numpy()
    a_val = O.fp8_scaled_values(ab, amx, fmt)
    oracle = O.fused_moe_fp64(a_val, wp, ws, 0.5, np.linspace(1, 2, e), w.numpy(), ids_np, True)
    oracle[ids_np == 1] = 0.0
    alpha = 0.5 * np.linspace(1, 2, e)[ids_np] * w.numpy()
    _assert_fp8_parity(C, oracle, a_val, wp, ws, ids_np, alpha, f"fp8 {fmt} block {block_m}")


@pytest.mark.parametrize("c_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("block_m", [32, 128])
def test_aiter_entry_fp8_output_dtypes(c_dtype, block_m):
    rng = np.random.default_rng(17 + block_m)
    m, n, e, top_k, k = 200, 192, 3, 2, 512
    wp, ws = rand_mxfp4(rng, (e, n), k, lo=118, hi=126)
    ab, amx = _mxfp8_quant(rng.standard_normal((m, k)), "e4m3")
    w, ids = _route(m, e, top_k, 31 + block_m)
    srt, exp_, npp = O.make_routing(ids.numpy(), block_m=block_m, num_experts=e)
    C = torch.empty((m, top_k, n), dtype=c_dtype, device="cuda")
    mx.fused_moe_mxfp4(torch.from_numpy(ab).view(torch.float8_e4m3fn).cuda(), cuda(wp), C,
                       torch.ones(1, device="cuda"), torch.ones(e, device="cuda"), cuda(amx),
                       cuda(ws), cuda(w), cuda(ids), cuda(srt), cuda(exp_), cuda(npp), False,
                       top_k, False, False, {"BLOCK_SIZE_M": block_m}, c_dtype)
    a_val = O.fp8_scaled_values(ab, amx, "e4m3")
    oracle = O.fused_moe_fp64(a_val, wp, ws, 1.0, np.ones(e), w.numpy(), ids.numpy(), False)
    assert np.isfinite(oracle).all()
    _assert_fp8_parity(C, oracle, a_val, wp, ws, ids.numpy(), np.ones(ids.shape),
                       f"fp8 out {c_dtype}", out_fmt="f16" if c_dtype == torch.float16 else None)


def test_soft_op_fp8_activations_convert_to_compute_dtype():
    # soft:472-475: unpacked A is A.to(C.dtype) (exact for e4m3 / e5m2 in
    # bf16), and A_mx_scale must be None
    rng = np.random.default_rng(55)
    m, n, e, top_k, k = 40, 96, 5, 2, 256
    wp, ws = rand_mxfp4(rng, (e, n), k)
    ab = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(
        torch.float8_e5m2).view(torch.uint8).numpy()
    A = torch.from_numpy(ab).view(torch.float8_e5m2).cuda()
    w, ids = _route(m, e, top_k, 56)
    C = torch.empty((m, top_k, n), dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4_soft(A, cuda(wp), C, torch.ones(1, device="cuda"),
                            torch.ones(e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                            _empty(), _empty(), _empty(), True, top_k, False, False)
    oracle = O.fused_moe_fp64(O.fp8_values(ab, "e5m2"), wp, ws, 1.0, np.ones(e), w.numpy(),
                              ids.numpy(), True)
    assert_parity(C, oracle, what="soft op fp8 A")
    with pytest.raises(ValueError, match="must not provide A_mx_scale"):
        mx.fused_moe_mxfp4_soft(A, cuda(wp), C, torch.ones(1, device="cuda"),
                                torch.ones(e, device="cuda"),
                                torch.full((m, k // 32), 127, dtype=torch.uint8, device="cuda"),
                                cuda(ws), cuda(w), cuda(ids), _empty(), _empty(), _empty(), True,
                                top_k, False, False)


def test_empty_token_batches():
    # zero tokens through every entry point: the reference returns empty
    # results (torch.matmul of [0, K]; the safe MoE loop finds no routes and
    # leaves C as zero_() made it, soft:476-494; the layer's sum over
    # nothing), and so must these -- no launch, no error
    rng = np.random.default_rng(3)
    e, top_k, k, n, inter = 4, 2, 256, 64, 64
    wp, ws = rand_mxfp4(rng, (e, n), k)
    B, Bs = cuda(wp), cuda(ws)
    x = torch.empty((0, k), dtype=torch.bfloat16, device="cuda")
    y = mx.linear_mxfp4_soft(x, B[0], Bs[0])
    assert y.shape == (0, n) and y.dtype == torch.bfloat16
    y3 = mx.linear_mxfp4_soft(torch.empty((2, 0, k), dtype=torch.float16, device="cuda"),
                              B[0], Bs[0])
    assert y3.shape == (2, 0, n) and y3.dtype == torch.float16
    tw = torch.empty((0, top_k), dtype=torch.float32, device="cuda")
    ti = torch.empty((0, top_k), dtype=torch.int64, device="cuda")
    C = torch.empty((0, top_k, n), dtype=torch.bfloat16, device="cuda")
    one, ones_e = torch.ones(1, device="cuda"), torch.ones(e, device="cuda")
    mx.fused_moe_mxfp4_soft(x, B, C, one, ones_e, None, Bs, tw, ti, _empty(), _empty(), _empty(),
                            True, top_k, False, False)
    empty_i = torch.empty(0, dtype=torch.int32, device="cuda")
    mx.fused_moe_mxfp4(x, B, C, one, ones_e, None, Bs, tw, ti, empty_i, empty_i,
                       torch.zeros(1, dtype=torch.int32, device="cuda"), True, top_k, False, False,
                       {"BLOCK_SIZE_M": 32}, torch.bfloat16)
    w13p, w13s = rand_mxfp4(rng, (e, 2 * inter), k)
    w2p, w2s = rand_mxfp4(rng, (e, k), inter)
    out = mx.moe_layer(x, cuda(w13p), cuda(w13s), cuda(w2p), cuda(w2s), tw, ti)
    assert out.shape == (0, k) and out.dtype == torch.bfloat16
    rw, ri = mx.route_topk(torch.empty((0, e), device="cuda"), top_k)
    assert rw.shape == (0, top_k) and ri.shape == (0, top_k)
    qp, qs = mx.dynamic_mxfp4_quant(x)
    assert qp.shape == (0, k // 2) and qs.shape == (0, k // 32)
    torch.cuda.synchronize()
