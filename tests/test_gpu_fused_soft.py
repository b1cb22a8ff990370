"""GPU parity: ``fused_moe_mxfp4_soft`` through its one library call
(``mxfp4_fused_moe``: device routing + the grouped GEMM, soft:379-494).

The safe path zero-fills C and then writes the rows of routes whose expert id
is in range (soft:476-494).  The library writes zeros only to the rows no GEMM
row covers (the routing gathers out-of-range ids in blocks of an extra
expert, which the GEMMs fill with zeros), so every test starts from a C full
of NaN: any row left unwritten fails.  The sizes pick each routing block
size (16 / 32 / 64 / 128 rows, from the routes per expert) and each compute
path (W4A16 bf16 / fp16, packed-A W4A4, C in FP32)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import mxfp4_oracle as O

from _helpers import assert_parity, cuda, rand_act, rand_mxfp4

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]


def _empty():
    return torch.empty(0, device="cuda")


def _route_with_dropped(m, e, top_k, seed, dropped):
    """softmax -> top-k of seeded logits; then `dropped` of the slots get ids
    outside [0, e) (-1, e, e + 7 in turn)."""
    g = torch.Generator().manual_seed(seed)
    w, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
    ids = ids.clone()
    if dropped:
        pick = torch.randperm(m * top_k, generator=g)[:dropped]
        bad = torch.tensor([-1, e, e + 7])[torch.arange(dropped) % 3]
        ids.view(-1)[pick] = bad
    return w.float(), ids


def _run(a, a_mx, wp, ws, ids, w, c_dtype, mul, a_scale=0.75, b_scale=None):
    m, top_k = ids.shape
    e, n = wp.shape[0], wp.shape[1]
    bs = torch.ones(e) if b_scale is None else b_scale
    C = torch.full((m, top_k, n), float("nan"), dtype=c_dtype, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.full((1,), a_scale, device="cuda"),
                            cuda(bs), None if a_mx is None else cuda(a_mx), cuda(ws), cuda(w),
                            cuda(ids), _empty(), _empty(), _empty(), mul, top_k, False, False)
    return C


# (tokens, experts, top_k) -> routes per expert 1 / 16 / 40 / 128: routing
# blocks of 16 / 32 / 64 / 128 rows
BLOCK_CASES = [(8, 64, 8), (64, 16, 4), (160, 16, 4), (512, 16, 4)]


@pytest.mark.parametrize("m,e,top_k", BLOCK_CASES, ids=["blk16", "blk32", "blk64", "blk128"])
@pytest.mark.parametrize("c_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("dropped", [0, 37], ids=["all_valid", "dropped"])
def test_soft_op_every_row_written(m, e, top_k, c_dtype, dropped):
    rng = np.random.default_rng(m + e)
    k, n = 256, 192  # a ragged last column tile for the 128- and 256-wide tiles
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(m + 3, (m, k))
    w, ids = _route_with_dropped(m, e, top_k, 1000 + m, min(dropped, m * top_k // 2))
    b_scale = torch.linspace(0.5, 1.5, e)
    C = _run(a, None, wp, ws, ids, w, c_dtype, True, b_scale=b_scale)
    out = C.float().cpu().numpy()
    assert not np.isnan(out).any(), "a row of C was left unwritten"
    ids_np = ids.numpy()
    bad = (ids_np < 0) | (ids_np >= e)
    assert np.all(out[bad] == 0), "rows of out-of-range ids must be zero (soft:476)"
    dt = "f16" if c_dtype == torch.float16 else "bf16"
    oracle = O.fused_moe_fp64(O.round_to_dtype(a.float().numpy(), dt), wp, ws, 0.75,
                              b_scale.numpy(), w.numpy(), ids_np, True, compute_dtype=dt)
    assert_parity(out, oracle, what=f"m={m} e={e} top_k={top_k} {dt} dropped={int(bad.sum())}")


@pytest.mark.parametrize("m,e,top_k", [(64, 16, 4), (512, 16, 4)], ids=["blk32", "blk64"])
def test_soft_op_w4a4_every_row_written(m, e, top_k):
    rng = np.random.default_rng(7 * m)
    k, n = 512, 160
    wp, ws = rand_mxfp4(rng, (e, n), k)
    ap, asc = O.quant_mxfp4_rne(rand_act(m + 5, (m, k)).float().numpy())
    w, ids = _route_with_dropped(m, e, top_k, 2000 + m, 23)
    C = _run(ap, asc, wp, ws, ids, w, torch.bfloat16, False)
    out = C.float().cpu().numpy()
    assert not np.isnan(out).any(), "a row of C was left unwritten"
    ids_np = ids.numpy()
    assert np.all(out[(ids_np < 0) | (ids_np >= e)] == 0)
    oracle = O.fused_moe_fp64(O.dequant_values(ap, asc, "bf16"), wp, ws, 0.75, np.ones(e),
                              w.numpy(), ids_np, False)
    assert_parity(out, oracle, what=f"w4a4 m={m}")


@pytest.mark.parametrize("m,e,top_k", [(8, 64, 8), (160, 16, 4)], ids=["blk16", "blk64"])
def test_soft_op_fp32_every_row_written(m, e, top_k):
    rng = np.random.default_rng(11 * m)
    k, n = 256, 96
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(m + 9, (m, k)).float()
    w, ids = _route_with_dropped(m, e, top_k, 3000 + m, 19)
    C = _run(a, None, wp, ws, ids, w, torch.float32, True)
    out = C.cpu().numpy()
    assert not np.isnan(out).any(), "a row of C was left unwritten"
    ids_np = ids.numpy()
    assert np.all(out[(ids_np < 0) | (ids_np >= e)] == 0)
    oracle = O.fused_moe_fp64(a.numpy(), wp, ws, 0.75, np.ones(e), w.numpy(), ids_np, True,
                              compute_dtype="f32")
    assert_parity(out, oracle, what=f"fp32 m={m}")


def test_soft_op_1024_experts_zero_fill():
    # 1024 experts leave no room for the extra expert of dropped routes: the
    # call zero-fills C with a fill kernel and routes the valid ids only
    rng = np.random.default_rng(1024)
    m, e, top_k, k, n = 96, 1024, 4, 128, 48
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(1025, (m, k))
    w, ids = _route_with_dropped(m, e, top_k, 1026, 31)
    C = _run(a, None, wp, ws, ids, w, torch.bfloat16, True)
    out = C.float().cpu().numpy()
    assert not np.isnan(out).any()
    ids_np = ids.numpy()
    assert np.all(out[(ids_np < 0) | (ids_np >= e)] == 0)
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.75, np.ones(e), w.numpy(), ids_np,
                              True)
    assert_parity(out, oracle, what="1024 experts")


def test_soft_op_gate_up_shape_512_tokens():
    # BASELINE config 3's gate_up at 512 tokens (the bench row): 64-row
    # blocks on 64 x 128 tiles of the checkpoint layout; sampled rows vs the
    # FP64 oracle, every row written
    rng = np.random.default_rng(20260818)
    m, e, top_k, k, n = 512, 128, 8, 2048, 1536
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(20260819, (m, k))
    w, ids = _route_with_dropped(m, e, top_k, 20260820, 0)
    C = _run(a, None, wp, ws, ids, w, torch.bfloat16, True, a_scale=1.0)
    out = C.float().cpu().numpy()
    assert not np.isnan(out).any()
    rows = np.arange(0, m, 37)
    oracle = O.fused_moe_fp64(a.float().numpy()[rows], wp, ws, 1.0, np.ones(e),
                              w.numpy()[rows], ids.numpy()[rows], True)
    assert_parity(out[rows], oracle, what="gate_up 512 tokens")


@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
def test_soft_op_triton_backend_uses_caller_metadata(block_m, monkeypatch):
    # MXFP4_GFX936_BACKEND=triton (soft:409-464): C zero-filled, then the
    # grouped GEMM over the caller's metadata; an expert -1 block writes
    # zeros and routes the metadata leaves out stay zero
    rng = np.random.default_rng(block_m + 50)
    m, k, n, e, top_k = 40, 256, 96, 5, 2
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(block_m + 51, (m, k))
    w, ids = _route_with_dropped(m, e, top_k, 500 + block_m, 0)
    ids_np = ids.numpy()
    srt, exp_, npp = O.make_routing(ids_np, block_m=block_m, num_experts=e)
    srt, exp_ = srt.copy(), exp_.copy()
    exp_[exp_ == 2] = -1                            # not on this device
    left_out = srt[(srt < m * top_k)][:3].copy()    # three routes the metadata omits
    srt[np.isin(srt, left_out)] = m * top_k
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "triton")
    C = torch.full((m, top_k, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(a), cuda(wp), C, torch.tensor([0.5], device="cuda"),
                            torch.linspace(1, 2, e, device="cuda"), None, cuda(ws), cuda(w),
                            cuda(ids), cuda(srt), cuda(exp_), cuda(npp), True, top_k, False,
                            False)
    out = C.float().cpu().numpy()
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.5, np.linspace(1, 2, e), w.numpy(),
                              ids_np, True)
    oracle[ids_np == 2] = 0.0
    oracle.reshape(m * top_k, n)[left_out] = 0.0
    assert not np.isnan(out).any()
    assert np.all(out.reshape(m * top_k, n)[left_out] == 0)
    assert_parity(out, oracle, what=f"triton backend block {block_m}")


def test_soft_op_activations_beyond_2gib():
    # A [270000, 4096] bf16 (2.2 GB) routed top-1 over 2 experts: the
    # routed GEMM on the kernel with 64-bit operand addressing, and the
    # routing over 264 chunks of 1024 routes (the separate scan and
    # placement launches beyond 64 chunks); sampled rows near the start,
    # the 2^31-byte mark and the end against the FP64 oracle
    m, k, n, e, top_k = 270000, 4096, 128, 2, 1
    rng = np.random.default_rng(4096)
    wp, ws = rand_mxfp4(rng, (e, n), k)
    g = torch.Generator(device="cuda").manual_seed(4097)
    a = torch.randn((m, k), generator=g, device="cuda", dtype=torch.bfloat16)
    ids = torch.randint(0, e, (m, top_k), generator=g, device="cuda")
    w = torch.rand((m, top_k), generator=g, device="cuda") + 0.5
    C = torch.full((m, top_k, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    b_scale = torch.tensor([0.5, 1.5], device="cuda")
    mx.fused_moe_mxfp4_soft(a, cuda(wp), C, torch.tensor([0.75], device="cuda"), b_scale, None,
                            cuda(ws), w, ids, _empty(), _empty(), _empty(), True, top_k, False,
                            False)
    rows = np.array([0, 1, (1 << 31) // (k * 2) - 1, (1 << 31) // (k * 2), m - 2, m - 1])
    sel = torch.from_numpy(rows).cuda()
    oracle = O.fused_moe_fp64(a[sel].float().cpu().numpy(), wp, ws, 0.75, b_scale.cpu().numpy(),
                              w[sel].cpu().numpy(), ids[sel].cpu().numpy(), True)
    assert not torch.isnan(C).any()
    assert_parity(C[sel], oracle, what="2.2 GB of activations")
    del a, C
    torch.cuda.empty_cache()


def test_triton_value_matches_safe_on_the_reference_inputs(monkeypatch):
    # test:144-213 on the test's own inputs (its seed, randn drawn on the
    # device; the reference's quantizer): one expert, top-1, 16 tokens, the
    # triton value fed identity metadata of one 16-row block.  The reference
    # asserts the two values bitwise equal.  Here they take different
    # kernels -- the safe value's device routing puts the 16 routes in a
    # 32-row block (prefill tile, sequential K), the caller's 16-row block
    # takes the decode kernel (K split across waves, partial sums added in
    # a fixed order) -- so their FP32 sums of the exact products may differ
    # by a few FP32 steps; no output of these inputs lies that close to a
    # bf16 rounding boundary.
    torch.manual_seed(20260812)
    m, n, k, e, top_k = 16, 256, 2048, 1, 1
    activations = torch.randn((m, k), device="cuda", dtype=torch.bfloat16)
    weights = torch.randn((e, n, k), device="cuda", dtype=torch.bfloat16)
    packed, scales = (cuda(t) for t in O.quant_mxfp4_ties_away(weights.float().cpu().numpy()))
    tw = torch.ones((m, top_k), device="cuda", dtype=torch.float32)
    ti = torch.zeros((m, top_k), device="cuda", dtype=torch.int64)
    one, ones_e = torch.ones(1, device="cuda"), torch.ones(e, device="cuda")
    empty = torch.empty(0, device="cuda", dtype=torch.int32)
    expected = torch.empty((m, top_k, n), device="cuda", dtype=torch.bfloat16)
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "safe")
    mx.fused_moe_mxfp4_soft(activations, packed, expected, one, ones_e, None, scales, tw, ti,
                            empty, empty, empty, False, top_k, False, False)
    actual = torch.empty_like(expected)
    monkeypatch.setenv("MXFP4_GFX936_BACKEND", "triton")
    mx.fused_moe_mxfp4_soft(activations, packed, actual, one, ones_e, None, scales, tw, ti,
                            torch.arange(m, device="cuda", dtype=torch.int32),
                            torch.zeros(1, device="cuda", dtype=torch.int32),
                            torch.tensor([m], device="cuda", dtype=torch.int32), False, top_k,
                            False, False)
    assert torch.equal(actual, expected)
    oracle = O.fused_moe_fp64(activations.float().cpu().numpy(), packed.cpu().numpy(),
                              scales.cpu().numpy(), 1.0, np.ones(e), tw.cpu().numpy(),
                              ti.cpu().numpy(), False)
    assert_parity(actual, oracle, what="triton vs safe, reference inputs")


# routes per expert 16 (32-row blocks either way) and 128 (128-row blocks on
# the checkpoint layout, 64 with a copy); N 200 leaves a ragged 16-row group
@pytest.mark.parametrize("m,e,top_k,n", [(64, 16, 4, 192), (512, 16, 4, 200)],
                         ids=["blk32", "blk128"])
@pytest.mark.parametrize("c_dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "f16", "f32"])
def test_registered_copy_is_bitwise_the_checkpoint_result(m, e, top_k, n, c_dtype, monkeypatch):
    # a registered prepacked copy of B is read by the soft op (device
    # routing), its triton-backend value (caller metadata) and AITER's entry;
    # each C equals the unregistered call's bit for bit (C in FP32: bf16 A on
    # the W4A16 tiles storing FP32)
    from mxfp4_amd import prepack as P
    print(f"registered copy m={m} e={e} n={n} {c_dtype}", flush=True)
    rng = np.random.default_rng(3 * m + n)
    k = 512
    wp, ws = rand_mxfp4(rng, (e, n), k)
    B, Bs = cuda(wp), cuda(ws)
    A = cuda(rand_act(m + 77, (m, k))).to(torch.bfloat16 if c_dtype == torch.float32 else c_dtype)
    w, ids = _route_with_dropped(m, e, top_k, 4000 + m, 11)
    w, ids = cuda(w), cuda(ids)
    a_scale = torch.tensor([0.75], device="cuda")
    b_scale = torch.linspace(0.5, 1.5, e, device="cuda")
    srt, exp_, npp = (cuda(t) for t in O.make_routing(ids.cpu().numpy(), block_m=64,
                                                         num_experts=e))

    def soft():
        C = torch.full((m, top_k, n), float("nan"), dtype=c_dtype, device="cuda")
        mx.fused_moe_mxfp4_soft(A, B, C, a_scale, b_scale, None, Bs, w, ids, _empty(), _empty(),
                                _empty(), True, top_k, False, False)
        return C

    def triton():
        monkeypatch.setenv("MXFP4_GFX936_BACKEND", "triton")
        C = torch.full((m, top_k, n), float("nan"), dtype=c_dtype, device="cuda")
        mx.fused_moe_mxfp4_soft(A, B, C, a_scale, b_scale, None, Bs, w, ids, srt, exp_, npp,
                                True, top_k, False, False)
        monkeypatch.delenv("MXFP4_GFX936_BACKEND")
        return C

    def aiter():
        C = torch.full((m, top_k, n), 3.0, dtype=c_dtype, device="cuda")
        mx.fused_moe_mxfp4(A, B, C, a_scale, b_scale, None, Bs, w, ids, srt, exp_, npp, True,
                           top_k, False, False, {"BLOCK_SIZE_M": 64}, c_dtype)
        return C

    plain = [f() for f in (soft, triton, aiter)]
    pre = P.register_prepacked(B, Bs)
    try:
        assert P.lookup_prepacked(B, Bs) is pre
        fast = [f() for f in (soft, triton, aiter)]
        torch.cuda.synchronize()
        for name, x, y in zip(("soft", "triton", "aiter"), plain, fast):
            assert torch.equal(x, y), name
            assert not torch.isnan(x).any(), name
        # an in-place weight update makes the copy stale: the calls read the
        # new checkpoint weights (and the entry is dropped)
        wp2, _ = rand_mxfp4(rng, (e, n), k)
        B.copy_(cuda(wp2))
        after = soft()
        assert P.lookup_prepacked(B, Bs) is None
        P.unregister_prepacked(B)
        assert torch.equal(after, soft())
        assert not torch.equal(after, plain[0])
    finally:
        P.unregister_prepacked(B)


# the FP32 path's 32-deep stages run in pairs with two register sets: one
# stage (K=32), an odd count (K=96, 160) and an even one (K=256); ragged N;
# 16- and 32-row routing blocks (4 and 40 routes per expert)
@pytest.mark.parametrize("k", [32, 96, 160, 256])
@pytest.mark.parametrize("m,e,top_k,n", [(8, 16, 8, 40), (160, 16, 4, 130)],
                         ids=["blk16", "blk32"])
def test_soft_op_fp32_stage_counts(k, m, e, top_k, n):
    rng = np.random.default_rng(k * 3 + m)
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(k + m, (m, k)).float()
    w, ids = _route_with_dropped(m, e, top_k, 6000 + k + m, 5)
    C = _run(a, None, wp, ws, ids, w, torch.float32, True)
    out = C.cpu().numpy()
    assert not np.isnan(out).any(), "a row of C was left unwritten"
    ids_np = ids.numpy()
    assert np.all(out[(ids_np < 0) | (ids_np >= e)] == 0)
    oracle = O.fused_moe_fp64(a.numpy(), wp, ws, 0.75, np.ones(e), w.numpy(), ids_np, True,
                              compute_dtype="f32")
    assert_parity(out, oracle, what=f"fp32 k={k} m={m} n={n}")


# C in FP32 with bf16 activations: routing blocks of 32 / 64 / 128 rows run
# the W4A16 prefill tiles storing FP32 (the bf16 MFMA's products of bf16 A
# and the E2M1 x 2^k weights are exact, summed in FP32); the same values as
# FP32 A run the FP32 MFMA, and so do 16-row blocks, where bf16 A is widened
# on the way in (bitwise the FP32-A result).  AITER's entry on caller
# metadata (an expert -1 block writes zeros, dropped routes stay untouched)
# and the soft op; both paths on the FP64 oracle and within FP32 summation
# noise of each other
@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
def test_fp32_c_bf16_activations_prefill_tiles(block_m):
    print(f"fp32 C, bf16 A, block {block_m}", flush=True)
    rng = np.random.default_rng(700 + block_m)
    m, e, top_k, k, n = 384, 16, 4, 1024, 200
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(701 + block_m, (m, k))
    w, ids = _route_with_dropped(m, e, top_k, 702 + block_m, 9)
    ids_np = ids.numpy()
    srt, eid, npp = O.make_routing(ids_np, block_m=block_m, num_experts=e)
    eid = eid.copy()
    eid[eid == 5] = -1

    def aiter(act):
        C = torch.full((m, top_k, n), 3.0, dtype=torch.float32, device="cuda")
        mx.fused_moe_mxfp4(cuda(act), cuda(wp), C, torch.full((1,), 0.75, device="cuda"),
                           torch.ones(e, device="cuda"), None, cuda(ws), cuda(w), cuda(ids),
                           cuda(srt), cuda(eid), cuda(npp), True, top_k, False, False,
                           {"BLOCK_SIZE_M": block_m}, torch.float32)
        return C.cpu().numpy()

    got, ref32 = aiter(a), aiter(a.float())
    oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.75, np.ones(e), w.numpy(), ids_np,
                              True, compute_dtype="f32")
    dropped = (ids_np < 0) | (ids_np >= e)
    assert np.all(got[dropped] == 3.0) and np.all(got[ids_np == 5] == 0)
    oracle[ids_np == 5] = 0.0
    oracle[dropped] = 3.0
    assert_parity(got, oracle, what=f"bf16 A, C fp32, block {block_m}")
    assert_parity(ref32, oracle, what=f"fp32 A, C fp32, block {block_m}")
    scale = np.abs(oracle[~dropped]).max()
    assert np.abs(got - ref32).max() <= 1e-5 * scale
    if block_m == 16:
        assert np.array_equal(got, ref32)
    if block_m == 32:
        # the soft op (device routing) on the same inputs
        soft = _run(a, None, wp, ws, ids, w, torch.float32, True).cpu().numpy()
        assert np.all(soft[dropped] == 0)
        soft_oracle = O.fused_moe_fp64(a.float().numpy(), wp, ws, 0.75, np.ones(e), w.numpy(),
                                       ids_np, True, compute_dtype="f32")
        soft_oracle[dropped] = 0.0
        assert_parity(soft, soft_oracle, what="soft op, bf16 A, C fp32")


@pytest.mark.parametrize("ids_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("m,top_k", [(1, 8), (3, 4), (8, 8)])
def test_soft_op_direct_routing_writes_dropped_rows(m, top_k, ids_dtype):
    # <= 64 routes on the W4A16 path: the decode kernels route from the ids
    # themselves (no routing launch); a route with an id outside [0, E) gets
    # a row of zeros from its own workgroup
    e, k, n = 32, 512, 96
    rng = np.random.default_rng(m * 10 + top_k)
    wp, ws = rand_mxfp4(rng, (e, n), k)
    a = rand_act(m + 90, (m, k))
    w, ids = _route_with_dropped(m, e, top_k, 7000 + m, max(1, m * top_k // 4))
    ids = ids.to(ids_dtype)
    C = _run(a, None, wp, ws, ids, w, torch.bfloat16, True)
    out = C.float().cpu().numpy()
    assert not np.isnan(out).any(), "a row of C was left unwritten"
    ids_np = ids.numpy().astype(np.int64)
    bad = (ids_np < 0) | (ids_np >= e)
    assert bad.any() and np.all(out[bad] == 0)
    oracle = O.fused_moe_fp64(O.round_to_dtype(a.float().numpy(), "bf16"), wp, ws, 0.75,
                              np.ones(e), w.numpy(), ids_np, True, compute_dtype="bf16")
    assert_parity(out, oracle, what=f"direct m={m} top_k={top_k} {ids_dtype}")
