"""GPU: the prepacked weight copy (prepack_w4a16) is the layout its numpy
statement gives, and every prefill kernel that reads it (dense, split K,
routed SiLU*mul, routed with route weights, persistent) returns bitwise the
result of the checkpoint-layout call."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx

from _helpers import cuda, prepack_layout_np, rand_act, rand_mxfp4

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("e,rows,k", [(1, 200, 256), (3, 48, 128), (2, 5, 64)])
def test_prepack_bytes_match_layout(e, rows, k):
    rng = np.random.default_rng(e * 1000 + rows)
    packed, scales = rand_mxfp4(rng, (e, rows), k, lo=0, hi=255)
    pre = mx.prepack_w4a16(cuda(packed), cuda(scales))
    nib, sc = prepack_layout_np(packed, scales)
    assert (pre.experts, pre.rows, pre.k) == (e, rows, k)
    assert np.array_equal(pre.nibbles.cpu().numpy(), nib.reshape(-1))
    assert np.array_equal(pre.scales.cpu().numpy().view(np.uint16), sc.reshape(-1))
    # the 2D (dense) form is the one-expert case
    if e == 1:
        pre2 = mx.prepack_w4a16(cuda(packed[0]), cuda(scales[0]))
        assert torch.equal(pre2.nibbles, pre.nibbles)
        assert torch.equal(pre2.scales, pre.scales)


# (m, k, n): 128 x 320 tiles (the qkv headline), 128 x 256, 64 x 128,
# split K (o_proj at 370 tokens), 32 x 128, a ragged N (partial 16-row
# group), the skinny decode kernel (no prefill kernel: copy unused)
# (1536, 2048, 5120): dense 128 x 128 tiles, which read checkpoint weights in
# 2-stage weight-line groups
LINEAR_CASES = [(4096, 2048, 5120), (4096, 4096, 4096), (1024, 2048, 5120), (370, 4096, 2048),
                (256, 2048, 1536), (300, 512, 200), (8, 2048, 5120), (1536, 2048, 5120)]


@pytest.mark.parametrize("m,k,n", LINEAR_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_prepacked_bitwise(m, k, n, dtype):
    print(f"linear prepacked m={m} k={k} n={n} {dtype}", flush=True)
    rng = np.random.default_rng(m + k + n)
    packed, scales = rand_mxfp4(rng, (n,), k)
    w, s = cuda(packed), cuda(scales)
    x = cuda(rand_act(m + n, (m, k), dtype))
    bias = cuda(rand_act(n, (n,), dtype)) if n % 3 == 0 or n == 200 else None
    pre = mx.prepack_w4a16(w, s)
    plain = mx.linear_mxfp4_soft(x, w, s, bias)
    fast = mx.linear_mxfp4_soft(x, w, s, bias, prepacked=pre)
    torch.cuda.synchronize()
    assert torch.equal(plain, fast)
    assert torch.isfinite(plain).all()


@pytest.fixture(scope="module")
def moe_weights():
    e, h, i = 32, 2048, 768
    rng = np.random.default_rng(99)
    w13, s13 = rand_mxfp4(rng, (e, 2 * i), h)
    w2, s2 = rand_mxfp4(rng, (e, h), i)
    w13, s13, w2, s2 = cuda(w13), cuda(s13), cuda(w2), cuda(s2)
    return e, h, i, (w13, s13, w2, s2), (mx.prepack_w4a16(w13, s13), mx.prepack_w4a16(w2, s2))


# 4096 tokens: persistent routed kernel for gate_up, 128 x 320 for down;
# 512: one round of tiles; 64 (16 routes per expert over the 32 experts):
# 32-row blocks, whose checkpoint-layout tiles take 4-stage weight-line
# groups; 4: the direct-routed decode path (copies unused)
@pytest.mark.parametrize("m", [4096, 512, 64, 4])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_moe_layer_prepacked_bitwise(m, ids_dtype, moe_weights):
    print(f"moe layer prepacked m={m} ids={ids_dtype}", flush=True)
    e, h, _, (w13, s13, w2, s2), (p13, p2) = moe_weights
    top_k = 8
    g = torch.Generator().manual_seed(m)
    logits = torch.randn((m, e), generator=g)
    tw, ti = torch.topk(torch.softmax(logits, -1), top_k, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True)).cuda()
    ti = ti.to(ids_dtype).cuda()
    if m >= 512:
        ti[::97, 3] = -1  # a few slots routed off this device
    x = cuda(rand_act(m, (m, h)))
    plain = mx.moe_layer(x, w13, s13, w2, s2, tw, ti)
    fast = mx.moe_layer(x, w13, s13, w2, s2, tw, ti, prepacked13=p13, prepacked2=p2)
    torch.cuda.synchronize()
    assert torch.equal(plain, fast)
    assert torch.isfinite(plain).all()


def test_prepacked_copy_of_other_weights_is_refused(moe_weights):
    _, h, i, (w13, s13, w2, s2), (p13, p2) = moe_weights
    x = cuda(rand_act(1, (16, h)))
    tw = torch.full((16, 2), 0.5, device="cuda")
    ti = torch.zeros((16, 2), dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError, match="prepacked copy"):
        mx.moe_layer(x, w13, s13, w2, s2, tw, ti, prepacked13=p2, prepacked2=p13)
    with pytest.raises(ValueError, match="prepacked copy"):
        mx.linear_mxfp4_soft(x, w13[0], s13[0], prepacked=p13)


def test_stale_prepacked_copy_is_refused_and_the_hooks_refresh():
    # an in-place update of the weights makes the copy stale: the operator
    # refuses it, and the vLLM apply hook prepacks again before the call
    import types

    from torch.nn import Parameter

    from mxfp4_amd import vllm_adapter as va
    rng = np.random.default_rng(401)
    m, k, n = 512, 1024, 640  # a prefill grid (it reads the prepacked copy)
    w0, s0 = rand_mxfp4(rng, (n,), k)
    w1, _ = rand_mxfp4(rng, (n,), k)
    x = cuda(rand_act(402, (m, k)))
    w, s = cuda(w0), cuda(s0)
    pre = mx.prepack_w4a16(w, s)
    assert torch.equal(mx.linear_mxfp4_soft(x, w, s, prepacked=pre), mx.linear_mxfp4_soft(x, w, s))
    w.copy_(cuda(w1))
    with pytest.raises(ValueError, match="stale"):
        mx.linear_mxfp4_soft(x, w, s, prepacked=pre)
    pre = mx.prepack_w4a16(w, s)
    assert torch.equal(mx.linear_mxfp4_soft(x, w, s, prepacked=pre), mx.linear_mxfp4_soft(x, w, s))

    layer = types.SimpleNamespace(weight_packed=cuda(w0), weight_scale=cuda(s0))
    va._dense_process_weights_after_loading(None, layer)
    first = layer.mxfp4_prepacked
    y0 = va._dense_apply_weights(None, layer, x)
    assert torch.equal(y0, mx.linear_mxfp4_soft(x, cuda(w0), cuda(s0)))
    assert layer.mxfp4_prepacked is first
    with torch.no_grad():  # a weight sync writing the parameter in place
        layer.weight_packed.copy_(cuda(w1))
    y1 = va._dense_apply_weights(None, layer, x)
    assert layer.mxfp4_prepacked is not first
    assert torch.equal(y1, mx.linear_mxfp4_soft(x, cuda(w1), cuda(s0)))
    # a write through .data is not versioned: refresh_prepacked picks it up
    layer.weight_packed.data.copy_(cuda(w0))
    va.refresh_prepacked(layer)
    assert torch.equal(va._dense_apply_weights(None, layer, x), y0)
    assert isinstance(layer.weight_packed, Parameter)


def test_registered_dense_copy_serves_the_reference_signature():
    # linear_mxfp4_soft(x, packed, block_scales) -- soft:310's signature, no
    # copy argument -- reads a copy registered for those tensors: bitwise the
    # explicit-copy and the checkpoint results; stale after an in-place write
    from mxfp4_amd import prepack as P
    rng = np.random.default_rng(411)
    m, k, n = 1024, 2048, 1536
    wp, ws = rand_mxfp4(rng, (n,), k)
    w, s = cuda(wp), cuda(ws)
    x = cuda(rand_act(412, (m, k)))
    plain = mx.linear_mxfp4_soft(x, w, s)
    pre = P.register_prepacked(w, s)
    try:
        assert P.lookup_prepacked(w, s) is pre
        assert torch.equal(mx.linear_mxfp4_soft(x, w, s), plain)
        assert torch.equal(mx.linear_mxfp4_soft(x, w, s, prepacked=pre), plain)
        w2, _ = rand_mxfp4(rng, (n,), k)
        w.copy_(cuda(w2))
        after = mx.linear_mxfp4_soft(x, w, s)
        assert P.lookup_prepacked(w, s) is None
        assert not torch.equal(after, plain)
        P.register_prepacked(w, s)
        assert torch.equal(mx.linear_mxfp4_soft(x, w, s), after)
    finally:
        P.unregister_prepacked(w)


# AITER's entry with BLOCK_SIZE_M 32, E=128, top-8.  1024 tokens: more than
# ten 32 x 128 tiles per CU, so the checkpoint layout runs 32 x 256 tiles
# with 2-stage weight-line groups; 256 tokens (16 routes per expert): 32 x
# 128 tiles with 4-stage groups.  The registered prepacked copy runs its own
# 32-row tiles; bitwise the same C, and sampled rows on the FP64 oracle
@pytest.mark.parametrize("m", [1024, 256])
def test_routed_32x256_line_groups_bitwise(m):
    from mxfp4_amd import prepack as P
    from oracle import mxfp4_oracle as O
    from _helpers import assert_parity
    print(f"routed 32-row line groups m={m}", flush=True)
    rng = np.random.default_rng(m)
    e, top_k, k, n = 128, 8, 2048, 1536
    wp, ws = rand_mxfp4(rng, (e, n), k)
    B, Bs = cuda(wp), cuda(ws)
    a = cuda(rand_act(m + 1, (m, k)))
    g = torch.Generator().manual_seed(m + 2)
    tw, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
    tw, ids = tw.cuda(), ids.cuda()
    srt, eid, npp = mx.make_routing_device(ids, e, 32)
    one, ones_e = torch.ones(1, device="cuda"), torch.ones(e, device="cuda")

    def run():
        C = torch.full((m, top_k, n), 3.0, dtype=torch.bfloat16, device="cuda")
        mx.fused_moe_mxfp4(a, B, C, one, ones_e, None, Bs, tw, ids, srt, eid, npp, True, top_k,
                           False, False, {"BLOCK_SIZE_M": 32}, torch.bfloat16)
        return C
    plain = run()
    P.register_prepacked(B, Bs)
    try:
        fast = run()
    finally:
        P.unregister_prepacked(B)
    torch.cuda.synchronize()
    assert torch.equal(plain, fast)
    rows = np.arange(0, m, 53 if m > 512 else 13)
    oracle = O.fused_moe_fp64(a.float().cpu().numpy()[rows], wp, ws, 1.0, np.ones(e),
                              tw.cpu().numpy()[rows], ids.cpu().numpy()[rows], True)
    assert_parity(plain.float().cpu().numpy()[rows], oracle, what="routed 32 x 256 groups")


# 4-stage weight-line groups whose last group is half past the end of K
# (K / 64 = 6 or 10 stages: the last group's load covers two stages that do
# not exist, reading the next row's bytes or zeros past the buffer, which no
# stage uses) and a ragged last column tile (N = 200): 12.5 routes per
# expert on 32-row blocks take the 32 x 128 tiles with 4-stage groups
@pytest.mark.parametrize("k", [384, 640])
def test_routed_line_groups_partial_last_group(k):
    from mxfp4_amd import prepack as P
    from oracle import mxfp4_oracle as O
    from _helpers import assert_parity
    print(f"routed 4-stage line groups k={k}", flush=True)
    rng = np.random.default_rng(k)
    m, e, top_k, n = 100, 16, 2, 200
    wp, ws = rand_mxfp4(rng, (e, n), k)
    B, Bs = cuda(wp), cuda(ws)
    a = cuda(rand_act(k + 1, (m, k)))
    g = torch.Generator().manual_seed(k + 2)
    tw, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
    tw, ids = tw.cuda(), ids.cuda()
    srt, eid, npp = mx.make_routing_device(ids, e, 32)
    one, ones_e = torch.ones(1, device="cuda"), torch.ones(e, device="cuda")

    def run():
        C = torch.full((m, top_k, n), 3.0, dtype=torch.bfloat16, device="cuda")
        mx.fused_moe_mxfp4(a, B, C, one, ones_e, None, Bs, tw, ids, srt, eid, npp, True, top_k,
                           False, False, {"BLOCK_SIZE_M": 32}, torch.bfloat16)
        return C
    plain = run()
    P.register_prepacked(B, Bs)
    try:
        fast = run()
    finally:
        P.unregister_prepacked(B)
    torch.cuda.synchronize()
    assert torch.equal(plain, fast)
    oracle = O.fused_moe_fp64(a.float().cpu().numpy(), wp, ws, 1.0, np.ones(e),
                              tw.cpu().numpy(), ids.cpu().numpy(), True)
    assert_parity(plain.float().cpu().numpy(), oracle, what=f"4-stage groups k={k}")
