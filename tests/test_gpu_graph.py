"""GPU: the operators inside a captured HIP graph.  The library synchronises
nothing and records no memset (only kernels), so the router, the MoE layer,
the dense linear, the soft op and AITER's entry can be captured once and
replayed with new inputs copied in place.  Every replay must equal eager calls on the same inputs
bitwise (the kernels are deterministic), with the program's own eager work
and synchronisations between replays.  Calls on two streams at once and
from two host threads at once must equal sequential calls the same way."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxfp4_amd as mx

from _helpers import cuda, rand_act, rand_mxfp4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    rng = np.random.default_rng(20260815)
    w13, s13 = rand_mxfp4(rng, (128, 1536), 2048)
    w2, s2 = rand_mxfp4(rng, (128, 2048), 768)
    wl, sl = rand_mxfp4(rng, (1536,), 2048)
    return tuple(cuda(t) for t in (w13, s13, w2, s2, wl, sl))


def _logits(m, seed):
    return cuda(torch.randn((m, 128), generator=torch.Generator().manual_seed(seed)))


# m = 8: direct routing and the fused decode down projection; m = 512: the
# routing metadata, 64-row expert blocks and the prefill GEMMs
@pytest.mark.parametrize("m", [8, 512])
def test_graph_replays_equal_eager(m, weights):
    w13, s13, w2, s2, wl, sl = weights
    x = cuda(rand_act(30 + m, (m, 2048)))
    logits = _logits(m, 31 + m)

    def step():
        w, ids = mx.route_topk(logits, 8)
        y = mx.moe_layer(x, w13, s13, w2, s2, w, ids)
        z = mx.linear_mxfp4_soft(y, wl, sl)
        return w, ids, y, z

    step()  # warm-up outside the capture (allocator, library load)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            captured = step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    for rep in range(3):
        print(f"graph m={m} replay {rep}", flush=True)
        x.copy_(cuda(rand_act(40 + rep, (m, 2048))))
        logits.copy_(_logits(m, 50 + rep))
        graph.replay()
        torch.cuda.synchronize()
        eager = step()
        torch.cuda.synchronize()
        for name, a, b in zip(("weights", "ids", "layer", "linear"), captured, eager):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
        # eager work between replays that reuses freed memory
        torch.empty((m, 4096), device="cuda").fill_(7.0)
        torch.cuda.synchronize()


# the soft op (device routing + routed GEMM in one library call) on plain
# weights, on a registered prepacked copy, with C in FP32; and AITER's entry
# on metadata the device builds inside the same graph
@pytest.mark.parametrize("case", ["soft_bf16", "soft_registered", "soft_f32", "aiter"])
def test_graph_soft_op_replays_equal_eager(case, weights):
    from mxfp4_amd import prepack as P
    w13, s13 = weights[0], weights[1]
    if case == "soft_registered":
        w13, s13 = w13.clone(), s13.clone()
        P.register_prepacked(w13, s13)
    m, top_k, e, n = (64 if case == "soft_f32" else 512), 8, 128, 1536
    c_dtype = torch.float32 if case == "soft_f32" else torch.bfloat16
    x = cuda(rand_act(60, (m, 2048)))
    logits = _logits(m, 61)
    one, ones_e, empty = (torch.ones(1, device="cuda"), torch.ones(e, device="cuda"),
                          torch.empty(0, device="cuda"))

    def step():
        w, ids = mx.route_topk(logits, top_k)
        C = torch.full((m, top_k, n), 5.0, dtype=c_dtype, device="cuda")
        if case == "aiter":
            srt, eid, npp = mx.make_routing_device(ids, e, 64)
            mx.fused_moe_mxfp4(x, w13, C, one, ones_e, None, s13, w, ids, srt, eid, npp, True,
                               top_k, False, False, {"BLOCK_SIZE_M": 64}, c_dtype)
        else:
            mx.fused_moe_mxfp4_soft(x, w13, C, one, ones_e, None, s13, w, ids, empty, empty,
                                    empty, True, top_k, False, False)
        return C

    try:
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                captured = step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for rep in range(3):
            print(f"graph {case} replay {rep}", flush=True)
            x.copy_(cuda(rand_act(70 + rep, (m, 2048))))
            logits.copy_(_logits(m, 80 + rep))
            graph.replay()
            torch.cuda.synchronize()
            eager = step()
            torch.cuda.synchronize()
            assert torch.equal(captured, eager), f"replay {rep} differs from the eager call"
            assert torch.isfinite(captured).all()
            torch.empty((m, 4096), device="cuda").fill_(7.0)
            torch.cuda.synchronize()
    finally:
        P.unregister_prepacked(w13)


def test_concurrent_streams_and_host_threads_equal_sequential(weights):
    # The library keeps no state between calls but per-device constants and
    # a thread-local error message; workspaces come with each call.  The MoE
    # layer and the dense linear on two streams at once, then from two host
    # threads at once (each on its own stream), give the results of
    # sequential calls bit for bit.
    import threading
    w13, s13, w2, s2, wl, sl = weights
    cases = []
    for i, m in enumerate((8, 512)):
        x = cuda(rand_act(900 + i, (m, 2048)))
        tw, ti = mx.route_topk(_logits(m, 910 + i), 8)
        cases.append((x, tw, ti))

    def run(x, tw, ti):
        return (mx.moe_layer(x, w13, s13, w2, s2, tw, ti), mx.linear_mxfp4_soft(x, wl, sl))

    ref = [run(*c) for c in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        print(f"two streams, round {rep}", flush=True)
        outs = []
        for c, s in zip(cases, streams):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                outs.append(run(*c))
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o[0], r[0]) and torch.equal(o[1], r[1])
    results, errors = [None, None], []

    def worker(i):
        try:
            with torch.cuda.stream(streams[i]):
                got = [run(*cases[i]) for _ in range(10)]
            streams[i].synchronize()
            results[i] = got
        except Exception as e:  # reported by the main thread
            errors.append(e)

    print("two host threads", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for got, r in zip(results, ref):
        assert got is not None and len(got) == 10
        for o in got:
            assert torch.equal(o[0], r[0]) and torch.equal(o[1], r[1])
