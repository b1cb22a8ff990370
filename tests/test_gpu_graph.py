"""GPU: the operators inside a captured HIP graph.  The library synchronises
nothing and records no memset (only kernels), so the router, the MoE layer
and the dense linear can be captured once and replayed with new inputs
copied in place.  Every replay must equal eager calls on the same inputs
bitwise (the kernels are deterministic), with the program's own eager work
and synchronisations between replays."""

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
