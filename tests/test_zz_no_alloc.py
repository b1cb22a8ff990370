"""The allocation-free MoE layer entry point, mxfp4_moe_layer_noalloc,
called through the C ABI: its output equals mxfp4_moe_layer's (the entry
point with a caller workspace; they share every kernel) bit for bit, on two
calls in a row, the second with fewer tokens; a size whose workspace
exceeds the fixed scratch is refused with ERR_VALUE before anything is
enqueued."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from mxfp4_amd import _lib

from _helpers import cuda, rand_act, rand_mxfp4

pytestmark = [pytest.mark.gpu]

E, H, I, TOPK = 128, 2048, 768, 8
SCRATCH_BYTES = 32 << 20  # MXFP4_NOALLOC_SCRATCH_BYTES


def _noalloc(x, w13, s13, w2, s2, w, ids, out):
    lib = _lib.load()
    m, hidden = x.shape
    return lib.mxfp4_moe_layer_noalloc(
        _lib.ptr(x), _lib.dtype_code(x.dtype), m, hidden, _lib.ptr(w13), _lib.ptr(s13),
        _lib.ptr(w2), _lib.ptr(s2), w13.shape[0], w13.shape[1] // 2, _lib.ptr(w), _lib.ptr(ids),
        _lib.dtype_code(ids.dtype), ids.shape[1], _lib.ptr(out), _lib.stream_of(x.device))


def _route(m, seed, ids_dtype):
    g = torch.Generator().manual_seed(seed)
    w, ids = torch.topk(torch.softmax(torch.randn((m, E), generator=g), -1), TOPK, dim=-1)
    return cuda((w / w.sum(-1, keepdim=True)).float()), cuda(ids.to(ids_dtype))


def _workspace_bytes(m):
    nb = ctypes.c_int64()
    _lib.check(_lib.load().mxfp4_moe_layer_workspace_size(m, TOPK, E, H, I, ctypes.byref(nb)))
    return nb.value


def test_noalloc_layer_equals_workspace_layer():
    rng = np.random.default_rng(7000)
    # E8M0 116..121 keep every fp16 intermediate of the second call finite
    w13, s13 = rand_mxfp4(rng, (E, 2 * I), H, lo=116, hi=121)
    w2, s2 = rand_mxfp4(rng, (E, H), I, lo=116, hi=121)
    w13, s13, w2, s2 = cuda(w13), cuda(s13), cuda(w2), cuda(s2)
    # 512 tokens (routing metadata, routed prefill tiles), then 8 (direct
    # routing, the fused down + top-k decode kernel) in fp16 with int32 ids:
    # the second call reuses the scratch the first one filled
    for m, dt, ids_dt in ((512, torch.bfloat16, torch.int64), (8, torch.float16, torch.int32)):
        assert 0 < _workspace_bytes(m) <= SCRATCH_BYTES
        x = cuda(rand_act(7001 + m, (m, H), dt))
        w, ids = _route(m, 7002 + m, ids_dt)
        ref = mx.moe_layer(x, w13, s13, w2, s2, w, ids)
        out = torch.full((m, H), 7.0, dtype=dt, device="cuda")
        rc = _noalloc(x, w13, s13, w2, s2, w, ids, out)
        assert rc == _lib.OK, _lib.load().mxfp4_last_error().decode()
        torch.cuda.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(out, ref), f"m={m}: differs from the workspace entry point"


def test_noalloc_layer_refuses_sizes_beyond_the_scratch():
    # the largest token count that fits, and the first that does not
    lo, hi = 1, 1 << 16
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if _workspace_bytes(mid) <= SCRATCH_BYTES else (lo, mid)
    assert lo >= 512
    m = hi
    x = torch.zeros((m, H), dtype=torch.bfloat16, device="cuda")
    w13 = torch.zeros((E, 2 * I, H // 2), dtype=torch.uint8, device="cuda")
    s13 = torch.zeros((E, 2 * I, H // 32), dtype=torch.uint8, device="cuda")
    w2 = torch.zeros((E, H, I // 2), dtype=torch.uint8, device="cuda")
    s2 = torch.zeros((E, H, I // 32), dtype=torch.uint8, device="cuda")
    w, ids = _route(m, 7003, torch.int64)
    out = torch.full((m, H), 7.0, dtype=torch.bfloat16, device="cuda")
    rc = _noalloc(x, w13, s13, w2, s2, w, ids, out)
    assert rc == _lib.ERR_VALUE
    assert "fixed scratch" in _lib.load().mxfp4_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was enqueued
