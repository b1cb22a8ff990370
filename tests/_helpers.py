"""Shared helpers for the GPU parity tests: seeded synthetic inputs (the
BASELINE distributions: codes uniform over 0..15, E8M0 scales uniform over
120..128, activations ~N(0, 1) in bf16) and the parity assertion."""

from __future__ import annotations

import numpy as np
import torch

from oracle import mxfp4_oracle as O


def rand_mxfp4(rng: np.random.Generator, rows_shape, k, lo=120, hi=128):
    packed = rng.integers(0, 256, size=(*rows_shape, k // 2), dtype=np.uint8)
    scales = rng.integers(lo, hi + 1, size=(*rows_shape, k // 32), dtype=np.uint8)
    return packed, scales


def rand_act(seed: int, shape, dtype=torch.bfloat16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def cuda(a) -> torch.Tensor:
    if isinstance(a, np.ndarray):
        a = torch.from_numpy(np.ascontiguousarray(a))
    return a.to("cuda")


def assert_parity(y, oracle, elem_tol=O.ELEM_TOL, norm_tol=O.NORM_TOL, ref=None, what=""):
    """Elementwise (denominator floor 1e-3 * rms) and norm-wise parity vs the
    FP64 oracle; with ``ref`` (the reference safe path's output on the same
    inputs) also that ours is no worse than it (10% slack for run-to-run
    BF16 rounding noise of two FP32-accumulated results)."""
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else np.asarray(y)
    e = O.parity_errors(y, oracle)
    assert e["elem_rel"] <= elem_tol, f"{what} elementwise {e['elem_rel']:.3e} > {elem_tol}"
    assert e["norm_rel"] <= norm_tol, f"{what} norm-wise {e['norm_rel']:.3e} > {norm_tol}"
    if ref is not None:
        r = ref.float().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
        er = O.parity_errors(r, oracle)
        assert e["norm_rel"] <= 1.1 * er["norm_rel"] + 1e-7, (
            f"{what} worse than the reference safe path: {e['norm_rel']:.3e} vs {er['norm_rel']:.3e}")
    return e


def assert_layer_parity(y, oracle, ref, what=""):
    """Parity for the MoE layer, whose reference composition rounds every
    route's down output to bf16 before the top-k sum (vllm:255-265): where
    routes cancel, that rounding alone exceeds the 1e-2 elementwise bar for
    the reference itself.  Bars: norm-wise <= 2e-3 (strict); elementwise
    no worse than the reference safe path on the same inputs (and <= 1e-2
    for all but 1e-3 of the elements)."""
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else np.asarray(y)
    r = ref.float().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
    e = O.parity_errors(y, oracle)
    er = O.parity_errors(r, oracle)
    o = np.asarray(oracle, dtype=np.float64)
    floor = 1e-3 * np.sqrt(np.mean(o * o))
    frac = float(np.mean(np.abs(y - o) / np.maximum(np.abs(o), floor) > O.ELEM_TOL))
    assert e["norm_rel"] <= O.NORM_TOL, f"{what} norm-wise {e['norm_rel']:.3e}"
    assert e["elem_rel"] <= max(O.ELEM_TOL, er["elem_rel"]), (
        f"{what} elementwise {e['elem_rel']:.3e} > reference {er['elem_rel']:.3e}")
    assert frac <= 1e-3, f"{what} {frac:.2e} of elements beyond {O.ELEM_TOL}"
    assert e["norm_rel"] <= er["norm_rel"] * 1.1 + 1e-7, (
        f"{what} worse than the reference: {e['norm_rel']:.3e} vs {er['norm_rel']:.3e}")
    return e, er
