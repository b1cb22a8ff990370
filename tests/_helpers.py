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


def _format_floor(o: np.ndarray, fmt: str) -> float:
    """Norm-wise error of the oracle itself correctly rounded to ``fmt``:
    what the output format alone costs, for any implementation."""
    fin = np.isfinite(o)
    return O.parity_errors(O.round_to_dtype(o[fin], fmt), o[fin])["norm_rel"]


def assert_parity(y, oracle, elem_tol=O.ELEM_TOL, norm_tol=O.NORM_TOL, ref=None, what="",
                  fmt=None):
    """Elementwise (denominator floor 1e-3 * rms) and norm-wise parity vs the
    FP64 oracle; with ``ref`` (the reference safe path's output on the same
    inputs) also that ours is no worse than it (10% slack for run-to-run
    BF16 rounding noise of two FP32-accumulated results).

    With ``fmt`` (the output dtype: "bf16" / "f16") the bars also admit what
    the output format itself imposes: an element may miss by up to one grid
    step of ``fmt`` at the oracle's value (subnormal outputs have a fixed,
    coarse step), and the norm-wise bar is no tighter than the error of the
    oracle correctly rounded to ``fmt`` (x1.1): structured inputs (the
    BASELINE edge sweep) can make that rounding alone exceed 2e-3."""
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else np.asarray(y)
    e = O.parity_errors(y, oracle)
    if fmt is None:
        assert e["elem_rel"] <= elem_tol, f"{what} elementwise {e['elem_rel']:.3e} > {elem_tol}"
    else:
        o = np.asarray(oracle, dtype=np.float64)
        floor = 1e-3 * np.sqrt(np.mean(o * o))
        diff = np.abs(y - o)
        bad = (diff / np.maximum(np.abs(o), floor) > elem_tol) & (diff > O.format_ulp(o, fmt))
        assert not bad.any(), (f"{what} {int(bad.sum())} elements beyond {elem_tol} and beyond "
                               f"one {fmt} step (max elementwise {e['elem_rel']:.3e})")
        norm_tol = max(norm_tol, 1.1 * _format_floor(o, fmt))
    assert e["norm_rel"] <= norm_tol, f"{what} norm-wise {e['norm_rel']:.3e} > {norm_tol:.3e}"
    if ref is not None:
        r = ref.float().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
        er = O.parity_errors(r, oracle)
        assert e["norm_rel"] <= 1.1 * er["norm_rel"] + 1e-7, (
            f"{what} worse than the reference safe path: {e['norm_rel']:.3e} vs {er['norm_rel']:.3e}")
    return e


def assert_layer_parity(y, oracle, ref, what="", routes=None, fmt="bf16"):
    """Parity for the MoE layer, whose reference composition rounds every
    route's down output to ``fmt`` before the top-k sum (vllm:253-265).  An
    FP32-accumulated route value sits within one ``fmt`` step of the FP64
    oracle's rounded one, but where it lands on the other side of a
    rounding boundary the token's sum moves by that step -- which, where
    routes cancel, exceeds 1e-2 of the sum for the reference itself.

    Bars: norm-wise <= 2e-3 (or, where the output format alone costs more,
    no worse than the oracle correctly rounded to ``fmt``, x1.1) and no
    worse than the reference safe path (x1.1; below a tenth of 2e-3 both
    sit at the rounding-flip noise of the same rounding points and this leg
    is not applied); elementwise <= 1e-2 for all but 1e-3 of the elements,
    and every element within 1e-2, or within one ``fmt`` step per route
    value (``routes``: the oracle's rounded per-route outputs
    [M, top_k, H]) plus one of the output, or no further from the oracle
    than the reference plus that budget (a gate / up / h value one step
    apart moves a route by more than its own step, for the reference as
    for us).  Without ``routes``, elementwise no worse than the reference."""
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else np.asarray(y)
    r = ref.float().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
    e = O.parity_errors(y, oracle)
    er = O.parity_errors(r, oracle)
    o = np.asarray(oracle, dtype=np.float64)
    floor = 1e-3 * np.sqrt(np.mean(o * o))
    diff = np.abs(y - o)
    rel = diff / np.maximum(np.abs(o), floor)
    frac = float(np.mean(rel > O.ELEM_TOL))
    if routes is not None:
        budget = O.format_ulp(routes, fmt).sum(axis=1) + O.format_ulp(o, fmt)
        bad = (rel > O.ELEM_TOL) & (diff > budget) & (diff > np.abs(r - o) + budget)
        assert not bad.any(), (
            f"{what} {int(bad.sum())} elements beyond {O.ELEM_TOL} and beyond one {fmt} step per "
            f"route (max elementwise {e['elem_rel']:.3e})")
    else:
        assert e["elem_rel"] <= max(O.ELEM_TOL, er["elem_rel"]), (
            f"{what} elementwise {e['elem_rel']:.3e} > reference {er['elem_rel']:.3e}")
    norm_tol = max(O.NORM_TOL, 1.1 * _format_floor(o, fmt))
    assert e["norm_rel"] <= norm_tol, f"{what} norm-wise {e['norm_rel']:.3e} > {norm_tol:.3e}"
    assert frac <= 1e-3, f"{what} {frac:.2e} of elements beyond {O.ELEM_TOL}"
    assert e["norm_rel"] <= max(er["norm_rel"] * 1.1 + 1e-7, 0.1 * O.NORM_TOL), (
        f"{what} worse than the reference: {e['norm_rel']:.3e} vs {er['norm_rel']:.3e}")
    return e, er


def dequant_device(packed: np.ndarray, scales: np.ndarray, dt: str = "bf16") -> torch.Tensor:
    """The exact dequantized weights (the oracle's bits) as a device tensor."""
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    bits = O.dequant_bits(packed, scales, dt)
    view = np.int32 if dt == "f32" else np.int16
    return torch.from_numpy(bits.view(view)).view(tdt).cuda()


def safe_linear_device(x: torch.Tensor, packed: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """soft:371-373 on the device: exact dequant (oracle bits), then the
    library GEMM in x's dtype (FP32 accumulation inside it)."""
    dt = "bf16" if x.dtype == torch.bfloat16 else "f16"
    w = dequant_device(packed, scales, dt)
    return torch.matmul(x.reshape(-1, w.shape[1]), w.T)


def fp32_gemm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b.T in FP32 on the device from operands exact in FP32 (bf16 /
    fp16 values), with TF32-style reduced precision switched off: an
    FP32-accumulated oracle for whole outputs at sizes the FP64 oracle
    cannot cover in seconds (its error, ~1e-6 relative, is pinned against
    the FP64 oracle on sampled rows by each test that uses it)."""
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        return torch.matmul(a.float(), b.float().T)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev


def assert_rows_parity(y: torch.Tensor, o: torch.Tensor, ref: torch.Tensor | None = None,
                       what: str = "", row_block: int = 1, fmt: torch.dtype | None = None):
    """Whole-output parity on the device.  Elementwise relative error <=
    ELEM_TOL with the denominator floored at 1e-3 * rms of the whole output;
    norm-wise <= NORM_TOL for every block of ``row_block`` rows (1: every
    row), so a wrong tile anywhere fails; with ``ref`` (the reference safe
    path on the same inputs) every block must also be no worse than it
    (10% slack for bf16 rounding noise).  With ``fmt`` (the output dtype) a
    block's norm-wise bar is no tighter than 1.1x the error of ``o``
    correctly rounded to ``fmt``: a short row (a few hundred outputs) can
    exceed 2e-3 from the output rounding alone."""
    y2 = y.reshape(y.shape[0], -1).double()
    o2 = o.reshape(o.shape[0], -1).double()
    rms = o2.square().mean().sqrt().item()
    floor = max(1e-3 * rms, 1e-300)
    elem = ((y2 - o2).abs() / o2.abs().clamp(min=floor)).max().item()
    assert elem <= O.ELEM_TOL, f"{what} elementwise {elem:.3e}"
    rows = y2.shape[0]
    nb = (rows + row_block - 1) // row_block
    pad = nb * row_block - rows

    def block_norm(t):
        t = torch.nn.functional.pad(t, (0, 0, 0, pad)) if pad else t
        return t.reshape(nb, -1).norm(dim=1)

    on = block_norm(o2)
    err = block_norm(y2 - o2) / on.clamp(min=1e-300)
    bar = torch.full_like(err, O.NORM_TOL)
    if fmt is not None:
        floor = block_norm(o.reshape(o.shape[0], -1).to(fmt).double() - o2) / on.clamp(min=1e-300)
        bar = torch.maximum(bar, 1.1 * floor)
    worst = (err / bar).max().item()
    assert worst <= 1.0, (
        f"{what} norm-wise {err[(err / bar).argmax()].item():.3e} (bar "
        f"{bar[(err / bar).argmax()].item():.3e}) in block {int((err / bar).argmax())} of "
        f"{row_block} rows")
    worst = err.max().item()
    if ref is not None:
        r2 = ref.reshape(ref.shape[0], -1).double()
        rerr = block_norm(r2 - o2) / on.clamp(min=1e-300)
        bad = err > 1.1 * rerr + 1e-7
        assert not bool(bad.any()), (
            f"{what} worse than the reference safe path in {int(bad.sum())} blocks, e.g. "
            f"{err[bad][0].item():.3e} vs {rerr[bad][0].item():.3e}")
    return elem, worst


def moe_layer_device(x: torch.Tensor, w13d: torch.Tensor, w2d: torch.Tensor,
                     topk_w: torch.Tensor, topk_ids: torch.Tensor, gemm: str,
                     return_routes: bool = False):
    """vllm:233-265 composed on the device over the safe op (soft:476-494
    with unit scales), from the exact dequantized experts w13d [E, 2I, H]
    and w2d [E, H, I] in x's dtype.  gemm="ref": the reference safe path
    itself -- each expert GEMM in x's dtype rounded to it, silu*mul on
    tensors of x's dtype (vllm:249-252), the route weight applied in FP32
    and rounded, the top-k sum of x's dtype (vllm:263-265).  gemm="f32": the
    same rounding points with FP32-accumulated GEMMs of the exact operands
    and a float64 top-k sum (an FP32 oracle for whole outputs).  With
    ``return_routes`` also the rounded per-route down outputs [M, top_k, H]."""
    m, top_k = topk_ids.shape
    num_experts, two_i, hidden = w13d.shape
    inter = two_i // 2
    dt = x.dtype
    ids = topk_ids.reshape(-1).long()
    tok = torch.arange(m * top_k, device=x.device) // top_k
    wts = topk_w.reshape(-1).float()
    gu = torch.zeros((m * top_k, two_i), dtype=dt, device=x.device)
    sels = [(e, (ids == e).nonzero().flatten()) for e in range(num_experts)]
    for e, sel in sels:
        if sel.numel() == 0:
            continue
        a = x[tok[sel]]
        gu[sel] = torch.matmul(a, w13d[e].T) if gemm == "ref" else fp32_gemm(a, w13d[e]).to(dt)
    h = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    d = torch.zeros((m * top_k, hidden), dtype=dt, device=x.device)
    for e, sel in sels:
        if sel.numel() == 0:
            continue
        v = torch.matmul(h[sel], w2d[e].T) if gemm == "ref" else fp32_gemm(h[sel], w2d[e])
        d[sel] = (v * wts[sel, None]).to(dt)
    d = d.reshape(m, top_k, hidden)
    y = d.sum(1) if gemm == "ref" else d.double().sum(1)
    return (y, d) if return_routes else y


def prepack_layout_np(packed: np.ndarray, scales: np.ndarray):
    """numpy statement of the prepacked weight layout (prepack.hip): for
    [E, rows, K/2] / [E, rows, K/32] uint8 weights, the nibble blocks
    [E, G, K/64, 64 lanes, 8 bytes] and scale operand high halves
    [E, G, K/64, 16, 2] (uint16).  Lane l of group g holds the bytes
    s*32 + j*16 + (l//16)*4 .. +3 (j = 0, 1) of row g*16 + l%16; scale (r, j)
    is (byte[2s + j] << 7) | 0x40 of row g*16 + r (the float
    (byte << 23) | 0x400000 without its zero low half); rows past the end
    are zero nibbles with byte 127."""
    e, rows, half_k = packed.shape
    k = half_k * 2
    g = (rows + 15) // 16
    nk = k // 64
    p = np.zeros((e, g * 16, half_k), np.uint8)
    p[:, :rows] = packed
    s = np.full((e, g * 16, k // 32), 127, np.uint8)
    s[:, :rows] = scales
    # [e, g, r, s, j, quad, 4 bytes] -> [e, g, s, lane = quad * 16 + r, j, 4]
    pv = p.reshape(e, g, 16, nk, 2, 4, 4).transpose(0, 1, 3, 5, 2, 4, 6)
    nib = pv.reshape(e, g, nk, 64, 8)
    ops = ((s.astype(np.uint16) << 7) | np.uint16(0x40)).astype(np.uint16)
    sc = ops.reshape(e, g, 16, nk, 2).transpose(0, 1, 3, 2, 4)
    return np.ascontiguousarray(nib), np.ascontiguousarray(sc)


def assert_layer_blocks(y, o, ref, routes, what, row_block=128):
    """The MoE layer bar (tests/_helpers.assert_layer_parity) on whole
    outputs, per block of ``row_block`` tokens: norm-wise <= NORM_TOL and no
    worse than the reference per block; every element within ELEM_TOL or
    within one bf16 step per route value (``routes``, the oracle's rounded
    per-route outputs) plus one of the output; <= ELEM_TOL on all but 1e-3
    of the elements."""
    y2, o2, r2 = y.double(), o.double(), ref.double()
    floor = 1e-3 * o2.square().mean().sqrt()
    diff = (y2 - o2).abs()
    rel = diff / o2.abs().clamp(min=floor)
    budget = (O.format_ulp(routes.double().cpu().numpy(), "bf16").sum(axis=1)
              + O.format_ulp(o2.cpu().numpy(), "bf16"))
    budget = torch.from_numpy(budget).to(diff.device)
    # an upstream rounding flip (gate, up or h one bf16 step apart) moves a
    # route by more than its own step; the reference composition takes such
    # flips too, so an element no further from the oracle than the
    # reference's (plus the budget) passes
    bad = (rel > O.ELEM_TOL) & (diff > budget) & (diff > (r2 - o2).abs() + budget)
    if bool(bad.any()):
        i, j = (int(v) for v in bad.nonzero()[0])
        raise AssertionError(
            f"{what} {int(bad.sum())} elements beyond {O.ELEM_TOL} and one bf16 step per route "
            f"(max {rel.max():.3e}); first at [{i}, {j}]: y {y2[i, j].item():.6g} oracle "
            f"{o2[i, j].item():.6g} reference {r2[i, j].item():.6g} budget {budget[i, j]:.3g} "
            f"routes {routes[i, :, j].double().cpu().numpy().tolist()}")
    frac = (rel > O.ELEM_TOL).double().mean().item()
    assert frac <= 1e-3, f"{what} {frac:.2e} of elements beyond {O.ELEM_TOL}"
    # blocks of row_block tokens, the last one partial (zero rows padded in
    # add nothing to its norms)
    nb = (y2.shape[0] + row_block - 1) // row_block
    pad = nb * row_block - y2.shape[0]

    def blocks(t):
        t = torch.nn.functional.pad(t, (0, 0, 0, pad))
        return t.reshape(nb, -1)
    on = blocks(o2).norm(dim=1)
    err = blocks(y2 - o2).norm(dim=1) / on
    rerr = blocks(r2 - o2).norm(dim=1) / on
    assert err.max() <= O.NORM_TOL, f"{what} norm-wise {err.max():.3e}"
    # below a tenth of the bar both sit at the rounding-flip noise of the
    # same rounding points, where "no worse" is a coin toss
    ok = (err <= 1.1 * rerr + 1e-7) | (err <= 0.1 * O.NORM_TOL)
    assert bool(ok.all()), (f"{what} worse than the reference in a block: "
                            f"{err[~ok][0].item():.3e} vs {rerr[~ok][0].item():.3e}")
