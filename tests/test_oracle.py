"""Pins the CPU oracle (CPU only).

Each check is chosen so that a plausible mistake in the oracle -- a wrong
nibble order, a dropped or shifted scale, a sign error, a wrong rounding
rule, a transposed operand -- fails at least one of them:

* closed forms of OCP E2M1 / E8M0 and torch's own float8_e8m0fnu decode;
* the reference's only known-answer test (tests/test_moe_mxfp4_soft.py:81-92);
* two independent derivations of dequant (numpy ldexp vs C integer bit
  construction) over every (code, scale, dtype), and the torch restatement of
  soft:295-307;
* the committed golden fixtures;
* exact-rational characterisations of both quantizers (nearest with ties
  away / ties to even, amax rules) and brute force on tiny routing inputs;
* composition invariants of the safe path (test:95-111, test:270-285).
"""

from __future__ import annotations

import math
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import c_oracle, mxfp4_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def _all_pairs():
    codes = np.concatenate([np.arange(16), np.arange(16)]).astype(np.uint8)
    packed = np.tile(O.pack_codes(codes), (256, 1))
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    return packed, scales


# ---------------------------------------------------------------- formats

def test_e2m1_table_closed_form():
    # OCP E2M1: sign bit 3, exponent bits 2:1 (bias 1), mantissa bit 0;
    # exponent 0 is subnormal: 0.5 * m.
    for code in range(16):
        sign = -1.0 if code & 8 else 1.0
        e, m = (code >> 1) & 3, code & 1
        mag = 0.5 * m if e == 0 else (1 + 0.5 * m) * 2.0 ** (e - 1)
        v = O.E2M1_VALUES[code]
        assert v == sign * mag
        assert np.signbit(v) == bool(code & 8)


def test_e8m0_matches_torch_float8_e8m0fnu():
    s = np.arange(256, dtype=np.uint8)
    ours = O.e8m0_to_f32(s)
    theirs = torch.from_numpy(s.copy()).view(torch.float8_e8m0fnu).float().numpy()
    assert np.isnan(ours[255]) and np.isnan(theirs[255])
    assert np.array_equal(ours[:255].view(np.uint32), theirs[:255].view(np.uint32))
    assert ours[0] == np.float32(2.0 ** -127) and ours[254] == np.float32(2.0 ** 127)


def test_reference_known_answer_all_codes():
    # tests/test_moe_mxfp4_soft.py:81-92: codes 0..15 at scale 127 -> LUT, exact
    packed = np.array([[c | ((c + 1) << 4) for c in range(0, 16, 2)] * 2], dtype=np.uint8)
    scales = np.full((1, 1), 127, dtype=np.uint8)
    got = O.dequant_f32(packed, scales)
    want = np.array([O.E2M1_VALUES * 2], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_dequant_two_derivations_agree(dtype):
    packed, scales = _all_pairs()
    assert np.array_equal(O.dequant_bits(packed, scales, dtype),
                          c_oracle.dequant_bits(packed, scales, dtype))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_dequant_golden_table(dtype):
    g = np.load(os.path.join(GOLDEN, "dequant_table.npz"))
    assert np.array_equal(O.dequant_bits(g["packed"], g["scales"], dtype), g[dtype])


@pytest.mark.parametrize("dtype,tdt", [("f32", torch.float32), ("bf16", torch.bfloat16),
                                       ("f16", torch.float16)])
def test_dequant_torch_restatement_bitwise(dtype, tdt):
    packed, scales = _all_pairs()
    t = O.dequant_safe(packed, scales, tdt)
    bits = t.view(torch.int32 if dtype == "f32" else torch.int16).numpy()
    ours = O.dequant_bits(packed, scales, dtype)
    nan = np.isnan(O.dequant_f32(packed, scales))
    assert np.array_equal(bits.view(ours.dtype)[~nan], ours[~nan])
    assert np.all(np.isnan(t.float().numpy()[nan]))


def test_dequant_special_cases():
    packed, scales = _all_pairs()
    f = O.dequant_f32(packed, scales)  # [256 scales, 32]
    bits = f.view(np.uint32)
    # -0 keeps its sign bit (code 8) for every finite scale
    assert np.all(bits[:255, 8] == 0x80000000) and np.all(bits[:255, 0] == 0)
    # s = 0: subnormal products, e.g. 0.5 * 2^-127 = 2^-128, 1.5 * 2^-127
    assert f[0, 1] == np.float32(2.0 ** -128) and f[0, 3] == np.float32(1.5 * 2.0 ** -127)
    # s = 253: |v| >= 4 overflows; s = 254: |v| >= 2 overflows; 1.5*2^127 is finite
    assert np.all(np.isinf(f[253, [6, 7, 14, 15]])) and np.isfinite(f[253, 5])
    assert np.all(np.isinf(f[254, [4, 5, 6, 7]])) and f[254, 3] == np.float32(1.5 * 2.0 ** 127)
    assert np.all(f[254, [12, 13]] < 0)
    # s = 255: NaN for every code, including +-0
    assert np.all(np.isnan(f[255]))
    # exact otherwise: value * 2^(s-127) as a rational
    for s in (1, 60, 127, 200, 252):
        for c in range(16):
            assert Fraction(float(f[s, c])) == Fraction(O.E2M1_VALUES[c]) * Fraction(2) ** (s - 127)


def test_dequant_f16_rounding_closed_forms():
    packed, scales = _all_pairs()
    h = O.dequant_bits(packed, scales, "f16").view(np.float16)
    assert np.isinf(h[141, 7]) and h[140, 7] == np.float16(49152.0)  # 6*2^14 > 65504
    assert np.all(np.isinf(h[144, [1, 2, 3, 4, 5, 6, 7]]))            # 0.5*2^17 = 65536
    assert h[103, 1] == 0.0 and h[103, 2] == np.float16(2.0 ** -24)   # tie at 2^-25 -> even 0
    assert h[103, 3] == np.float16(2.0 ** -23)                        # 1.5 ulp tie -> even 2
    assert h[102, 3] == np.float16(2.0 ** -24)                        # 0.75 ulp -> 1 ulp
    assert h[101, 3] == 0.0                                           # 0.375 ulp -> 0


def test_rounding_helpers_match_torch():
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(20000) * np.exp2(rng.integers(-140, 120, 20000))).astype(np.float32)
    v[:4] = [np.inf, -np.inf, 0.0, -0.0]
    tb = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(v), tb)
    th = torch.from_numpy(v).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_f16_bits(v), th)


def test_dequant_validation_order():
    with pytest.raises(TypeError, match="packed must be uint8"):
        O.check_dequant_args(np.zeros((1, 16), np.int8), np.zeros((1, 1), np.uint8))
    with pytest.raises(TypeError, match="block_scales must be uint8"):
        O.check_dequant_args(np.zeros((1, 16), np.uint8), np.zeros((1, 1), np.int8))
    with pytest.raises(ValueError, match="divisible by 32"):
        O.check_dequant_args(np.zeros((1, 8), np.uint8), np.zeros((1, 1), np.uint8))
    with pytest.raises(ValueError, match="leading dimensions"):
        O.check_dequant_args(np.zeros((2, 16), np.uint8), np.zeros((1, 1), np.uint8))
    with pytest.raises(ValueError, match="every 32"):
        O.check_dequant_args(np.zeros((1, 16), np.uint8), np.zeros((1, 2), np.uint8))


# ---------------------------------------------------------------- quantizers

_GRID = [Fraction(v) for v in (0, 0.5, 1, 1.5, 2, 3, 4, 6)]


def _nearest(q: Fraction, ties: str) -> int:
    mag = abs(q)
    if mag >= 6:
        return 7
    best = min(range(8), key=lambda i: abs(_GRID[i] - mag))
    d = abs(_GRID[best] - mag)
    tied = [i for i in range(8) if abs(_GRID[i] - mag) == d]
    if len(tied) > 1:
        best = max(tied) if ties == "away" else [i for i in tied if i % 2 == 0][0]
    return best


def _closed_form_quant(x: np.ndarray, mode: str):
    """Exact rational characterisation of both quantizers, block by block."""
    codes, scales = [], []
    for blk in x.reshape(-1, 32):
        amax = float(np.max(np.abs(blk)))
        if mode == "away":
            # test:37: amax rounded up to the next power of two iff its
            # mantissa fraction is >= 0.75, else down
            if amax == 0:
                e = -127
            else:
                m, ex = np.frexp(np.float32(amax))  # amax = m * 2^ex, m in [0.5, 1)
                fl = int(ex) - 1
                e = fl + (1 if (2 * m - 1) >= 0.75 else 0) - 2
        else:
            e = -127 if amax == 0 else int(np.floor(np.log2(np.float64(amax)))) - 2
        e = max(-127, min(127, e))
        scales.append((e + 127) & 0xFF)
        for v in blk:
            q = Fraction(float(v)) / Fraction(2) ** e
            c = _nearest(q, mode)
            codes.append(c | (8 if np.signbit(v) else 0))
    return np.array(codes, np.uint8).reshape(x.shape), np.array(scales, np.uint8)


@pytest.mark.parametrize("mode", ["away", "rne"])
def test_quantizer_closed_form(mode):
    rng = np.random.default_rng(11 if mode == "away" else 12)
    x = (rng.standard_normal((6, 64)) * np.exp2(rng.integers(-8, 8, (6, 1)))).astype(np.float32)
    x[0, :16] = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 5.5, -0.25, -0.75, -1.25,
                            -1.75, -2.5, -3.5, -5.0, -0.01])
    x[1, :32] = 0.0
    x[2, 5] = 6.0 * 0.999
    fn = O.quant_mxfp4_ties_away if mode == "away" else O.quant_mxfp4_rne
    packed, scales = fn(x)
    codes, sc = _closed_form_quant(x, mode)
    assert np.array_equal(O.unpack_codes(packed), codes)
    assert np.array_equal(scales.reshape(-1), sc)
    cmode = "ties_away" if mode == "away" else "rne"
    cp, cs = c_oracle.quant(x, cmode)
    assert np.array_equal(cp, packed) and np.array_equal(cs, scales)


def test_quantizer_tie_cases():
    # scale 2^0 (amax 5 -> E = 0) so q = x exactly
    x = np.zeros((1, 32), np.float32)
    x[0, :4] = [0.25, 1.25, 2.5, 5.0]
    pa, sa = O.quant_mxfp4_ties_away(x)
    pr, sr = O.quant_mxfp4_rne(x)
    assert sa[0, 0] == 127 and sr[0, 0] == 127
    va = O.dequant_f32(pa, sa)[0, :4]
    vr = O.dequant_f32(pr, sr)[0, :4]
    assert list(va) == [0.5, 1.5, 3.0, 6.0]   # ties away from zero
    assert list(vr) == [0.0, 1.0, 2.0, 4.0]   # ties to even


@pytest.mark.parametrize("fn", [O.quant_mxfp4_ties_away, O.quant_mxfp4_rne])
def test_quantizer_roundtrip_representable(fn):
    # values on the E2M1 grid times 2^e with amax 6 * 2^e round-trip exactly
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 16, (8, 64)).astype(np.uint8)
    codes[:, ::32] = 7  # amax = 6 * 2^e in every block
    e = rng.integers(-20, 20, (8, 2))
    vals = np.array(O.E2M1_VALUES, np.float32)[codes] * np.repeat(np.exp2(e), 32, axis=1)
    p, s = fn(vals.astype(np.float32))
    assert np.array_equal(O.dequant_f32(p, s), vals.astype(np.float32))


def test_quantizer_golden():
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    pa, sa = O.quant_mxfp4_ties_away(g["quant_x"])
    pr, sr = O.quant_mxfp4_rne(g["quant_x"])
    assert np.array_equal(pa, g["quant_ta_p"]) and np.array_equal(sa, g["quant_ta_s"])
    assert np.array_equal(pr, g["quant_rne_p"]) and np.array_equal(sr, g["quant_rne_s"])


# ---------------------------------------------------------------- routing

def _check_routing_format(ids, sorted_ids, expert_ids, npp, block_m, num_experts):
    flat = ids.reshape(-1)
    n = flat.size
    assert npp[0] == sorted_ids.size and sorted_ids.size == expert_ids.size * block_m
    assert np.all(np.diff(expert_ids) >= 0)  # ascending experts
    seen = []
    for b, e in enumerate(expert_ids):
        blk = sorted_ids[b * block_m:(b + 1) * block_m]
        real = blk[blk < n]
        assert np.all(blk[len(real):] == n)        # padding only at the tail
        assert np.all(flat[real] == e)             # one expert per block
        seen.extend(real.tolist())
    valid = [r for r in range(n) if 0 <= flat[r] < num_experts]
    assert sorted(seen) == valid                   # every valid route exactly once
    by_expert = {}
    for r in seen:
        by_expert.setdefault(int(flat[r]), []).append(r)
    assert all(v == sorted(v) for v in by_expert.values())  # ascending inside an expert


@pytest.mark.parametrize("block_m", [16, 64])
def test_routing_format_and_c_agree(block_m):
    rng = np.random.default_rng(block_m)
    ids = rng.integers(-1, 9, (37, 4))
    r_np = O.make_routing(ids, block_m=block_m, num_experts=8)
    r_c = c_oracle.make_routing(ids, 8, block_m)
    for a, b in zip(r_np, r_c):
        assert np.array_equal(a, b)
    _check_routing_format(ids, *r_np, block_m, 8)


def test_routing_golden_and_reference_sentinel():
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    srt, exp_, npp = O.make_routing(g["moe_ids"], block_m=16, num_experts=4)
    assert np.array_equal(srt, g["route_sorted"]) and np.array_equal(exp_, g["route_experts"])
    assert npp[0] == g["route_npp"][0]
    # vllm:119-146 keeps every distinct id; with num_experts=None so does the oracle
    srt2, exp2, _ = O.make_routing(np.array([[0, 5]]), block_m=16)
    assert list(exp2) == [0, 5] and srt2[0] == 0 and srt2[16] == 1 and srt2[1] == 2


# ---------------------------------------------------------------- GEMM oracles

def test_linear_fp64_brute_force_and_golden():
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    x, w, s = g["lin_x"], g["lin_w"], g["lin_s"]
    y = O.linear_fp64(x, w, s)
    assert np.array_equal(y, g["lin_y"])
    wv = O.dequant_f32(w, s).astype(np.float64)
    i, j = 3, 17
    brute = sum(float(x[i, k]) * float(wv[j, k]) for k in range(x.shape[1]))
    assert abs(brute - y[i, j]) <= 1e-12 * max(1.0, abs(brute))
    # a transposed / nibble-swapped weight is caught
    swapped = ((w >> 4) | (w << 4)).astype(np.uint8)
    assert O.parity_errors(O.linear_fp64(x, swapped, s), y)["norm_rel"] > 0.1


def test_linear_safe_composition_and_tolerance():
    # test:95-111: the safe path equals x @ dequant(W).T bitwise
    rng = np.random.default_rng(20260811)
    x = torch.randn(8, 256, generator=torch.Generator().manual_seed(20260811)).to(torch.bfloat16)
    w = rng.integers(0, 256, (64, 128), dtype=np.uint8)
    s = rng.integers(120, 129, (64, 8), dtype=np.uint8)
    got = O.linear_safe(x, torch.from_numpy(w), torch.from_numpy(s))
    want = x @ O.dequant_safe(w, s, torch.bfloat16).T
    assert torch.equal(got, want)
    err = O.parity_errors(got.float().numpy(), O.linear_fp64(x.float().numpy(), w, s))
    assert err["elem_rel"] <= O.ELEM_TOL and err["norm_rel"] <= O.NORM_TOL


def test_moe_oracles_agree_with_gemv_loop():
    # test:216-285 in miniature: the safe per-expert loop vs a per-(token, slot)
    # GEMV loop, and the FP64 oracle vs both
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    a = torch.from_numpy(g["moe_a"]).to(torch.bfloat16)
    B = torch.from_numpy(g["moe_b"])
    Bs = torch.from_numpy(g["moe_bs"])
    ids = torch.from_numpy(g["moe_ids"])
    w = torch.from_numpy(g["moe_w"])
    bsc = torch.from_numpy(g["moe_bscale"])
    C = torch.empty(6, 2, 40, dtype=torch.bfloat16)
    O.fused_moe_safe(a, B, C, torch.tensor([0.75]), bsc, None, Bs, w, ids, True)
    assert torch.all(C[5, 1] == 0)  # out-of-range id: slot stays zero
    loop = torch.zeros_like(C)
    for t in range(6):
        for s_ in range(2):
            e = int(ids[t, s_])
            if not 0 <= e < 4:
                continue
            wt = O.dequant_safe(g["moe_b"][e], g["moe_bs"][e], torch.bfloat16)
            v = torch.matmul(a[t], wt.T) * 0.75 * bsc[e] * w[t, s_]
            loop[t, s_] = v.to(torch.bfloat16)
    torch.testing.assert_close(C, loop, rtol=1e-2, atol=1e-2)
    assert np.array_equal(
        O.fused_moe_fp64(g["moe_a"], g["moe_b"], g["moe_bs"], 0.75, g["moe_bscale"], g["moe_w"],
                         g["moe_ids"], True), g["moe_c"])
    err = O.parity_errors(C.float().numpy(), g["moe_c"])
    assert err["elem_rel"] <= 2e-2 and err["norm_rel"] <= 5e-3


def test_moe_layer_oracles_agree():
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    y64 = O.moe_layer_fp64(g["layer_x"], g["layer_w13"], g["layer_s13"], g["layer_w2"],
                           g["layer_s2"], g["layer_w"], g["layer_ids"])
    assert np.array_equal(y64, g["layer_y"])
    t = lambda k: torch.from_numpy(g[k])  # noqa: E731
    y = O.moe_layer_safe(t("layer_x").to(torch.bfloat16), t("layer_w13"), t("layer_s13"),
                         t("layer_w2"), t("layer_s2"), t("layer_w"), t("layer_ids"))
    err = O.parity_errors(y.float().numpy(), y64)
    assert err["norm_rel"] <= 1e-2
    # dropping the route weight is caught
    bad = O.moe_layer_fp64(g["layer_x"], g["layer_w13"], g["layer_s13"], g["layer_w2"],
                           g["layer_s2"], np.ones_like(g["layer_w"]), g["layer_ids"])
    assert O.parity_errors(bad, y64)["norm_rel"] > 0.1


def test_parity_metric_floor():
    o = np.array([1.0, -2.0, 1e-9, 3.0])
    e = O.parity_errors(o + np.array([0, 0, 1e-6, 0]), o)
    # the 1e-6 miss at a ~0 entry is judged against 1e-3 * rms, not 1e-9
    assert e["elem_rel"] < 1e-2
    assert O.parity_errors(o * 1.01, o)["elem_rel"] == pytest.approx(0.01)


def test_router_oracle_pinned():
    # test:242-244 through torch itself (float64 softmax, torch.topk), then
    # the renormalisation; closed forms at two experts; ties by definition
    import torch
    rng = np.random.default_rng(242)
    x = rng.standard_normal((64, 128))
    p = torch.softmax(torch.from_numpy(x), dim=-1)
    tw, ti = torch.topk(p, k=8, dim=-1)
    w, ids = O.route_topk_fp64(x, 8, renormalize=False)
    assert np.array_equal(ids, ti.numpy())
    np.testing.assert_allclose(w, tw.numpy(), rtol=1e-13, atol=0)
    wr, idr = O.route_topk_fp64(x, 8, renormalize=True)
    assert np.array_equal(idr, ids)
    np.testing.assert_allclose(wr, (tw / tw.sum(-1, keepdim=True)).numpy(), rtol=1e-13, atol=0)
    # two experts: the larger logit wins with weight sigmoid(l0 - l1)
    w2, i2 = O.route_topk_fp64(np.array([[0.7, -0.4]]), 1, renormalize=False)
    assert i2[0, 0] == 0 and abs(w2[0, 0] - 1.0 / (1.0 + math.exp(-1.1))) < 1e-15
    w3, _ = O.route_topk_fp64(np.array([[0.7, -0.4]]), 1, renormalize=True)
    assert w3[0, 0] == 1.0
    # ties: descending logit, then ascending expert id (brute force)
    t = np.array([[1.0, 3.0, 3.0, 0.0, 3.0, 1.0]])
    wt, it = O.route_topk_fp64(t, 4, renormalize=True)
    brute = sorted(range(6), key=lambda e: (-t[0, e], e))[:4]
    assert it[0].tolist() == brute == [1, 2, 4, 0]
    assert wt[0, 0] == wt[0, 1] == wt[0, 2] and abs(wt.sum() - 1.0) < 1e-15


def test_moe_oracle_predequantized_path_and_ieee_specials():
    # the b_values / w13_values / w2_values hooks give the default results
    # bit for bit; with +-inf weights (E8M0 254) the oracle's library matmul
    # gives the IEEE outcome of the exact product sum (0 * inf and
    # inf - inf are NaN, a lone inf keeps its sign), checked against
    # products summed elementwise
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    args = (g["layer_x"], g["layer_w13"], g["layer_s13"], g["layer_w2"], g["layer_s2"],
            g["layer_w"], g["layer_ids"])
    v13 = lambda e: O.dequant_values(g["layer_w13"][e], g["layer_s13"][e], "bf16")  # noqa: E731
    v2 = lambda e: O.dequant_values(g["layer_w2"][e], g["layer_s2"][e], "bf16")  # noqa: E731
    assert np.array_equal(O.moe_layer_fp64(*args, w13_values=v13, w2_values=v2), g["layer_y"])
    rng = np.random.default_rng(254)
    k, n, m = 64, 24, 5
    codes = np.zeros((2, n, k), dtype=np.uint8)
    codes[:, :, 7] = 4          # +inf at s = 254 in every row, block 0 ...
    codes[:, :12, 40] = 12      # ... -inf in block 1 of half the rows
    codes[:, 12:, 33] = 1       # ... the finite 2^126 in the other half
    scales = np.full((2, n, k // 32), 254, dtype=np.uint8)
    packed = O.pack_codes(codes)
    a = rng.standard_normal((m, k))
    a[0, 7] = 0.0               # 0 * inf
    ids = np.array([[0, 1]] * m)
    w = np.ones((m, 2))
    got = O.fused_moe_fp64(a, packed, scales, 1.0, np.ones(2), w, ids, False)
    for e in range(2):
        wv = O.dequant_values(packed[e], scales[e], "bf16")
        brute = (a[:, None, :] * wv[None, :, :]).sum(-1)
        np.testing.assert_array_equal(got[:, e], brute)
    assert np.all(np.isnan(got[0]))  # 0 * inf
    # rows with +inf and -inf: NaN exactly where the two activations agree in sign
    same = np.sign(a[1:, 7]) == np.sign(a[1:, 40])
    assert np.array_equal(np.isnan(got[1:, :, :12]), np.broadcast_to(same[:, None, None],
                                                                     (m - 1, 2, 12)))
    assert np.array_equal(got[1:, :, 12:], np.broadcast_to(
        (np.sign(a[1:, 7]) * np.inf)[:, None, None], (m - 1, 2, n - 12)))


def test_format_ulp_is_the_grid_spacing():
    # the gap to the next representable value, from the bit patterns
    rng = np.random.default_rng(7)
    b16 = rng.integers(0, 0x7F7F, 4000, dtype=np.uint16)  # finite positive bf16, below max
    v = O.bf16_bits_to_f32(b16).astype(np.float64)
    nxt = O.bf16_bits_to_f32(b16 + 1).astype(np.float64)
    np.testing.assert_array_equal(O.format_ulp(v, "bf16"), nxt - v)
    np.testing.assert_array_equal(O.format_ulp(-v, "bf16"), nxt - v)
    h = rng.integers(0, 0x7BFF, 4000, dtype=np.uint16).view(np.float16)
    np.testing.assert_array_equal(O.format_ulp(h, "f16"),
                                  np.nextafter(h, np.float16(np.inf)).astype(np.float64) - h)
    f = rng.integers(0, 0x7F7FFFFF, 4000, dtype=np.uint32).view(np.float32)
    np.testing.assert_array_equal(O.format_ulp(f, "f32"),
                                  np.nextafter(f, np.float32(np.inf)).astype(np.float64) - f)
    assert O.format_ulp(np.array([0.0]), "bf16")[0] == 2.0 ** -133
    assert O.format_ulp(np.array([np.nan, np.inf]), "bf16").tolist() == [0.0, 0.0]


@pytest.mark.parametrize("fmt,tdt", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_fp8_decode_matches_torch_on_every_byte(fmt, tdt):
    # the FP8 activation formats of aiter:11-20: every one of the 256 bytes
    # decoded from the bit fields equals torch's own float8 -> float32
    # conversion (NaN bytes: NaN-ness), plus a few values by hand
    codes = np.arange(256, dtype=np.uint8)
    ours = O.fp8_values(codes, fmt)
    theirs = torch.from_numpy(codes).view(tdt).float().numpy().astype(np.float64)
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    fin = ~np.isnan(ours)
    assert np.array_equal(ours[fin], theirs[fin])
    assert np.array_equal(np.signbit(ours[fin]), np.signbit(theirs[fin]))  # -0
    if fmt == "e4m3":
        assert O.fp8_values(np.array([0x7E, 0x01, 0x38, 0xB8]), fmt).tolist() == \
            [448.0, 2.0 ** -9, 1.0, -1.0]
        assert np.isnan(O.fp8_values(np.array([0x7F, 0xFF]), fmt)).all()
    else:
        assert O.fp8_values(np.array([0x7B, 0x01, 0x3C, 0x7C]), fmt).tolist() == \
            [57344.0, 2.0 ** -16, 1.0, np.inf]


def test_fp8_scaled_values_apply_the_block_scale():
    codes = np.full((2, 64), 0x38, dtype=np.uint8)  # e4m3 1.0
    scales = np.array([[127, 130], [0, 254]], dtype=np.uint8)
    v = O.fp8_scaled_values(codes, scales, "e4m3")
    assert np.array_equal(v[0, :32], np.ones(32)) and np.array_equal(v[0, 32:], np.full(32, 8.0))
    assert np.array_equal(v[1, :32], np.full(32, 2.0 ** -127))
    assert np.array_equal(v[1, 32:], np.full(32, 2.0 ** 127))
    assert np.array_equal(O.fp8_scaled_values(codes, None, "e4m3"), np.ones((2, 64)))
