"""CPU restatement of the reference MXFP4 path, plus FP64 oracles.

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker; the product never
imports it.

Every function names the reference lines it restates (paths relative to the
reference repository ``lutianshu824/mxfp4-gfx936``):

* ``soft`` = ``src/aiter/ops/triton/moe_op_mxfp4_soft.py``
* ``vllm`` = ``integration/vllm/vllm_mxfp4_gfx936.py``
* ``aiter`` = ``integration/aiter/moe_op_mxfp4.py``
* ``test`` = ``tests/test_moe_mxfp4_soft.py``

Two kinds of function live here:

* *Restatements* (``*_safe``) reproduce the reference safe path operation by
  operation with the same rounding points (explicit dequant, then
  ``torch.matmul`` in the activation dtype with FP32 accumulation inside the
  library GEMM).  They run on CPU tensors and are the "reference itself" that
  the HIP path must be no worse than, and the CPU baseline in ``bench.py``.
* *FP64 oracles* (``*_fp64``) accumulate in float64 from the exact
  dequantized values.  The parity bars (elementwise relative error <= 1e-2
  with a denominator floor of 1e-3 * rms, norm-wise <= 2e-3) are measured
  against these.

Pinning (what makes this oracle trustworthy) is done in
``tests/test_oracle.py``: closed forms for E2M1/E8M0, the reference
known-answer test (test:81-92), torch's own ``float8_e8m0fnu`` decode, an
independent integer bit construction in ``mxfp4_oracle.c``, brute force over
every (code, scale) pair, and exact-rational checks of both quantizers.
"""

from __future__ import annotations

import math

import numpy as np

# soft:12-29 -- OCP E2M1 code -> value; bit 3 is the sign, so code 8 is -0.0.
E2M1_VALUES = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)
_E2M1_F32 = np.array(E2M1_VALUES, dtype=np.float32)

BLOCK = 32  # one E8M0 scale per 32 E2M1 values (soft:288-294)


# ----------------------------------------------------------------------------
# Element formats
# ----------------------------------------------------------------------------

def e8m0_to_f32(scales: np.ndarray) -> np.ndarray:
    """E8M0 byte -> float32 scale, restating soft:299-306.

    ``2 ** (s - 127)`` computed with ldexp (as the independent reference in
    vllm:82-85 does), so s = 0 gives the FP32 subnormal 2**-127; s = 255 is
    NaN (soft:302-306).
    """
    s = np.asarray(scales, dtype=np.uint8).astype(np.int32)
    out = np.ldexp(np.ones(s.shape, dtype=np.float32), s - 127).astype(np.float32)
    out[s == 255] = np.float32("nan")
    return out


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-to-nearest-even.

    Matches torch's CPU conversion: NaN becomes the canonical 0x7FC0 (the
    reference casts with ``.to(dtype)``, soft:307).
    """
    a = np.ascontiguousarray(values, dtype=np.float32)
    bits = a.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    rounded[np.isnan(a)] = 0x7FC0
    return rounded


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> float16 bit patterns (numpy's IEEE RNE conversion, with
    subnormals, overflow to +-inf, and NaN -> 0x7E00 for the canonical
    0x7FC00000 input)."""
    a = np.ascontiguousarray(values, dtype=np.float32)
    out = a.astype(np.float16).view(np.uint16).copy()
    out[np.isnan(a)] = 0x7E00
    return out


def round_to_dtype(values: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values through ``dtype`` ("f32", "bf16", "f16") and return
    them as float64 (the value the reference would hold after ``.to``)."""
    a = np.asarray(values)
    if dtype == "f32":
        return a.astype(np.float32).astype(np.float64)
    a32 = a.astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(a32)).astype(np.float64)
    if dtype == "f16":
        return a32.astype(np.float16).astype(np.float64)
    raise ValueError(dtype)


# ----------------------------------------------------------------------------
# Dequant (soft:277-307)
# ----------------------------------------------------------------------------

_FMT_BITS = {"bf16": (7, -133), "f16": (10, -24), "f32": (23, -149)}


def format_ulp(values: np.ndarray, dtype: str) -> np.ndarray:
    """Spacing of the ``dtype`` grid (bf16 / f16 / f32) at |values|: 2^(e - p)
    for |v| in [2^e, 2^(e+1)) with p explicit mantissa bits, never below
    the format's smallest subnormal.  0 at non-finite values."""
    mant, sub = _FMT_BITS[dtype]
    v = np.abs(np.asarray(values, dtype=np.float64))
    fin = np.isfinite(v)
    _, ex = np.frexp(np.where(fin & (v > 0), v, 1.0))
    ulp = np.where(v > 0, np.ldexp(1.0, ex - 1 - mant), 0.0)
    ulp = np.maximum(ulp, np.ldexp(1.0, sub))
    return np.where(fin, ulp, 0.0)


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """Packed bytes [..., K/2] -> codes [..., K]; the low nibble is the even k
    (soft:295)."""
    p = np.asarray(packed, dtype=np.uint8)
    codes = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    codes[..., 0::2] = p & 0x0F
    codes[..., 1::2] = p >> 4
    return codes


def pack_codes(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def check_dequant_args(packed: np.ndarray, scales: np.ndarray) -> None:
    """The validation of soft:283-294 (types first, then shapes)."""
    if packed.dtype != np.uint8:
        raise TypeError(f"packed must be uint8, got {packed.dtype}")
    if scales.dtype != np.uint8:
        raise TypeError(f"block_scales must be uint8, got {scales.dtype}")
    logical_k = packed.shape[-1] * 2
    if logical_k % 32 != 0:
        raise ValueError(f"logical K must be divisible by 32, got {logical_k}")
    if scales.shape[:-1] != packed.shape[:-1]:
        raise ValueError("packed and block_scales leading dimensions must match")
    if scales.shape[-1] * 32 != logical_k:
        raise ValueError("one E8M0 scale is required for every 32 MXFP4 values")


def dequant_f32(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """The exact FP32 product LUT[nibble] * 2**(s-127) (soft:295-306).

    The product of an E2M1 value and a power of two is exact in FP32 except
    where it overflows to +-inf (s = 253 with |v| >= 4, s = 254 with |v| >= 2)
    or where the scale is NaN (s = 255, also for +-0 codes).
    """
    packed = np.asarray(packed)
    scales = np.asarray(scales)
    check_dequant_args(packed, scales)
    values = _E2M1_F32[unpack_codes(packed)]
    block_scale = np.repeat(e8m0_to_f32(scales), BLOCK, axis=-1)
    with np.errstate(over="ignore", invalid="ignore"):
        return (values * block_scale).astype(np.float32)


def dequant_bits(packed: np.ndarray, scales: np.ndarray, dtype: str) -> np.ndarray:
    """``dequant_mxfp4(packed, scales, dtype)`` as raw bit patterns
    (uint32 for "f32", uint16 for "bf16"/"f16"): soft:307's ``.to(dtype)``."""
    v = dequant_f32(packed, scales)
    if dtype == "f32":
        return v.view(np.uint32)
    if dtype == "bf16":
        return f32_to_bf16_bits(v)
    if dtype == "f16":
        return f32_to_f16_bits(v)
    raise ValueError(f"unsupported dtype {dtype}")


def dequant_values(packed, scales, dtype: str) -> np.ndarray:
    """Dequantized values after rounding to ``dtype``, as float64."""
    v = dequant_f32(packed, scales)
    return round_to_dtype(v, dtype)


def fp8_values(codes: np.ndarray, fmt: str) -> np.ndarray:
    """OCP FP8 byte -> exact value (float64): the activation formats that
    aiter:11-20 hands to ``tl.dot_scaled`` as "e4m3" (``tl.float8e4nv``,
    torch.float8_e4m3fn: bias 7, no infinities, S.1111.111 is NaN) and "e5m2"
    (``tl.float8e5``, torch.float8_e5m2: bias 15, IEEE-style inf / NaN).
    Closed form from the bit fields; subnormals for exponent field 0."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    if fmt == "e4m3":
        e, m = (c >> 3) & 0xF, c & 0x7
        mag = np.where(e == 0, np.ldexp(m / 8.0, -6), np.ldexp(1.0 + m / 8.0, e - 7))
        mag = np.where((e == 0xF) & (m == 0x7), np.nan, mag)
    elif fmt == "e5m2":
        e, m = (c >> 2) & 0x1F, c & 0x3
        mag = np.where(e == 0, np.ldexp(m / 4.0, -14), np.ldexp(1.0 + m / 4.0, e - 15))
        mag = np.where(e == 0x1F, np.where(m == 0, np.inf, np.nan), mag)
    else:
        raise ValueError(f"unsupported fp8 format {fmt}")
    return sign * mag


def fp8_scaled_values(codes: np.ndarray, scales: np.ndarray | None, fmt: str) -> np.ndarray:
    """FP8 activations times their E8M0 block scales (one per 32 along the
    last axis; None = every scale 1): the exact values the block-scaled MFMA
    multiplies (aiter:206-214, 329-338 with an FP8 A)."""
    v = fp8_values(codes, fmt)
    if scales is None:
        return v
    s = np.repeat(e8m0_to_f32(np.asarray(scales, np.uint8)).astype(np.float64), BLOCK, axis=-1)
    return v * s


# ----------------------------------------------------------------------------
# Quantizers
# ----------------------------------------------------------------------------

def quant_mxfp4_ties_away(x: np.ndarray):
    """The reference test quantizer ``torch_dynamic_mxfp4_quant`` (test:28-60).

    * amax per 32-block is pre-rounded to a power of two by adding 0x200000
      to its FP32 bits and masking the mantissa (test:35-37);
    * E = clamp(floor(log2 amax') - 2, -127, 127) (test:38);
    * each q = x * 2**-E is rounded to the E2M1 grid by truncating to three
      bits and rounding the last one half-up, i.e. nearest with ties away
      from zero, saturating at 6 (test:39-54);
    * scale byte = (E + 127) mod 256 (test:57; torch's negative-float ->
      uint8 cast wraps).
    Returns (packed uint8 [..., K/2], scales uint8 [..., K/32]).
    """
    x = np.asarray(x, dtype=np.float32)
    if x.shape[-1] % BLOCK:
        raise ValueError("test quantizer requires K divisible by 32")
    shape = x.shape
    blocks = x.reshape(-1, shape[-1] // BLOCK, BLOCK)
    amax = np.max(np.abs(blocks), axis=-1)
    amax_bits = amax.view(np.int32).astype(np.int64)
    amax_bits = ((amax_bits + 0x200000) & 0xFF800000).astype(np.uint32).astype(np.int64)
    amax_r = amax_bits.astype(np.uint32).view(np.float32)
    with np.errstate(divide="ignore"):
        e = np.clip(np.floor(np.log2(amax_r)) - 2, -127, 127).astype(np.float32)
    q = (blocks * np.exp2(-e)[..., None]).astype(np.float32)
    qi = q.view(np.int32).astype(np.int64) & 0xFFFFFFFF
    signs = qi & 0x80000000
    exps = (qi >> 23) & 0xFF
    mants = qi & 0x7FFFFF
    shift = 127 - exps - 1
    # shifts of 32 or more leave nothing (torch's >> on int32 sign-fills, and
    # the shifted value is non-negative here).
    sub = np.where(shift < 32, (0x400000 | (mants >> 1)) >> np.clip(shift, 0, 63), 0)
    mants = np.where(exps < 127, sub, mants)
    exps = np.where(exps > 126, exps, 126) - 126
    combined = (((exps << 2) | (mants >> 21)) + 1) >> 1
    mag = np.where(combined < 7, combined, 7)
    codes = (((signs >> 28) & 0xF) | mag).astype(np.uint8)
    packed = pack_codes(codes).reshape(*shape[:-1], shape[-1] // 2)
    scales = ((e.astype(np.int64) + 127) & 0xFF).astype(np.uint8).reshape(
        *shape[:-1], shape[-1] // BLOCK)
    return packed, scales


_E2M1_POS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def quant_mxfp4_rne(x: np.ndarray):
    """OCP MX v1.0 quantizer used by the W4A4 benchmark configuration:
    E = floor(log2(amax)) - 2 per 32-block (clamped to the E8M0 range
    [-127, 127]; an all-zero block gets E = -127), then each x * 2**-E is
    rounded to the nearest E2M1 value with ties to the even code and
    saturated to +-6.  No amax pre-rounding (unlike test:37).
    Returns (packed uint8 [..., K/2], scales uint8 [..., K/32])."""
    x = np.asarray(x, dtype=np.float32)
    if x.shape[-1] % BLOCK:
        raise ValueError("quantizer requires K divisible by 32")
    shape = x.shape
    blocks = x.reshape(-1, shape[-1] // BLOCK, BLOCK).astype(np.float64)
    amax = np.max(np.abs(blocks), axis=-1)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - 2, -127)
    e = np.clip(e, -127, 127)
    q = blocks * np.exp2(-e)[..., None]
    mag = np.abs(q)
    # index of the nearest grid point; ties -> even code index
    idx = np.searchsorted(_E2M1_POS, mag)  # first grid >= mag
    idx = np.clip(idx, 1, 7)
    lo = _E2M1_POS[idx - 1]
    hi = _E2M1_POS[idx]
    choose_hi = (mag - lo > hi - mag) | ((mag - lo == hi - mag) & (idx % 2 == 0))
    code = np.where(choose_hi, idx, idx - 1)
    code = np.where(mag >= 6.0, 7, code)
    code = np.where(mag <= 0.0, 0, code)
    # the sign bit follows the input, also where the magnitude rounds to 0
    # (as test:54 does for the reference quantizer)
    codes = (code | np.where(np.signbit(q), 8, 0)).astype(np.uint8)
    packed = pack_codes(codes).reshape(*shape[:-1], shape[-1] // 2)
    scales = (e.astype(np.int64) + 127).astype(np.uint8).reshape(*shape[:-1], shape[-1] // BLOCK)
    return packed, scales


# ----------------------------------------------------------------------------
# Routing metadata (vllm:119-146)
# ----------------------------------------------------------------------------

def make_routing(topk_ids: np.ndarray, block_m: int = 64, num_experts: int | None = None):
    """Expert-sorted, ``block_m``-padded route ids (vllm:119-146).

    Route id r = token * top_k + slot (the flattened index).  Experts are
    visited in ascending order; within an expert, route ids ascend; each
    expert's list is cut into ``block_m`` chunks padded with the sentinel
    ``topk_ids.size``; ``expert_ids`` holds one expert per chunk and
    ``num_tokens_post_padded = len(sorted_ids)``.

    With ``num_experts`` given, ids outside [0, num_experts) are dropped,
    which is what the safe path does with them (their slots stay zero,
    soft:476-481); vllm:124 would instead emit a block for every distinct id.
    Unlike vllm:137-138 an empty routing is allowed and gives zero blocks.
    """
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    sentinel = flat.size
    sorted_blocks, expert_blocks = [], []
    for expert in np.unique(flat):
        if num_experts is not None and not (0 <= expert < num_experts):
            continue
        route_ids = np.nonzero(flat == expert)[0]
        for start in range(0, route_ids.size, block_m):
            chunk = route_ids[start:start + block_m]
            padded = np.full(block_m, sentinel, dtype=np.int32)
            padded[:chunk.size] = chunk
            sorted_blocks.append(padded)
            expert_blocks.append(int(expert))
    if sorted_blocks:
        sorted_ids = np.concatenate(sorted_blocks).astype(np.int32)
    else:
        sorted_ids = np.zeros(0, dtype=np.int32)
    expert_ids = np.array(expert_blocks, dtype=np.int32)
    return sorted_ids, expert_ids, np.array([sorted_ids.size], dtype=np.int32)


def route_topk_fp64(logits: np.ndarray, top_k: int, renormalize: bool = True):
    """Router: softmax over the experts, top-k, optional renormalisation, in
    float64 -- the ``topk_weights`` / ``topk_ids`` the MoE layer consumes
    (vllm:233-265), built as test:242-244 builds them (softmax, then
    ``torch.topk``) and, with ``renormalize``, divided by their sum.  Slots
    in descending probability; ties to the lower expert id (``torch.topk``
    leaves tie order unspecified).  Returns (weights float64, ids int64)."""
    x = np.asarray(logits, dtype=np.float64)
    ne = x.shape[-1]
    flat = x.reshape(-1, ne)
    # descending logit, then ascending expert id
    order = np.lexsort((np.broadcast_to(np.arange(ne), flat.shape), -flat), axis=-1)
    ids = order[:, :top_k]
    p = np.exp(flat - flat.max(-1, keepdims=True))
    p = p / p.sum(-1, keepdims=True)
    w = np.take_along_axis(p, ids, -1)
    if renormalize:
        w = w / w.sum(-1, keepdims=True)
    shape = x.shape[:-1] + (top_k,)
    return w.reshape(shape), ids.astype(np.int64).reshape(shape)


# ----------------------------------------------------------------------------
# FP64 oracles
# ----------------------------------------------------------------------------

def linear_fp64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray,
                bias: np.ndarray | None = None, w_dtype: str = "bf16") -> np.ndarray:
    """y = x . dequant(W)^T (+ bias) accumulated in float64 (soft:371-376).

    The weights enter at the value the reference multiplies with: the
    dequantized FP32 value rounded to the activation dtype (exact for bf16
    unless it overflows; rounded for fp16)."""
    w = dequant_values(packed, scales, w_dtype)
    y = np.asarray(x, dtype=np.float64).reshape(-1, w.shape[1]) @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def fused_moe_fp64(a_values: np.ndarray, b_packed: np.ndarray, b_mx: np.ndarray,
                   a_scale: float, b_scale: np.ndarray, topk_weights: np.ndarray,
                   topk_ids: np.ndarray, mul_routed_weight: bool,
                   compute_dtype: str = "bf16", b_values=None) -> np.ndarray:
    """C[t, s, :] = a[t] . dequant(B[e])^T * a_scale * b_scale[e] (* w[t, s])
    for e = topk_ids[t, s] in [0, E); other slots are 0 (soft:476-494).

    ``a_values`` are the activations already at the compute dtype (the caller
    dequantizes packed A, soft:468-475).  Accumulates in float64.
    ``b_values`` (optional): a callable e -> ``dequant_values(b_packed[e],
    b_mx[e], compute_dtype)`` computed once by the caller, for tests that
    evaluate many cases over the same experts."""
    a = np.asarray(a_values, dtype=np.float64)
    ids = np.asarray(topk_ids).astype(np.int64)
    m, top_k = ids.shape
    num_experts, n = b_packed.shape[0], b_packed.shape[1]
    out = np.zeros((m, top_k, n), dtype=np.float64)
    for e in range(num_experts):
        t, s = np.nonzero(ids == e)
        if t.size == 0:
            continue
        if b_values is not None:
            w = np.asarray(b_values(e), dtype=np.float64)
        else:
            w = dequant_values(b_packed[e], b_mx[e], compute_dtype)
        v = (a[t] @ w.T) * float(a_scale) * float(b_scale[e])
        if mul_routed_weight:
            v = v * np.asarray(topk_weights, dtype=np.float64)[t, s, None]
        out[t, s] = v
    return out


def silu_mul_bf16(gate_up_bf16: np.ndarray) -> np.ndarray:
    """``F.silu(g) * u`` on bf16 tensors (vllm:248-252): silu evaluated in
    float on the bf16 gate and rounded to bf16, then the bf16 product rounded
    to bf16.  Input and output are float64 arrays holding bf16 values."""
    inter = gate_up_bf16.shape[-1] // 2
    g = gate_up_bf16[..., :inter]
    u = gate_up_bf16[..., inter:]
    silu = round_to_dtype(g / (1.0 + np.exp(-g)), "bf16")
    return round_to_dtype(silu * u, "bf16")


def moe_layer_fp64(x: np.ndarray, w13: np.ndarray, s13: np.ndarray, w2: np.ndarray,
                   s2: np.ndarray, topk_weights: np.ndarray, topk_ids: np.ndarray,
                   w13_values=None, w2_values=None, return_routes: bool = False):
    """The vLLM MoE layer (vllm:233-265) with float64 GEMMs and the
    reference's rounding points: gate_up rounded to bf16 per route, silu*mul
    in bf16, the route-weighted down output rounded to bf16 per route, then
    the top-k sum (accumulated in float64 here).  Returns float64 [M, H].
    ``w13_values`` / ``w2_values``: optional pre-dequantized experts, as
    ``b_values`` of fused_moe_fp64.  With ``return_routes`` also returns the
    per-route down outputs after their bf16 rounding, [M, top_k, H] (the
    values the reference rounds before the top-k sum, vllm:253-265)."""
    m, top_k = np.asarray(topk_ids).shape
    ones_e = np.ones(w13.shape[0])
    gu = fused_moe_fp64(x, w13, s13, 1.0, ones_e, topk_weights, topk_ids, False,
                        b_values=w13_values)
    gu = round_to_dtype(gu, "bf16")
    h = silu_mul_bf16(gu).reshape(m * top_k, -1)
    down = fused_moe_fp64(h, w2, s2, 1.0, ones_e, np.asarray(topk_weights).reshape(-1, 1),
                          np.asarray(topk_ids).reshape(-1, 1), True, b_values=w2_values)
    down = round_to_dtype(down, "bf16")[:, 0].reshape(m, top_k, -1)
    y = down.sum(axis=1)
    return (y, down) if return_routes else y


# ----------------------------------------------------------------------------
# Restatements of the safe path (torch on CPU; same rounding points)
# ----------------------------------------------------------------------------

def _torch():
    import torch
    return torch


_TORCH_DT = {"f32": "float32", "bf16": "bfloat16", "f16": "float16"}


def dequant_safe(packed, scales, dtype):
    """soft:277-307 with torch CPU ops: explicit dequant to ``dtype``."""
    torch = _torch()
    p = torch.as_tensor(np.asarray(packed))
    s = torch.as_tensor(np.asarray(scales))
    codes = torch.stack((p & 0x0F, p >> 4), dim=-1).flatten(-2)
    table = torch.tensor(E2M1_VALUES, dtype=torch.float32)
    values = table[codes.long()]
    scale_codes = s.repeat_interleave(32, dim=-1)
    sc = torch.exp2((scale_codes.to(torch.int16) - 127).to(torch.float32))
    sc = torch.where(scale_codes == 255, torch.full_like(sc, float("nan")), sc)
    return (values * sc).to(dtype)


def linear_safe(x, packed, scales, bias=None):
    """soft:371-376: ``x_2d @ dequant(W, S, x.dtype).T (+ bias)`` on CPU
    torch tensors (BF16/FP16 GEMM, FP32 accumulation inside the BLAS)."""
    torch = _torch()
    k = packed.shape[1] * 2
    x2 = x.reshape(-1, k).contiguous()
    w = dequant_safe(packed, scales, x.dtype)
    out = torch.matmul(x2, w.transpose(0, 1))
    if bias is not None:
        out = out + bias
    return out.reshape(*x.shape[:-1], packed.shape[0])


def fused_moe_safe(A, B, C, A_scale, B_scale, A_mx_scale, B_mx_scale, topk_weights,
                   topk_ids, mul_routed_weight):
    """soft:466-494 on CPU torch tensors: writes C in place."""
    torch = _torch()
    dt = C.dtype
    if A.dtype == torch.uint8:
        act = dequant_safe(A, A_mx_scale, dt)
    else:
        act = A.to(dt)
    C.zero_()
    g = A_scale.reshape(-1)[0].to(torch.float32)
    for e in range(B.shape[0]):
        pos = torch.nonzero(topk_ids == e, as_tuple=False)
        if pos.numel() == 0:
            continue
        t, s = pos[:, 0], pos[:, 1]
        w = dequant_safe(B[e], B_mx_scale[e], dt)
        out = torch.matmul(act[t], w.transpose(0, 1))
        out = out * g * B_scale[e].to(torch.float32)
        if mul_routed_weight:
            out = out * topk_weights[t, s, None]
        C[t, s] = out.to(dt)


def moe_layer_safe(x, w13, s13, w2, s2, topk_weights, topk_ids):
    """vllm:233-265 composed over the safe op (vllm:149-185 with A_scale =
    B_scale = 1), on CPU torch tensors."""
    torch = _torch()
    F = torch.nn.functional
    m, top_k = topk_ids.shape
    ones_a = torch.ones(1, dtype=torch.float32)
    ones_b = torch.ones(w13.shape[0], dtype=torch.float32)
    gu = torch.empty((m, top_k, w13.shape[1]), dtype=x.dtype)
    fused_moe_safe(x, w13, gu, ones_a, ones_b, None, s13, topk_weights, topk_ids, False)
    inter = gu.shape[-1] // 2
    h = (F.silu(gu[..., :inter]) * gu[..., inter:]).reshape(m * top_k, inter)
    down = torch.empty((m * top_k, 1, w2.shape[1]), dtype=x.dtype)
    fused_moe_safe(h, w2, down, ones_a, ones_b, None, s2, topk_weights.reshape(-1, 1),
                   topk_ids.reshape(-1, 1), True)
    return down[:, 0].reshape(m, top_k, -1).sum(dim=1)


# ----------------------------------------------------------------------------
# Parity metrics
# ----------------------------------------------------------------------------

def parity_errors(y: np.ndarray, oracle: np.ndarray) -> dict:
    """Elementwise relative error with the denominator floored at
    1e-3 * rms(oracle), and the norm-wise error ||y - o|| / ||o||."""
    y = np.asarray(y, dtype=np.float64)
    o = np.asarray(oracle, dtype=np.float64)
    rms = math.sqrt(float(np.mean(o * o))) if o.size else 0.0
    floor = max(1e-3 * rms, np.finfo(np.float64).tiny)
    diff = np.abs(y - o)
    elem = float(np.max(diff / np.maximum(np.abs(o), floor))) if o.size else 0.0
    norm_o = float(np.linalg.norm(o))
    norm = float(np.linalg.norm(y - o) / norm_o) if norm_o > 0 else float(np.linalg.norm(y - o))
    return {"elem_rel": elem, "norm_rel": norm}


ELEM_TOL = 1e-2
NORM_TOL = 2e-3
