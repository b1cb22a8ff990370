"""The SiLU lookup tables the gate_up epilogue reads (built by
``mxfp4-gfx936_amd/silu_table.py`` into ``_build/gen/silu_table.inc``):
torch's FP32 steps ``x / (1 + exp(-x))`` on every bf16 / fp16 value, rounded
back to the type (vllm:249-252)."""

import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "mxfp4-gfx936_amd"))
import silu_table as S  # noqa: E402

import oracle.mxfp4_oracle as O  # noqa: E402


def _inputs(kind):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    if kind == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def _values(kind, t):
    if kind == "bf16":
        return (t.astype(np.uint32) << 16).view(np.float32)
    return t.view(np.float16).astype(np.float32)


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_table_matches_float32_steps(kind):
    # numpy float32 arithmetic (its own exp) on every finite input.  The
    # table rounds exp correctly; a result may differ only where numpy's
    # float32 exp is off by an ulp, and then by one unit of the type
    t = S.silu_table(kind)
    x = _inputs(kind)[np.isfinite(_inputs(kind))]
    with np.errstate(all="ignore"):
        e32 = np.exp(-x)
        q = (x / (np.float32(1.0) + e32)).astype(np.float32)
        e_cr = np.exp(-x.astype(np.float64)).astype(np.float32)
    ref = O.round_to_dtype(q.astype(np.float64), kind)
    got = _values(kind, t)[np.isfinite(_inputs(kind))].astype(np.float64)
    both_nan = np.isnan(ref) & np.isnan(got)
    diff = (got != ref) & ~both_nan
    assert np.all(e32[diff] != e_cr[diff])
    assert diff.sum() <= 8
    unit = np.abs(np.spacing(ref[diff].astype(np.float16 if kind == "f16" else np.float32)))
    if kind == "bf16":
        unit = unit * 65536.0
    assert np.all(np.abs(got[diff] - ref[diff]) <= unit.astype(np.float64) * 1.0001)


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_table_against_float64_silu(kind):
    # the oracle's single-rounding float64 SiLU: equal except where the FP32
    # steps round differently, by at most one unit of the type
    t = S.silu_table(kind)
    x = _inputs(kind)
    fin = np.isfinite(x) & (np.abs(x) < 80)
    x64 = x[fin].astype(np.float64)
    ref = O.round_to_dtype(x64 / (1.0 + np.exp(-x64)), kind).astype(np.float64)
    got = _values(kind, t)[fin].astype(np.float64)
    diff = got != ref
    assert diff.mean() < 1e-3
    ulp = np.abs(np.spacing(ref.astype(np.float16 if kind == "f16" else np.float32)))
    if kind == "bf16":
        ulp = ulp * 65536.0
    assert np.all(np.abs(got - ref)[diff] <= ulp[diff] * 1.0001)


def test_table_special_values():
    tb, tf = S.silu_table("bf16"), S.silu_table("f16")
    def bfv(b):
        return float((np.uint32(b) << np.uint32(16)).view(np.float32))
    assert tb[0x0000] == 0x0000                  # silu(0) = 0
    assert tb[0x8000] == 0x8000                  # silu(-0) = -0
    assert bfv(tb[0x3F80]) == 0.73046875         # silu(1) = 0.7310586 -> bf16
    assert tb[0x41A0] == 0x41A0                  # silu(20) rounds to 20
    assert tb[0x7F80] == 0x7F80                  # silu(+inf) = +inf
    assert np.isnan(bfv(tb[0xFF80]))             # silu(-inf) = -inf / inf
    assert tb[0xC2C8] == 0x8000                  # exp(100) overflows FP32: -100 / inf = -0
    assert np.isnan(bfv(tb[0x7FC0]))             # NaN stays NaN
    assert np.uint16(tf[np.float16(1.0).view(np.uint16)]).view(np.float16) == np.float16(0.731)
    assert np.isnan(np.uint16(tf[0x7E00]).view(np.float16))
