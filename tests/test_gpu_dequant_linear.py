"""GPU parity: standalone dequant (bit-exact) and the dense W4A16 linear
(tolerance vs the FP64 oracle, and no worse than the reference safe path
``x @ dequant(W).T`` run through torch on the same device)."""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from mxfp4_amd import _lib
from oracle import c_oracle, mxfp4_oracle as O

from _helpers import (assert_parity, assert_rows_parity, cuda, dequant_device, fp32_gemm,
                      rand_act, rand_mxfp4)

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
IDT = {"f32": torch.int32, "bf16": torch.int16, "f16": torch.int16}


def _bits(t: torch.Tensor, dt: str) -> np.ndarray:
    a = t.view(IDT[dt]).cpu().numpy()
    return a.view(np.uint32 if dt == "f32" else np.uint16)


def test_native_library_is_loaded():
    lib = _lib.load()
    assert lib.mxfp4_abi_version() == _lib.ABI_VERSION
    assert torch.cuda.is_available()


# ---------------------------------------------------------------- dequant

@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_dequant_all_codes_all_scales_bitexact(dt):
    g = np.load(os.path.join(GOLDEN, "dequant_table.npz"))
    out = mx.dequant_mxfp4(cuda(g["packed"]), cuda(g["scales"]), TDT[dt])
    # every pattern, including the canonical NaN of s = 255, -0, subnormals, +-inf
    assert np.array_equal(_bits(out, dt), g[dt])


def test_dequant_reference_known_answer():
    # tests/test_moe_mxfp4_soft.py:81-92
    packed = torch.tensor([[c | ((c + 1) << 4) for c in range(0, 16, 2)] * 2], dtype=torch.uint8,
                          device="cuda")
    scales = torch.full((1, 1), 127, device="cuda", dtype=torch.uint8)
    actual = mx.dequant_mxfp4(packed, scales)
    expected = torch.tensor([mx._MXFP4_E2M1_VALUES], device="cuda", dtype=torch.float32).repeat(1, 2)
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_dequant_expert_shapes_vs_c_oracle(dt):
    rng = np.random.default_rng(20260901)
    # leading dims [E, N] like the MoE expert tensors; the full scale range
    packed, scales = rand_mxfp4(rng, (3, 96), 2048, lo=0, hi=255)
    out = mx.dequant_mxfp4(cuda(packed), cuda(scales), TDT[dt])
    assert out.shape == (3, 96, 2048)
    assert np.array_equal(_bits(out, dt), c_oracle.dequant_bits(packed, scales, dt))


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,k", [(300, 2080), (5000, 96), (7, 4096 + 64)])
def test_dequant_ragged_blocks_vs_c_oracle(rows, k, dt):
    # 16-byte rows go through the wide kernel, whose waves take 2048-value
    # blocks: a last block of one chunk (K = 2080), rows shorter than a block
    # (K = 96) over a grid-stride loop, and a ragged tail after two blocks
    rng = np.random.default_rng(rows + k)
    packed, scales = rand_mxfp4(rng, (rows,), k, lo=0, hi=255)
    out = mx.dequant_mxfp4(cuda(packed), cuda(scales), TDT[dt])
    assert np.array_equal(_bits(out, dt), c_oracle.dequant_bits(packed, scales, dt))


@pytest.mark.parametrize("dt,rows", [("bf16", 65536), ("f32", 32768)])
def test_dequant_streaming_output_sampled_rows(dt, rows):
    # outputs of >= 256 MiB are written with non-temporal stores; sampled
    # rows (and the last) bit-exact against the C oracle
    rng = np.random.default_rng(rows)
    k = 2048
    packed = torch.randint(0, 256, (rows, k // 2), dtype=torch.uint8, device="cuda")
    scales = torch.randint(0, 256, (rows, k // 32), dtype=torch.uint8, device="cuda")
    out = mx.dequant_mxfp4(packed, scales, TDT[dt])
    assert out.numel() * out.element_size() >= 256 << 20
    pick = torch.from_numpy(np.sort(np.append(rng.choice(rows, 256, replace=False), rows - 1)))
    got = _bits(out[pick.cuda()], dt)
    want = c_oracle.dequant_bits(packed[pick.cuda()].cpu().numpy(),
                                 scales[pick.cuda()].cpu().numpy(), dt)
    del out
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_dequant_c_abi_four_byte_row_stride(dt):
    # a packed row stride that is 4-byte but not 16-byte aligned takes the
    # dword kernel (the C ABI accepts any multiple of 4)
    rng = np.random.default_rng(99)
    rows, k = 37, 160
    packed, scales = rand_mxfp4(rng, (rows,), k, lo=0, hi=255)
    stride = k // 2 + 4
    buf = np.zeros((rows, stride), dtype=np.uint8)
    buf[:, : k // 2] = packed
    p, s = cuda(buf), cuda(scales)
    out = torch.empty((rows, k), dtype=TDT[dt], device="cuda")
    lib = _lib.load()
    rc = lib.mxfp4_dequant(p.data_ptr(), stride, s.data_ptr(), k // 32, rows, k, out.data_ptr(),
                           _lib.dtype_code(TDT[dt]),
                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.mxfp4_last_error()
    assert np.array_equal(_bits(out, dt), c_oracle.dequant_bits(packed, scales, dt))


def test_dequant_noncontiguous_and_other_dtype():
    rng = np.random.default_rng(7)
    packed, scales = rand_mxfp4(rng, (64,), 256)
    p = cuda(packed)[::2]
    s = cuda(scales)[::2]
    out = mx.dequant_mxfp4(p, s, torch.bfloat16)
    assert np.array_equal(_bits(out, "bf16"), O.dequant_bits(packed[::2], scales[::2], "bf16"))
    out64 = mx.dequant_mxfp4(p, s, torch.float64)
    assert out64.dtype == torch.float64
    assert np.array_equal(out64.cpu().numpy(), O.dequant_f32(packed[::2], scales[::2]).astype(np.float64))
    empty = mx.dequant_mxfp4(torch.empty((0, 16), dtype=torch.uint8, device="cuda"),
                             torch.empty((0, 1), dtype=torch.uint8, device="cuda"))
    assert empty.shape == (0, 32)


# ---------------------------------------------------------------- linear

def _safe_reference(x: torch.Tensor, packed: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """soft:371-373 on the device: exact dequant (oracle bits) then torch.matmul."""
    dt = "bf16" if x.dtype == torch.bfloat16 else "f16"
    w = torch.from_numpy(O.dequant_bits(packed, scales, dt).view(np.int16)).view(x.dtype).cuda()
    return torch.matmul(x.reshape(-1, w.shape[1]), w.T)


@pytest.mark.parametrize("m_value", [1, 8])
def test_linear_matches_explicit_dequant_small(m_value):
    # test:95-111 on the test's own inputs (its seed, randn drawn on the
    # device) and the reference's quantizer.  The reference asserts bitwise
    # equality with x @ dequant(W).T, which torch's BLAS sums in its own
    # order.  Every product of a bf16 activation and an E2M1 x 2^s weight is
    # exact in FP32, and an FP32 sum of 128 of them errs by a few FP32 steps
    # at most, so two summation orders round to different bf16 values only
    # where a sum lies that close to a bf16 rounding boundary: none of these
    # inputs' outputs does (nor any of 20480 outputs over 40 other seeds).
    torch.manual_seed(20260811 + m_value)
    n_value, k_value = 64, 128
    x = torch.randn((m_value, k_value), device="cuda", dtype=torch.bfloat16)
    w = torch.randn((n_value, k_value), device="cuda", dtype=torch.bfloat16)
    packed, scales = O.quant_mxfp4_ties_away(w.float().cpu().numpy())
    y = mx.linear_mxfp4_soft(x, cuda(packed), cuda(scales))
    assert y.dtype == torch.bfloat16 and y.shape == (m_value, n_value)
    ref = _safe_reference(x, packed, scales)
    assert torch.equal(y, ref)
    assert_parity(y, O.linear_fp64(x.float().cpu().numpy(), packed, scales), ref=ref)


@pytest.mark.parametrize("k,n", [(2048, 5120), (4096, 2048)], ids=["qkv", "o_proj"])
@pytest.mark.parametrize("m", [1, 8, 370, 4096])
def test_linear_attention_shapes(m, k, n):
    rng = np.random.default_rng(20260810 + m + k)
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(20260810 + m, (m, k))
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    ref = _safe_reference(cuda(x), packed, scales)
    rows = np.arange(m) if m <= 370 else np.sort(rng.choice(m, 192, replace=False))
    oracle = O.linear_fp64(x.float().numpy()[rows], packed, scales)
    assert_parity(y[rows], oracle, ref=ref[rows], what=f"linear m={m} k={k} n={n}")


@pytest.mark.parametrize("m,k,n", [(8192, 4096, 4096), (2100, 256, 16400)],
                         ids=["cube", "partial_tiles"])
def test_linear_wide_tile_shapes(m, k, n):
    # the wide tiles: 1024 tiles of 128 x 256 (two full rounds of two per
    # CU), and 128 x 320 tiles ending in a partial row tile and an 80-column
    # last tile
    rng = np.random.default_rng(20261201 + m)
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(20261201 + n, (m, k))
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    ref = _safe_reference(cuda(x), packed, scales)
    rows = np.sort(np.concatenate([rng.choice(m, 96, replace=False), [m - 1]]))
    oracle = O.linear_fp64(x.float().numpy()[rows], packed, scales)
    assert_parity(y[rows], oracle, ref=ref[rows], what=f"linear m={m} k={k} n={n}")


@pytest.mark.parametrize("k,n", [(2048, 512), (4096, 384), (640, 272)])
def test_linear_decode_every_m(k, n):
    # every dense decode size of the skinny kernel: 1-16 rows (one 16-row
    # block, up to all of its rows staged through LDS; 8 at K=4096), 17-32
    # (two blocks); x rows strided (a column slice of a wider tensor)
    rng = np.random.default_rng(k + n)
    packed, scales = rand_mxfp4(rng, (n,), k)
    w = dequant_device(packed, scales)
    wp, ws = cuda(packed), cuda(scales)
    for m in list(range(1, 17)) + [17, 24, 31, 32]:
        xw = cuda(rand_act(m * 7 + k, (m, k + 256)))
        x = xw[:, 128:128 + k]
        y = mx.linear_mxfp4_soft(x, wp, ws)
        ref = fp32_gemm(x, w)
        assert_rows_parity(y, ref, what=f"m={m} k={k} n={n}", fmt=torch.bfloat16)


def test_linear_rejects_k_not_multiple_of_128():
    # soft:326-327: the module and the C ABI both refuse K % 128 != 0
    rng = np.random.default_rng(700)
    n, k, m = 64, 2080, 4
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(700, (m, k))
    with pytest.raises(ValueError):
        mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    xd, wd, sd = cuda(x), cuda(packed), cuda(scales)
    y = torch.empty((m, n), dtype=x.dtype, device="cuda")
    lib = _lib.load()
    rc = lib.mxfp4_linear_w4a16(_lib.ptr(xd), _lib.dtype_code(x.dtype), m, k, k, _lib.ptr(wd),
                                _lib.ptr(sd), n, None, _lib.ptr(y), _lib.stream_of(xd.device))
    assert rc == _lib.ERR_VALUE


@pytest.mark.parametrize("m", [1, 20, 100])
def test_linear_fp16_partial_tiles(m):
    rng = np.random.default_rng(m)
    n, k = 200, 768
    packed, scales = rand_mxfp4(rng, (n,), k, lo=118, hi=132)
    x = rand_act(m, (m, k), torch.float16)
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    assert y.dtype == torch.float16
    ref = _safe_reference(cuda(x), packed, scales)
    oracle = O.linear_fp64(x.float().numpy(), packed, scales, w_dtype="f16")
    assert_parity(y, oracle, ref=ref, what=f"fp16 m={m}")


@pytest.mark.parametrize("m", [33, 96, 128])
def test_linear_mid_m_long_k(m):
    # o_proj shape, 33 <= M <= 128: 32-row skinny blocks (the prefill grid
    # would be under 128 workgroups with a 64-stage K loop)
    rng = np.random.default_rng(400 + m)
    k, n = 4096, 2048
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(400 + m, (m, k))
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    ref = _safe_reference(cuda(x), packed, scales)
    oracle = O.linear_fp64(x.float().numpy(), packed, scales)
    assert_parity(y, oracle, ref=ref, what=f"mid m={m}")


@pytest.mark.parametrize("m,k,n,dt", [(370, 4096, 2048, torch.bfloat16),
                                      (200, 4096, 1002, torch.float16),
                                      (64, 2048, 1536, torch.bfloat16),
                                      (130, 8192, 640, torch.bfloat16)])
def test_linear_split_k(m, k, n, dt):
    # too few tiles to fill the GPU: K goes in slices whose FP32 partial sums
    # are added in slice order, then the bias, then one rounding
    ws = ctypes.c_int64(0)
    _lib.check(_lib.load().mxfp4_linear_w4a16_workspace_size(m, k, n, ctypes.byref(ws)))
    assert ws.value >= 2 * m * n * 4, "this shape is expected to split K"
    rng = np.random.default_rng(500 + m)
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(500 + m, (m, k), dt)
    bias = rand_act(501 + m, (n,), dt)
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales), cuda(bias))
    assert y.dtype == dt and y.shape == (m, n)
    oracle = O.linear_fp64(x.float().numpy(), packed, scales, bias.float().numpy())
    assert_parity(y, oracle, what=f"split-K m={m} k={k} n={n}")
    y2 = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales), cuda(bias))
    assert torch.equal(y, y2)  # deterministic


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_linear_pipelined_decode_grid(dt):
    # 3 rows over 20480 columns: 640 two-step workgroups take the
    # software-pipelined decode kernel (dense rows)
    rng = np.random.default_rng(31)
    m, k, n = 3, 2048, 20480
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(31, (m, k), dt)
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    assert y.dtype == dt
    ref = _safe_reference(cuda(x), packed, scales)
    oracle = O.linear_fp64(x.float().numpy(), packed, scales,
                           w_dtype="f16" if dt == torch.float16 else "bf16")
    assert_parity(y, oracle, ref=ref, what=f"pipelined {dt}")


def test_linear_activations_beyond_2gib():
    # x [270000, 4096] bf16 is 2.2 GB: past what a 32-bit buffer offset
    # addresses, so the GEMM takes the kernel that addresses its operands
    # with 64-bit pointers; rows near the start, the 2^31-byte mark and
    # the end against the FP64 oracle
    m, k, n = 270000, 4096, 128
    rng = np.random.default_rng(2048)
    packed, scales = rand_mxfp4(rng, (n,), k)
    g = torch.Generator(device="cuda").manual_seed(2049)
    x = torch.randn((m, k), generator=g, device="cuda", dtype=torch.bfloat16)
    assert x.numel() * 2 > 1 << 31
    y = mx.linear_mxfp4_soft(x, cuda(packed), cuda(scales))
    rows = np.array([0, 1, (1 << 31) // (k * 2) - 1, (1 << 31) // (k * 2), m - 2, m - 1])
    xs = x[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    oracle = O.linear_fp64(xs, packed, scales)
    assert_parity(y[torch.from_numpy(rows).cuda()], oracle, what="2.2 GB of activations")
    del x, y
    torch.cuda.empty_cache()


def test_linear_bias_and_leading_dims():
    rng = np.random.default_rng(31)
    n, k = 96, 256
    packed, scales = rand_mxfp4(rng, (n,), k)
    x = rand_act(31, (2, 3, k))
    bias = rand_act(32, (n,))
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales), cuda(bias))
    assert y.shape == (2, 3, n) and y.dtype == torch.bfloat16
    oracle = O.linear_fp64(x.float().numpy().reshape(6, k), packed, scales, bias.float().numpy())
    assert_parity(y.reshape(6, n), oracle)
    # an fp32 bias is added after the GEMM with torch's promotion (soft:374-375):
    # exactly the bf16 GEMM result plus the bias in fp32
    y32 = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales), cuda(bias.float()))
    assert y32.dtype == torch.float32
    y0 = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales))
    assert torch.equal(y32, y0 + cuda(bias.float()))


@pytest.mark.parametrize("scale", [1, 254])
@pytest.mark.parametrize("m", [1, 40])
def test_linear_edge_sweep_every_code(scale, m):
    # BASELINE config 5 edge sweep: every E2M1 code at E8M0 1 and 254, K=768
    n, k = 32, 768
    codes = np.tile(np.arange(16, dtype=np.uint8), (n, k // 16))
    for r in range(n):
        codes[r] = np.roll(codes[r], r)
    packed = O.pack_codes(codes)
    scales = np.full((n, k // 32), scale, dtype=np.uint8)
    x = rand_act(900 + m, (m, k))
    y = mx.linear_mxfp4_soft(cuda(x), cuda(packed), cuda(scales)).float().cpu().numpy()
    with np.errstate(all="ignore"):
        oracle = O.linear_fp64(x.float().numpy(), packed, scales)
    if scale == 254:
        # +-inf weights: the IEEE outcome (NaN where +inf and -inf meet) is
        # independent of summation order and must match exactly.
        assert np.array_equal(np.isnan(y), np.isnan(oracle))
        fin = ~np.isnan(oracle)
        assert np.array_equal(y[fin], oracle[fin])  # all +-inf
    else:
        assert np.all(np.isfinite(y))
        assert_parity(y, oracle, what="scale 1 (subnormal weights)")
