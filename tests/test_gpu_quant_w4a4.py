"""GPU parity: the activation quantizer (bit-exact vs the oracle, both
modes) and W4A4 on the block-scaled FP4 MFMA (tolerance vs FP64)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import mxfp4_amd as mx
from oracle import c_oracle, mxfp4_oracle as O

from _helpers import assert_parity, cuda, rand_act, rand_mxfp4

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("mode", ["ties_away", "rne"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_quant_matches_oracle(mode, dtype):
    g = torch.Generator().manual_seed(99)
    x = torch.randn((64, 2048), generator=g) * torch.exp2(torch.randint(-20, 20, (64, 1),
                                                                           generator=g).float())
    x[0, :32] = 0.0
    x[1, :8] = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -5.0])
    x[2, 3] = -0.0
    x = x.to(dtype)
    p, s = mx.dynamic_mxfp4_quant(cuda(x), mode=mode)
    rp, rs = c_oracle.quant(x.float().numpy(), mode)
    assert np.array_equal(p.cpu().numpy(), rp) and np.array_equal(s.cpu().numpy(), rs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_rne_encoder_path_matches_scalar_path(dtype):
    # 16-bit inputs with aligned rows take the FP4-encoder kernel; a view
    # one element off the alignment takes the scalar kernel.  Both must give
    # the same bytes, also for NaN, inf, subnormal and all-zero blocks.
    g = torch.Generator().manual_seed(7)
    rows, k = 96, 1024
    x = torch.randn((rows, k), generator=g) * torch.exp2(
        torch.randint(-30, 30, (rows, k // 32), generator=g).float()).repeat_interleave(32, 1)
    x = x.to(dtype)
    info = torch.finfo(dtype)
    x[0, 5] = float("nan")
    x[1, :32] = float("nan")
    x[2, 7] = float("inf")
    x[3, 9] = -float("inf")
    x[4, :32] = 0.0
    x[5, :32] = info.tiny * torch.linspace(-1, 1, 32).to(dtype)  # near the subnormal range
    x[6, :32] = info.max
    x[7, 0] = -0.0
    x[8, 40] = float("nan")
    x[8, 41] = info.max
    big = torch.zeros((rows, k + 8), dtype=dtype)
    big[:, 1:1 + k] = x
    xa = cuda(x)
    xm = cuda(big)[:, 1:1 + k]  # base pointer 2 bytes off a 16-byte boundary
    assert xa.data_ptr() % 16 == 0 and xm.data_ptr() % 16 == 2
    pa, sa = mx.dynamic_mxfp4_quant(xa, mode="rne")
    pm, sm = mx.dynamic_mxfp4_quant(xm, mode="rne")
    assert torch.equal(pa, pm) and torch.equal(sa, sm)
    finite = torch.isfinite(x).all(dim=1)
    rp, rs = c_oracle.quant(x[finite].float().numpy(), "rne")
    assert np.array_equal(pa[cuda(finite)].cpu().numpy(), rp)
    assert np.array_equal(sa[cuda(finite)].cpu().numpy(), rs)


def test_quant_golden_fixture():
    g = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    x = cuda(g["quant_x"])
    p, s = mx.dynamic_mxfp4_quant(x, "ties_away")
    assert np.array_equal(p.cpu().numpy(), g["quant_ta_p"])
    assert np.array_equal(s.cpu().numpy(), g["quant_ta_s"])
    p, s = mx.dynamic_mxfp4_quant(x, "rne")
    assert np.array_equal(p.cpu().numpy(), g["quant_rne_p"])
    assert np.array_equal(s.cpu().numpy(), g["quant_rne_s"])


@pytest.mark.parametrize("m,k,n", [(1, 128, 64), (16, 4096, 256), (100, 2080, 300),
                                   (256, 1024, 512)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_w4a4_linear(m, k, n, out_dtype):
    rng = np.random.default_rng(m * 31 + n)
    a = rand_act(m + k, (m, k)).float().numpy()
    w = (rand_act(n + k, (n, k)).float() * 0.02).numpy()
    ap, asc = O.quant_mxfp4_rne(a)
    wp, wsc = O.quant_mxfp4_rne(w)
    y = mx.linear_mxfp4_w4a4(cuda(ap), cuda(asc), cuda(wp), cuda(wsc), out_dtype)
    oracle = O.dequant_values(ap, asc, "f32") @ O.dequant_values(wp, wsc, "f32").T
    assert_parity(y, oracle, what=f"w4a4 {m}x{k}x{n}")
    del rng


@pytest.mark.parametrize("m,n,out_dtype", [(4096, 4096, torch.bfloat16), (2048, 2048, torch.float16),
                                           (2048, 4096, torch.float32), (1000, 4100, torch.bfloat16),
                                           (4096, 4096, torch.float32), (4000, 4100, torch.float16)],
                         ids=["256x256", "128x128", "f32_out", "partial", "f32_256x256",
                              "partial_256x256"])
@pytest.mark.parametrize("k", [256, 1536], ids=["scale_stage", "scale_group4"])
def test_w4a4_tile_configs(m, n, out_dtype, k):
    # grids large enough for the 256 x 256 (>= 256 tiles) / 128 x 128 tiles,
    # FP32 output, and partial row / column tiles; checked on sampled rows.
    # K = 256 stages the scales one 128-deep stage at a time, K = 1536
    # (a multiple of 512) four stages per 16-byte load.
    a = rand_act(m + 1, (m, k)).float().numpy()
    w = (rand_act(n + 2, (n, k)).float() * 0.02).numpy()
    ap, asc = O.quant_mxfp4_rne(a)
    wp, wsc = O.quant_mxfp4_rne(w)
    y = mx.linear_mxfp4_w4a4(cuda(ap), cuda(asc), cuda(wp), cuda(wsc), out_dtype)
    assert y.dtype == out_dtype and y.shape == (m, n)
    rows = np.sort(np.concatenate([np.random.default_rng(m).choice(m, 48, replace=False), [m - 1]]))
    oracle = O.dequant_values(ap[rows], asc[rows], "f32") @ O.dequant_values(wp, wsc, "f32").T
    assert_parity(y[torch.from_numpy(rows).cuda()], oracle, what=f"w4a4 {m}x{k}x{n}")


@pytest.mark.parametrize("m,n", [(5000, 9000), (4000, 4100)], ids=["720_tiles", "partial"])
def test_w4a4_multi_round_grid(m, n):
    # more 256 x 256 tiles than CUs on a dense grid (K % 512 == 0: grouped
    # scales, 256-deep stages): 720 / 272 tiles in rounds of 256
    # workgroups, partial row and column tiles; sampled rows, the last one
    # included
    k = 1024
    a = rand_act(m + 3, (m, k)).float().numpy()
    w = (rand_act(n + 4, (n, k)).float() * 0.02).numpy()
    ap, asc = O.quant_mxfp4_rne(a)
    wp, wsc = O.quant_mxfp4_rne(w)
    y = mx.linear_mxfp4_w4a4(cuda(ap), cuda(asc), cuda(wp), cuda(wsc), torch.bfloat16)
    assert y.shape == (m, n)
    rows = np.sort(np.concatenate([np.random.default_rng(m).choice(m - 1, 40, replace=False),
                                   [m - 1]]))
    oracle = O.dequant_values(ap[rows], asc[rows], "f32") @ O.dequant_values(wp, wsc, "f32").T
    assert_parity(y[torch.from_numpy(rows).cuda()], oracle, what=f"w4a4 multi-round {m}x{k}x{n}")


@pytest.mark.parametrize("which", ["a", "w"])
@pytest.mark.parametrize("m,n", [(4096, 4096), (2048, 2048)], ids=["256x256", "128x128"])
def test_w4a4_scale_rows_off_16_bytes(which, m, n):
    # scale rows that start 4 bytes past a 16-byte boundary take the
    # per-stage-scale kernel (3 stages of 128) instead of the grouped-scale
    # one (2 stages of 256); both accumulate in the same K order, so the
    # outputs are bitwise equal; and both match the oracle on sampled rows
    # (256 x 256 tiles at 4096 x 4096, 128 x 128 at 2048 x 2048)
    k = 1024
    a = rand_act(11, (m, k)).float().numpy()
    w = (rand_act(12, (n, k)).float() * 0.02).numpy()
    ap, asc = O.quant_mxfp4_rne(a)
    wp, wsc = O.quant_mxfp4_rne(w)
    ap_d, asc_d, wp_d, wsc_d = cuda(ap), cuda(asc), cuda(wp), cuda(wsc)
    ref = mx.linear_mxfp4_w4a4(ap_d, asc_d, wp_d, wsc_d)

    def off4(t):
        buf = torch.zeros(t.numel() + 16, dtype=torch.uint8, device="cuda")
        v = buf[4:4 + t.numel()].view(t.shape)
        v.copy_(t)
        assert v.is_contiguous() and v.data_ptr() % 16 == 4
        return v

    if which == "a":
        y = mx.linear_mxfp4_w4a4(ap_d, off4(asc_d), wp_d, wsc_d)
    else:
        y = mx.linear_mxfp4_w4a4(ap_d, asc_d, wp_d, off4(wsc_d))
    assert torch.equal(y, ref)
    rows = np.sort(np.random.default_rng(13).choice(m, 32, replace=False))
    oracle = O.dequant_values(ap[rows], asc[rows], "f32") @ O.dequant_values(wp, wsc, "f32").T
    assert_parity(y[torch.from_numpy(rows).cuda()], oracle, what=f"w4a4 scales off 16 ({which}, {m}x{n})")


def test_w4a4_baseline_shape_sampled():
    # M=8192, K=4096, N=4096 (checked on sampled rows)
    m, k, n = 8192, 4096, 4096
    a = rand_act(4, (m, k))
    w = rand_act(5, (n, k)).float() * 0.02
    ap, asc = mx.dynamic_mxfp4_quant(cuda(a), "rne")
    wp, wsc = mx.dynamic_mxfp4_quant(cuda(w), "rne")
    y = mx.linear_mxfp4_w4a4(ap, asc, wp, wsc)
    rows = np.sort(np.random.default_rng(6).choice(m, 64, replace=False))
    apn, ascn = ap.cpu().numpy()[rows], asc.cpu().numpy()[rows]
    oracle = O.dequant_values(apn, ascn, "f32") @ O.dequant_values(
        wp.cpu().numpy(), wsc.cpu().numpy(), "f32").T
    assert_parity(y[torch.from_numpy(rows).cuda()], oracle)


@pytest.mark.parametrize("m", [3, 64])
def test_w4a4_through_fused_moe(m):
    rng = np.random.default_rng(m)
    e, k, n, top_k = 6, 256, 128, 2
    wp, ws = rand_mxfp4(rng, (e, n), k)
    ap, asc = O.quant_mxfp4_ties_away(rand_act(m, (m, k)).float().numpy())
    g = torch.Generator().manual_seed(m)
    w, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
    C = torch.empty((m, top_k, n), dtype=torch.bfloat16, device="cuda")
    mx.fused_moe_mxfp4_soft(cuda(ap), cuda(wp), C, torch.tensor([0.75], device="cuda"),
                            torch.linspace(0.5, 1.25, e, device="cuda"), cuda(asc), cuda(ws),
                            cuda(w), cuda(ids), torch.empty(0, device="cuda"),
                            torch.empty(0, device="cuda"), torch.empty(0, device="cuda"), True,
                            top_k, False, False)
    oracle = O.fused_moe_fp64(O.dequant_values(ap, asc, "bf16"), wp, ws, 0.75,
                              np.linspace(0.5, 1.25, e), w.numpy(), ids.numpy(), True)
    assert_parity(C, oracle)
