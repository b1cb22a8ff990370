"""Write the committed golden fixtures under tests/golden/.

    python tests/golden/gen_golden.py

The reference repository commits no data fixtures (its only known answer is
tests/test_moe_mxfp4_soft.py:81-92), so these are generated from the
closed-form oracle, which tests/test_oracle.py pins independently:

* ``dequant_table.npz`` -- for every E8M0 scale s (rows) and every E2M1 code
  (columns, 16 codes twice = one 32-value block): the dequantized bit
  patterns for float32, bfloat16 and float16 outputs (soft:277-307), plus
  the packed input bytes.  Built by the C integer construction and checked
  against the numpy ldexp construction before it is written.
* ``small_cases.npz`` -- seeded tiny linear / routed-MoE / MoE-layer inputs
  with their FP64-accumulated oracle outputs and routing metadata, and both
  quantizers' codes for a seeded activation block including tie values.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import c_oracle, mxfp4_oracle as O  # noqa: E402


def dequant_table():
    codes = np.concatenate([np.arange(16), np.arange(16)]).astype(np.uint8)
    packed = np.tile(O.pack_codes(codes), (256, 1))
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    out = {"packed": packed, "scales": scales}
    for dt in ("f32", "bf16", "f16"):
        c_bits = c_oracle.dequant_bits(packed, scales, dt)
        np_bits = O.dequant_bits(packed, scales, dt)
        assert np.array_equal(c_bits, np_bits), dt
        out[dt] = c_bits
    return out


def random_mxfp4(rng, shape_rows, k, lo=120, hi=128):
    packed = rng.integers(0, 256, size=(*shape_rows, k // 2), dtype=np.uint8)
    scales = rng.integers(lo, hi + 1, size=(*shape_rows, k // 32), dtype=np.uint8)
    return packed, scales


def bf16_round(a):
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.asarray(a, dtype=np.float32)))


def small_cases():
    rng = np.random.default_rng(20260810)
    out = {}
    # dense linear: M=5, N=48, K=256 (bf16 x)
    x = bf16_round(rng.standard_normal((5, 256)))
    w, s = random_mxfp4(rng, (48,), 256)
    out.update(lin_x=x, lin_w=w, lin_s=s, lin_y=O.linear_fp64(x, w, s))
    # routed MoE: M=6, E=4, top_k=2, N=40, K=128, with an out-of-range id
    a = bf16_round(rng.standard_normal((6, 128)))
    bw, bs = random_mxfp4(rng, (4, 40), 128)
    ids = rng.integers(0, 4, size=(6, 2)).astype(np.int64)
    ids[5, 1] = 7  # outside [0, E): slot stays zero
    tw = rng.random((6, 2)).astype(np.float32)
    b_scale = np.linspace(0.5, 1.25, 4).astype(np.float32)
    out.update(moe_a=a, moe_b=bw, moe_bs=bs, moe_ids=ids, moe_w=tw, moe_bscale=b_scale,
               moe_ascale=np.array([0.75], np.float32),
               moe_c=O.fused_moe_fp64(a, bw, bs, 0.75, b_scale, tw, ids, True))
    srt, exp_, npp = O.make_routing(ids, block_m=16, num_experts=4)
    out.update(route_sorted=srt, route_experts=exp_, route_npp=npp)
    # MoE layer: M=3, E=4, top_k=2, H=64, I=32
    xl = bf16_round(rng.standard_normal((3, 64)))
    w13, s13 = random_mxfp4(rng, (4, 64), 64)
    w2, s2 = random_mxfp4(rng, (4, 64), 32)
    lids = np.array([[0, 3], [1, 0], [2, 2]], dtype=np.int64)
    lw = np.array([[0.7, 0.3], [0.6, 0.4], [0.5, 0.5]], dtype=np.float32)
    out.update(layer_x=xl, layer_w13=w13, layer_s13=s13, layer_w2=w2, layer_s2=s2,
               layer_ids=lids, layer_w=lw,
               layer_y=O.moe_layer_fp64(xl, w13, s13, w2, s2, lw, lids))
    # quantizers on a block with exact ties (q = 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5)
    q = rng.standard_normal((4, 64)).astype(np.float32)
    q[0, :8] = np.array([4.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    q[0, 8:16] = -q[0, :8]
    pa, sa = O.quant_mxfp4_ties_away(q)
    pr, sr = O.quant_mxfp4_rne(q)
    out.update(quant_x=q, quant_ta_p=pa, quant_ta_s=sa, quant_rne_p=pr, quant_rne_s=sr)
    return out


def main():
    np.savez_compressed(os.path.join(HERE, "dequant_table.npz"), **dequant_table())
    np.savez_compressed(os.path.join(HERE, "small_cases.npz"), **small_cases())
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
