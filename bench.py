#!/usr/bin/env python
"""Benchmark of the MXFP4 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]

Prints ONE JSON line.  The headline (``value``) is BASELINE config 2's
prefill point: the dense W4A16 linear at qkv_proj shape M=4096, K=2048,
N=5120 (bf16 activations ~N(0,1), E2M1 codes uniform 0..15, E8M0 scales
uniform 120..128, seeded), in TFLOP/s.  A step is one
``linear_mxfp4_soft`` call on HBM-resident inputs, with the weights'
prepacked copy (``prepack_w4a16``, made once before timing, as the vLLM
adapter does when the weights are loaded); the same call on the checkpoint
layout alone is timed beside it (``roofline.checkpoint_layout_kernel_us``).
K steps are timed with a
device synchronisation on both sides, after W untimed warmup steps that
follow an untimed clock ramp (RAMP_MS of back-to-back calls: MI355X takes
~10-15 ms of sustained work to reach its steady clocks, and every timing
here is of the steady state).  ``roofline`` is for that step's only
kernel (w4a16_pf, the direct-to-LDS prefill GEMM), its average duration
taken from HIP events on the stream it is launched on; ``traffic`` is the
HBM bytes per launch measured with rocprofv3 counters (FETCH_SIZE and
WRITE_SIZE, each scaled by what the counter reads for a copy of known size)
on ``bench.py --traffic-probe`` and recorded in
profiles/w4a16_pf_qkv_prefill_traffic.md, or null when that file is absent.  ``sweep`` carries the other BASELINE points:
decode W4A16 GEMV (HBM GB/s, weights rotated over >= 512 MB so the 256 MB
MALL cannot serve them, launches replayed from a HIP graph), the routed MoE
layer (us, 3 weight copies rotated), the soft op (C bf16 at 512 and 4096
tokens, C FP32 on the FP32 MFMA at 512) and the AITER entry on caller
metadata (3 weight copies rotated; ``us_one_copy`` replays a single copy,
whose weights the MALL then serves), W4A4 on the
block-scaled FP4 MFMA, and the standalone dequant.
``cpu_baseline`` times the reference safe path (explicit dequant +
torch.matmul bf16, restated in oracle/) on this host's cores on a bounded
row sample of the headline workload; ``cpu_config1`` times it on BASELINE
config 1 (M=64, K=2048, N=2048; seconds and GFLOP/s), and every sweep row
carries ``cpu_ms``, the same restatement at that row's shape (the MoE layer
as the per-expert loop of the safe op composed as the vLLM layer), under a
per-row time cap.
"""

from __future__ import annotations

import argparse
import itertools
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mxfp4-gfx936_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP4_PEAK_TFLOPS = 10100.0
FP32_PEAK_TFLOPS = 157.3
METRIC = ("W4A16 GEMM TFLOP/s (prefill) & HBM GB/s (decode), % roofline; MoE layer µs")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def rand_weights(rng, rows, k, copies=1):
    import numpy as np
    import torch
    out = []
    for _ in range(copies):
        p = torch.from_numpy(rng.integers(0, 256, size=(*rows, k // 2), dtype=np.uint8)).cuda()
        s = torch.from_numpy(rng.integers(120, 129, size=(*rows, k // 32), dtype=np.uint8)).cuda()
        out.append((p, s))
    return out


def randn_bf16(seed, shape):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16).cuda()


RAMP_MS = 40.0


def ramp_clocks(fn, ms=RAMP_MS):
    """Call fn back to back for `ms` of wall time, untimed.  After an idle
    spell MI355X raises its clocks over the first ~10-15 ms of sustained
    work (measured on the headline kernel: ~86 us per launch for the first
    20 launches, ~78 us from about the 140th on, flat for the next 0.5 s),
    so timing right after start-up measures the ramp, not the kernel."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_eager(fn, steps, warmup):
    """(wall ms per step, HIP-event ms per step) over `steps` calls, after
    the clock ramp and `warmup` untimed calls."""
    import torch
    ramp_clocks(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, start.elapsed_time(end) / steps


def time_graph(fns, replays=20):
    """Capture one call of each fn (rotating inputs) in a HIP graph; return
    the device time per call (ms), from events around graph replays."""
    import torch
    for f in fns:  # warm up outside capture (allocator, library load)
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for f in fns:
                f()
    torch.cuda.current_stream().wait_stream(s)
    ramp_clocks(g.replay)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * len(fns))


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "w4a16_pf_qkv_prefill_traffic.md")
COPY_BYTES = 256 << 20  # the calibration copy of --traffic-probe, each direction


def recorded_traffic():
    """HBM bytes per headline launch from the committed counter summary:
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the prefill kernel, each
    scaled by COPY_BYTES / (the counter's reading for the calibration copy)."""
    vals = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("- ") and ":" in line:
                    key, _, val = line[2:].partition(":")
                    try:
                        vals[key.strip()] = float(val.split()[0])
                    except (ValueError, IndexError):
                        pass
    except OSError:
        return None
    need = ("kernel_fetch_kib", "kernel_write_kib", "copy_fetch_kib", "copy_write_kib")
    if not all(k in vals and vals[k] > 0 for k in need):
        return None
    fetch = vals["kernel_fetch_kib"] * COPY_BYTES / vals["copy_fetch_kib"]
    write = vals["kernel_write_kib"] * COPY_BYTES / vals["copy_write_kib"]
    return int(round(fetch + write))


def traffic_probe() -> int:
    """Headline kernel launches plus a 256 MiB device copy, for counter runs
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE -- python3 bench.py --traffic-probe)."""
    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    m, k, n = 4096, 2048, 5120
    rng = np.random.default_rng(20260810 + 1)
    (w, s), = rand_weights(rng, (n,), k)
    x = randn_bf16(20260810, (m, k))
    pre = mx.prepack_w4a16(w, s)
    for _ in range(12):
        mx.linear_mxfp4_soft(x, w, s, prepacked=pre)
    a = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "traffic", "linear_launches": 12, "copy_bytes": COPY_BYTES}))
    return 0


def headline_probe() -> int:
    """Headline launches for trace and counter runs: qkv M=4096, K=2048,
    N=5120 with the prepacked copy, then on the checkpoint layout, each
    after an untimed clock ramp, 20 launches."""
    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    m, k, n = 4096, 2048, 5120
    rng = np.random.default_rng(20260810 + 1)
    (w, s), = rand_weights(rng, (n,), k)
    x = randn_bf16(20260810, (m, k))
    pre = mx.prepack_w4a16(w, s)
    for name, q in (("prepacked", pre), ("checkpoint", None)):
        ramp_clocks(lambda: mx.linear_mxfp4_soft(x, w, s, prepacked=q))
        for _ in range(20):
            mx.linear_mxfp4_soft(x, w, s, prepacked=q)
        torch.cuda.synchronize()
        log(f"headline probe {name} done")
    print(json.dumps({"probe": "headline", "m": m, "k": k, "n": n}))
    return 0


def decode_probe() -> int:
    """Decode launches for counter and trace runs of the bandwidth-bound
    kernels: dense W4A16 GEMV (qkv M=1 and 8, o_proj M=1) over rotated weight
    copies (>= 256 MB, so the MALL cannot hold them), the MoE layer at M=1
    and 8 over 2 weight copies, then the 256 MiB calibration copy."""
    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    for name, k, n, ms in (("qkv", 2048, 5120, (1, 8)), ("o_proj", 4096, 2048, (1,))):
        rng = np.random.default_rng(20260811 + k)
        copies = (300 << 20) // (n * k // 2 + n * k // 32) + 1
        ws = rand_weights(rng, (n,), k, copies)
        for m in ms:
            x = randn_bf16(20260811 + m, (m, k))
            for p, s in ws:
                mx.linear_mxfp4_soft(x, p, s)
        del ws
    e, hidden, inter, top_k = 128, 2048, 768, 8
    rng = np.random.default_rng(20260815)
    layers = []
    for _ in range(2):
        (w13, s13), = rand_weights(rng, (e, 2 * inter), hidden)
        (w2, s2), = rand_weights(rng, (e, hidden), inter)
        layers.append((w13, s13, w2, s2))
    for m in (1, 8):
        g = torch.Generator().manual_seed(20260817 + m)
        w, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
        w = (w / w.sum(-1, keepdim=True)).cuda()
        ids = ids.cuda()
        x = randn_bf16(20260816 + m, (m, hidden))
        for _ in range(3):
            for c in layers:
                mx.moe_layer(x, *c, w, ids)
    a = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "decode", "copy_bytes": COPY_BYTES}))
    return 0


def moe_probe() -> int:
    """MoE layer prefill launches for trace and counter runs of the routed
    GEMMs: E=128, top-8, H=2048, I=768 with prepacked weights, 512 and 4096
    tokens, each after an untimed clock ramp, 20 launches; then the 256 MiB
    calibration copy of --traffic-probe (FETCH_SIZE / WRITE_SIZE scale)."""
    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    e, hidden, inter, top_k = 128, 2048, 768, 8
    rng = np.random.default_rng(20260815)
    (w13, s13), = rand_weights(rng, (e, 2 * inter), hidden)
    (w2, s2), = rand_weights(rng, (e, hidden), inter)
    pre = {"prepacked13": mx.prepack_w4a16(w13, s13), "prepacked2": mx.prepack_w4a16(w2, s2)}
    for m in (512, 4096):
        g = torch.Generator().manual_seed(20260817 + m)
        w, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
        w = (w / w.sum(-1, keepdim=True)).cuda()
        ids = ids.cuda()
        x = randn_bf16(20260816 + m, (m, hidden))
        ramp_clocks(lambda: mx.moe_layer(x, w13, s13, w2, s2, w, ids, **pre))
        for _ in range(20):
            mx.moe_layer(x, w13, s13, w2, s2, w, ids, **pre)
        torch.cuda.synchronize()
        log(f"moe probe m={m} done")
    del pre
    a = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "moe", "m": [512, 4096], "copy_bytes": COPY_BYTES}))
    return 0


def w4a4_probe() -> int:
    """W4A4 launches for trace and counter runs: packed MXFP4 activations x
    packed MXFP4 weights at M=8192, K=N=4096, bf16 out,
    an untimed clock ramp, then 20 launches."""
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    m, k, n = 8192, 4096, 4096
    a = randn_bf16(4, (m, k))
    wt = randn_bf16(5, (n, k)).float() * 0.02
    ap, asc = mx.dynamic_mxfp4_quant(a, "rne")
    wp, wsc = mx.dynamic_mxfp4_quant(wt, "rne")
    ramp_clocks(lambda: mx.linear_mxfp4_w4a4(ap, asc, wp, wsc))
    for _ in range(20):
        mx.linear_mxfp4_w4a4(ap, asc, wp, wsc)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "w4a4", "m": m, "k": k, "n": n}))
    return 0


def data_probe() -> int:
    """Steady-clock time of the headline GEMM on random inputs (the bench's)
    and on all-zero / constant ones.  The kernel and the work are the same;
    only the data differs, so a gap is the chip's power management lowering
    the clock while random operands keep the MFMAs switching."""
    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    m, k, n = 4096, 2048, 5120
    rng = np.random.default_rng(20260810 + 1)
    (w, s), = rand_weights(rng, (n,), k)
    x = randn_bf16(20260810, (m, k))
    cases = {
        "random": (x, w),
        "zeros": (torch.zeros_like(x), torch.zeros_like(w)),
        "x_zero": (torch.zeros_like(x), w),
        "codes_zero": (x, torch.zeros_like(w)),
        "constant": (torch.full_like(x, 1.5), torch.full_like(w, 0x22)),
    }
    res = {}
    for name, (xa, wa) in cases.items():
        pre = mx.prepack_w4a16(wa, s)
        ramp_clocks(lambda: mx.linear_mxfp4_soft(xa, wa, s, prepacked=pre))
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(300):
            mx.linear_mxfp4_soft(xa, wa, s, prepacked=pre)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / 300 * 1e3
        res[name] = {"us": round(us, 2), "tflops": round(2.0 * m * n * k / us / 1e6, 1)}
        log(f"data probe {name}: {us:.2f} us")
    print(json.dumps({"probe": "data", "m": m, "k": k, "n": n, "results": res}))
    return 0


PROBE_LIB = os.path.join(ROOT, "mxfp4-gfx936_amd", "mxfp4_amd", "libmxfp4_probe.so")
_floor_cache = {}


def read_floor_us(torch, nbytes):
    """Device time (us) of one launch of a plain HBM read of `nbytes`
    (csrc/probe/read_floor.hip: every load in flight before any is used),
    graph-replayed over rotating buffers of >= 600 MB in all, as the decode
    rows are: the floor a single decode launch over those bytes cannot beat.
    None when the probe library is not built."""
    import ctypes
    nbytes = (int(nbytes) + 15) // 16 * 16
    if nbytes in _floor_cache:
        return _floor_cache[nbytes]
    if not os.path.exists(PROBE_LIB):
        return None
    lib = ctypes.CDLL(PROBE_LIB)
    lib.mxfp4_probe_read_floor_sink_words.restype = ctypes.c_int64
    lib.mxfp4_probe_read_floor_sink_words.argtypes = [ctypes.c_int64]
    lib.mxfp4_probe_read_floor.restype = ctypes.c_int
    lib.mxfp4_probe_read_floor.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_void_p]
    copies = max(1, min(128, (600 << 20) // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 256)
            for _ in range(copies)]
    words = int(lib.mxfp4_probe_read_floor_sink_words(nbytes))
    sink = torch.empty(words, dtype=torch.int32, device="cuda")

    def fn(b):
        rc = lib.mxfp4_probe_read_floor(b.data_ptr(), nbytes, sink.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError("read-floor probe launch failed")

    t = time_graph([lambda b=b: fn(b) for b in bufs], replays=10) * 1e3
    del bufs, sink
    _floor_cache[nbytes] = t
    return t


def linear_bytes(m, n, k, prepacked=False):
    """Algorithmic bytes of one W4A16 linear: weights (nibbles + scales: one
    byte per 32 on the checkpoint layout, two in the prepacked copy), x, out."""
    return n * k // 2 + n * k // (16 if prepacked else 32) + 2 * m * k + 2 * m * n


def soft_op_cases(mx, torch, np, copies=3):
    """(name, calls, FLOPs, peak) of the soft-op and AITER-entry rows: BASELINE
    config 3's gate_up shape (E=128, top-8, K=2048, N=1536), seeded.  `calls`
    holds one call per weight copy: the 201 MB of one copy fit the 256 MB
    MALL, so replaying a single copy would time MALL-resident weights, where
    a serving step finds a layer's weights in HBM."""
    e, k, n, top_k = 128, 2048, 1536, 8
    rng = np.random.default_rng(20260818)
    wcs = rand_weights(rng, (e, n), k, copies)
    one, ones_e, empty = (torch.ones(1, device="cuda"), torch.ones(e, device="cuda"),
                          torch.empty(0, device="cuda"))
    regs = []
    cases = []
    for m, cdt, name in ((512, torch.bfloat16, "bf16"), (4096, torch.bfloat16, "bf16"),
                         (512, torch.float32, "f32")):
        a = randn_bf16(20260819, (m, k))
        g = torch.Generator().manual_seed(20260820)
        tw, ids = torch.topk(torch.softmax(torch.randn((m, e), generator=g), -1), top_k, dim=-1)
        tw, ids = tw.cuda(), ids.cuda()
        C = torch.empty((m, top_k, n), dtype=cdt, device="cuda")
        fl = 2.0 * m * top_k * n * k
        peak = FP32_PEAK_TFLOPS if cdt == torch.float32 else BF16_PEAK_TFLOPS

        def soft(ws, a=a, C=C, tw=tw, ids=ids):
            return [lambda wp=wp, wsc=wsc: mx.fused_moe_mxfp4_soft(
                a, wp, C, one, ones_e, None, wsc, tw, ids, empty, empty, empty, True, top_k,
                False, False) for wp, wsc in ws]

        def aiter(ws, bm, a=a, C=C, tw=tw, ids=ids):
            srt, eid, npp = mx.make_routing_device(ids, e, bm)
            return [lambda wp=wp, wsc=wsc: mx.fused_moe_mxfp4(
                a, wp, C, one, ones_e, None, wsc, tw, ids, srt, eid, npp, True, top_k, False,
                False, {"BLOCK_SIZE_M": bm}, torch.bfloat16) for wp, wsc in ws]

        cases.append((f"fused_moe_soft_c{name}_m{m}", soft(wcs), fl, peak))
        if m == 512 and cdt == torch.bfloat16:
            for bm in (32, 64):
                cases.append((f"aiter_fused_moe_bm{bm}_m{m}", aiter(wcs, bm), fl,
                              BF16_PEAK_TFLOPS))
        if cdt == torch.bfloat16:
            # the same calls with a registered prepacked copy of B (second
            # weight tensors, so the rows above keep the checkpoint layout)
            if not regs:
                for wp, wsc in wcs:
                    wp_r, wsc_r = wp.clone(), wsc.clone()
                    mx.register_prepacked(wp_r, wsc_r)
                    regs.append((wp_r, wsc_r))
            cases.append((f"fused_moe_soft_c{name}_m{m}_registered", soft(regs), fl, peak))
            if m == 512:
                cases.append((f"aiter_fused_moe_bm64_m{m}_registered", aiter(regs, 64), fl,
                              BF16_PEAK_TFLOPS))
    return cases


def soft_probe() -> int:
    """Soft-op and AITER-entry launches for trace runs (the soft_op_cases
    rows): per row an untimed clock ramp and 20 timed calls, both over the
    rotated weight copies, then a one-element fill kernel as the row's end
    marker."""
    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    for key, fns, _, _ in soft_op_cases(mx, torch, np):
        # the ramp rotates the copies too: after a ramp on one (MALL-served)
        # copy the rotated calls of the prepacked rows ran 8-10 us slower
        rot = itertools.cycle(fns)
        ramp_clocks(lambda: next(rot)())
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(20):
            fns[i % len(fns)]()
        end.record()
        # a one-element fill marks the end of the case's launches in a trace
        torch.full((1,), 0.0, device="cuda")
        torch.cuda.synchronize()
        log(f"soft probe {key}: {start.elapsed_time(end) * 1e3 / 20:.2f} us per call "
            "(20 calls over the rotated copies)")
    print(json.dumps({"probe": "soft"}))
    return 0


def sweep(mx, torch, np):
    res = {}
    # --- decode / mid W4A16
    for name, k, n in (("qkv", 2048, 5120), ("o_proj", 4096, 2048)):
        for m in (1, 8, 370) + ((4096,) if name == "o_proj" else ()):
            rng = np.random.default_rng(20260811 + m + k)
            wbytes = n * k // 2 + n * k // 32
            copies = max(1, min(128, (600 << 20) // wbytes)) if m <= 370 else 1
            ws = rand_weights(rng, (n,), k, copies)
            x = randn_bf16(20260811 + m, (m, k))
            # prepacked copies as loaded by the vLLM adapter (the decode
            # kernels read the checkpoint layout; the copy serves prefill)
            pres = [mx.prepack_w4a16(p, s) if m >= 370 else None for p, s in ws]
            fns = [lambda p=p, s=s, q=q: mx.linear_mxfp4_soft(x, p, s, prepacked=q)
                   for (p, s), q in zip(ws, pres)]
            if m <= 370:
                t = time_graph(fns, replays=10)
            else:
                t = time_eager(fns[0], 20, 5)[1]
            b = linear_bytes(m, n, k)
            fl = 2.0 * m * n * k
            res[f"w4a16_{name}_m{m}"] = {
                "us": round(t * 1e3, 3), "GB/s": round(b / t / 1e6, 1),
                "hbm_frac": round(b / t / 1e6 / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(fl / t / 1e9, 2),
                "mfma_frac": round(fl / t / 1e9 / BF16_PEAK_TFLOPS, 4),
                "weight_copies": copies}
            del ws, pres
            if m <= 8:
                fl_us = read_floor_us(torch, b)
                if fl_us is not None:
                    res[f"w4a16_{name}_m{m}"].update(
                        {"read_floor_us": round(fl_us, 3),
                         "floor_frac": round(fl_us / (t * 1e3), 4)})
            log(f"{name} m={m}: {res[f'w4a16_{name}_m{m}']}")
    torch.cuda.empty_cache()
    # --- routed MoE layer (BASELINE configs 3 and 5)
    e, hidden, inter, top_k = 128, 2048, 768, 8
    rng = np.random.default_rng(20260815)
    layer_copies = []
    for _ in range(3):
        (w13, s13), = rand_weights(rng, (e, 2 * inter), hidden)
        (w2, s2), = rand_weights(rng, (e, hidden), inter)
        layer_copies.append(((w13, s13, w2, s2),
                             {"prepacked13": mx.prepack_w4a16(w13, s13),
                              "prepacked2": mx.prepack_w4a16(w2, s2)}))
    per_expert = 2 * inter * hidden // 2 + 2 * inter * hidden // 32 + hidden * inter // 2 + \
        hidden * inter // 32
    for m in (1, 8, 32, 512, 4096):
        g = torch.Generator().manual_seed(20260817 + m)
        logits = torch.randn((m, e), generator=g)
        w, ids = torch.topk(torch.softmax(logits, -1), top_k, dim=-1)
        w = (w / w.sum(-1, keepdim=True)).cuda()
        ids = ids.cuda()
        x = randn_bf16(20260816 + m, (m, hidden))
        e_active = int(torch.unique(ids).numel())
        fns = [lambda c=c, q=q: mx.moe_layer(x, *c, w, ids, **q) for c, q in layer_copies]
        if m <= 512:
            t = time_graph(fns, replays=10)
        else:
            t = time_eager(fns[0], 10, 3)[1]
        b = e_active * per_expert + 4 * m * hidden + 8 * m * top_k
        fl = 2.0 * m * top_k * (hidden * 2 * inter + inter * hidden)
        res[f"moe_layer_m{m}"] = {
            "us": round(t * 1e3, 2), "e_active": e_active, "GB/s": round(b / t / 1e6, 1),
            "hbm_frac": round(b / t / 1e6 / HBM_PEAK_GBS, 4), "TFLOP/s": round(fl / t / 1e9, 2),
            "mfma_frac": round(fl / t / 1e9 / BF16_PEAK_TFLOPS, 4)}
        if m <= 32:
            fl_us = read_floor_us(torch, b)
            if fl_us is not None:
                res[f"moe_layer_m{m}"].update({"read_floor_us": round(fl_us, 3),
                                               "floor_frac": round(fl_us / (t * 1e3), 4)})
        log(f"moe m={m}: {res[f'moe_layer_m{m}']}")
    del layer_copies
    torch.cuda.empty_cache()
    # --- the soft op (soft:379-494) on BASELINE config 3's gate_up shape
    # (E=128, top-8, K=2048, N=1536): C bf16 at 512 and 4096 tokens, C fp32
    # (the FP32 compute path, soft:405-407) at 512; each call builds the
    # routing on the device and writes all of C.  Beside it the AITER entry
    # (aiter:367-472) on caller metadata of BLOCK_SIZE_M 32 and 64 at 512
    # tokens (the metadata is built once, outside the timing, as a caller
    # would pass it in).
    for key, fns, fl, peak in soft_op_cases(mx, torch, np):
        t = time_graph(fns, replays=10)
        t1 = time_graph([fns[0]] * len(fns), replays=10)
        rot = itertools.cycle(fns)
        te = time_eager(lambda: next(rot)(), 21, 3)[1]
        res[key] = {"us": round(t * 1e3, 2), "TFLOP/s": round(fl / t / 1e9, 2),
                    "peak_frac": round(fl / t / 1e9 / peak, 4), "peak": peak,
                    "eager_us": round(te * 1e3, 2), "weight_copies": len(fns),
                    "us_one_copy": round(t1 * 1e3, 2)}
        log(f"{key}: {res[key]}")
    torch.cuda.empty_cache()
    # --- W4A4, activations/weights quantized with the RNE rule
    m, k, n = 8192, 4096, 4096
    a = randn_bf16(4, (m, k))
    wt = (randn_bf16(5, (n, k)).float() * 0.02)
    ap, asc = mx.dynamic_mxfp4_quant(a, "rne")
    wp, wsc = mx.dynamic_mxfp4_quant(wt, "rne")
    t = time_eager(lambda: mx.linear_mxfp4_w4a4(ap, asc, wp, wsc), 20, 5)[1]
    fl = 2.0 * m * n * k
    res["w4a4_8192x4096x4096"] = {"us": round(t * 1e3, 2), "TFLOP/s": round(fl / t / 1e9, 1),
                                  "fp4_frac": round(fl / t / 1e9 / FP4_PEAK_TFLOPS, 4)}
    log(f"w4a4: {res['w4a4_8192x4096x4096']}")
    tq = time_eager(lambda: mx.dynamic_mxfp4_quant(a, "rne"), 20, 5)[1]
    qb = m * k * 2 + m * k // 2 + m * k // 32
    res["quant_rne_8192x4096"] = {"us": round(tq * 1e3, 2), "GB/s": round(qb / tq / 1e6, 1)}
    # --- standalone dequant: all 128 experts' w13 -> bf16
    (p, s), = rand_weights(np.random.default_rng(9), (128 * 1536,), 2048)
    t = time_eager(lambda: mx.dequant_mxfp4(p, s, torch.bfloat16), 10, 3)[1]
    db = p.numel() + s.numel() + p.numel() * 4
    res["dequant_bf16_128x1536x2048"] = {"us": round(t * 1e3, 1), "GB/s": round(db / t / 1e6, 1),
                                         "hbm_frac": round(db / t / 1e6 / HBM_PEAK_GBS, 4)}
    log(f"dequant: {res['dequant_bf16_128x1536x2048']}")
    # --- router: logits f32 [4096, 128] -> top-8 weights and ids
    # (graph replays of 16 calls: the kernel is shorter than an eager call's
    # Python overhead)
    logits = torch.randn((4096, 128), generator=torch.Generator().manual_seed(12)).cuda()
    t = time_graph([lambda: mx.route_topk(logits, 8)] * 16, replays=20)
    rb = logits.numel() * 4 + 4096 * 8 * (4 + 8)
    res["route_topk_4096x128_k8"] = {"us": round(t * 1e3, 2), "GB/s": round(rb / t / 1e6, 1)}
    log(f"router: {res['route_topk_4096x128_k8']}")
    return res


def cpu_baseline(np, m, k, n, budget_s=20.0):
    """The reference safe path restated (oracle/mxfp4_oracle.py: explicit
    dequant -> torch.matmul bf16), timed on this host on a row sample."""
    import torch
    from oracle import mxfp4_oracle as O
    threads, isa = _cpu_setup()
    rng = np.random.default_rng(20260812)
    w = torch.from_numpy(rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8))
    s = torch.from_numpy(rng.integers(120, 129, size=(n, k // 32), dtype=np.uint8))
    probe_m = 64
    x = torch.randn((probe_m, k), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    O.linear_safe(x, w, s)  # warm-up
    t0 = time.perf_counter()
    O.linear_safe(x, w, s)
    t_probe = time.perf_counter() - t0
    # rows so that one call takes about budget/6, capped at the workload's M
    rows = int(min(m, max(probe_m, probe_m * (budget_s / 6) / max(t_probe, 1e-3))))
    x = torch.randn((rows, k), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    O.linear_safe(x, w, s)
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        O.linear_safe(x, w, s)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    flops = 2.0 * rows * n * k
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"safe path (dequant + torch.matmul bf16) on x[{rows},{k}] x W[{n},{k}], "
                      f"median of {len(times)} calls ({t * 1e3:.1f} ms each), torch "
                      f"{torch.__version__}, isa {isa}"}


def _cpu_setup():
    """Threads for the CPU legs (the host share given to this job) and the ISA."""
    import torch
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = max(1, min(threads, int(os.environ["OMP_NUM_THREADS"])))
    torch.set_num_threads(threads)
    isa = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            flags = next((ln for ln in f if ln.startswith("flags")), "")
        isa = ",".join(x for x in ("avx512_bf16", "amx_bf16", "avx512f", "avx2") if x in flags.split())
    except OSError:
        pass
    return threads, isa


def _time_cpu(fn, cap_s, max_runs=5):
    """One warm-up call, then up to max_runs timed calls while the timed total
    stays under cap_s (at least one); returns (median seconds, runs)."""
    import numpy as np
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_runs and (not times or time.perf_counter() - t_start < cap_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_config1(np):
    """the reference safe path (oracle/mxfp4_oracle.py
    linear_safe: explicit dequant -> torch.matmul bf16) on the host, x bf16
    [64, 2048] ~ N(0, 1), W u8 [2048, 1024] codes uniform 0..15, S u8
    [2048, 64] uniform 120..128; seconds and GFLOP/s per call."""
    import torch
    from oracle import mxfp4_oracle as O
    threads, isa = _cpu_setup()
    m, k, n = 64, 2048, 2048
    rng = np.random.default_rng(20260810)
    w = torch.from_numpy(rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8))
    s = torch.from_numpy(rng.integers(120, 129, size=(n, k // 32), dtype=np.uint8))
    x = torch.randn((m, k), generator=torch.Generator().manual_seed(20260810)).to(torch.bfloat16)
    t, runs = _time_cpu(lambda: O.linear_safe(x, w, s), cap_s=10.0, max_runs=9)
    flops = 2.0 * m * n * k
    return {"seconds": round(t, 6), "GFLOP/s": round(flops / t / 1e9, 2), "flops": int(flops),
            "runs": runs, "cores": threads, "isa": isa, "torch": torch.__version__,
            "kind": "port", "what": "safe path restated: dequant_safe + torch.matmul bf16"}


CPU_CAP_S = {"linear": 3.0, "moe": 12.0, "w4a4": 6.0}


def cpu_beside_sweep(np, res):
    """The same CPU restatement of the safe path at each sweep row's shape,
    added to that row as cpu_ms (median of up to 5 calls after one warm-up,
    within CPU_CAP_S seconds per row; cpu_runs says how many were timed)."""
    import torch
    from oracle import mxfp4_oracle as O
    _cpu_setup()
    g = torch.Generator().manual_seed(20260813)
    rng = np.random.default_rng(20260813)

    def weights(rows, k):
        return (torch.from_numpy(rng.integers(0, 256, size=(*rows, k // 2), dtype=np.uint8)),
                torch.from_numpy(rng.integers(120, 129, size=(*rows, k // 32), dtype=np.uint8)))

    def put(key, fn, cap):
        if key not in res:
            return
        t, runs = _time_cpu(fn, cap)
        res[key]["cpu_ms"] = round(t * 1e3, 3)
        res[key]["cpu_runs"] = runs
        res[key]["gpu_speedup"] = round(t * 1e3 / res[key]["us"] * 1e3, 1)
        log(f"cpu {key}: {t * 1e3:.1f} ms ({runs} runs)")

    for name, k, n in (("qkv", 2048, 5120), ("o_proj", 4096, 2048)):
        w, s = weights((n,), k)
        for m in (1, 8, 370, 4096):
            x = torch.randn((m, k), generator=g).to(torch.bfloat16)
            put(f"w4a16_{name}_m{m}", lambda x=x, w=w, s=s: O.linear_safe(x, w, s),
                CPU_CAP_S["linear"])
    e, hidden, inter, top_k = 128, 2048, 768, 8
    w13, s13 = weights((e, 2 * inter), hidden)
    w2, s2 = weights((e, hidden), inter)
    for m in (1, 8, 32, 512, 4096):
        logits = torch.randn((m, e), generator=g)
        tw, ids = torch.topk(torch.softmax(logits, -1), top_k, dim=-1)
        tw = tw / tw.sum(-1, keepdim=True)
        x = torch.randn((m, hidden), generator=g).to(torch.bfloat16)
        put(f"moe_layer_m{m}",
            lambda x=x, tw=tw, ids=ids: O.moe_layer_safe(x, w13, s13, w2, s2, tw, ids),
            CPU_CAP_S["moe"])
    # W4A4 = the soft op with one expert and packed A (soft:468-494)
    m, k, n = 8192, 4096, 4096
    ap, asc = weights((m,), k)
    bp, bsc = weights((1, n), k)
    c = torch.empty((m, 1, n), dtype=torch.bfloat16)
    ones, ids1 = torch.ones(1), torch.zeros((m, 1), dtype=torch.int64)
    put("w4a4_8192x4096x4096",
        lambda: O.fused_moe_safe(ap, bp, c, ones, ones, asc, bsc, ones.expand(m, 1), ids1, False),
        CPU_CAP_S["w4a4"])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the launches the counter runs measure")
    ap.add_argument("--decode-probe", action="store_true",
                    help="only run decode launches for counter / trace runs")
    ap.add_argument("--data-probe", action="store_true",
                    help="time the headline GEMM on random vs zero / constant inputs")
    ap.add_argument("--moe-probe", action="store_true",
                    help="only run MoE layer prefill launches for trace runs")
    ap.add_argument("--headline-probe", action="store_true",
                    help="only run headline launches (prepacked, then checkpoint layout)")
    ap.add_argument("--soft-probe", action="store_true",
                    help="only run soft-op / AITER-entry launches for trace runs")
    ap.add_argument("--w4a4-probe", action="store_true",
                    help="only run W4A4 launches (8192 x 4096 x 4096) for trace / counter runs")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    if args.traffic_probe:
        return traffic_probe()
    if args.decode_probe:
        return decode_probe()
    if args.data_probe:
        return data_probe()
    if args.moe_probe:
        return moe_probe()
    if args.w4a4_probe:
        return w4a4_probe()
    if args.soft_probe:
        return soft_probe()
    if args.headline_probe:
        return headline_probe()

    import numpy as np
    import torch

    import mxfp4_amd as mx
    mx._lib.load()
    torch.cuda.set_device(0)

    m, k, n = 4096, 2048, 5120
    rng = np.random.default_rng(20260810 + 1)
    (w, s), = rand_weights(rng, (n,), k)
    x = randn_bf16(20260810, (m, k))
    pre = mx.prepack_w4a16(w, s)  # once, as at weight load
    log(f"headline: w4a16 linear m={m} k={k} n={n} (prepacked weights), clock ramp "
        f"{RAMP_MS:.0f} ms, warmup {args.warmup}, steps {args.steps}")

    def step():
        mx.linear_mxfp4_soft(x, w, s, prepacked=pre)

    ramp_clocks(step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kernel_ms = start.elapsed_time(end) / args.steps
    # the same call without the prepacked copy (checkpoint layout), untimed
    # for `value`: reported beside it
    ckpt_ms = time_eager(lambda: mx.linear_mxfp4_soft(x, w, s), args.steps, args.warmup)[1]
    flops = 2.0 * m * n * k
    value = flops / (wall_ms * 1e-3) / 1e12
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    log(f"headline: {wall_ms:.4f} ms/step wall, {kernel_ms:.4f} ms/kernel, {value:.1f} TFLOP/s; "
        f"checkpoint layout {ckpt_ms:.4f} ms/kernel")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded: E2M1 codes uniform 0..15, E8M0 120..128, x ~ N(0,1) bf16)",
        "config": {"workload": "w4a16_linear_qkv_prefill", "m": m, "k": k, "n": n,
                   "op": "linear_mxfp4_soft", "weights": "MXFP4 E2M1 + E8M0/32",
                   "weight_layout": "prepacked at load (prepack_w4a16)",
                   "activations": "bf16"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                     "traffic": recorded_traffic(),
                     "kernel": "w4a16_pf<bf16, prepacked> 256x320 tile, 2 x 4 waves of 128x80 "
                               "(direct-to-LDS)",
                     "kernel_us": round(kernel_ms * 1e3, 3),
                     "checkpoint_layout_kernel_us": round(ckpt_ms * 1e3, 3),
                     "algorithmic_bytes": linear_bytes(m, n, k, prepacked=True)},
    }
    if not args.no_sweep:
        out["sweep"] = sweep(mx, torch, np)
    if not args.no_cpu:
        log("cpu baseline (bounded sample)")
        out["cpu_baseline"] = cpu_baseline(np, m, k, n)
        log("cpu: BASELINE config 1")
        out["cpu_config1"] = cpu_config1(np)
        if "sweep" in out:
            log("cpu: the safe path beside each sweep row")
            cpu_beside_sweep(np, out["sweep"])
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
