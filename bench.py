"""Benchmark of the H3 per-block hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--only fused,block_order,copy,swiglu,select,cond,heads,attn,proj,fc1,rms_f32,block,ref,share]
                    [--no-cpu] [--no-compare]

A step is one pass of the headline kernel -- the fused adaLN-modulated RMS norm + gated residual -- over the
768p-shaped batch (129,536 rows = 32x48x84 video + 512 text, x 5120, bf16), inputs resident in HBM. value is its
achieved algorithmic HBM bandwidth (6 bytes an element: read x and residual, write out). The same run also times the
other ops of the path at their shapes (SwiGLU split and fused-row, the cube selector, the int8 fc1 + SwiGLU GEMM, the
fp32 modulated RMS norm, heads_partial, the sparse attention, the other projections) and reports each as ms, GB/s or
TFLOP/s and a fraction of the MI355X roofline; `block` times one whole H3 block at 768p as one sequence of
launches; `share` repeats the main ones at one GPU's share of an 8-way split;
`ref` times the reference's own published workloads at H3's dimensions beside its published Apple M5 Max times
(`reference_shapes`), and sums a forward's kernels (dense and sparse) against the reference's GPU time a forward.
Kernel times come from HIP events recorded on the stream the kernels run on (torch's current stream): the mean over the timed
launches, with the median beside it for the row and selector workloads. Launches run back to back with warm caches;
`cold_ms` beside the fused op, SwiGLU, the select kernel, fc1 and the fp32 norm times each launch after a 512 MiB
overwrite of L2 and the MALL instead. The CPU baseline is the scalar C oracle on one host core, on a bounded sample of
the same workload.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "mako-video_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA
INT8_PEAK_TOPS = 5000.0        # dense int8 MFMA
METRIC = "ms/op + achieved HBM GB/s (% peak) at 768p rows; int8 GEMM MFMA util %"

ROWS, DIM, FFN = 32 * 48 * 84 + 512, 5120, 13824
GRID, HEADS = (32, 48, 84), 40


LAST_MEDIAN_MS = [0.0]  # the median of the last time_launches call's per-launch event times


_FLUSH: list = []


def flush_caches() -> None:
    """Overwrite 512 MiB on the current stream: twice the 256 MB MALL and far more than the 8 x 4 MB of L2, so the
    launch after it starts with cold caches."""
    if not _FLUSH:
        _FLUSH.append(torch.empty(512 << 20, dtype=torch.uint8, device="cuda"))
    _FLUSH[0].zero_()


def time_launches(fn, steps: int, warmup: int, cold: bool = False) -> tuple[float, float]:
    """(mean ms per launch from HIP events on the current stream, wall ms per launch) over `steps` launches; the
    median of the per-launch times is left in LAST_MEDIAN_MS[0]. With `cold`, `flush_caches` runs before each timed
    launch, outside its events (the wall time then includes the flushes)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        if cold:
            flush_caches()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    LAST_MEDIAN_MS[0] = float(np.median(ev))
    return float(np.mean(ev)), wall


def mod_params(dev, dim, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (1 + 0.02 * torch.randn(dim, generator=g, device=dev)).float()
    shift = (0.1 * torch.randn(dim, generator=g, device=dev)).float()
    scale = (0.1 * torch.randn(dim, generator=g, device=dev)).float()
    gate = (0.1 * torch.randn(dim, generator=g, device=dev)).float()
    return w, shift, scale, gate


def bench_fused(mh, dev, steps, warmup):
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    res = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    w, shift, scale, gate = mod_params(dev, DIM, 1)
    out = torch.empty_like(x)
    ms, wall = time_launches(lambda: mh.rms_mod_gate_add_rows(x, res, w, shift, scale, gate, out=out), steps, warmup)
    med = LAST_MEDIAN_MS[0]
    cold_ms, _ = time_launches(lambda: mh.rms_mod_gate_add_rows(x, res, w, shift, scale, gate, out=out), steps,
                               warmup, cold=True)
    nbytes = ROWS * DIM * 6
    return {"ms": ms, "median_ms": med, "median_GBs": nbytes / med / 1e6, "wall_ms": wall, "bytes": nbytes,
            "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS, "shape": [ROWS, DIM],
            "cold_ms": cold_ms, "cold_GBs": nbytes / cold_ms / 1e6}


def bench_block_order(mh, dev, steps, warmup):
    """The block's own order in one pass: x += gate * y, h = modulated RMS norm of the new x (8 bytes an element:
    read x and y, write x and h), against the two kernels it replaces (10 bytes an element)."""
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    y = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    w, shift, scale, gate = mod_params(dev, DIM, 3)
    h = torch.empty_like(x)
    ms, _ = time_launches(lambda: mh.gate_add_rms_mod_rows(x, y, gate, w, shift, scale, h=h), steps, warmup)

    def two():
        mh.gate_add_rows(x, y, gate)
        mh.rms_mod_rows(x, w, shift, scale, out=h)
    ms2, _ = time_launches(two, steps, warmup)
    nbytes = ROWS * DIM * 8
    res = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS,
           "two_kernel_ms": ms2, "two_kernel_bytes": ROWS * DIM * 10, "shape": [ROWS, DIM]}
    del x, y, h
    torch.cuda.empty_cache()
    # The reference's float residual stream: x float, y (the out projection's bf16 output) and h (fc1's bf16 input)
    # bf16; 12 bytes an element (read x 4 and y 2, write x 4 and h 2). And the modulated norm alone from the float x
    # to the bf16 GEMM row (6 bytes an element).
    xf = torch.randn((ROWS, DIM), generator=g, device=dev)
    yb = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    hb = torch.empty((ROWS, DIM), dtype=torch.bfloat16, device=dev)
    fms, _ = time_launches(lambda: mh.gate_add_rms_mod_rows(xf, yb, gate, w, shift, scale, h=hb), steps, warmup)
    rms, _ = time_launches(lambda: mh.rms_mod_rows(xf, w, shift, scale, out=hb), steps, warmup)
    fb, rb = ROWS * DIM * 12, ROWS * DIM * 6
    res["float_stream"] = {"ms": fms, "bytes": fb, "GBs": fb / fms / 1e6, "frac": fb / fms / 1e6 / HBM_PEAK_GBS,
                           "rms_mod_f32_to_bf16": {"ms": rms, "bytes": rb, "GBs": rb / rms / 1e6,
                                                   "frac": rb / rms / 1e6 / HBM_PEAK_GBS}}
    return res


def bench_copy(dev, steps, warmup):
    """Calibration: a plain device-to-device copy of a 768p-sized bf16 tensor (read + write, 2.65 GB)."""
    src = torch.empty((ROWS, DIM), dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    ms, _ = time_launches(lambda: dst.copy_(src), steps, warmup)
    nbytes = ROWS * DIM * 4
    return {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}


def bench_stream(dev, steps, warmup):
    """The streaming ceiling: a plain HIP kernel reading, copying, reading two streams into a third (the fused row
    op's and SwiGLU's mix) and reading two streams into two (the block's own order: x += gate y and h = norm of x),
    16-byte non-temporal accesses over 768p-sized bf16 buffers (1.33 GB each), swept over the access form (global or
    buffer instructions), unroll (2, 4, 8 vectors a thread) and grid (flat; 4, 8, 16 workgroups a CU, grid-stride,
    for the global form); the best of each mix is reported. Also the MFMA peaks from the device's CU count and peak
    clock (flops a clock a CU: bf16 4096, int8 8192)."""
    import ctypes as C

    lib = C.CDLL(str(REPO / "mako-video_amd" / "lib" / "libmh3_stream_probe.so"))
    lib.mh3_probe_stream.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_int, C.c_uint32,
                                     C.c_void_p]
    lib.mh3_probe_device.argtypes = [C.POINTER(C.c_int), C.POINTER(C.c_int)]
    cus, khz = C.c_int(0), C.c_int(0)
    if lib.mh3_probe_device(C.byref(cus), C.byref(khz)) != 0:
        raise RuntimeError("mh3_probe_device failed")
    nbytes = ROWS * DIM * 2
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a).fill_(2)
    c = torch.empty(2 * nbytes, dtype=torch.uint8, device=dev)  # two write streams for r2w2
    stream = torch.cuda.current_stream().cuda_stream
    res = {"bytes_per_stream": nbytes}
    # Each mix in both access forms: global loads and stores (kinds 0-3, flat or grid-stride) and buffer loads and
    # stores (kinds 4-7, flat), the best of all reported as the mix's ceiling.
    for kinds, name, moved in (((0, 4), "read", 1), ((1, 5), "copy", 2), ((2, 6), "r2w1", 3), ((3, 7), "r2w2", 4)):
        best = None
        for kind in kinds:
            for unroll in (2, 4, 8):
                for per_cu in ((0, 4, 8, 16) if kind < 4 else (0,)):
                    blocks = per_cu * cus.value

                    def run():
                        rc = lib.mh3_probe_stream(kind, a.data_ptr(), b.data_ptr(), c.data_ptr(), nbytes // 16,
                                                  unroll, blocks, stream)
                        if rc != 0:
                            raise RuntimeError(f"mh3_probe_stream({name}) returned {rc}")
                    ms, _ = time_launches(run, max(5, steps // 2), 2)
                    if best is None or ms < best[0]:
                        best = (ms, unroll, per_cu, kind)
        ms, unroll, per_cu, kind = best
        res[name] = {"ms": ms, "GBs": moved * nbytes / ms / 1e6, "frac": moved * nbytes / ms / 1e6 / HBM_PEAK_GBS,
                     "unroll": unroll, "grid": "flat" if per_cu == 0 else f"{per_cu} workgroups a CU",
                     "access": "buffer" if kind >= 4 else "global"}
    # The fused row op's own shape with no arithmetic (one 5120-wide row a wave, all of a's row then all of b's, an
    # 8-wave workgroup of 8 rows), at one, two and three workgroups a CU (the dynamic LDS sets it; the fused op runs
    # two): the ceiling for that access pattern.
    lib.mh3_probe_rows.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
                                   C.c_void_p]
    rows_res = {}
    for per_cu, lds in ((1, 81 * 1024), (2, 54 * 1024), (3, 41 * 1024)):
        def run_rows():
            rc = lib.mh3_probe_rows(a.data_ptr(), b.data_ptr(), c.data_ptr(), ROWS, DIM // 8, lds, stream)
            if rc != 0:
                raise RuntimeError(f"mh3_probe_rows returned {rc}")
        ms, _ = time_launches(run_rows, max(5, steps // 2), 2)
        rows_res[f"{per_cu}_workgroups_a_cu"] = {"ms": ms, "GBs": 3 * nbytes / ms / 1e6,
                                                 "frac": 3 * nbytes / ms / 1e6 / HBM_PEAK_GBS}
    best = max(rows_res.values(), key=lambda r: r["GBs"])
    res["rows_r2w1"] = {**rows_res, "GBs": best["GBs"], "frac": best["frac"], "ms": best["ms"],
                        "shape": "one row a wave, 10 vectors a lane of two inputs, one output, no arithmetic"}
    clk = khz.value * 1e3
    res["device"] = {"cus": cus.value, "peak_clock_mhz": khz.value / 1e3,
                     "bf16_mfma_peak_tflops": cus.value * clk * 4096 / 1e12,
                     "int8_mfma_peak_tops": cus.value * clk * 8192 / 1e12}
    return res


def bench_mfma_ceiling(dev, steps, warmup):
    """The matrix cores' sustained rate on this GPU under its power limit: a register-only loop of the GEMMs' own
    instructions, v_mfma_f32_16x16x32_bf16 and v_mfma_i32_16x16x64_i8 (and of the 32 x 32 forms beside them), 16 (8)
    independent accumulators a wave, two waves a SIMD, one 8-wave workgroup a CU, the operands cycling through 8
    fragments of random bits, ~40 ms a launch (the power limit acts within it). The clock each workgroup ran at is its
    shader clock counter's advance over the 100 MHz real-time counter's (s_memtime, s_memrealtime): the median over
    workgroups is reported."""
    import ctypes as C

    lib = C.CDLL(str(REPO / "mako-video_amd" / "lib" / "libmh3_stream_probe.so"))
    lib.mh3_probe_mfma.argtypes = [C.c_int, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]
    lib.mh3_probe_device.argtypes = [C.POINTER(C.c_int), C.POINTER(C.c_int)]
    cus, khz = C.c_int(0), C.c_int(0)
    if lib.mh3_probe_device(C.byref(cus), C.byref(khz)) != 0:
        raise RuntimeError("mh3_probe_device failed")
    blocks = cus.value
    out = torch.empty(blocks * 512, dtype=torch.float32, device=dev)
    clocks = torch.zeros(2 * blocks, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    res = {}
    # (kind, name, ops an instruction, accumulators a wave, cycles an instruction at the nameplate rate, peak)
    for kind, name, flops_per, accs, cyc, peak in ((0, "bf16", 2 * 16 * 16 * 32, 16, 16, BF16_PEAK_TFLOPS),
                                                   (1, "int8", 2 * 16 * 16 * 64, 16, 16, INT8_PEAK_TOPS),
                                                   (2, "bf16_32x32", 2 * 32 * 32 * 16, 8, 32, BF16_PEAK_TFLOPS),
                                                   (3, "int8_32x32", 2 * 32 * 32 * 32, 8, 32, INT8_PEAK_TOPS)):
        iters = 40000 if kind in (0, 2) else 20000  # ~40 ms a launch at 2 GHz

        def run():
            rc = lib.mh3_probe_mfma(kind, blocks, iters, out.data_ptr(), clocks.data_ptr(), stream)
            if rc != 0:
                raise RuntimeError(f"mh3_probe_mfma returned {rc}")
        ms, _ = time_launches(run, max(3, steps // 4), max(1, warmup // 2))
        ck = clocks.view(blocks, 2).double().cpu()
        ghz = float((ck[:, 0] / ck[:, 1]).median()) * 0.1  # 100 MHz real-time counter
        ops = float(blocks) * 512 / 64 * iters * accs * flops_per
        rate = ops / ms / 1e9
        res[name] = {"ms": ms, "rate": rate, "unit": "TOP/s" if "int8" in name else "TFLOP/s", "frac": rate / peak,
                     "clock_ghz": ghz,
                     "mfma_busy_at_clock": rate / (cus.value * ghz * 1e9 * 4 * flops_per / cyc / 1e12) if ghz else None}
    return res


def bench_rms_f32(mh, dev, steps, warmup):
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn((4096, 1024), generator=g, device=dev)
    w, shift, scale, _ = mod_params(dev, 1024, 4)
    out = torch.empty_like(x)
    ms, _ = time_launches(lambda: mh.rms_mod_rows(x, w, shift, scale, out=out), steps, warmup)
    cold_ms, _ = time_launches(lambda: mh.rms_mod_rows(x, w, shift, scale, out=out), steps, warmup, cold=True)
    nbytes = 4096 * 1024 * 8
    return {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "shape": [4096, 1024],
            "cold_ms": cold_ms, "cold_GBs": nbytes / cold_ms / 1e6,
            "note": "33.6 MB: launch- and L2-bound, not an HBM measurement"}


def bench_swiglu(mh, dev, steps, warmup):
    g = torch.Generator(device=dev).manual_seed(5)
    res = {}
    nbytes = ROWS * FFN * 6
    gate = torch.randn((ROWS, FFN), generator=g, device=dev).to(torch.bfloat16)
    up = torch.randn((ROWS, FFN), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(gate)
    ms, _ = time_launches(lambda: mh.swiglu_rows(gate, up, out=out), steps, warmup)
    res["split"] = {"ms": ms, "median_ms": LAST_MEDIAN_MS[0], "GBs": nbytes / ms / 1e6,
                    "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}
    res["split"]["cold_ms"], _ = time_launches(lambda: mh.swiglu_rows(gate, up, out=out), steps, warmup, cold=True)
    del gate, up
    gu = torch.randn((ROWS, 2 * FFN), generator=g, device=dev).to(torch.bfloat16)
    ms, _ = time_launches(lambda: mh.swiglu_rows(gu, out=out), steps, warmup)
    res["fused_row"] = {"ms": ms, "median_ms": LAST_MEDIAN_MS[0], "GBs": nbytes / ms / 1e6,
                        "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}
    res["bytes"] = nbytes
    res["shape"] = [ROWS, FFN]
    return res


def selector_qk(dev, extra_rows=0, shared=False):
    """q and k [40][rows + extra_rows][128] bf16: N(0,1) plus, on the video rows, four low-frequency waves over
    (t, y, x) along random unit directions (amplitude 0.5), so cube means separate above the pooled noise; the
    extra (dense) rows are N(0,1). q and k draw their own waves, unless `shared`: then a head's waves are the same in
    q and k (only the noise differs), so cubes of similar phase score high, as similar content does in a video, and
    neighbouring query cubes select overlapping key cubes."""
    T, Y, X = GRID
    rows = T * Y * X
    g = torch.Generator(device=dev).manual_seed(7)
    rng = np.random.default_rng(7)
    tt = torch.arange(T, device=dev, dtype=torch.float32).view(T, 1, 1) / T
    yy = torch.arange(Y, device=dev, dtype=torch.float32).view(1, Y, 1) / Y
    xx = torch.arange(X, device=dev, dtype=torch.float32).view(1, 1, X) / X
    waves = {}
    qk = []
    for which in range(2):
        t = torch.empty((HEADS, rows + extra_rows, 128), dtype=torch.bfloat16, device=dev)
        for h in range(HEADS):
            acc = torch.randn((rows, 128), generator=g, device=dev)
            for j in range(4):
                if not shared or which == 0:
                    f = rng.integers(0, 3, 3)
                    u = rng.standard_normal(128)
                    waves[h, j] = (f, torch.from_numpy(u / np.linalg.norm(u)).float().to(dev), rng.uniform(0, 6.283))
                f, u, phase = waves[h, j]
                wave = torch.cos(2 * math.pi * (f[0] * tt + f[1] * yy + f[2] * xx) + phase)
                acc += 0.5 * wave.reshape(-1, 1) * u
            t[h, :rows] = acc.to(torch.bfloat16)
            if extra_rows:
                t[h, rows:] = torch.randn((extra_rows, 128), generator=g, device=dev).to(torch.bfloat16)
        qk.append(t)
    return qk


def bench_select(mh, dev, steps, warmup):
    T, Y, X = GRID
    rows = T * Y * X
    q, k = selector_qk(dev)
    cubes = mh.cube_count(*GRID)
    kk = mh.topk_k(0.1, cubes)
    a = mh.cube_args(HEADS, GRID, k=kk, local=1)
    qc = torch.empty((HEADS, cubes, 128), dtype=torch.float32, device=dev)
    kc = torch.empty_like(qc)
    idx = torch.empty((HEADS, cubes, kk + 1), dtype=torch.int32, device=dev)
    cnt = torch.empty((HEADS, cubes), dtype=torch.int32, device=dev)
    ws = torch.empty(mh.cube_select_workspace_bytes(a), dtype=torch.uint8, device=dev)
    pool_ms, _ = time_launches(lambda: mh.cube_pool(a, q, k, qc=qc, kc=kc), steps, warmup)
    sel_ms, _ = time_launches(lambda: mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt), steps, warmup)
    # The pooled inputs (83 MB) fit in the MALL, so back-to-back launches start warm; this timing starts each cold.
    sel_cold_ms, _ = time_launches(lambda: mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt), steps, warmup,
                                   cold=True)

    def both():
        mh.cube_pool(a, q, k, qc=qc, kc=kc)
        mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt)
    total_ms, _ = time_launches(both, steps, warmup)
    total_median = LAST_MEDIAN_MS[0]
    # The unfused pair, scores through HBM: for comparison with the fused select.
    del q, k
    s = torch.empty((HEADS, cubes, cubes), dtype=torch.float32, device=dev)
    scores_ms, _ = time_launches(lambda: mh.cube_scores(a, qc, kc, out=s), steps, warmup)
    topk_ms, _ = time_launches(lambda: mh.cube_topk(a, s, idx=idx, cnt=cnt), steps, warmup)
    del s
    pool_bytes = 2 * HEADS * rows * 128 * 2 + 2 * HEADS * cubes * 128 * 4
    sel_bytes = 2 * HEADS * cubes * 128 * 4 + HEADS * cubes * (kk + 2) * 4
    alg_bytes = 2 * HEADS * rows * 128 * 2 + HEADS * cubes * (kk + 1) * 4
    flops = 2.0 * HEADS * cubes * cubes * 128
    return {"pool_ms": pool_ms, "select_ms": sel_ms, "select_cold_ms": sel_cold_ms, "ms": total_ms, "median_ms": total_median, "k": kk,
            "cubes": cubes,
            "pool_GBs": pool_bytes / pool_ms / 1e6, "pool_frac": pool_bytes / pool_ms / 1e6 / HBM_PEAK_GBS,
            "alg_bytes": alg_bytes, "GBs": alg_bytes / total_ms / 1e6,
            "frac": alg_bytes / total_ms / 1e6 / HBM_PEAK_GBS,
            "score_gflop": flops / 1e9, "select_TFLOPs": flops / sel_ms / 1e9,
            # The scores are three bf16 MFMA products of split float operands: 3 x the flops on the bf16 matrix cores.
            "select_split_bf16_mfma_frac": 3.0 * flops / sel_ms / 1e9 / BF16_PEAK_TFLOPS,
            "select_bytes": sel_bytes, "unfused_scores_ms": scores_ms, "unfused_topk_ms": topk_ms}


def pass_list_overlap(idx, cnt, cubes):
    """Mean share of a query cube's selected cubes that the next query cube (same head, next in raster order) also
    selected: how much K/V a neighbouring tile could find in L2."""
    heads = idx.shape[0]
    sel = torch.zeros((heads, cubes, cubes + 1), dtype=torch.bool, device=idx.device)
    sel.scatter_(2, torch.where(idx >= 0, idx, cubes).long(), True)
    sel = sel[..., :cubes]
    both = (sel[:, :-1] & sel[:, 1:]).sum(-1).float()
    return float((both / cnt[:, :-1].float()).mean())


def bench_attn(mh, dev, steps, warmup, shared=False):
    """flash_attn_sparse_128 at the 768p shape: 40 heads, grid 32 x 48 x 84 (2016 cubes) in the model's row order,
    512 text rows after the video rows; the pass lists from cube_pool + cube_select at ratio 0.1 (k = 202), local 1;
    the query cubes scheduled in cube_order's order, as the block runs them (`plain_order_ms`: without it).
    Algorithmic work: 4 x 128 flops (q.k and p.v) per (query, attended key) pair; K/V bytes: 512 per attended key
    a query tile (one K and one V row per tile that attends it). `shared`: the q/k data whose smooth waves q and k
    share (selector_qk), so neighbouring query cubes' pass lists overlap."""
    T, Y, X = GRID
    video, n_dense = T * Y * X, 512
    rows = video + n_dense
    q, k = selector_qk(dev, n_dense, shared=shared)
    v = torch.randn((HEADS, rows, 128), generator=torch.Generator(device=dev).manual_seed(8),
                    device=dev).to(torch.bfloat16)
    cubes = mh.cube_count(*GRID)
    kk = mh.topk_k(0.1, cubes)
    a = mh.cube_args(HEADS, GRID, head_stride=rows * 128, k=kk, local=1)
    qc, kc = mh.cube_pool(a, q, k)
    idx, cnt = mh.cube_select(a, qc, kc)
    order = mh.cube_order(a, idx, cnt)
    out = torch.empty_like(q)
    # The block's launch: the query cubes in cube_order's order (the plain order timed beside it).
    ms, _ = time_launches(lambda: mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense,
                                                           out=out, order=order), steps, warmup)
    plain_ms, _ = time_launches(lambda: mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video,
                                                                 n_dense=n_dense, out=out), steps, warmup)
    order_ms, _ = time_launches(lambda: mh.cube_order(a, idx, cnt, order=order), steps, warmup)
    sel = int(cnt.to(torch.int64).sum())
    pairs = 64 * (sel * 64 + HEADS * cubes * n_dense) + HEADS * n_dense * rows
    flops = 4.0 * 128 * pairs
    kv_tile_rows = sel * 64 + HEADS * cubes * n_dense + HEADS * (n_dense // 64) * rows
    dense_flops = 4.0 * 128 * HEADS * rows * rows
    # Each 64-key tile a query tile attends brings 32 KB of K and V for 64 x 64 x 128 x 4 flops: 64 flop a byte, far
    # below the ridge point (2.5 PFLOP/s / 8 TB/s = 312), so the K/V stream bounds the kernel. kv_tile_GBs is the rate
    # at which the CUs' loads receive K/V tile bytes: most of them come from L2 and the MALL (a tile serves several
    # query tiles), so it is not an HBM figure and is not compared with the HBM peak; the HBM-side rate comes from the
    # counters (bytes past L2, FETCH_SIZE) in the profile summaries.
    res = {"ms": ms, "tflops": flops / ms / 1e9, "mfma_util": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
           "plain_order_ms": plain_ms, "cube_order_ms": order_ms,
           "flops": flops, "mean_cubes_selected": sel / (HEADS * cubes), "kv_tile_bytes": kv_tile_rows * 512,
           "kv_tile_GBs": kv_tile_rows * 512 / ms / 1e6,
           "flop_per_kv_byte": flops / (kv_tile_rows * 512), "dense_equivalent_flops": dense_flops,
           "pass_list_overlap": pass_list_overlap(idx, cnt, cubes),
           "shape": {"heads": HEADS, "grid": list(GRID), "cubes": cubes, "dense_rows": n_dense, "k": kk}}
    del q, k, v, out, qc, kc
    torch.cuda.empty_cache()
    if not shared:
        res["shared_waves"] = bench_attn(mh, dev, steps, warmup, shared=True)
    return res


def bench_cond(mh, dev, steps, warmup):
    """The modulation table's producer at H3's shapes (docs/architecture.md:49-52): the time MLP (256 -> 5376 -> 2688,
    float weights, 63 MB) for three levels, and one block's AdaLN projection (bf16 [96,768][2688], 520 MB) for one
    and three levels, each against HBM: their bytes are the weights read once (plus the small vectors)."""
    g = torch.Generator(device=dev).manual_seed(11)
    res = {}
    w_in = torch.randn((5376, 256), generator=g, device=dev) / 16
    b_in = torch.randn(5376, generator=g, device=dev) * 0.1
    w_out = torch.randn((2688, 5376), generator=g, device=dev) / 73
    b_out = torch.randn(2688, generator=g, device=dev) * 0.1
    t = torch.tensor([0.9230769, 0.5, 0.999], device=dev)
    ws = torch.empty(mh.time_embed_workspace_bytes(3, 256, 5376, 2688), dtype=torch.uint8, device=dev)
    temb = torch.empty((3, 2688), device=dev)
    cond = torch.empty((3, 2688), dtype=torch.bfloat16, device=dev)
    ms, _ = time_launches(lambda: mh.time_embed(t, w_in, b_in, w_out, b_out, workspace=ws, temb=temb, cond=cond),
                          steps, warmup)
    nb = (5376 * 256 + 5376 + 2688 * 5376 + 2688) * 4
    res["time_embed"] = {"ms": ms, "bytes": nb, "GBs": nb / ms / 1e6, "frac": nb / ms / 1e6 / HBM_PEAK_GBS,
                         "shape": {"levels": 3, "freq_dim": 256, "hidden": 5376, "out_dim": 2688}}
    n, k = 18 * 5376, 2688
    w = (0.02 * torch.randn((n, k), generator=g, device=dev)).to(torch.bfloat16)
    bias = torch.randn(n, generator=g, device=dev) * 0.01
    for levels in (1, 3):
        c = cond[:levels].contiguous()
        out = torch.empty((levels, n), device=dev)
        ms, _ = time_launches(lambda: mh.adaln_mod(c, w, bias, out=out), steps, warmup)
        cold, _ = time_launches(lambda: mh.adaln_mod(c, w, bias, out=out), steps, warmup, cold=True)
        nb = n * k * 2 + n * 4 + levels * n * 4
        res[f"adaln_mod_{levels}_levels"] = {"ms": ms, "cold_ms": cold, "bytes": nb, "GBs": nb / ms / 1e6,
                                             "frac": nb / ms / 1e6 / HBM_PEAK_GBS,
                                             "cold_frac": nb / cold / 1e6 / HBM_PEAK_GBS,
                                             "shape": {"levels": levels, "n": n, "k": k}}
    return res


def bench_heads(mh, dev, steps, warmup):
    """heads_partial at the 768p shape: qkv [129,536][3 x 40 x 128] bf16 (the QKV GEMM's rows: 512 text + the
    32 x 48 x 84 video grid), per-head RMS norm + rotary on 96 of 128 values for q and k, v copied, out as head tiles
    [40][rows][128]; and the same with the cube map (the gathered order: 2016 cubes x 64 slots + 512 text rows).
    Algorithmic bytes: 4 per element of q, k and v (read once, written once), plus the rows' cos / sin tables."""
    g = torch.Generator(device=dev).manual_seed(11)
    T, Y, X = GRID
    video, n_dense = T * Y * X, 512
    rows = ROWS
    x = torch.randn((rows, 3 * HEADS * 128), generator=g, device=dev).to(torch.bfloat16)
    ang = torch.rand((rows, 48), generator=g, device=dev) * 6.2831853 - 3.1415927
    ct, st = torch.cos(ang), torch.sin(ang)
    qw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    kw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    outs = [torch.empty((HEADS, rows, 128), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    ms, _ = time_launches(lambda: mh.heads_partial(x, HEADS, qw, kw, ct, st, q=outs[0], k=outs[1], v=outs[2]),
                          steps, warmup)
    nbytes = rows * 3 * HEADS * 128 * 4 + rows * 48 * 8
    res = {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS,
           "shape": {"rows": rows, "heads": HEADS, "rot": 96}}
    # Gathered through the cube map (mh3_cube_map): text rows first in the model (rows 0..511), the video grid after them.
    cmap, _ = mh.cube_map(GRID, n_dense=n_dense, video_row0=n_dense, dense_row0=0, device=dev)
    del outs
    gout = [torch.empty((HEADS, cmap.numel(), 128), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    gms, _ = time_launches(lambda: mh.heads_partial(x, HEADS, qw, kw, ct, st, map=cmap, q=gout[0], k=gout[1],
                                                    v=gout[2]), steps, warmup)
    gbytes = cmap.numel() * 3 * HEADS * 128 * 4 + cmap.numel() * (48 * 8 + 4)
    res["gathered"] = {"ms": gms, "bytes": gbytes, "GBs": gbytes / gms / 1e6,
                       "frac": gbytes / gms / 1e6 / HBM_PEAK_GBS, "rows": cmap.numel()}
    # The same pass with cube_pool fused in (mh3_heads_partial_pool): the selector's cube means from the values as
    # they are stored, against the gathered heads_partial followed by cube_pool over its output.
    cubes = mh.cube_count(*GRID)
    qc = torch.empty((HEADS, cubes, 128), dtype=torch.float32, device=dev)
    kc = torch.empty_like(qc)
    pa = mh.cube_args(HEADS, GRID, layout=mh.CUBES_GATHERED, row0=0, head_stride=cmap.numel() * 128)
    pool_ms, _ = time_launches(lambda: mh.cube_pool(pa, gout[0], gout[1], qc=qc, kc=kc), steps, warmup)
    fms, _ = time_launches(lambda: mh.heads_partial_pool(x, HEADS, GRID, qw, kw, ct, st, map=cmap, q=gout[0],
                                                         k=gout[1], v=gout[2], qc=qc, kc=kc), steps, warmup)
    fbytes = gbytes + 2 * HEADS * cubes * 128 * 4
    res["gathered_pool"] = {"ms": fms, "bytes": fbytes, "GBs": fbytes / fms / 1e6,
                            "frac": fbytes / fms / 1e6 / HBM_PEAK_GBS, "two_kernel_ms": gms + pool_ms,
                            "pool_ms": pool_ms, "pool_cost_in_pass_ms": fms - gms}
    # The same in the model's order (MH3_CUBES_GRID, no map): the sparse path then needs no gather either way.
    del gout
    outs = [torch.empty((HEADS, rows, 128), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    ga = mh.cube_args(HEADS, GRID, layout=mh.CUBES_GRID, row0=n_dense, head_stride=rows * 128)
    gpool_ms, _ = time_launches(lambda: mh.cube_pool(ga, outs[0], outs[1], qc=qc, kc=kc), steps, warmup)
    gfms, _ = time_launches(lambda: mh.heads_partial_pool(x, HEADS, GRID, qw, kw, ct, st, row0=n_dense,
                                                          cube_layout=mh.CUBES_GRID, q=outs[0], k=outs[1], v=outs[2],
                                                          qc=qc, kc=kc), steps, warmup)
    pbytes = nbytes + 2 * HEADS * cubes * 128 * 4
    res["grid_pool"] = {"ms": gfms, "bytes": pbytes, "GBs": pbytes / gfms / 1e6,
                        "frac": pbytes / gfms / 1e6 / HBM_PEAK_GBS, "two_kernel_ms": ms + gpool_ms,
                        "pool_ms": gpool_ms, "pool_cost_in_pass_ms": gfms - ms}
    return res


# The reference's own published timings (docs/performance.md, Apple M5 Max, 40-core GPU): its dense GEMM bench at
# 19,456 rows (:52-62), the per-forward kernel times of a 960x544, 124-frame forward of 50 blocks at 19,308 rows
# (:36-46) and the sparse path at that shape (:165-177, 37 x 17 x 30 patch grid -> 400 cubes, 435 dense rows).
REF_HW = "Apple M5 Max, 40-core GPU (docs/performance.md)"
H3_D, H3_HEADS, H3_FFN, H3_BLOCKS = 5376, 56, 14336, 50


def bench_reference_shapes(mh, dev, steps, warmup):
    """The reference's own headline workloads at H3's real dimensions (D 5376, 56 heads, fc1 5376 -> 2 x 14,336), timed
    here beside the reference's published M5 Max times for the same work. Per-forward figures are one block's kernels
    times the forward's 50 blocks. GEMMs are the bf16 forms (the reference's table is bf16) plus the int8 fc1 it
    quotes; our fc1 includes the SwiGLU epilogue the reference runs as a separate kernel."""
    g = torch.Generator(device=dev).manual_seed(31)
    rnd = lambda *shape: torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)  # noqa: E731
    out = {"reference_hardware": REF_HW}

    def entry(ms, ref_ms, what):
        return {"ms": ms, "reference_ms": ref_ms, "speedup": ref_ms / ms, "work": what}

    # Dense GEMMs at 19,456 rows (docs/performance.md:55-58, the 64 x 128-tile column).
    m = 19456
    gemms = {}
    x = rnd(m, H3_D)
    w = (0.02 * torch.randn((2 * H3_FFN, H3_D), generator=g, device=dev)).to(torch.bfloat16)
    ms, _ = time_launches(lambda: mh.gemm_bf16_swiglu(x, w), steps, warmup)
    gemms["fc1_bf16"] = entry(ms, 99.0, "19,456 x 5376 -> 28,672 (+ SwiGLU here)")
    wq, ws = mh.quant_rows_i8(w)

    def fc1_i8():
        xq, xs = mh.quant_rows_i8(x)
        mh.gemm_i8_swiglu(xq, xs, wq, ws)
    ms, _ = time_launches(fc1_i8, steps, warmup)
    gemms["fc1_int8"] = entry(ms, 62.0, "the same, W8A8 with the activations quantized each call (+ SwiGLU here)")
    del w, wq, ws
    wqkv = (0.02 * torch.randn((3 * H3_HEADS * 128, H3_D), generator=g, device=dev)).to(torch.bfloat16)
    ms, _ = time_launches(lambda: mh.gemm(x, wqkv), steps, warmup)
    gemms["qkv_bf16"] = entry(ms, 74.0, "19,456 x 5376 -> 21,504")
    del wqkv
    for name, k_in, ref in (("out_bf16", H3_HEADS * 128, 25.0), ("fc2_bf16", H3_FFN, 54.0)):
        xi = rnd(m, k_in)
        wi = (0.02 * torch.randn((H3_D, k_in), generator=g, device=dev)).to(torch.bfloat16)
        ms, _ = time_launches(lambda: mh.gemm(xi, wi), steps, warmup)
        gemms[name] = entry(ms, ref, f"19,456 x {k_in} -> 5376")
        del xi, wi
    del x
    out["gemm_19456_rows"] = gemms

    # The row kernels of one block at 19,308 rows (docs/performance.md:44: heads_partial, swiglu_rows,
    # gate_add_rows and rms_mod_rows, 1.3-1.5 s a forward): rms_mod_rows and gate_add_rows twice (attention and MLP
    # halves), swiglu_rows once over fc1's [gate | up] rows, heads_partial once (56 heads).
    rows = 19308
    xr, yr = rnd(rows, H3_D), rnd(rows, H3_D)
    wv, shv, scv, gav = mod_params(dev, H3_D, 32)
    hbuf = torch.empty_like(xr)
    fc1o = rnd(rows, 2 * H3_FFN)
    sw = torch.empty((rows, H3_FFN), dtype=torch.bfloat16, device=dev)
    qkv = rnd(rows, 3 * H3_HEADS * 128)
    ang = torch.rand((rows, 48), generator=g, device=dev) * 6.2831853 - 3.1415927
    ct, st = torch.cos(ang), torch.sin(ang)
    heads_out = [torch.empty((H3_HEADS, rows, 128), dtype=torch.bfloat16, device=dev) for _ in range(3)]

    def block_rows():
        for _ in range(2):
            mh.rms_mod_rows(xr, wv, shv, scv, out=hbuf)
            mh.gate_add_rows(xr, yr, gav)
        mh.swiglu_rows(fc1o, out=sw)
        mh.heads_partial(qkv, H3_HEADS, None, None, ct, st, q=heads_out[0], k=heads_out[1], v=heads_out[2])
    ms, _ = time_launches(block_rows, steps, warmup)
    out["row_kernels_per_forward"] = entry(ms * H3_BLOCKS, 1400.0,
                                           "a block's rms_mod_rows x2, gate_add_rows x2, swiglu_rows, heads_partial at "
                                           "19,308 rows, x 50 blocks (reference 1.3-1.5 s; its midpoint)")
    del xr, yr, hbuf, fc1o, sw, qkv, heads_out

    # The sparse path at 960x544 (docs/performance.md:165-177): 37 x 17 x 30 patch grid (400 cubes), 435 dense rows,
    # 56 heads, ratio 0.1 (k = 40), local 1; selection 0.3 s and attention 4.7 s a forward.
    grid = (37, 17, 30)
    video, n_dense = grid[0] * grid[1] * grid[2], 435
    arows = video + n_dense
    cubes = mh.cube_count(*grid)
    kk = mh.topk_k(0.1, cubes)
    q, k, v = rnd(H3_HEADS, arows, 128), rnd(H3_HEADS, arows, 128), rnd(H3_HEADS, arows, 128)
    a = mh.cube_args(H3_HEADS, grid, head_stride=arows * 128, k=kk, local=1)
    qc = torch.empty((H3_HEADS, cubes, 128), dtype=torch.float32, device=dev)
    kc = torch.empty_like(qc)
    idx = torch.empty((H3_HEADS, cubes, kk + 1), dtype=torch.int32, device=dev)
    cnt = torch.empty((H3_HEADS, cubes), dtype=torch.int32, device=dev)
    ws = torch.empty(mh.cube_select_workspace_bytes(a), dtype=torch.uint8, device=dev)
    order = torch.empty((H3_HEADS, cubes), dtype=torch.int32, device=dev)

    def select():
        mh.cube_pool(a, q, k, qc=qc, kc=kc)
        mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt)
        mh.cube_order(a, idx, cnt, order=order)
    ms, _ = time_launches(select, steps, warmup)
    out["sparse_selection_per_forward"] = entry(ms * H3_BLOCKS, 300.0,
                                                "cube_pool + cube_select + cube_order, 56 heads, 400 cubes, k = 40, "
                                                "x 50 blocks")
    ao = torch.empty_like(q)
    ms, _ = time_launches(lambda: mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense,
                                                           out=ao, order=order), steps, warmup)
    out["sparse_attention_per_forward"] = entry(ms * H3_BLOCKS, 4700.0,
                                                "flash_attn_sparse_128 over those pass lists, 19,305 rows, x 50 blocks")
    # Dense attention (docs/performance.md:168-169: 17.2 s a forward) is the same kernel with every cube selected
    # (ratio 1, which the reference's tests treat as dense).
    ad = mh.cube_args(H3_HEADS, grid, head_stride=arows * 128, k=cubes, local=0)
    idx_d = torch.arange(cubes, dtype=torch.int32, device=dev).expand(H3_HEADS, cubes, cubes).contiguous()
    cnt_d = torch.full((H3_HEADS, cubes), cubes, dtype=torch.int32, device=dev)
    ms_d, _ = time_launches(lambda: mh.flash_attn_sparse_128(ad, q, k, v, idx_d, cnt_d, dense_row0=video,
                                                             n_dense=n_dense, out=ao), steps, warmup)
    out["dense_attention_per_forward"] = entry(ms_d * H3_BLOCKS, 17200.0,
                                               "flash_attn_sparse_128 with every cube selected, 19,305 rows, x 50 "
                                               "blocks")
    del q, k, v, ao, idx_d, cnt_d

    # The AdaLN projections (docs/performance.md:45: gemm BF16 2688 x 96768, 50 a forward, 70-85 ms).
    cond = rnd(1, 2688)
    wa = (0.02 * torch.randn((6 * 3 * H3_D, 2688), generator=g, device=dev)).to(torch.bfloat16)
    mod = torch.empty((1, 6 * 3 * H3_D), dtype=torch.float32, device=dev)
    ms, _ = time_launches(lambda: mh.adaln_mod(cond, wa, out=mod), steps, warmup)
    out["adaln_projections_per_forward"] = entry(ms * H3_BLOCKS, 77.5,
                                                 "cond [1][2688] -> [96,768] table, x 50 blocks (reference 70-85 ms)")
    # A forward's kernels summed, against the reference's GPU time a forward at 960x544 (docs/performance.md:167-168:
    # dense 34.4 s, sparse at ratio 0.1 21.3 s, nominal thermal state): the four bf16 GEMMs (at 19,456 rows; fc1
    # with SwiGLU in its epilogue, which the row kernels time again) x 50, the row kernels, the AdaLN projections, and
    # the attention (with its selection when sparse).
    gemm_fwd = sum(gemms[n]["ms"] for n in ("fc1_bf16", "qkv_bf16", "out_bf16", "fc2_bf16")) * H3_BLOCKS
    common = gemm_fwd + out["row_kernels_per_forward"]["ms"] + out["adaln_projections_per_forward"]["ms"]
    out["sparse_forward_kernels"] = entry(common + out["sparse_selection_per_forward"]["ms"] +
                                          out["sparse_attention_per_forward"]["ms"], 21300.0,
                                          "the entries above summed for a sparse (ratio 0.1) forward")
    out["dense_forward_kernels"] = entry(common + out["dense_attention_per_forward"]["ms"], 34400.0,
                                         "the entries above summed for a dense forward")
    return out


def bench_block(mh, dev, steps, warmup):
    """One whole H3 block at the 768p shape through the library, in the model's row order from end to end (no gather
    or scatter): rms_mod_rows; the qkv projection (int8 weights, W8A16); heads_partial with cube_pool in its pass,
    its outputs [rows][heads x 128]; cube_select at ratio 0.1; flash_attn_sparse_128 over those rows; the out
    projection with gate_add_rows in its epilogue; rms_mod_rows; fc1 W8A16 + SwiGLU; fc2 with gate_add_rows. Weights
    are random normals quantized per row by quant_rows_i8, rows and modulation synthetic; the residual is updated in
    place by every timed block. The sequence of launches is timed as one step. `w8a8_ms` is the same block with the
    reference's own --int8 all (each GEMM's activations quantized per row, the int8 MFMA)."""
    T, Y, X = GRID
    video, n_dense = T * Y * X, ROWS - T * Y * X
    g = torch.Generator(device=dev).manual_seed(51)

    def w8(n, k):
        w = (0.02 * torch.randn((n, k), generator=g, device=dev)).to(torch.bfloat16)
        return mh.quant_rows_i8(w)
    wqkv, sqkv = w8(3 * HEADS * 128, DIM)
    wo, so = w8(DIM, HEADS * 128)
    w1, s1 = w8(2 * FFN, DIM)
    w2, s2 = w8(DIM, FFN)
    n1, sh_a, sc_a, ga_a = mod_params(dev, DIM, 52)
    n2, sh_m, sc_m, ga_m = mod_params(dev, DIM, 53)
    ang = torch.rand((ROWS, 48), generator=g, device=dev) * 6.2831853 - 3.1415927
    cs, sn = torch.cos(ang), torch.sin(ang)
    x = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    h = torch.empty_like(x)
    qkv = torch.empty((ROWS, 3 * HEADS * 128), dtype=torch.bfloat16, device=dev)
    q, k, v = (torch.empty((ROWS, HEADS * 128), dtype=torch.bfloat16, device=dev) for _ in range(3))
    cubes = mh.cube_count(*GRID)
    kk = mh.topk_k(0.1, cubes)
    a = mh.cube_args(HEADS, GRID, head_stride=128, row_stride=HEADS * 128, k=kk, local=1)
    qc = torch.empty((HEADS, cubes, 128), dtype=torch.float32, device=dev)
    kc = torch.empty_like(qc)
    idx = torch.empty((HEADS, cubes, kk + 1), dtype=torch.int32, device=dev)
    cnt = torch.empty((HEADS, cubes), dtype=torch.int32, device=dev)
    ws = torch.empty(mh.cube_select_workspace_bytes(a), dtype=torch.uint8, device=dev)
    order = torch.empty((HEADS, cubes), dtype=torch.int32, device=dev)
    att = torch.empty((ROWS, HEADS * 128), dtype=torch.bfloat16, device=dev)
    f = torch.empty((ROWS, FFN), dtype=torch.bfloat16, device=dev)

    def block():
        mh.rms_mod_rows(x, n1, sh_a, sc_a, out=h)
        mh.gemm(h, wqkv, w_scale=sqkv, out=qkv)
        mh.heads_partial_pool(qkv, HEADS, GRID, None, None, cs, sn, rot=96, layout="rows", cube_layout=mh.CUBES_GRID,
                              q=q, k=k, v=v, qc=qc, kc=kc)
        mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt)
        mh.cube_order(a, idx, cnt, order=order)
        mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense, out=att, order=order)
        mh.gemm_gate_add(att, wo, x, ga_a, w_scale=so)
        mh.rms_mod_rows(x, n2, sh_m, sc_m, out=h)
        mh.gemm_w8a16_swiglu(h, w1, s1, out=f)
        mh.gemm_gate_add(f, w2, x, ga_m, w_scale=s2)
    ms, wall = time_launches(block, steps, warmup)
    med = LAST_MEDIAN_MS[0]
    finite = bool(torch.isfinite(x.float()).all())

    # The same block under the reference's own --int8 all (W8A8): each GEMM's activations quantized per row by
    # quant_rows_i8 first, then the int8 MFMA.
    xq = torch.empty((ROWS, max(DIM, FFN)), dtype=torch.int8, device=dev)
    xs = torch.empty(ROWS, dtype=torch.float32, device=dev)

    def quant(t):
        n = t.shape[1]
        q8 = xq.view(-1)[:ROWS * n].view(ROWS, n)
        mh.quant_rows_i8(t, q=q8, scale=xs)
        return q8

    def block_w8a8():
        mh.rms_mod_rows(x, n1, sh_a, sc_a, out=h)
        mh.gemm(quant(h), wqkv, x_scale=xs, w_scale=sqkv, out=qkv)
        mh.heads_partial_pool(qkv, HEADS, GRID, None, None, cs, sn, rot=96, layout="rows", cube_layout=mh.CUBES_GRID,
                              q=q, k=k, v=v, qc=qc, kc=kc)
        mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt)
        mh.cube_order(a, idx, cnt, order=order)
        mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense, out=att, order=order)
        mh.gemm_gate_add(quant(att), wo, x, ga_a, x_scale=xs, w_scale=so)
        mh.rms_mod_rows(x, n2, sh_m, sc_m, out=h)
        mh.gemm_i8_swiglu(quant(h), xs, w1, s1, out=f)
        mh.gemm_gate_add(quant(f), w2, x, ga_m, x_scale=xs, w_scale=s2)
    ms8, _ = time_launches(block_w8a8, steps, warmup)
    finite = finite and bool(torch.isfinite(x.float()).all())
    return {"ms": ms, "median_ms": med, "wall_ms": wall, "rows": ROWS, "finite": finite,
            "shape": {"rows": ROWS, "dim": DIM, "ffn": FFN, "heads": HEADS, "grid": list(GRID), "k": kk},
            "weights": "int8 (W8A16)", "w8a8_ms": ms8, "w8a8_median_ms": LAST_MEDIAN_MS[0]}


def bench_proj(mh, dev, steps, warmup):
    """The block's other projections at the 768p rows (129,536): qkv 5120 -> 3 x 40 x 128 = 15,360 (plain store), the
    out projection 5120 -> 5120 and fc2 13,824 -> 5120 with gate_add_rows folded into the epilogue (residual += gate *
    y, in place), each with int8 weights (weight-only, the --int8 path) and qkv also with bf16 weights. 2 flop a MAC."""
    g = torch.Generator(device=dev).manual_seed(12)
    res = {}
    for name, k, n, epi in (("qkv", DIM, 3 * HEADS * 128, "store"), ("out", DIM, DIM, "gate_add"),
                            ("fc2", FFN, DIM, "gate_add")):
        x = torch.randn((ROWS, k), generator=g, device=dev).to(torch.bfloat16)
        w = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
        s = (torch.rand(n, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
        y = torch.zeros((ROWS, n), dtype=torch.bfloat16, device=dev)
        gate = (0.1 * torch.randn(n, generator=g, device=dev)).float()
        if epi == "store":
            fn = lambda: mh.gemm(x, w, w_scale=s, out=y)  # noqa: E731
        else:
            fn = lambda: mh.gemm_gate_add(x, w, y, gate, w_scale=s)  # noqa: E731
        ms, _ = time_launches(fn, steps, warmup)
        flops = 2.0 * ROWS * k * n
        res[name] = {"ms": ms, "tflops": flops / ms / 1e9, "mfma_util": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
                     "shape": [ROWS, k, n], "weights": "int8 (W8A16)", "epilogue": epi}
        if name == "out":
            # The same on the reference's float residual stream: residual float [rows][5120] += gate * y.
            yf = torch.zeros((ROWS, n), dtype=torch.float32, device=dev)
            fms, _ = time_launches(lambda: mh.gemm_gate_add(x, w, yf, gate, w_scale=s), steps, warmup)
            res[name]["float_residual_ms"] = fms
            res[name]["float_residual_tflops"] = flops / fms / 1e9
            del yf
        if name == "qkv":
            wb = (w.float() * s[:, None]).to(torch.bfloat16)
            bms, _ = time_launches(lambda: mh.gemm(x, wb, out=y), steps, warmup)
            res[name]["bf16_ms"] = bms
            res[name]["bf16_tflops"] = flops / bms / 1e9
            res[name]["bf16_mfma_util"] = flops / bms / 1e9 / BF16_PEAK_TFLOPS
            del wb
        del x, w, y
        torch.cuda.empty_cache()
    return res


def bench_fc1(mh, dev, steps, warmup, compare):
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randint(-127, 128, (2 * FFN, DIM), generator=g, device=dev, dtype=torch.int8)
    s = (torch.rand(2 * FFN, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
    out = torch.empty((ROWS, FFN), dtype=torch.bfloat16, device=dev)
    ms, _ = time_launches(lambda: mh.gemm_w8a16_swiglu(x, w, s, out=out), steps, warmup)
    flops = 2.0 * ROWS * DIM * 2 * FFN
    # The int8 weights (141 MB) fit in the MALL; each launch reads them once per row band anyway. Timed cold too.
    cold_ms, _ = time_launches(lambda: mh.gemm_w8a16_swiglu(x, w, s, out=out), max(3, steps // 2), 1, cold=True)
    res = {"ms": ms, "tflops": flops / ms / 1e9, "mfma_util": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
           "flops": flops, "shape": [ROWS, DIM, 2 * FFN], "cold_ms": cold_ms}
    # The dense bf16 fc1 the int8 path replaces: this library's bf16 kernel (GEMM + SwiGLU epilogue) and, with
    # compare, hipBLASLt through torch.matmul (GEMM only, no epilogue).
    wb = (w.float() * s[:, None]).to(torch.bfloat16)
    bms, _ = time_launches(lambda: mh.gemm_bf16_swiglu(x, wb, out=out), steps, warmup)
    res["bf16_fc1_ms"] = bms
    res["bf16_fc1_tflops"] = flops / bms / 1e9
    res["bf16_fc1_mfma_util"] = flops / bms / 1e9 / BF16_PEAK_TFLOPS
    del wb
    # The reference's own --int8 form, W8A8: x quantized per row (quant_rows_i8), the int8 GEMM on the int8 MFMA.
    xq = torch.empty((ROWS, DIM), dtype=torch.int8, device=dev)
    xs = torch.empty(ROWS, dtype=torch.float32, device=dev)
    qms, _ = time_launches(lambda: mh.quant_rows_i8(x, q=xq, scale=xs), steps, warmup)
    ims, _ = time_launches(lambda: mh.gemm_i8_swiglu(xq, xs, w, s, out=out), steps, warmup)
    res["w8a8_quant_x_ms"] = qms
    res["w8a8_quant_x_GBs"] = ROWS * (DIM * 3 + 4) / qms / 1e6       # read bf16 x; write int8 x and a scale a row
    res["w8a8_quant_x_frac"] = res["w8a8_quant_x_GBs"] / HBM_PEAK_GBS
    res["w8a8_fc1_ms"] = ims
    res["w8a8_fc1_tops"] = flops / ims / 1e9
    res["w8a8_fc1_int8_mfma_util"] = flops / ims / 1e9 / INT8_PEAK_TOPS
    del xq, xs
    if compare:
        # hipBLASLt's bf16 GEMM on the same weight layout (w [2 F][5120], x w^T: its fastest form here) and on w^T
        # stored [5120][2 F]; no epilogue.
        wb = (w.float() * s[:, None]).to(torch.bfloat16)
        y = torch.empty((ROWS, 2 * FFN), dtype=torch.bfloat16, device=dev)
        cms, _ = time_launches(lambda: torch.matmul(x, wb.t(), out=y), max(3, steps // 2), 2)
        res["bf16_hipblaslt_gemm_ms"] = cms
        res["bf16_hipblaslt_tflops"] = flops / cms / 1e9
        wt = wb.t().contiguous()
        nms, _ = time_launches(lambda: torch.matmul(x, wt, out=y), max(3, steps // 2), 2)
        res["bf16_hipblaslt_gemm_wt_ms"] = nms
        del wt
        res.update(hipblaslt_tuned_replay(lambda: torch.matmul(x, wb.t(), out=y), flops, max(3, steps // 2)))
        del y, wb
    return res


TUNABLEOP_FC1 = Path(__file__).resolve().parent / "bench_tunableop_fc1.csv"


def hipblaslt_tuned_replay(run, flops, steps):
    """The fc1 GEMM with the solution PyTorch's TunableOp found best for it (`bench.py --only tuned --tunableop-out
    bench_tunableop_fc1.csv` on this image), read from that file with tuning off, so the default run times it in
    seconds instead of tuning for minutes. The file's validators (PyTorch, ROCm, hipBLASLt versions, the GPU) must match
    the running ones, else TunableOp refuses the file and no figure is reported."""
    if not TUNABLEOP_FC1.exists():
        return {"bf16_hipblaslt_tuned_ms": None, "bf16_hipblaslt_tuned_note": "no tuning file"}
    tun = torch.cuda.tunable
    try:
        tun.enable(True)
        tun.tuning_enable(False)
        if not tun.read_file(str(TUNABLEOP_FC1)):
            return {"bf16_hipblaslt_tuned_ms": None, "bf16_hipblaslt_tuned_note": "tuning file refused"}
        sol = [r for r in tun.get_results() if r[0].startswith("GemmTunableOp_BFloat16") and r[2] != "Default"]
        ms, _ = time_launches(run, steps, 2)
    finally:
        tun.enable(False)
    return {"bf16_hipblaslt_tuned_ms": ms, "bf16_hipblaslt_tuned_tflops": flops / ms / 1e9,
            "bf16_hipblaslt_tuned_solution": " ".join(map(str, sol[0][:3])) if sol else None}


def bench_hipblaslt_tuned(dev, steps, warmup, max_ms_per_solution=200, out_file=None):
    """hipBLASLt's (and rocBLAS's) best solution for fc1's GEMM (x [129,536][5120] bf16 times w^T, w the weight's
    [27,648][5120] rows, no epilogue), found by PyTorch's TunableOp, which times every candidate solution for this
    shape; beside the default solution torch.matmul picks. The tuning results file goes to a temporary directory,
    and is copied to `out_file` when one is given (the file the default run's fc1 leg replays)."""
    import tempfile

    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn((2 * FFN, DIM), generator=g, device=dev).to(torch.bfloat16)  # the weight's [out][in] rows
    wt = w.t()
    y = torch.empty((ROWS, 2 * FFN), dtype=torch.bfloat16, device=dev)
    flops = 2.0 * ROWS * DIM * 2 * FFN
    dms, _ = time_launches(lambda: torch.matmul(x, wt, out=y), max(3, steps), warmup)
    tun = torch.cuda.tunable
    t0 = time.perf_counter()
    with tempfile.TemporaryDirectory() as tmp:
        tun.set_filename(str(Path(tmp) / "tunableop_results.csv"))
        tun.enable(True)
        tun.tuning_enable(True)
        tun.set_max_tuning_duration(max_ms_per_solution)
        tun.set_max_tuning_iterations(3)
        torch.matmul(x, wt, out=y)  # tunes this shape
        torch.cuda.synchronize()
        tune_s = time.perf_counter() - t0
        tun.tuning_enable(False)
        tms, _ = time_launches(lambda: torch.matmul(x, wt, out=y), max(3, steps), warmup)
        results = tun.get_results()
        if out_file:
            # TunableOp's results-file format: its validators, then one line a tuned GEMM
            lines = [f"Validator,{k},{v}" for k, v in tun.get_validators()]
            lines += [",".join(map(str, r)) for r in results]
            Path(out_file).write_text("\n".join(lines) + "\n")
        tun.enable(False)
    return {"default_ms": dms, "default_tflops": flops / dms / 1e9, "tuned_ms": tms, "tuned_tflops": flops / tms / 1e9,
            "tuned_mfma_util": flops / tms / 1e9 / BF16_PEAK_TFLOPS, "tuning_s": tune_s,
            "results": [" ".join(map(str, r)) for r in results]}


def bench_share(mh, dev, steps, warmup, gpus=8):
    """The hot path at one GPU's share of a `gpus`-way split, on this one GPU: the row ops and fc1 shard by rows
    (N / gpus rows, fc1's weights whole), the selector and the attention by heads (40 / gpus heads). Each figure is the
    share's own throughput; `vs_full` is it over the full shape's (1 = no loss from the smaller launch)."""
    rows = (ROWS + gpus - 1) // gpus
    heads = HEADS // gpus
    g = torch.Generator(device=dev).manual_seed(17)
    res = {"gpus": gpus, "rows": rows, "heads": heads}
    x = torch.randn((rows, DIM), generator=g, device=dev).to(torch.bfloat16)
    r = torch.randn((rows, DIM), generator=g, device=dev).to(torch.bfloat16)
    w, shift, scale, gate = mod_params(dev, DIM, 1)
    out = torch.empty_like(x)
    ms, _ = time_launches(lambda: mh.rms_mod_gate_add_rows(x, r, w, shift, scale, gate, out=out), steps, warmup)
    nb = rows * DIM * 6
    res["fused_rms_mod_gate_add"] = {"ms": ms, "GBs": nb / ms / 1e6, "frac": nb / ms / 1e6 / HBM_PEAK_GBS}
    del r, out
    gt = torch.randn((rows, FFN), generator=g, device=dev).to(torch.bfloat16)
    up = torch.randn((rows, FFN), generator=g, device=dev).to(torch.bfloat16)
    so = torch.empty_like(gt)
    ms, _ = time_launches(lambda: mh.swiglu_rows(gt, up, out=so), steps, warmup)
    nb = rows * FFN * 6
    res["swiglu"] = {"ms": ms, "GBs": nb / ms / 1e6, "frac": nb / ms / 1e6 / HBM_PEAK_GBS}
    del gt, up
    wq = torch.randint(-127, 128, (2 * FFN, DIM), generator=g, device=dev, dtype=torch.int8)
    ws = (torch.rand(2 * FFN, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
    ms, _ = time_launches(lambda: mh.gemm_w8a16_swiglu(x, wq, ws, out=so), max(3, steps // 2), max(1, warmup // 2))
    fl = 2.0 * rows * DIM * 2 * FFN
    res["fc1_w8a16_swiglu"] = {"ms": ms, "tflops": fl / ms / 1e9, "mfma_util": fl / ms / 1e9 / BF16_PEAK_TFLOPS}
    del x, so, wq, ws
    torch.cuda.empty_cache()
    # Selector and attention on the first `heads` heads of the 768p q / k.
    T, Y, X = GRID
    video, n_dense = T * Y * X, 512
    q, k = (t[:heads].contiguous() for t in selector_qk(dev, n_dense))
    torch.cuda.empty_cache()
    v = torch.randn((heads, video + n_dense, 128), generator=g, device=dev).to(torch.bfloat16)
    cubes = mh.cube_count(*GRID)
    kk = mh.topk_k(0.1, cubes)
    a = mh.cube_args(heads, GRID, head_stride=(video + n_dense) * 128, k=kk, local=1)
    qc = torch.empty((heads, cubes, 128), dtype=torch.float32, device=dev)
    kc = torch.empty_like(qc)
    idx = torch.empty((heads, cubes, kk + 1), dtype=torch.int32, device=dev)
    cnt = torch.empty((heads, cubes), dtype=torch.int32, device=dev)
    ws = torch.empty(mh.cube_select_workspace_bytes(a), dtype=torch.uint8, device=dev)

    def selector():
        mh.cube_pool(a, q, k, qc=qc, kc=kc)
        mh.cube_select(a, qc, kc, workspace=ws, idx=idx, cnt=cnt)
    ms, _ = time_launches(selector, steps, warmup)
    nb = 2 * heads * video * 128 * 2 + heads * cubes * (kk + 1) * 4
    res["cube_selector"] = {"ms": ms, "GBs": nb / ms / 1e6, "frac": nb / ms / 1e6 / HBM_PEAK_GBS}
    o = torch.empty_like(q)
    order = mh.cube_order(a, idx, cnt)
    ms, _ = time_launches(lambda: mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense,
                                                           out=o, order=order), max(3, steps // 2),
                          max(1, warmup // 2))
    sel = int(cnt.to(torch.int64).sum())
    rows_all = video + n_dense
    fl = 4.0 * 128 * (64 * (sel * 64 + heads * cubes * n_dense) + heads * n_dense * rows_all)
    res["flash_attn_sparse_128"] = {"ms": ms, "tflops": fl / ms / 1e9, "mfma_util": fl / ms / 1e9 / BF16_PEAK_TFLOPS}
    del q, k, v, o, qc, kc, idx, cnt, order
    torch.cuda.empty_cache()
    return res


def cpu_model() -> str:
    """The host CPU from /proc/cpuinfo: its model name, with the family / model / stepping numbers (a virtualized host
    may report a bare family name) and the logical CPUs the file lists; the machine type where the file has none."""
    try:
        fields, cpus = {}, 0
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "processor":
                cpus += 1
            elif key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                fields[key] = val.strip()
        if "model name" in fields:
            ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
            return f"{fields['model name']} ({ids}; {cpus} logical CPUs)" if ids else fields["model name"]
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(seconds: float = 10.0) -> dict:
    """The scalar C oracle of the fused op on one host core, on a sample of the 768p rows sized to ~`seconds`."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as orc

    rng = np.random.default_rng(0)

    def run(n):
        x = orc.bf16_from_f64(rng.standard_normal((n, DIM)))
        r = orc.bf16_from_f64(rng.standard_normal((n, DIM)))
        w = (1 + 0.02 * rng.standard_normal(DIM)).astype(np.float32)
        sh, sc, ga = [(0.1 * rng.standard_normal((1, DIM))).astype(np.float32) for _ in range(3)]
        t0 = time.perf_counter()
        orc.rms_mod_gate_add_rows(x, r, w, sh, sc, ga)
        return time.perf_counter() - t0

    t = run(64)
    n = int(min(ROWS, max(64, 64 * seconds / max(t, 1e-6))))
    t = run(n)
    gbs = n * DIM * 6 / t / 1e9
    # The same port row-parallel on every core this process may use (the oracle releases the GIL in its C call).
    cores = len(os.sched_getaffinity(0))
    x = orc.bf16_from_f64(rng.standard_normal((n, DIM)))
    r = orc.bf16_from_f64(rng.standard_normal((n, DIM)))
    w = (1 + 0.02 * rng.standard_normal(DIM)).astype(np.float32)
    sh, sc, ga = [(0.1 * rng.standard_normal((1, DIM))).astype(np.float32) for _ in range(3)]
    chunks = np.array_split(np.arange(n), cores)
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(cores) as ex:
        t0 = time.perf_counter()
        list(ex.map(lambda c: orc.rms_mod_gate_add_rows(x[c[0]:c[-1] + 1], r[c[0]:c[-1] + 1], w, sh, sc, ga),
                    [c for c in chunks if len(c)]))
        tp = time.perf_counter() - t0
    return {"value": gbs, "unit": "GB/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
            "sample": f"fused modulated RMS norm + gated residual over {n} of the {ROWS} rows x {DIM} bf16 "
                      f"({t:.1f} s), scalar C oracle, one thread on {cpu_model()}",
            "row_parallel": {"value": n * DIM * 6 / tp / 1e9, "unit": "GB/s", "cores": cores,
                             "sample": f"the same {n} rows split over {cores} threads ({tp:.2f} s)"}}


def _parallel(fn, parts, cores):
    """Run fn(part) for every part on `cores` threads (the oracle's C calls release the GIL); wall seconds."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(cores) as ex:
        t0 = time.perf_counter()
        list(ex.map(fn, parts))
        return time.perf_counter() - t0


def cpu_baseline_configs(gpu: dict) -> dict:
    """The scalar C oracle on the other workloads, one thread and row-parallel on every host core, each on a sample
    of a few seconds; figures for the full workload are extrapolated linearly from the sample and say so."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as orc

    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(5)
    out = {}

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    # modulated RMS norm, f32 [4096][1024], full size
    x = rng.standard_normal((4096, 1024)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(1024)).astype(np.float32)
    sh, sc = [(0.1 * rng.standard_normal((1, 1024))).astype(np.float32) for _ in range(2)]
    t1 = timed(lambda: orc.rms_mod_rows(x, w, sh, sc))
    parts = np.array_split(np.arange(4096), cores)
    tp = _parallel(lambda c: orc.rms_mod_rows(x[c[0]:c[-1] + 1], w, sh, sc), parts, cores)
    nb = 4096 * 1024 * 8
    out["rms_mod_f32_4096x1024"] = {"unit": "GB/s", "single": nb / t1 / 1e9, "row_parallel": nb / tp / 1e9,
                                    "sample": "full size", "gpu": gpu.get("rms_mod_f32_4096x1024", {}).get("GBs")}

    # SwiGLU, split gate and up [129,536][13,824] bf16: a row sample
    base = orc.bf16_from_f64(rng.standard_normal((64, FFN)))
    n1 = 64 * max(1, int(1.0 / max(timed(lambda: orc.swiglu_rows(base, base)), 1e-3) // 1))
    n1 = min(n1, 4096)
    g = np.tile(base, (n1 // 64, 1))
    u = np.roll(g, 1, axis=1)
    t1 = timed(lambda: orc.swiglu_rows(g, u))
    gp, up = np.tile(g, (cores, 1)), np.tile(u, (cores, 1))
    parts = [slice(i * n1, (i + 1) * n1) for i in range(cores)]
    tp = _parallel(lambda sl: orc.swiglu_rows(gp[sl], up[sl]), parts, cores)
    single, par = n1 * FFN * 6 / t1 / 1e9, cores * n1 * FFN * 6 / tp / 1e9
    out["swiglu_129536x13824"] = {"unit": "GB/s", "single": single, "row_parallel": par,
                                  "full_ms_extrapolated": {"single": ROWS * FFN * 6 / single / 1e6,
                                                           "row_parallel": ROWS * FFN * 6 / par / 1e6},
                                  "sample": f"{n1} rows on one thread, {cores} x {n1} rows on {cores} threads",
                                  "gpu": gpu.get("swiglu", {}).get("split", {}).get("GBs")}
    del gp, up, g, u

    # cube selector (pool, scores, top-k) per head: one head on one thread, one head a thread on all cores
    rows_h = GRID[0] * GRID[1] * GRID[2]
    k = math.ceil(0.1 * (GRID[0] // 4) * (GRID[1] // 4) * (GRID[2] // 4))
    q0 = orc.bf16_from_f64(rng.standard_normal((1, rows_h, 128)))
    heads_p = min(cores, HEADS)
    qs = [np.roll(q0, 7 * h, axis=1) for h in range(heads_p)]
    ks = [np.roll(q0, 7 * h + 3, axis=1) for h in range(heads_p)]

    def one_head(h):
        qc, kc, _ = orc.cube_pool(qs[h], ks[h], 1, GRID)
        orc.cube_topk(orc.cube_scores(qc, kc), GRID, k, 1, sorted_form=True)
    t1 = timed(lambda: one_head(0))
    tp = _parallel(one_head, range(heads_p), cores)
    sel = gpu.get("cube_selector", {})
    out["cube_selector_40x2016"] = {"unit": "ms for 40 heads (extrapolated)", "single": 1e3 * t1 * HEADS,
                                    "row_parallel": 1e3 * tp * math.ceil(HEADS / heads_p),
                                    "sample": f"1 head on one thread; {heads_p} heads, one a thread",
                                    "gpu": sel.get("ms")}
    del qs, ks

    # fc1 W8A16 + SwiGLU [129,536] x 5120 x 27,648: a row slice
    wq = rng.integers(-127, 128, (2 * FFN, DIM), dtype=np.int8)
    ws = rng.uniform(0.5e-3, 2e-3, 2 * FFN).astype(np.float32)
    xr = orc.bf16_from_f64(rng.standard_normal((4 * cores, DIM)))
    t1 = timed(lambda: orc.gemm_w8a16_swiglu(xr[:4], wq, ws))
    tp = _parallel(lambda i: orc.gemm_w8a16_swiglu(xr[4 * i:4 * i + 4], wq, ws), range(cores), cores)
    fl = 2 * DIM * 2 * FFN
    fc = gpu.get("fc1_w8a16_swiglu", {})
    out["fc1_w8a16_swiglu"] = {"unit": "TFLOP/s", "single": 4 * fl / t1 / 1e12, "row_parallel": 4 * cores * fl / tp / 1e12,
                               "full_ms_extrapolated": {"single": 1e3 * t1 * ROWS / 4,
                                                        "row_parallel": 1e3 * tp * ROWS / (4 * cores)},
                               "sample": f"4 rows on one thread, {cores} x 4 rows on {cores} threads",
                               "gpu": fc.get("tflops")}
    out["cores"] = cores
    out["cpu"] = cpu_model()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="fused,block_order,copy,swiglu,select,cond,heads,attn,proj,fc1,mfma,rms_f32,"
                                      "block,ref,share")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-compare", action="store_true")
    ap.add_argument("--tunableop-out", default=None, help="with --only tuned: where to copy TunableOp's results file")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: these kernels run on a single MI355X and have no multi-GPU path (the row "
              "ops and fc1 would shard by rows, the selector and attention by heads, each GPU running the same "
              "kernel on its share). Run with --gpus 1.", file=sys.stderr)
        return 2
    import mako_h3 as mh

    dev = torch.device("cuda:0")
    ops = set(args.only.split(","))
    report = {}

    def done(name: str) -> None:
        # one progress line a leg, on stderr, so the JSON line stays alone on stdout
        print(f"bench: {name} done", file=sys.stderr, flush=True)

    if "fused" in ops:
        report["fused_rms_mod_gate_add"] = bench_fused(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        done("fused")
    if "block_order" in ops:
        report["gate_add_rms_mod"] = bench_block_order(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        done("block_order")
    if "copy" in ops:
        report["hbm_copy"] = bench_copy(dev, args.steps, args.warmup)
        report["stream_ceiling"] = bench_stream(dev, args.steps, args.warmup)
        head = report.get("fused_rms_mod_gate_add")
        if head:
            report["stream_ceiling"]["fused_vs_r2w1"] = head["GBs"] / report["stream_ceiling"]["r2w1"]["GBs"]
            rows2 = report["stream_ceiling"]["rows_r2w1"]["2_workgroups_a_cu"]
            report["stream_ceiling"]["fused_vs_rows_r2w1"] = head["GBs"] / rows2["GBs"]
        order = report.get("gate_add_rms_mod")
        if order:
            report["stream_ceiling"]["block_order_vs_r2w2"] = order["GBs"] / report["stream_ceiling"]["r2w2"]["GBs"]
            report["stream_ceiling"]["float_stream_block_order_vs_r2w2"] = (
                order["float_stream"]["GBs"] / report["stream_ceiling"]["r2w2"]["GBs"])
        torch.cuda.empty_cache()
        done("copy")
    if "rms_f32" in ops:
        report["rms_mod_f32_4096x1024"] = bench_rms_f32(mh, dev, args.steps, args.warmup)
        done("rms_f32")
    if "swiglu" in ops:
        report["swiglu"] = bench_swiglu(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        done("swiglu")
    if "select" in ops:
        report["cube_selector"] = bench_select(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        done("select")
    if "cond" in ops:
        report["modulation"] = bench_cond(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        done("cond")
    if "heads" in ops:
        report["heads_partial"] = bench_heads(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
        done("heads")
    sel, hp = report.get("cube_selector"), report.get("heads_partial")
    if sel and hp:
        # The selector with its pool folded into heads_partial: what the pool still costs in that pass (gathered
        # through the cube map, or in the model's order), plus cube_select.
        sel["pool_in_heads_partial"] = {
            lay: {"pool_ms": hp[key]["pool_cost_in_pass_ms"],
                  "ms": max(hp[key]["pool_cost_in_pass_ms"], 0.0) + sel["select_ms"]}
            for lay, key in (("gathered", "gathered_pool"), ("grid", "grid_pool"))}
    if "attn" in ops:
        report["flash_attn_sparse_128"] = bench_attn(mh, dev, max(3, args.steps // 2), max(1, args.warmup // 2))
        torch.cuda.empty_cache()
        done("attn")
    if "proj" in ops:
        report["projections"] = bench_proj(mh, dev, max(3, args.steps // 2), max(1, args.warmup // 2))
        torch.cuda.empty_cache()
        done("proj")
    if "fc1" in ops:
        report["fc1_w8a16_swiglu"] = bench_fc1(mh, dev, max(3, args.steps // 2), max(1, args.warmup // 2),
                                               not args.no_compare)
        torch.cuda.empty_cache()
        done("fc1")
    if "tuned" in ops:
        report["hipblaslt_tuned_fc1"] = bench_hipblaslt_tuned(dev, max(3, args.steps // 2),
                                                              max(1, args.warmup // 2), out_file=args.tunableop_out)
        torch.cuda.empty_cache()
        done("tuned")
    if "mfma" in ops:
        ceil = bench_mfma_ceiling(dev, args.steps, args.warmup)
        fc1 = report.get("fc1_w8a16_swiglu")
        if fc1:
            ceil["fc1_w8a16_vs_bf16_ceiling"] = fc1["tflops"] / ceil["bf16"]["rate"]
            ceil["fc1_w8a8_vs_int8_ceiling"] = fc1["w8a8_fc1_tops"] / ceil["int8"]["rate"]
        report["mfma_ceiling"] = ceil
        done("mfma")

    if "block" in ops:
        blk = bench_block(mh, dev, 3, 1)
        # The same stages timed on their own in the legs above (all but the two rms_mod_rows), summed, where those
        # legs ran: qkv, heads_partial with the pool (grid layout), cube_select, the attention, out, fc1, fc2.
        proj = report.get("projections") or {}
        parts = [(proj.get("qkv") or {}).get("ms"),
                 ((report.get("heads_partial") or {}).get("grid_pool") or {}).get("ms"),
                 (report.get("cube_selector") or {}).get("select_ms"),
                 (report.get("flash_attn_sparse_128") or {}).get("ms"),
                 (proj.get("out") or {}).get("ms"),
                 (report.get("fc1_w8a16_swiglu") or {}).get("ms"),
                 (proj.get("fc2") or {}).get("ms")]
        if all(t is not None for t in parts):
            blk["stages_ms_without_norms"] = sum(parts)
        report["block_768p"] = blk
        torch.cuda.empty_cache()
        done("block")

    if "ref" in ops:
        report["reference_shapes"] = bench_reference_shapes(mh, dev, max(3, args.steps // 2), max(1, args.warmup // 2))
        torch.cuda.empty_cache()
        done("ref")

    if "share" in ops:
        share = bench_share(mh, dev, args.steps, args.warmup)
        full = {"fused_rms_mod_gate_add": (report.get("fused_rms_mod_gate_add") or {}).get("GBs"),
                "swiglu": ((report.get("swiglu") or {}).get("split") or {}).get("GBs"),
                "fc1_w8a16_swiglu": (report.get("fc1_w8a16_swiglu") or {}).get("tflops"),
                "cube_selector": (report.get("cube_selector") or {}).get("GBs"),
                "flash_attn_sparse_128": (report.get("flash_attn_sparse_128") or {}).get("tflops")}
        for name, ref in full.items():
            mine = share[name].get("GBs", share[name].get("tflops"))
            share[name]["vs_full"] = mine / ref if ref else None
        report["per_gpu_share"] = share
        torch.cuda.empty_cache()
        done("share")

    head = report.get("fused_rms_mod_gate_add")
    traffic = None
    tf = REPO / "profiles" / "traffic_fused_rms_mod_gate_add_768p.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
    line = {
        "metric": METRIC,
        "value": round(head["GBs"], 1) if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4) if head else None,
        "median_ms": round(head["median_ms"], 4) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) rows, N(0,0.1) modulation vectors)",
        "config": {"workload": "fused adaLN-modulated RMSNorm + gated residual, 768p-shaped rows",
                   "rows": ROWS, "dim": DIM, "eps": 1e-6, "bytes_per_step": ROWS * DIM * 6},
    }
    if head:
        line["roofline"] = {"bound": "hbm", "achieved": round(head["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(head["frac"], 4), "traffic": traffic}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
        line["cpu_baseline"]["other_workloads"] = cpu_baseline_configs(report)
    line["ops"] = report
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
