"""Benchmark of the H3 per-block hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only fused,swiglu,select,fc1,rms_f32] [--no-cpu]

A step is one pass of the headline kernel -- the fused adaLN-modulated RMS norm + gated residual -- over the
768p-shaped batch (129,536 rows = 32x48x84 video + 512 text, x 5120, bf16), inputs resident in HBM. value is its
achieved algorithmic HBM bandwidth (6 bytes an element: read x and residual, write out). The same run also times the
other ops of the path at their shapes (SwiGLU split and fused-row, the cube selector, the int8 fc1 + SwiGLU GEMM, the
fp32 modulated RMS norm) and reports each as ms, GB/s or TFLOP/s and a fraction of the MI355X roofline. Kernel times
come from HIP events recorded on the stream the kernels run on (torch's current stream). The CPU baseline is the
scalar C oracle on one host core, on a bounded sample of the same workload.

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
FP32_MFMA_PEAK_TFLOPS = 157.3  # dense fp32 MFMA
METRIC = "ms/op + achieved HBM GB/s (% peak) at 768p rows; int8 GEMM MFMA util %"

ROWS, DIM, FFN = 32 * 48 * 84 + 512, 5120, 13824
GRID, HEADS = (32, 48, 84), 40


def time_launches(fn, steps: int, warmup: int) -> tuple[float, float]:
    """(mean ms per launch from HIP events on the current stream, wall ms per launch) over `steps` launches."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = [s.elapsed_time(e) for s, e in zip(starts, ends)]
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
    nbytes = ROWS * DIM * 6
    return {"ms": ms, "wall_ms": wall, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 /
            HBM_PEAK_GBS, "shape": [ROWS, DIM]}


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
    return {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "two_kernel_ms": ms2, "two_kernel_bytes": ROWS * DIM * 10, "shape": [ROWS, DIM]}


def bench_copy(dev, steps, warmup):
    """Calibration: a plain device-to-device copy of a 768p-sized bf16 tensor (read + write, 2.65 GB)."""
    src = torch.empty((ROWS, DIM), dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    ms, _ = time_launches(lambda: dst.copy_(src), steps, warmup)
    nbytes = ROWS * DIM * 4
    return {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}


def bench_rms_f32(mh, dev, steps, warmup):
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn((4096, 1024), generator=g, device=dev)
    w, shift, scale, _ = mod_params(dev, 1024, 4)
    out = torch.empty_like(x)
    ms, _ = time_launches(lambda: mh.rms_mod_rows(x, w, shift, scale, out=out), steps, warmup)
    nbytes = 4096 * 1024 * 8
    return {"ms": ms, "bytes": nbytes, "GBs": nbytes / ms / 1e6, "shape": [4096, 1024],
            "note": "33.6 MB: launch- and L2-bound, not an HBM measurement"}


def bench_swiglu(mh, dev, steps, warmup):
    g = torch.Generator(device=dev).manual_seed(5)
    res = {}
    nbytes = ROWS * FFN * 6
    gate = torch.randn((ROWS, FFN), generator=g, device=dev).to(torch.bfloat16)
    up = torch.randn((ROWS, FFN), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(gate)
    ms, _ = time_launches(lambda: mh.swiglu_rows(gate, up, out=out), steps, warmup)
    res["split"] = {"ms": ms, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}
    del gate, up
    gu = torch.randn((ROWS, 2 * FFN), generator=g, device=dev).to(torch.bfloat16)
    ms, _ = time_launches(lambda: mh.swiglu_rows(gu, out=out), steps, warmup)
    res["fused_row"] = {"ms": ms, "GBs": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}
    res["bytes"] = nbytes
    res["shape"] = [ROWS, FFN]
    return res


def bench_select(mh, dev, steps, warmup):
    T, Y, X = GRID
    rows = T * Y * X
    g = torch.Generator(device=dev).manual_seed(7)
    rng = np.random.default_rng(7)
    tt = torch.arange(T, device=dev, dtype=torch.float32).view(T, 1, 1) / T
    yy = torch.arange(Y, device=dev, dtype=torch.float32).view(1, Y, 1) / Y
    xx = torch.arange(X, device=dev, dtype=torch.float32).view(1, 1, X) / X
    qk = []
    for _ in range(2):
        t = torch.empty((HEADS, rows, 128), dtype=torch.bfloat16, device=dev)
        for h in range(HEADS):
            acc = torch.randn((rows, 128), generator=g, device=dev)
            for _j in range(4):
                f = rng.integers(0, 3, 3)
                u = rng.standard_normal(128)
                u = torch.from_numpy(u / np.linalg.norm(u)).float().to(dev)
                wave = torch.cos(2 * math.pi * (f[0] * tt + f[1] * yy + f[2] * xx) + rng.uniform(0, 6.283))
                acc += 0.5 * wave.reshape(-1, 1) * u
            t[h] = acc.to(torch.bfloat16)
        qk.append(t)
    q, k = qk
    cubes = mh.cube_count(*GRID)
    kk = mh.topk_k(0.1, cubes)
    a = mh.cube_args(HEADS, GRID, k=kk, local=1)
    qc = torch.empty((HEADS, cubes, 128), dtype=torch.float32, device=dev)
    kc = torch.empty_like(qc)
    idx = torch.empty((HEADS, cubes, kk + 1), dtype=torch.int32, device=dev)
    cnt = torch.empty((HEADS, cubes), dtype=torch.int32, device=dev)
    pool_ms, _ = time_launches(lambda: mh.cube_pool(a, q, k, qc=qc, kc=kc), steps, warmup)
    sel_ms, _ = time_launches(lambda: mh.cube_select(a, qc, kc, idx=idx, cnt=cnt), steps, warmup)

    def both():
        mh.cube_pool(a, q, k, qc=qc, kc=kc)
        mh.cube_select(a, qc, kc, idx=idx, cnt=cnt)
    total_ms, _ = time_launches(both, steps, warmup)
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
    return {"pool_ms": pool_ms, "select_ms": sel_ms, "ms": total_ms, "k": kk, "cubes": cubes,
            "pool_GBs": pool_bytes / pool_ms / 1e6, "pool_frac": pool_bytes / pool_ms / 1e6 / HBM_PEAK_GBS,
            "alg_bytes": alg_bytes, "GBs": alg_bytes / total_ms / 1e6,
            "frac": alg_bytes / total_ms / 1e6 / HBM_PEAK_GBS,
            "score_gflop": flops / 1e9, "select_TFLOPs": flops / sel_ms / 1e9,
            "select_fp32_mfma_frac": flops / sel_ms / 1e9 / FP32_MFMA_PEAK_TFLOPS,
            "select_bytes": sel_bytes, "unfused_scores_ms": scores_ms, "unfused_topk_ms": topk_ms}


def bench_fc1(mh, dev, steps, warmup, compare):
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn((ROWS, DIM), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randint(-127, 128, (2 * FFN, DIM), generator=g, device=dev, dtype=torch.int8)
    s = (torch.rand(2 * FFN, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
    out = torch.empty((ROWS, FFN), dtype=torch.bfloat16, device=dev)
    ms, _ = time_launches(lambda: mh.gemm_w8a16_swiglu(x, w, s, out=out), steps, warmup)
    flops = 2.0 * ROWS * DIM * 2 * FFN
    res = {"ms": ms, "tflops": flops / ms / 1e9, "mfma_util": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
           "flops": flops, "shape": [ROWS, DIM, 2 * FFN]}
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
    res["w8a8_fc1_ms"] = ims
    res["w8a8_fc1_tops"] = flops / ims / 1e9
    res["w8a8_fc1_int8_mfma_util"] = flops / ims / 1e9 / INT8_PEAK_TOPS
    del xq, xs
    if compare:
        wb = (w.float() * s[:, None]).to(torch.bfloat16)
        wt = wb.t().contiguous()
        y = torch.empty((ROWS, 2 * FFN), dtype=torch.bfloat16, device=dev)
        cms, _ = time_launches(lambda: torch.matmul(x, wt, out=y), max(3, steps // 2), 2)
        res["bf16_hipblaslt_gemm_ms"] = cms
        res["bf16_hipblaslt_tflops"] = flops / cms / 1e9
        del wt, y, wb
    return res


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
    return {"value": gbs, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"fused modulated RMS norm + gated residual over {n} of the {ROWS} rows x {DIM} bf16 "
                      f"({t:.1f} s), scalar C oracle, one thread on {platform.processor() or platform.machine()}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="fused,block_order,copy,swiglu,select,fc1,rms_f32")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-compare", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's kernels run on a single MI355X and have no multi-GPU path "
              "(see DESIGN.md for how they would shard). Run with --gpus 1.", file=sys.stderr)
        return 2
    import mako_h3 as mh

    dev = torch.device("cuda:0")
    ops = set(args.only.split(","))
    report = {}
    if "fused" in ops:
        report["fused_rms_mod_gate_add"] = bench_fused(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if "block_order" in ops:
        report["gate_add_rms_mod"] = bench_block_order(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if "copy" in ops:
        report["hbm_copy"] = bench_copy(dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if "rms_f32" in ops:
        report["rms_mod_f32_4096x1024"] = bench_rms_f32(mh, dev, args.steps, args.warmup)
    if "swiglu" in ops:
        report["swiglu"] = bench_swiglu(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if "select" in ops:
        report["cube_selector"] = bench_select(mh, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if "fc1" in ops:
        report["fc1_w8a16_swiglu"] = bench_fc1(mh, dev, max(3, args.steps // 2), max(1, args.warmup // 2),
                                               not args.no_compare)
        torch.cuda.empty_cache()

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
    line["ops"] = report
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
