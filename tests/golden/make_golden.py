"""Writes the small committed fixtures under tests/golden/: seeded inputs and the CPU oracle's outputs for each
hot-path op, plus manifest.json. The reference holds no vectors for these ops, so these are the build's own, made
by the oracle (which tests/test_oracle*.py pin against library routines, brute force and invariants).
tests/test_golden_gpu.py runs each fixture's inputs through the HIP kernels and compares them with the stored
outputs; tests/test_oracle.py checks the oracle still reproduces them.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
import oracle as orc  # noqa: E402


def _bf16(rng, shape, scale=1.0):
    f = (rng.standard_normal(shape) * scale).astype(np.float64)
    return orc.bf16_from_f64(f)


def _params(rng, dim, n_sets=1):
    return ((1 + rng.standard_normal(dim) * 0.02).astype(np.float32),
            (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32),
            (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32),
            (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32))


def make_inputs(case: dict) -> dict:
    rng = np.random.default_rng(case["seed"])
    op = case["op"]
    if op == "rms_mod_rows_f32":
        rows, dim = case["rows"], case["dim"]
        w, shift, scale, _ = _params(rng, dim)
        return {"x": rng.standard_normal((rows, dim)).astype(np.float32), "w": w, "shift": shift, "scale": scale}
    if op == "rms_mod_gate_add_rows_bf16":
        rows, dim, n_sets = case["rows"], case["dim"], case["n_sets"]
        w, shift, scale, gate = _params(rng, dim, n_sets)
        return {"x": _bf16(rng, (rows, dim)), "residual": _bf16(rng, (rows, dim)), "w": w, "shift": shift,
                "scale": scale, "gate": gate, "set_of_row": rng.integers(0, n_sets, rows).astype(np.uint8)}
    if op == "swiglu_rows_bf16_fused":
        return {"gu": _bf16(rng, (case["rows"], 2 * case["dim"]), 2.0)}
    if op == "cube_pool":
        gt, gh, gw = case["grid"]
        rows = gt * gh * gw
        return {"q": _bf16(rng, (case["heads"], rows, 128)), "k": _bf16(rng, (case["heads"], rows, 128))}
    if op == "cube_topk":
        C = orc.cube_count(*case["grid"])
        return {"scores": rng.integers(-20, 20, (case["heads"], C, C)).astype(np.float32) / 8}
    if op == "quant_rows_i8":
        return {"w": _bf16(rng, (case["rows"], case["cols"]), 0.02)}
    if op == "gemm_w8a16_swiglu":
        m, n, k = case["m"], case["n"], case["k"]
        return {"x": _bf16(rng, (m, k)), "w": rng.integers(-127, 128, (2 * n, k), dtype=np.int8),
                "scale": rng.uniform(0.5e-3, 2e-3, 2 * n).astype(np.float32)}
    if op == "cube_map":
        return {}
    if op == "time_embed":
        f, h, o = case["freq_dim"], case["hidden"], case["out_dim"]
        return {"t": np.array(case["t"], np.float32),
                "w_in": (rng.standard_normal((h, f)) / np.sqrt(f)).astype(np.float32),
                "b_in": (0.1 * rng.standard_normal(h)).astype(np.float32),
                "w_out": (rng.standard_normal((o, h)) / np.sqrt(h)).astype(np.float32),
                "b_out": (0.1 * rng.standard_normal(o)).astype(np.float32)}
    if op == "adaln_mod":
        return {"cond": _bf16(rng, (case["levels"], case["k"])), "w": _bf16(rng, (case["n"], case["k"]), 0.05),
                "bias": (0.1 * rng.standard_normal(case["n"])).astype(np.float32)}
    if op == "curve_mods":
        return {"t": np.array(case["t"], np.float32),
                "table": rng.standard_normal((case["points"], case["width"])).astype(np.float32),
                "w": rng.standard_normal((case["n"], case["width"])).astype(np.float32),
                "bias": rng.standard_normal(case["n"]).astype(np.float32)}
    raise ValueError(op)


def run_case(case: dict, data) -> dict:
    """The oracle's outputs for a case's inputs."""
    op = case["op"]
    if op == "rms_mod_rows_f32":
        return {"y": orc.rms_mod_rows(data["x"], data["w"], data["shift"], data["scale"], case["eps"])}
    if op == "rms_mod_gate_add_rows_bf16":
        return {"out": orc.rms_mod_gate_add_rows(data["x"], data["residual"], data["w"], data["shift"],
                                                 data["scale"], data["gate"], case["eps"], data["set_of_row"])}
    if op == "swiglu_rows_bf16_fused":
        return {"out": orc.swiglu_rows(data["gu"])}
    if op == "cube_pool":
        qc, kc, counts = orc.cube_pool(data["q"], data["k"], case["heads"], tuple(case["grid"]))
        return {"qc": qc, "kc": kc, "counts": counts}
    if op == "cube_topk":
        idx, cnt = orc.cube_topk(data["scores"].astype(np.float64), tuple(case["grid"]), case["k"], case["local"])
        return {"idx": idx, "cnt": cnt}
    if op == "quant_rows_i8":
        q, s = orc.quant_rows_i8(data["w"])
        return {"q": q, "s": s}
    if op == "gemm_w8a16_swiglu":
        return {"out": orc.gemm_w8a16_swiglu(data["x"], data["w"], data["scale"])}
    if op == "cube_map":
        m, c = orc.cube_map(tuple(case["grid"]), case["n_dense"], case["video_row0"], case["dense_row0"])
        return {"map": m, "counts": c}
    if op == "time_embed":
        temb, cond = orc.time_embed(data["t"], data["w_in"], data["b_in"], data["w_out"], data["b_out"])
        return {"temb": temb, "cond": cond}
    if op == "adaln_mod":
        return {"mod": orc.adaln_mod(data["cond"], data["w"], data["bias"])}
    if op == "curve_mods":
        return {"mod": orc.curve_mods(data["t"], data["table"], data["w"], data["bias"])}
    raise ValueError(op)


CASES = [
    {"name": "rms_mod_f32", "op": "rms_mod_rows_f32", "seed": 100, "rows": 16, "dim": 1024, "eps": 1e-6},
    {"name": "fused_bf16_sets", "op": "rms_mod_gate_add_rows_bf16", "seed": 101, "rows": 12, "dim": 5376,
     "n_sets": 3, "eps": 1e-6},
    {"name": "swiglu_fused", "op": "swiglu_rows_bf16_fused", "seed": 102, "rows": 6, "dim": 1152},
    {"name": "cube_pool_padded", "op": "cube_pool", "seed": 103, "heads": 2, "grid": [5, 6, 9]},
    {"name": "cube_topk_ties", "op": "cube_topk", "seed": 104, "heads": 2, "grid": [12, 8, 8], "k": 5, "local": 3},
    {"name": "quant_rows", "op": "quant_rows_i8", "seed": 105, "rows": 8, "cols": 512},
    {"name": "fc1_small", "op": "gemm_w8a16_swiglu", "seed": 106, "m": 5, "n": 128, "k": 256},
    {"name": "cube_map_padded", "op": "cube_map", "seed": 107, "grid": [5, 6, 9], "n_dense": 7, "video_row0": 7,
     "dense_row0": 0},
    {"name": "time_embed_small", "op": "time_embed", "seed": 108, "t": [0.0, 0.4, 0.9230769], "freq_dim": 256,
     "hidden": 96, "out_dim": 40},
    {"name": "adaln_mod_small", "op": "adaln_mod", "seed": 109, "levels": 3, "n": 54, "k": 264},
    {"name": "curve_mods_small", "op": "curve_mods", "seed": 110, "t": [0.0, 0.0769230769, 0.5, 1.0], "points": 1025,
     "width": 8, "n": 36},
]


def main() -> None:
    manifest = {"about": "inputs and CPU-oracle outputs of the H3 hot-path ops, written by make_golden.py",
                "cases": []}
    for case in CASES:
        data = make_inputs(case)
        data.update(run_case(case, data))
        f = f"{case['name']}.npz"
        np.savez_compressed(HERE / f, **data)
        manifest["cases"].append({**case, "file": f})
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(f"wrote {len(CASES)} fixtures")


if __name__ == "__main__":
    main()
