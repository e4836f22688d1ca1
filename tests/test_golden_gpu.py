"""The committed fixtures under tests/golden/ (seeded inputs and the CPU oracle's outputs, written by
tests/golden/make_golden.py) run through the HIP kernels: index, count and int8 outputs bit-exact, bf16 outputs within
1e-2 relative, float outputs within 1e-5."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import mako_h3 as mh
from helpers import assert_close, bits_to_f64, from_bits, to_bits

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = json.loads((GOLDEN / "manifest.json").read_text())["cases"]


def close_rows(got, want, rtol, width):
    """Within rtol of each element plus rtol of its row's RMS (sums that cancel toward zero)."""
    g, w = np.asarray(got, np.float64).reshape(-1, width), np.asarray(want, np.float64).reshape(-1, width)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True))
    assert (np.abs(g - w) <= rtol * (np.abs(w) + scale)).all(), float((np.abs(g - w) / (np.abs(w) + scale)).max())


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_fixture_on_gpu(dev, case):
    d = np.load(GOLDEN / case["file"])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    op = case["op"]
    if op == "rms_mod_rows_f32":
        got = mh.rms_mod_rows(t(d["x"]), t(d["w"]), t(d["shift"]), t(d["scale"]), eps=case["eps"])
        assert_close(got.cpu().numpy(), d["y"], 1e-5, 1e-6, case["name"])
    elif op == "rms_mod_gate_add_rows_bf16":
        got = mh.rms_mod_gate_add_rows(from_bits(d["x"], dev), from_bits(d["residual"], dev), t(d["w"]), t(d["shift"]),
                                       t(d["scale"]), t(d["gate"]), eps=case["eps"], set_of_row=t(d["set_of_row"]),
                                       n_sets=case["n_sets"])
        assert_close(bits_to_f64(to_bits(got)), bits_to_f64(d["out"]), 1e-2, 1e-5, case["name"])
    elif op == "swiglu_rows_bf16_fused":
        got = mh.swiglu_rows(from_bits(d["gu"], dev))
        assert_close(bits_to_f64(to_bits(got)), bits_to_f64(d["out"]), 1e-2, 1e-6, case["name"])
    elif op == "cube_pool":
        a = mh.cube_args(case["heads"], tuple(case["grid"]))
        counts = torch.empty(mh.cube_count(*case["grid"]), dtype=torch.int32, device=dev)
        qc, kc = mh.cube_pool(a, from_bits(d["q"], dev), from_bits(d["k"], dev), counts=counts)
        assert_close(qc.cpu().numpy(), d["qc"], 1e-5, 1e-6, case["name"])
        assert_close(kc.cpu().numpy(), d["kc"], 1e-5, 1e-6, case["name"])
        assert np.array_equal(counts.cpu().numpy(), d["counts"])
    elif op == "cube_topk":
        a = mh.cube_args(case["heads"], tuple(case["grid"]), k=case["k"], local=case["local"],
                         out_stride=d["idx"].shape[-1])
        idx, cnt = mh.cube_topk(a, t(d["scores"]))
        assert np.array_equal(idx.cpu().numpy(), d["idx"]) and np.array_equal(cnt.cpu().numpy(), d["cnt"])
    elif op == "quant_rows_i8":
        q, s = mh.quant_rows_i8(from_bits(d["w"], dev))
        assert np.array_equal(q.cpu().numpy(), d["q"]) and np.array_equal(s.cpu().numpy(), d["s"])
    elif op == "gemm_w8a16_swiglu":
        got = mh.gemm_w8a16_swiglu(from_bits(d["x"], dev), t(d["w"]), t(d["scale"]))
        assert_close(bits_to_f64(to_bits(got)), bits_to_f64(d["out"]), 1e-2, 1e-4, case["name"])
    elif op == "cube_map":
        m, c = mh.cube_map(tuple(case["grid"]), n_dense=case["n_dense"], video_row0=case["video_row0"],
                           dense_row0=case["dense_row0"], device=dev)
        assert np.array_equal(m.cpu().numpy(), d["map"]) and np.array_equal(c.cpu().numpy(), d["counts"])
    elif op == "time_embed":
        temb, cond = mh.time_embed(t(d["t"]), t(d["w_in"]), t(d["b_in"]), t(d["w_out"]), t(d["b_out"]))
        close_rows(temb.cpu().numpy(), d["temb"], 1e-5, case["out_dim"])
        g, w = bits_to_f64(to_bits(cond)), bits_to_f64(d["cond"])
        assert (np.abs(g - w) <= 2.0 ** -7 * np.abs(w) + 1e-5 * np.abs(w).max(1, keepdims=True)).all()
    elif op == "adaln_mod":
        got = mh.adaln_mod(from_bits(d["cond"], dev), from_bits(d["w"], dev), t(d["bias"]))
        close_rows(got.cpu().numpy(), d["mod"], 1e-5, case["n"])
    elif op == "curve_mods":
        got = mh.curve_mods(t(d["t"]), t(d["table"]), t(d["w"]), t(d["bias"]))
        close_rows(got.cpu().numpy(), d["mod"], 1e-5, case["n"])
    else:
        raise AssertionError(f"no GPU check for fixture op {op}")
