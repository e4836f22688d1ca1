"""Pins the oracle's qkv / out / fc2 projections (CPU): y = x w^T against torch.matmul in float64 for each operand
form (non-square shapes, so a transposed operand fails), exact integer results, and the gate-add epilogue against
gate_add_rows of the rounded product (they differ by at most the one extra rounding) with gate 0 leaving the
residual bit-exact."""
import numpy as np
import torch

import oracle as orc
from helpers import bits_to_f64, randn_bf16_bits


def torch_y(x, w, form, x_scale=None, w_scale=None):
    xf = torch.from_numpy(x.astype(np.float64) if form == orc.GEMM_W8A8 else bits_to_f64(x))
    wf = torch.from_numpy(w.astype(np.float64) if form != orc.GEMM_BF16 else bits_to_f64(w))
    y = xf @ wf.T
    if form != orc.GEMM_BF16:
        y = y * torch.from_numpy(w_scale.astype(np.float64))[None, :]
    if form == orc.GEMM_W8A8:
        y = y * torch.from_numpy(x_scale.astype(np.float64))[:, None]
    return y.numpy()


def operands(rng, form, m, n, k):
    if form == orc.GEMM_W8A8:
        x = rng.integers(-127, 128, (m, k), dtype=np.int8)
        xs = rng.uniform(0.5e-2, 2e-2, m).astype(np.float32)
    else:
        x, xs = randn_bf16_bits(rng, (m, k)), None
    if form == orc.GEMM_BF16:
        w, ws = randn_bf16_bits(rng, (n, k), 0.05), None
    else:
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ws = rng.uniform(0.5e-3, 2e-3, n).astype(np.float32)
    return x, xs, w, ws


def test_gemm_matches_torch_matmul_every_form():
    rng = np.random.default_rng(0)
    m, n, k = 9, 40, 72
    for form in (orc.GEMM_W8A16, orc.GEMM_BF16, orc.GEMM_W8A8):
        x, xs, w, ws = operands(rng, form, m, n, k)
        got = orc.gemm(x, w, form, xs, ws)
        want = orc.bf16_from_f64(torch_y(x, w, form, xs, ws))
        assert (got == want).mean() > 0.995, form
        assert np.allclose(bits_to_f64(got), bits_to_f64(want), rtol=2 ** -7, atol=1e-30), form


def test_gemm_exact_integers():
    rng = np.random.default_rng(1)
    m, n, k = 5, 24, 64
    xi = rng.integers(-3, 4, (m, k))
    wi = rng.integers(-1, 2, (n, k))
    want = (xi @ wi.T).astype(np.float64)                      # |y| <= 192: exact in bf16 only below 256
    x_bf = orc.bf16_from_f64(xi.astype(np.float64))
    for form, x, w, xs, ws in ((orc.GEMM_BF16, x_bf, orc.bf16_from_f64(wi.astype(np.float64)), None, None),
                               (orc.GEMM_W8A16, x_bf, wi.astype(np.int8), None, np.ones(n, np.float32)),
                               (orc.GEMM_W8A8, xi.astype(np.int8), wi.astype(np.int8), np.ones(m, np.float32),
                                np.ones(n, np.float32))):
        got = bits_to_f64(orc.gemm(x, w, form, xs, ws))
        assert np.array_equal(got, bits_to_f64(orc.bf16_from_f64(want))), form


def test_gemm_gate_add_epilogue():
    rng = np.random.default_rng(2)
    m, n, k = 11, 32, 48
    x, xs, w, ws = operands(rng, orc.GEMM_W8A16, m, n, k)
    res = randn_bf16_bits(rng, (m, n))
    gate = (0.1 * rng.standard_normal((3, n))).astype(np.float32)
    sets = rng.integers(0, 3, m).astype(np.uint8)
    got = orc.gemm_gate_add(x, w, orc.GEMM_W8A16, res, gate, None, ws, sets)
    y = torch_y(x, w, orc.GEMM_W8A16, None, ws)
    want = orc.bf16_from_f64(bits_to_f64(res) + gate[sets].astype(np.float64) * y)
    assert (got == want).mean() > 0.995
    # Against gate_add_rows of the bf16-rounded product: apart by at most the product's extra rounding (half an ulp of
    # y, times the gate) and the two final roundings.
    two_step = orc.gate_add_rows(res, orc.gemm(x, w, orc.GEMM_W8A16, None, ws), gate, set_of_row=sets)
    g, t = bits_to_f64(got), bits_to_f64(two_step)
    gy = np.abs(gate[sets].astype(np.float64) * y)
    assert np.all(np.abs(g - t) <= 2 ** -8 * (np.abs(t) + np.abs(g) + gy) + 1e-30)
    zero = orc.gemm_gate_add(x, w, orc.GEMM_W8A16, res, np.zeros(n, np.float32), None, ws)
    assert np.array_equal(zero, res)


def test_gemm_gate_add_float_residual():
    """The gate-add epilogue on a float residual (the reference's float residual stream): the float64 product added
    to the residual, rounded once to float; gate 0 leaves the residual bit-exact."""
    rng = np.random.default_rng(3)
    m, n, k = 7, 40, 64
    for form in (orc.GEMM_W8A16, orc.GEMM_BF16, orc.GEMM_W8A8):
        x, xs, w, ws = operands(rng, form, m, n, k)
        res = rng.standard_normal((m, n)).astype(np.float32)
        gate = (0.1 * rng.standard_normal((2, n))).astype(np.float32)
        sets = rng.integers(0, 2, m).astype(np.uint8)
        got = orc.gemm_gate_add(x, w, form, res, gate, xs, ws, sets)
        assert got.dtype == np.float32
        want = res.astype(np.float64) + gate[sets].astype(np.float64) * torch_y(x, w, form, xs, ws)
        assert np.all(np.abs(got - want) <= 2 ** -24 * np.abs(want) + 1e-12), form
        assert (orc.gemm_gate_add(x, w, form, res, np.zeros(n, np.float32), xs, ws) == res).all(), form
