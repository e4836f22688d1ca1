"""Parity of swiglu_rows (split and fused-row layouts) with the CPU oracle; bf16 at 1e-2, float at 1e-5."""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, bits_to_f64, check_rows_f64, diff, from_bits, nan_filled, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim", [8, 136, 1000, 13824])
@pytest.mark.parametrize("rows", [1, 5, 130])
@pytest.mark.parametrize("fused", [False, True])
def test_swiglu_bf16(dev, dim, rows, fused):
    rng = np.random.default_rng(dim + rows)
    if fused:
        gu = randn_bf16_bits(rng, (rows, 2 * dim), 2.0)
        want = orc.swiglu_rows(gu)
        got = mh.swiglu_rows(from_bits(gu, dev))
    else:
        g, u = randn_bf16_bits(rng, (rows, dim), 2.0), randn_bf16_bits(rng, (rows, dim), 2.0)
        want = orc.swiglu_rows(g, u)
        got = mh.swiglu_rows(from_bits(g, dev), from_bits(u, dev))
    assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), 1e-2, 1e-6, f"swiglu {rows}x{dim} fused={fused}")


@pytest.mark.parametrize("fused", [False, True])
def test_swiglu_f32(dev, fused):
    rng = np.random.default_rng(7)
    rows, dim = 37, 1028
    if fused:
        gu = (rng.standard_normal((rows, 2 * dim)) * 3).astype(np.float32)
        want = orc.swiglu_rows(gu)
        got = mh.swiglu_rows(torch.from_numpy(gu).to(dev))
    else:
        g = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
        u = rng.standard_normal((rows, dim)).astype(np.float32)
        want = orc.swiglu_rows(g, u)
        got = mh.swiglu_rows(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev))
    assert_close(got.cpu().numpy(), want, 1e-5, 1e-7, "swiglu f32")


def test_swiglu_special_values(dev):
    """silu(0) = 0; silu(g) -> g for large g and -> 0 for very negative g; infinities and NaN follow
    g / (1 + exp(-g)) * u (silu(-inf) is NaN, as torch's silu gives)."""
    gv = np.array([0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0, 100.0, -100.0, np.inf, -np.inf, np.nan, 1.0], np.float32)
    uv = np.array([3.0, 3.0, 1.0, 1.0, 2.0, 2.0, 1.0, 1.0, 1.0, 1.0, 1.0, np.inf], np.float32)
    g = np.tile(gv, (1, 4))
    u = np.tile(uv, (1, 4))
    want = orc.swiglu_rows(g, u)
    got = mh.swiglu_rows(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev)).cpu().numpy()
    assert_close(got, want, 1e-5, 1e-30, "swiglu special values")


@pytest.mark.parametrize("fused", [False, True])
def test_swiglu_768p_every_row(dev, fused):
    """gate and up [129,536 x 13,824] ~ N(0,1) bf16 (separate tensors, or the interleaved [N, 27,648] row), into a
    NaN-filled output: every element against a float64 restatement on the GPU (1e-2 relative), and 256 sampled rows
    (both ends included) against the oracle."""
    rows, dim = 129536, 13824
    gen = torch.Generator(device=dev).manual_seed(1)
    rng = np.random.default_rng(1)
    pick = np.unique(np.concatenate([[0, rows - 1], rng.integers(0, rows, 254)]))
    ti = torch.from_numpy(pick).to(dev)
    out = nan_filled((rows, dim), dev)
    if fused:
        gu = torch.randn((rows, 2 * dim), generator=gen, device=dev).to(torch.bfloat16)
        mh.swiglu_rows(gu, out=out)
        want = orc.swiglu_rows(to_bits(gu[ti]))
        g, u = gu[:, :dim], gu[:, dim:]
    else:
        g = torch.randn((rows, dim), generator=gen, device=dev).to(torch.bfloat16)
        u = torch.randn((rows, dim), generator=gen, device=dev).to(torch.bfloat16)
        mh.swiglu_rows(g, u, out=out)
        want = orc.swiglu_rows(to_bits(g[ti]), to_bits(u[ti]))
    for r0 in range(0, rows, 8192):
        gd, ud = g[r0:r0 + 8192].double(), u[r0:r0 + 8192].double()
        check_rows_f64(out[r0:r0 + 8192], gd * torch.sigmoid(gd) * ud, f"swiglu 768p rows {r0}..", 1e-2, 1e-6)
    got = bits_to_f64(to_bits(out[ti]))
    assert_close(got, bits_to_f64(want), 1e-2, 1e-6, "swiglu 768p")
    rel, cos = diff(got, bits_to_f64(want), dim)
    assert rel < 3e-3 and cos > 0.9999
