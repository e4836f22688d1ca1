"""Parity of the reference's float residual stream through the fused entry points (docs/architecture.md:69-70:
activations are fp32 and go into the bf16 GEMMs rounded to bf16).

- rms_mod_rows from a float x to the bf16 row the next GEMM takes, rounded once: against the oracle, 1e-2 relative
  plus 1e-5 of the row's RMS (one bf16 rounding on each side of float math).
- gate_add_rows of a bf16 y (a GEMM's output) into a float x: against the oracle within 1e-6 (one float rounding).
- gate_add_rms_mod_rows under the same flags: bit for bit the two kernels it replaces.
- the GEMM gate-add epilogue on a float residual, every form: against the oracle (float, 1e-5 relative plus 1e-5 of
  the row's RMS for the float32 accumulation), and at the 768p out-projection shape every element against float64 on
  the GPU.
- with LDS coefficient tables and, for several sets past 64 KiB of table, coefficients from the parameter vectors.
"""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, bits_to_f64, check_gemm_full, from_bits, nan_filled, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu


def t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def params(rng, dim, n_sets):
    w = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    shift = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    scale = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    gate = (rng.standard_normal((n_sets, dim)) * 0.5).astype(np.float32)
    return w, shift, scale, gate


def check_bf16(got_bits, want_bits, dim, what):
    g, w = bits_to_f64(got_bits).reshape(-1, dim), bits_to_f64(want_bits).reshape(-1, dim)
    rms = np.sqrt((w ** 2).mean(1, keepdims=True))
    err = np.abs(g - w)
    assert np.all(err <= 1e-2 * np.abs(w) + 1e-5 * rms), f"{what}: worst {(err / (np.abs(w) + rms)).max():.3g}"


# (dim 5120, 3 sets) and (6144, 2 sets): two-plane tables over 64 KiB, coefficients from the parameter vectors.
SHAPES = [(1, 8, 1), (67, 520, 1), (300, 5120, 1), (40, 5376, 1), (45, 5376, 3), (33, 5120, 3), (21, 6144, 2)]


@pytest.mark.parametrize("rows,dim,n_sets", SHAPES)
def test_rms_mod_rows_float_to_bf16(dev, rows, dim, n_sets):
    rng = np.random.default_rng(rows + dim + n_sets)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    w, shift, scale, _ = params(rng, dim, n_sets)
    sets = rng.integers(0, n_sets, rows).astype(np.uint8) if n_sets > 1 else None
    ts = t(sets, dev) if sets is not None else None
    h = mh.rms_mod_rows(t(x, dev), t(w, dev), t(shift, dev), t(scale, dev), set_of_row=ts, n_sets=n_sets,
                        out_dtype=torch.bfloat16)
    assert h.dtype == torch.bfloat16
    want = orc.rms_mod_rows(x, w, shift, scale, 1e-6, sets, out_dtype=np.uint16)
    check_bf16(to_bits(h), want, dim, f"rms_mod_rows f32 -> bf16 {rows}x{dim} sets {n_sets}")


@pytest.mark.parametrize("rows,dim,n_sets", SHAPES)
def test_gate_add_rows_bf16_y_into_float_x(dev, rows, dim, n_sets):
    rng = np.random.default_rng(rows * 3 + dim + n_sets)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    y = randn_bf16_bits(rng, (rows, dim))
    _, _, _, gate = params(rng, dim, n_sets)
    sets = rng.integers(0, n_sets, rows).astype(np.uint8) if n_sets > 1 else None
    tx = t(x, dev)
    mh.gate_add_rows(tx, from_bits(y, dev), t(gate, dev), set_of_row=t(sets, dev) if sets is not None else None,
                     n_sets=n_sets)
    want = orc.gate_add_rows(x, y, gate, sets)
    assert_close(tx.cpu().numpy(), want, 1e-6, 1e-30, f"gate_add_rows bf16 y {rows}x{dim}")


@pytest.mark.parametrize("y_bf16", [True, False])
@pytest.mark.parametrize("rows,dim,n_sets", SHAPES)
def test_block_order_equals_its_two_kernels(dev, rows, dim, n_sets, y_bf16):
    """x (float) += gate y, h = the bf16 modulated norm of the new x: bit for bit gate_add_rows then rms_mod_rows with
    the same flags, and against the oracle's chain."""
    rng = np.random.default_rng(rows * 5 + dim + n_sets + y_bf16)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    y = randn_bf16_bits(rng, (rows, dim)) if y_bf16 else rng.standard_normal((rows, dim)).astype(np.float32)
    w, shift, scale, gate = params(rng, dim, n_sets)
    sets = rng.integers(0, n_sets, rows).astype(np.uint8) if n_sets > 1 else None
    ts = t(sets, dev) if sets is not None else None
    ty = from_bits(y, dev) if y_bf16 else t(y, dev)
    g, tw, sh, sc = t(gate, dev), t(w, dev), t(shift, dev), t(scale, dev)
    x1, x2 = t(x, dev), t(x, dev)
    h = mh.gate_add_rms_mod_rows(x1, ty, g, tw, sh, sc, set_of_row=ts, n_sets=n_sets, h_dtype=torch.bfloat16)
    mh.gate_add_rows(x2, ty, g, set_of_row=ts, n_sets=n_sets)
    h2 = mh.rms_mod_rows(x2, tw, sh, sc, set_of_row=ts, n_sets=n_sets, out_dtype=torch.bfloat16)
    assert torch.equal(x1.view(torch.int32), x2.view(torch.int32)), "updated x differs from gate_add_rows"
    assert torch.equal(h.view(torch.int16), h2.view(torch.int16)), "h differs from rms_mod_rows of the updated x"
    ox = orc.gate_add_rows(x, y, gate, sets)
    assert_close(x1.cpu().numpy(), ox, 1e-6, 1e-30, "updated x against the oracle")
    oh = orc.rms_mod_rows(x1.cpu().numpy(), w, shift, scale, 1e-6, sets, out_dtype=np.uint16)
    check_bf16(to_bits(h), oh, dim, "h against the oracle's norm of the stored x")


def test_flags_refused_where_not_taken(dev):
    """A bf16 x with a flag, a bf16 y alone on the block order, a flag on the fused op, and an output over the float
    x (the rows no longer line up) are refused before any launch."""
    x = torch.zeros((4, 512), dtype=torch.float32, device=dev)
    xb = torch.zeros((4, 512), dtype=torch.bfloat16, device=dev)
    v = torch.zeros(512, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError):
        mh.rms_mod_rows(xb, v, v, v, out_dtype=torch.float32)
    with pytest.raises(RuntimeError):
        mh.gate_add_rms_mod_rows(x, xb, v, v, v, v)          # bf16 y with a float h
    over_x = x.view(-1).view(torch.bfloat16)[:2048].view(4, 512)  # a bf16 output on the float x's first rows
    with pytest.raises(RuntimeError):
        mh.rms_mod_rows(x, v, v, v, out=over_x)


@pytest.mark.parametrize("form", [mh.GEMM_W8A16, mh.GEMM_BF16, mh.GEMM_W8A8])
def test_gemm_gate_add_float_residual(dev, form):
    rng = np.random.default_rng(50 + form)
    m, n, k = 300, 512, 640
    if form == mh.GEMM_W8A8:
        xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
        xs = rng.uniform(0.5e-2, 2e-2, m).astype(np.float32)
        x, tx, txs = xq, t(xq, dev), t(xs, dev)
    else:
        x, xs = randn_bf16_bits(rng, (m, k)), None
        tx, txs = from_bits(x, dev), None
    if form == mh.GEMM_BF16:
        w, ws = randn_bf16_bits(rng, (n, k), 0.05), None
        tw, tws = from_bits(w, dev), None
    else:
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ws = rng.uniform(0.5e-3, 2e-3, n).astype(np.float32)
        tw, tws = t(w, dev), t(ws, dev)
    res = rng.standard_normal((m, n)).astype(np.float32)
    gate = (0.1 * rng.standard_normal((2, n))).astype(np.float32)
    sets = rng.integers(0, 2, m).astype(np.uint8)
    tr = t(res, dev)
    mh.gemm_gate_add(tx, tw, tr, t(gate, dev), x_scale=txs, w_scale=tws, set_of_row=t(sets, dev), n_sets=2)
    want = orc.gemm_gate_add(x, w, form, res, gate, xs, ws, sets)
    g = tr.cpu().numpy().astype(np.float64)
    rms = np.sqrt((want.astype(np.float64) ** 2).mean(1, keepdims=True))
    err = np.abs(g - want)
    assert np.all(err <= 1e-5 * np.abs(want) + 1e-5 * rms), f"form {form}: worst {(err / rms).max():.3g} of rms"


def test_gemm_gate_add_float_residual_768p_every_element(dev):
    """The out projection at 768p on the float stream: [129,536][5120] float residual += gate * (x W^T), W8A16, every
    element against float64 products on the GPU (1e-5 relative plus 1e-5 of the row's RMS)."""
    g = torch.Generator(device=dev).manual_seed(61)
    m, n, k = 129536, 5120, 5120
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
    ws = (torch.rand(n, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
    res = torch.randn((m, n), generator=g, device=dev)
    gate = (0.1 * torch.randn((3, n), generator=g, device=dev)).float()
    sets = torch.randint(0, 3, (m,), generator=g, device=dev).to(torch.uint8)
    res0 = res.clone()
    mh.gemm_gate_add(x, w, res, gate, w_scale=ws, set_of_row=sets, n_sets=3)
    torch.cuda.synchronize()
    rel, cos = check_gemm_full(res, x, w, "out projection, float residual", w_scale=ws, epi="gate_add",
                               residual0=res0, gate=gate, set_of_row=sets, rtol=1e-5, row_frac=1e-5)
    assert rel < 1e-6 and cos > 0.999999, (rel, cos)
