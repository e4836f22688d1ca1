"""Parity of gate_add_rms_mod_rows (the block's own order: x += gate * y, then h = modulated RMS norm of the new x).

- Against the two kernels it replaces, gate_add_rows then rms_mod_rows on the updated x: bit for bit, for x and h,
  at every width, dtype and modulation-set arrangement (both paths reduce in the same order).
- Against the CPU oracle: the updated x against its gate_add_rows, and h against its rms_mod_rows of the x the kernel
  stored; bf16 within 1e-2 relative (both round once at each output), float within 1e-5.
"""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, bits_to_f64, from_bits, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def inputs(rng, dev, rows, dim, dtype, n_sets):
    if dtype == "bf16":
        x, y = randn_bf16_bits(rng, (rows, dim)), randn_bf16_bits(rng, (rows, dim))
        tx, ty = from_bits(x, dev), from_bits(y, dev)
    else:
        x = rng.standard_normal((rows, dim)).astype(np.float32)
        y = rng.standard_normal((rows, dim)).astype(np.float32)
        tx, ty = dev_t(x, dev), dev_t(y, dev)
    gate = (rng.standard_normal((n_sets, dim)) * 0.5).astype(np.float32)
    shift = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    scale = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    w = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    sets = rng.integers(0, n_sets, rows).astype(np.uint8) if n_sets > 1 else None
    return x, y, tx, ty, gate, shift, scale, w, sets


def bits(t):
    return t.view(torch.int16).cpu().numpy() if t.dtype == torch.bfloat16 else t.view(torch.int32).cpu().numpy()


# dim 5120 with 9 sets and f32 at 5120 (1280 vectors a row) take the workgroup-per-row kernel; the rest one wave a row.
# bf16 (23, 6144, 1) and (21, 4096, 2): the wave kernel whose three-plane coefficient table (gate too) exceeds 64 KiB
# while rms_mod's two planes fit, so the block order reads its coefficients from the parameter vectors while
# rms_mod_rows reads them from LDS; the results must still agree bit for bit.
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,dim,n_sets", [(1, 8, 1), (67, 520, 1), (33, 5120, 1), (20, 5376, 1), (45, 5376, 3),
                                             (19, 5120, 9), (23, 6144, 1), (21, 4096, 2)])
def test_equals_gate_add_then_rms_mod(dev, dtype, rows, dim, n_sets):
    rng = np.random.default_rng(rows * 7 + dim + n_sets)
    x, y, tx, ty, gate, shift, scale, w, sets = inputs(rng, dev, rows, dim, dtype, n_sets)
    g, sh, sc, tw = dev_t(gate, dev), dev_t(shift, dev), dev_t(scale, dev), dev_t(w, dev)
    ts = dev_t(sets, dev) if sets is not None else None
    x2 = tx.clone()
    h = mh.gate_add_rms_mod_rows(tx, ty, g, tw, sh, sc, set_of_row=ts, n_sets=n_sets)
    mh.gate_add_rows(x2, ty, g, set_of_row=ts, n_sets=n_sets)
    h2 = mh.rms_mod_rows(x2, tw, sh, sc, set_of_row=ts, n_sets=n_sets)
    assert (bits(tx) == bits(x2)).all(), "updated x differs from gate_add_rows"
    assert (bits(h) == bits(h2)).all(), "h differs from rms_mod_rows of the updated x"

    # h is checked against the oracle's norm of the x the kernel stored: the two x values may differ by one ulp
    # (each rounds once), which the norm can magnify where the shift cancels the normed term.
    want_x = orc.gate_add_rows(x, y, gate, sets)
    got_x = to_bits(tx) if dtype == "bf16" else tx.cpu().numpy()
    want_h = orc.rms_mod_rows(got_x, w, shift, scale, 1e-6, sets)
    if dtype == "bf16":
        assert_close(bits_to_f64(to_bits(tx)), bits_to_f64(want_x), 1e-2, 1e-5, "x bf16")
        assert_close(bits_to_f64(to_bits(h)), bits_to_f64(want_h), 1e-2, 1e-5, "h bf16")
    else:
        assert_close(tx.cpu().numpy(), want_x, 1e-5, 1e-6, "x f32")
        assert_close(h.cpu().numpy(), want_h, 1e-5, 1e-6, "h f32")


def test_gate_zero_leaves_x_and_gives_rms_mod_of_x(dev):
    rng = np.random.default_rng(5)
    x, _, tx, ty, gate, shift, scale, w, _ = inputs(rng, dev, 12, 5120, "bf16", 1)
    x0 = tx.clone()
    h = mh.gate_add_rms_mod_rows(tx, ty, torch.zeros(1, 5120, device=dev), dev_t(w, dev), dev_t(shift, dev),
                                 dev_t(scale, dev))
    assert (bits(tx) == bits(x0)).all()
    assert (bits(h) == bits(mh.rms_mod_rows(x0, dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev)))).all()


def test_h_aliasing_x_is_rejected(dev):
    rng = np.random.default_rng(6)
    _, _, tx, ty, gate, shift, scale, w, _ = inputs(rng, dev, 4, 64, "bf16", 1)
    with pytest.raises(RuntimeError):
        mh.gate_add_rms_mod_rows(tx, ty, dev_t(gate, dev), dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev), h=tx)


def test_768p_rows_equal_two_kernel_sequence(dev):
    """129,536 x 5120 bf16: the fused pass equals the two-kernel sequence bit for bit on every row."""
    rows, dim = 32 * 48 * 84 + 512, 5120
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((rows, dim), generator=gen, device=dev).to(torch.bfloat16)
    y = torch.randn((rows, dim), generator=gen, device=dev).to(torch.bfloat16)
    gate, shift, scale = [0.1 * torch.randn((1, dim), generator=gen, device=dev) for _ in range(3)]
    w = 1 + 0.02 * torch.randn(dim, generator=gen, device=dev)
    x2 = x.clone()
    h = mh.gate_add_rms_mod_rows(x, y, gate, w, shift, scale)
    mh.gate_add_rows(x2, y, gate)
    h2 = mh.rms_mod_rows(x2, w, shift, scale)
    assert torch.equal(x.view(torch.int16), x2.view(torch.int16))
    assert torch.equal(h.view(torch.int16), h2.view(torch.int16))
    assert torch.isfinite(h.float()).all()
