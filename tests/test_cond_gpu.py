"""The modulation table's producer and the cube map on the GPU, against the oracle.

- mh3_cube_map: bit-exact at the 768p-shaped grid, H3's padded 37 x 24 x 42 grid and small padded grids, with the
  dense rows before or after the video rows.
- mh3_time_embed: the F32 time MLP at H3's shapes (256 -> 5376 -> 2688) for one to three levels and five (two level
  groups), float temb within 1e-5 of the oracle's float64 (relative to the level's largest value) and the reference's
  own bar (tests/h3_ref_test.cpp:228: relative RMS error 1e-4); cond = bf16(silu(temb)) within one bf16 rounding.
- mh3_adaln_mod: block 0's AdaLN projection at H3's shape (2688 -> 96,768, bf16 weights, 1 to 3 levels) and at every
  register shape the kernel has (k from 8 to 4096, n not a multiple of 4), within 1e-5 of the row scale; the
  reference's bar for the table is 5e-3 (tests/h3_ref_test.cpp:241).
- mh3_curve_mods: the pruned checkpoints' [1025][8] curve against the oracle.
- The chain: time_embed -> adaln_mod -> the fused row op reading its (level, tag) sets out of the [U][3][6][D] table
  through set_stride = 6 D, per row, against the oracle fed the same table.
"""
import math

import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, bits_to_f64, diff, from_bits, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("grid,n_dense,video_row0,dense_row0", [
    ((32, 48, 84), 512, 512, 0), ((37, 24, 42), 640, 640, 0), ((37, 24, 42), 512, 0, 37 * 24 * 42),
    ((5, 6, 9), 0, 0, 0), ((1, 1, 1), 3, 10, 0), ((7, 9, 10), 70, 70, 0)])
def test_cube_map_bit_exact(dev, grid, n_dense, video_row0, dense_row0):
    m, c = mh.cube_map(grid, n_dense=n_dense, video_row0=video_row0, dense_row0=dense_row0, device=dev)
    wm, wc = orc.cube_map(grid, n_dense, video_row0, dense_row0)
    assert np.array_equal(m.cpu().numpy(), wm)
    assert np.array_equal(c.cpu().numpy(), wc)


def mlp(dev, freq_dim, hidden, out_dim, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    w_in = torch.randn((hidden, freq_dim), generator=g, device=dev) / math.sqrt(freq_dim)
    b_in = 0.1 * torch.randn(hidden, generator=g, device=dev)
    w_out = torch.randn((out_dim, hidden), generator=g, device=dev) / math.sqrt(hidden)
    b_out = 0.1 * torch.randn(out_dim, generator=g, device=dev)
    return w_in, b_in, w_out, b_out


def check_temb(temb, cond, want_temb, want_cond):
    got = temb.cpu().numpy().astype(np.float64)
    want = want_temb.astype(np.float64)
    for u in range(got.shape[0]):
        scale = np.abs(want[u]).max()
        assert np.abs(got[u] - want[u]).max() <= 1e-5 * scale, f"level {u}"
    rel, cos = diff(got, want, want.shape[1])
    assert rel < 1e-4 and cos > 0.999999, (rel, cos)
    g, w = bits_to_f64(to_bits(cond)), bits_to_f64(want_cond)
    # one bf16 rounding each of silu(temb), from temb values 1e-5 of the level's scale apart: the two may round to
    # neighbouring bf16 values (one step, up to 2^-7 of the value), plus that 1e-5 where silu(temb) is near zero
    assert (np.abs(g - w) <= 2.0 ** -7 * np.abs(w) + 1e-5 * np.abs(w).max(1, keepdims=True)).all()


@pytest.mark.parametrize("t", [[0.9230769], [0.5, 0.999], [0.0, 0.25, 1.0], [0.1, 0.3, 0.5, 0.7, 0.9]])
def test_time_embed_h3(dev, t):
    w_in, b_in, w_out, b_out = mlp(dev, 256, 5376, 2688, 1)
    tt = torch.tensor(t, dtype=torch.float32, device=dev)
    temb, cond = mh.time_embed(tt, w_in, b_in, w_out, b_out)
    wt, wc = orc.time_embed(np.array(t, np.float32), w_in.cpu().numpy(), b_in.cpu().numpy(), w_out.cpu().numpy(),
                            b_out.cpu().numpy())
    check_temb(temb, cond, wt, wc)


@pytest.mark.parametrize("freq_dim,hidden,out_dim", [(64, 32, 8), (1024, 8192, 100), (8, 4, 1)])
def test_time_embed_shapes(dev, freq_dim, hidden, out_dim):
    """The embedding's width from 8 to 1024 (up to four pieces a lane), the widest hidden layer, no biases."""
    w_in, _, w_out, _ = mlp(dev, freq_dim, hidden, out_dim, 2)
    t = np.array([0.3, 0.75], np.float32)
    temb, cond = mh.time_embed(torch.from_numpy(t).to(dev), w_in, None, w_out, None)
    wt, wc = orc.time_embed(t, w_in.cpu().numpy(), None, w_out.cpu().numpy(), None)
    check_temb(temb, cond, wt, wc)


def test_time_embed_workspace_is_reused(dev):
    """A caller's workspace serves calls of different level counts; the second call's results do not depend on what
    the first left in it."""
    w_in, b_in, w_out, b_out = mlp(dev, 256, 5376, 2688, 3)
    ws = torch.empty(mh.time_embed_workspace_bytes(3, 256, 5376, 2688), dtype=torch.uint8, device=dev)
    t3 = torch.tensor([0.2, 0.4, 0.6], device=dev)
    a3, _ = mh.time_embed(t3, w_in, b_in, w_out, b_out, workspace=ws)
    a1, c1 = mh.time_embed(t3[2:], w_in, b_in, w_out, b_out, workspace=ws)
    fresh, _ = mh.time_embed(t3[2:], w_in, b_in, w_out, b_out)
    assert torch.equal(a1, fresh) and torch.equal(a1[0], a3[2])


def check_mod(got, want):
    g, w = got.cpu().numpy().astype(np.float64), want.astype(np.float64)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True)) + 1e-30
    assert (np.abs(g - w) <= 1e-5 * scale).all(), float((np.abs(g - w) / scale).max())
    rel, _ = diff(g, w, w.shape[1])
    assert rel < 1e-5


@pytest.mark.parametrize("levels", [1, 2, 3])
def test_adaln_mod_h3_block(dev, levels):
    """Block 0's AdaLN projection at H3's shape: cond [levels][2688] -> the [levels][3][6][5376] table."""
    g = torch.Generator(device=dev).manual_seed(40 + levels)
    k, n = 2688, 3 * 6 * 5376
    cond = torch.randn((levels, k), generator=g, device=dev).to(torch.bfloat16)
    w = (0.02 * torch.randn((n, k), generator=g, device=dev)).to(torch.bfloat16)
    bias = 0.1 * torch.randn(n, generator=g, device=dev)
    got = mh.adaln_mod(cond, w, bias)
    want = orc.adaln_mod(to_bits(cond), to_bits(w), bias.cpu().numpy())
    assert torch.isfinite(got).all()
    check_mod(got, want)


@pytest.mark.parametrize("levels,n,k", [(1, 37, 8), (3, 64, 520), (2, 100, 1024), (4, 41, 2560), (5, 29, 3072),
                                        (3, 33, 3584), (2, 18, 4096), (7, 5, 2688)])
def test_adaln_mod_shapes(dev, levels, n, k):
    """Every piece count a lane holds (1 to 8), the two-rows-a-wave form (k > 3072), row counts that leave a partial
    group, and more than four levels (two level groups)."""
    rng = np.random.default_rng(levels * 1000 + n + k)
    cond = randn_bf16_bits(rng, (levels, k))
    w = randn_bf16_bits(rng, (n, k), 0.05)
    bias = rng.standard_normal(n).astype(np.float32)
    got = mh.adaln_mod(from_bits(cond, dev), from_bits(w, dev), torch.from_numpy(bias).to(dev))
    check_mod(got, orc.adaln_mod(cond, w, bias))
    nob = mh.adaln_mod(from_bits(cond, dev), from_bits(w, dev))
    check_mod(nob, orc.adaln_mod(cond, w))


def test_curve_mods(dev):
    rng = np.random.default_rng(9)
    table = rng.standard_normal((1025, 8)).astype(np.float32)
    w = rng.standard_normal((96768, 8)).astype(np.float32)
    bias = rng.standard_normal(96768).astype(np.float32)
    t = np.array([0.0, 0.0769230769, 0.9230769, 1.0, 1.5], np.float32)
    got = mh.curve_mods(torch.from_numpy(t).to(dev), torch.from_numpy(table).to(dev), torch.from_numpy(w).to(dev),
                        torch.from_numpy(bias).to(dev))
    check_mod(got, orc.curve_mods(t, table, w, bias))


def test_modulation_chain_feeds_the_row_kernels(dev):
    """Three levels through the time MLP and block 0's projection (D = 5120: 2560 -> 92,160), then the fused row op
    with each row's (level, tag) set read from the [U][3][6][D] table through set_stride = 6 D (vectors 0, 1, 2:
    shift, scale, gate), against the oracle's row op fed the same table."""
    D, levels = 5120, 3
    w_in, b_in, w_out, b_out = mlp(dev, 256, D, D // 2, 5)
    g = torch.Generator(device=dev).manual_seed(6)
    w_ada = (0.02 * torch.randn((18 * D, D // 2), generator=g, device=dev)).to(torch.bfloat16)
    b_ada = 0.01 * torch.randn(18 * D, generator=g, device=dev)
    t = torch.tensor([0.9230769, 0.5, 0.999], device=dev)
    temb, cond = mh.time_embed(t, w_in, b_in, w_out, b_out)
    table = mh.adaln_mod(cond, w_ada, b_ada).view(levels, 3, 6, D)
    want_tab = orc.adaln_mod(to_bits(cond), to_bits(w_ada), b_ada.cpu().numpy()).reshape(levels, 3, 6, D)
    check_mod(table.view(levels * 18, D), want_tab.reshape(levels * 18, D))
    rows = 384
    rng = np.random.default_rng(7)
    x, res = randn_bf16_bits(rng, (rows, D)), randn_bf16_bits(rng, (rows, D))
    level, tag = rng.integers(0, levels, rows), rng.integers(0, 3, rows)
    sets = (level * 3 + tag).astype(np.uint8)
    nw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    shift, scale, gate = table[:, :, 0, :], table[:, :, 1, :], table[:, :, 2, :]
    got = mh.rms_mod_gate_add_rows(from_bits(x, dev), from_bits(res, dev), torch.from_numpy(nw).to(dev), shift, scale,
                                   gate, set_of_row=torch.from_numpy(sets).to(dev), n_sets=levels * 3)
    tab = table.cpu().numpy().reshape(levels * 3, 6, D)
    want = orc.rms_mod_gate_add_rows(x, res, nw, np.ascontiguousarray(tab[:, 0]), np.ascontiguousarray(tab[:, 1]),
                                     np.ascontiguousarray(tab[:, 2]), 1e-6, sets)
    assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), 1e-2, 1e-5, "rows from the modulation table")
