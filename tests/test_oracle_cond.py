"""Pins the oracle's cube map and time conditioning (CPU only).

- cube_map: a brute-force gather written per attention row in Python (the oracle scatters per token), the per-axis
  product for the counts, and the map's use: gathering q through it and pooling in the gathered layout gives the grid
  layout's means.
- time_embed: torch float64, restating the reference's own torch statement of the path
  (tools/check_pruned_curve.py:57-67, temb()); t = 0 has the closed form emb = [1 .. 1, 0 .. 0].
- adaln_mod: torch float64 matmul; small-integer operands give exact integer results.
- curve_mods: numpy interp per coordinate (a library routine), then matmul; t on a table point reads that row.
A slip such as sin before cos, a missing silu, the bias dropped or an off-by-one interpolation index fails one of these.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as orc


def brute_map(grid, n_dense, video_row0, dense_row0):
    T, Y, X = grid
    ct, ch, cw = (T + 3) // 4, (Y + 3) // 4, (X + 3) // 4
    out, counts = [], []
    for c in range(ct * ch * cw):
        a, rem = divmod(c, ch * cw)
        b, d = divmod(rem, cw)
        n = 0
        for l in range(64):
            t, y, x = 4 * a + l // 16, 4 * b + (l // 4) % 4, 4 * d + l % 4
            if t < T and y < Y and x < X:
                out.append(video_row0 + (t * Y + y) * X + x)
                n += 1
            else:
                out.append(-1)
        counts.append(n)
    out += [dense_row0 + j for j in range(n_dense)]
    return np.array(out, np.int32), np.array(counts, np.int32)


@pytest.mark.parametrize("grid,n_dense,video_row0,dense_row0", [
    ((5, 6, 9), 0, 0, 0), ((5, 7, 9), 7, 7, 0), ((8, 8, 12), 40, 0, 768), ((1, 1, 1), 3, 10, 0),
    ((37, 24, 42), 640, 640, 0)])
def test_cube_map_brute_force(grid, n_dense, video_row0, dense_row0):
    m, c = orc.cube_map(grid, n_dense, video_row0, dense_row0)
    bm, bc = brute_map(grid, n_dense, video_row0, dense_row0)
    assert np.array_equal(m, bm) and np.array_equal(c, bc)
    T, Y, X = grid
    assert (m >= 0).sum() == T * Y * X + n_dense                    # every token once, padding the rest
    assert np.array_equal(np.sort(m[m >= 0]), np.sort(np.r_[video_row0 + np.arange(T * Y * X),
                                                            dense_row0 + np.arange(n_dense)]))


def test_cube_map_h3_768p_cube_count():
    """H3's 768p grid 37 x 24 x 42 pads to 40 x 24 x 44: 660 cubes (docs/performance.md:175-177)."""
    m, c = orc.cube_map((37, 24, 42))
    assert c.size == 660 and m.size == 660 * 64 and c.sum() == 37 * 24 * 42
    # full cubes, the last frame group (1 frame of 4), the last column group (2 of 4), and both
    assert set(np.unique(c).tolist()) == {64, 16, 32, 8}


def test_cube_map_gather_pools_like_grid():
    rng = np.random.default_rng(5)
    grid, n_dense = (5, 6, 9), 4
    rows = 5 * 6 * 9
    q = rng.integers(0, 0x3f80, (1, n_dense + rows, 128)).astype(np.uint16)
    m, _ = orc.cube_map(grid, n_dense=n_dense)
    g = np.zeros((1, m.size, 128), np.uint16)
    g[0, m >= 0] = q[0, m[m >= 0]]
    qg, _, cg = orc.cube_pool(g, g, 1, grid, layout=orc.CUBES_GATHERED, head_stride=m.size * 128)
    qq, _, cq = orc.cube_pool(q, q, 1, grid, row0=n_dense, head_stride=(n_dense + rows) * 128)
    assert np.array_equal(qg, qq) and np.array_equal(cg, cq)


def torch_temb(t, w_in, b_in, w_out, b_out, max_period=10000.0):
    """tools/check_pruned_curve.py:57-63 in torch float64, for several levels."""
    half = w_in.shape[1] // 2
    i = torch.arange(half, dtype=torch.float64)
    freq = torch.exp(-math.log(max_period) * i / half)
    out = []
    for tv in t:
        arg = float(tv) * freq
        emb = torch.cat([torch.cos(arg), torch.sin(arg)])
        h = torch.nn.functional.silu(torch.from_numpy(w_in).double() @ emb + torch.from_numpy(b_in).double())
        out.append(torch.from_numpy(w_out).double() @ h + torch.from_numpy(b_out).double())
    return torch.stack(out)


def mlp_weights(rng, freq_dim, hidden, out_dim):
    return ((rng.standard_normal((hidden, freq_dim)) / math.sqrt(freq_dim)).astype(np.float32),
            (0.1 * rng.standard_normal(hidden)).astype(np.float32),
            (rng.standard_normal((out_dim, hidden)) / math.sqrt(hidden)).astype(np.float32),
            (0.1 * rng.standard_normal(out_dim)).astype(np.float32))


@pytest.mark.parametrize("freq_dim,hidden,out_dim", [(256, 96, 40), (256, 5376, 2688), (64, 32, 8)])
def test_time_embed_against_torch(freq_dim, hidden, out_dim):
    rng = np.random.default_rng(11)
    w_in, b_in, w_out, b_out = mlp_weights(rng, freq_dim, hidden, out_dim)
    t = np.array([0.0, 0.25, 0.9230769, 1.0], np.float32)
    temb, cond = orc.time_embed(t, w_in, b_in, w_out, b_out)
    want = torch_temb(t, w_in, b_in, w_out, b_out)
    assert np.abs(temb - want.numpy()).max() <= 1e-6 * np.abs(want.numpy()).max()
    sil = torch.nn.functional.silu(want).numpy()
    got = (cond.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert (np.abs(got - sil) <= 2.0 ** -8 * np.abs(sil) + 1e-30).all()    # one bf16 rounding


def test_time_embed_t0_closed_form():
    """At t = 0 every cos is 1 and every sin 0, so temb = w_out silu(sum of w_in's first half + b_in) + b_out."""
    rng = np.random.default_rng(12)
    w_in, b_in, w_out, b_out = mlp_weights(rng, 256, 64, 16)
    temb, _ = orc.time_embed(np.zeros(1, np.float32), w_in, b_in, w_out, b_out)
    s = w_in[:, :128].astype(np.float64).sum(1) + b_in
    want = w_out.astype(np.float64) @ (s / (1 + np.exp(-s))) + b_out
    assert np.abs(temb[0] - want).max() <= 1e-6 * np.abs(want).max()


def test_time_embed_order_is_cos_first():
    """Weights that read only the embedding's first half see cos(t f), the second half sin(t f)."""
    w_in = np.zeros((2, 256), np.float32)
    w_in[0, 0] = 1.0      # cos(t f_0) = cos(t)
    w_in[1, 128] = 1.0    # sin(t f_0) = sin(t)
    w_out = np.eye(2, dtype=np.float32)
    temb, _ = orc.time_embed(np.array([0.7], np.float32), w_in, np.zeros(2, np.float32), w_out,
                             np.zeros(2, np.float32))
    s = np.array([math.cos(np.float32(0.7)), math.sin(np.float32(0.7))])
    assert np.allclose(temb[0], s / (1 + np.exp(-s)), rtol=1e-6)


def test_adaln_mod_against_torch_and_exact():
    rng = np.random.default_rng(13)
    cond = orc.bf16_from_f64(rng.standard_normal((3, 264)))
    w = orc.bf16_from_f64(0.05 * rng.standard_normal((37, 264)))
    bias = rng.standard_normal(37).astype(np.float32)
    got = orc.adaln_mod(cond, w, bias)
    f = lambda a: torch.from_numpy((a.astype(np.uint32) << 16).view(np.float32)).double()  # noqa: E731
    want = (f(cond) @ f(w).T + torch.from_numpy(bias).double()).numpy()
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    ci = rng.integers(-8, 9, (2, 64)).astype(np.float64)
    wi = rng.integers(-8, 9, (5, 64)).astype(np.float64)
    got = orc.adaln_mod(orc.bf16_from_f64(ci), orc.bf16_from_f64(wi))
    assert np.array_equal(got, (ci @ wi.T).astype(np.float32))


def test_curve_mods_against_numpy_interp():
    rng = np.random.default_rng(14)
    table = rng.standard_normal((1025, 8)).astype(np.float32)
    w = rng.standard_normal((21, 8)).astype(np.float32)
    bias = rng.standard_normal(21).astype(np.float32)
    t = np.array([0.0, 0.0769230769, 0.5, 0.999, 1.0, -0.5, 1.5], np.float32)
    got = orc.curve_mods(t, table, w, bias)
    grid = np.arange(1025) / 1024.0
    for u, tv in enumerate(t):
        c = np.array([np.interp(np.clip(float(tv), 0, 1), grid, table[:, j].astype(np.float64)) for j in range(8)])
        want = w.astype(np.float64) @ c + bias
        assert np.abs(got[u] - want).max() <= 1e-5 * np.abs(want).max()
    on_point = orc.curve_mods(np.array([512 / 1024], np.float32), table, w)
    assert np.array_equal(on_point[0], (w.astype(np.float64) @ table[512].astype(np.float64)).astype(np.float32))
