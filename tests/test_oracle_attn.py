"""Pins of the oracle's sparse attention (flash_attn_sparse_128): torch's scaled_dot_product_attention in float64
with a boolean mask that numpy builds from the pass lists, written independently of the oracle's row mapping.
Every case checks to one bf16 ulp (the oracle rounds its double result once)."""
import numpy as np
import pytest
import torch

import oracle as orc


def layout_rows(grid, layout, row0):
    """(row, cube) of every token of the grid, in a numpy restatement of the two layouts."""
    gt, gh, gw = grid
    ch, cw = (gh + 3) // 4, (gw + 3) // 4
    t, y, x = np.meshgrid(np.arange(gt), np.arange(gh), np.arange(gw), indexing="ij")
    t, y, x = t.ravel(), y.ravel(), x.ravel()
    cube = ((t // 4) * ch + y // 4) * cw + x // 4
    if layout == orc.CUBES_GRID:
        row = row0 + (t * gh + y) * gw + x
    else:
        row = row0 + 64 * cube + ((t % 4) * 4 + y % 4) * 4 + x % 4
    return row, cube


def reference(q, k, v, idx, cnt, grid, layout, row0, dense_row0, n_dense):
    heads = q.shape[0]
    vrow, vcube = layout_rows(grid, layout, row0)
    drow = dense_row0 + np.arange(n_dense)
    rows = np.concatenate([vrow, drow])
    is_dense = np.concatenate([np.zeros(len(vrow), bool), np.ones(n_dense, bool)])
    cube = np.concatenate([vcube, -np.ones(n_dense, int)])
    out = {}
    for h in range(heads):
        C = idx.shape[1]
        sel = np.zeros((C, C), bool)
        for i in range(C):
            sel[i, idx[h, i, :cnt[h, i]]] = True
        mask = np.ones((len(rows), len(rows)), bool)
        vq = ~is_dense
        mask[np.ix_(vq, ~is_dense)] = sel[np.ix_(cube[vq], cube[~is_dense])]
        f = lambda a: torch.from_numpy(orc.bf16_to_f32(a[h, rows]).astype(np.float64))  # noqa: E731
        o = torch.nn.functional.scaled_dot_product_attention(f(q)[None], f(k)[None], f(v)[None],
                                                             attn_mask=torch.from_numpy(mask)[None])[0]
        out[h] = (rows, o.numpy())
    return out


def make(rng, heads, grid, layout, row0, dense_row0, n_dense, k_sel, local, total_rows):
    C = orc.cube_count(*grid)
    q, kk, v = [orc.bf16_from_f64(rng.standard_normal((heads, total_rows, 128))) for _ in range(3)]
    s = rng.standard_normal((heads, C, C))
    idx, cnt = orc.cube_topk(s, grid, k_sel, local, out_stride=k_sel + 3)
    return q, kk, v, idx, cnt


CASES = [
    # grid, layout, row0, dense_row0, n_dense, k, local
    ((8, 8, 12), orc.CUBES_GRID, 0, 768, 40, 4, 1),
    ((7, 9, 10), orc.CUBES_GATHERED, 70, 0, 70, 5, 3),
    ((8, 8, 12), orc.CUBES_GRID, 5, 0, 0, 3, 0),
    ((4, 5, 4), orc.CUBES_GRID, 64, 0, 64, 1, 1),
]


@pytest.mark.parametrize("grid,layout,row0,dense_row0,n_dense,k_sel,local", CASES)
def test_attn_sparse_matches_masked_sdpa(grid, layout, row0, dense_row0, n_dense, k_sel, local):
    rng = np.random.default_rng(sum(grid) + n_dense)
    C = orc.cube_count(*grid)
    video = C * 64 if layout == orc.CUBES_GATHERED else grid[0] * grid[1] * grid[2]
    total = max(row0 + video, dense_row0 + n_dense)
    q, k, v, idx, cnt = make(rng, 2, grid, layout, row0, dense_row0, n_dense, k_sel, local, total)
    got = orc.attn_sparse(q, k, v, idx, cnt, grid, dense_row0, n_dense, layout, row0)
    for h, (rows, want) in reference(q, k, v, idx, cnt, grid, layout, row0, dense_row0, n_dense).items():
        g = orc.bf16_to_f32(got[h, rows]).astype(np.float64)
        assert np.all(np.abs(g - want) <= 2.0 ** -8 * np.abs(want) + 1e-30), np.abs(g - want).max()
    if layout == orc.CUBES_GATHERED:                        # padding slots of gathered cubes are written zero
        vrow, _ = layout_rows(grid, layout, row0)
        pad = np.setdiff1d(np.arange(row0, row0 + 64 * C), vrow)
        assert len(pad) and (got[:, pad] == 0).all()


def test_attn_sparse_every_cube_is_dense_attention():
    """ratio 1: every cube selected, so every query attends every token: the unmasked attention."""
    rng = np.random.default_rng(3)
    grid = (8, 8, 8)
    C = orc.cube_count(*grid)
    q, k, v, _, _ = make(rng, 1, grid, orc.CUBES_GRID, 0, 512, 30, 1, 1, 542)
    idx = np.tile(np.arange(C, dtype=np.int32), (1, C, 1))
    cnt = np.full((1, C), C, np.int32)
    got = orc.attn_sparse(q, k, v, idx, cnt, grid, 512, 30)
    f = lambda a: torch.from_numpy(orc.bf16_to_f32(a[0]).astype(np.float64))  # noqa: E731
    want = torch.nn.functional.scaled_dot_product_attention(f(q)[None], f(k)[None], f(v)[None])[0].numpy()
    g = orc.bf16_to_f32(got[0]).astype(np.float64)
    assert np.all(np.abs(g - want) <= 2.0 ** -8 * np.abs(want) + 1e-30)


def test_attn_sparse_tile_subset_equals_whole():
    """The per-tile entry (used to sample large cases) writes exactly the whole call's rows for its tiles."""
    rng = np.random.default_rng(4)
    grid = (8, 8, 12)
    q, k, v, idx, cnt = make(rng, 2, grid, orc.CUBES_GRID, 0, 768, 40, 4, 1, 808)
    whole = orc.attn_sparse(q, k, v, idx, cnt, grid, 768, 40)
    part = orc.attn_sparse(q, k, v, idx, cnt, grid, 768, 40, tiles=[(1, 0), (0, 3), (1, 12)])
    rows_t3 = orc.attn_tile_rows(grid, orc.CUBES_GRID, 0, 768, 40, 3)
    assert (part[0, rows_t3] == whole[0, rows_t3]).all() and (part[1, 768:808] == whole[1, 768:808]).all()
