"""heads_partial fused with cube_pool (mh3_heads_partial_pool): every output bit-identical to heads_partial followed
by cube_pool over its gathered head tiles - q, k and v including the padding and dense rows, the cube means, the token
counts - on padded grids, with rows before and after the cubes, both output layouts, and the 768p shape. The oracle
pins the two separate kernels (test_heads_gpu.py, test_cubes_gpu.py); here the fused pass is held to them bit for
bit, which covers it to the same bar."""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import from_bits, randn_bf16_bits

pytestmark = pytest.mark.gpu


def inputs(dev, rows, heads, rot, seed):
    rng = np.random.default_rng(seed)
    x = from_bits(randn_bf16_bits(rng, (rows, 3 * heads * 128), 1.5), dev)
    ang = rng.uniform(-np.pi, np.pi, (rows, max(rot // 2, 1)))
    ct = torch.from_numpy(np.cos(ang).astype(np.float32)).to(dev)
    st = torch.from_numpy(np.sin(ang).astype(np.float32)).to(dev)
    qw = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(np.float32)).to(dev)
    kw = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(np.float32)).to(dev)
    return x, qw, kw, ct, st


def same(a, b):
    return a is None and b is None or torch.equal(a.view(torch.int32 if a.dtype == torch.float32 else torch.int16),
                                                  b.view(torch.int32 if b.dtype == torch.float32 else torch.int16))


def two_kernels(x, heads, grid, qw, kw, ct, st, rot, dm, with_v, layout, row0, counts):
    q, k, v = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot, map=dm, with_v=with_v, layout=layout)
    rows = q.numel() // (heads * 128)
    hs, rs = (rows * 128, 128) if layout == "heads" else (128, heads * 128)
    a = mh.cube_args(heads, grid, layout=mh.CUBES_GATHERED, row0=row0, head_stride=hs, row_stride=rs)
    qc, kc = mh.cube_pool(a, q, k, counts=counts)
    return q, k, v, qc, kc


CASES = [
    # grid, heads, rot, dense rows after the cubes, rows before them, with v, layout
    ((8, 8, 12), 2, 96, 70, 0, True, "heads"),
    ((7, 9, 10), 2, 96, 70, 0, True, "heads"),
    ((5, 3, 6), 5, 128, 0, 0, True, "rows"),
    ((3, 5, 9), 40, 96, 33, 19, True, "heads"),
    ((6, 7, 5), 3, 16, 12, 40, False, "heads"),
    ((4, 4, 4), 1, 0, 0, 0, True, "rows"),
]


@pytest.mark.parametrize("grid,heads,rot,n_after,n_before,with_v,layout", CASES)
def test_heads_partial_pool_matches_the_two_kernels(dev, grid, heads, rot, n_after, n_before, with_v, layout):
    C = orc.cube_count(*grid)
    video = grid[0] * grid[1] * grid[2]
    model_rows = n_before + n_after + video
    x, qw, kw, ct, st = inputs(dev, model_rows, heads, rot, seed=sum(grid) + heads + rot)
    # Attention rows: n_before text rows, the cubes, n_after more dense rows; model rows: text, video, dense.
    cm, _ = mh.cube_map(grid, n_dense=n_after, video_row0=n_before, dense_row0=n_before + video, device=dev)
    dm = torch.cat([torch.arange(n_before, dtype=torch.int32, device=dev), cm])
    counts_a = torch.full((C,), -7, dtype=torch.int32, device=dev)
    counts_b = torch.full((C,), -9, dtype=torch.int32, device=dev)
    want = two_kernels(x, heads, grid, qw, kw, ct, st, rot, dm, with_v, layout, n_before, counts_a)
    got = mh.heads_partial_pool(x, heads, grid, qw, kw, ct, st, rot=rot, map=dm, with_v=with_v, layout=layout,
                                row0=n_before, counts=counts_b)
    torch.cuda.synchronize()
    for name, g, w in zip(("q", "k", "v", "qc", "kc"), got, want):
        assert same(g, w), f"{name} differs for grid {grid} heads {heads} rot {rot} layout {layout}"
    assert torch.equal(counts_a, counts_b)
    assert torch.equal(counts_b.cpu(), torch.from_numpy(orc.cube_map(grid, 0, 0, 0)[1]).to(torch.int32))


def test_heads_partial_pool_without_a_map(dev):
    """No map: output row r is model row r, and the cube rows are simply rows row0 .. (their pool is what cube_pool
    makes of whatever heads_partial wrote there)."""
    grid, heads, rot = (5, 6, 7), 3, 96
    C = orc.cube_count(*grid)
    rows = 64 * C + 21
    x, qw, kw, ct, st = inputs(dev, rows, heads, rot, seed=3)
    want = two_kernels(x, heads, grid, qw, kw, ct, st, rot, None, True, "heads", 10, None)
    got = mh.heads_partial_pool(x, heads, grid, qw, kw, ct, st, rot=rot, row0=10)
    for name, g, w in zip(("q", "k", "v", "qc", "kc"), got, want):
        assert same(g, w), name


def test_heads_partial_pool_768p(dev):
    """768p: 512 text rows and the 32 x 48 x 84 video grid (2016 cubes), 40 heads, gathered through the cube map."""
    grid, heads, rot, n_dense = (32, 48, 84), 40, 96, 512
    video = grid[0] * grid[1] * grid[2]
    rows = n_dense + video
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn((rows, 3 * heads * 128), generator=g, device=dev).to(torch.bfloat16)
    ang = torch.rand((rows, rot // 2), generator=g, device=dev) * 6.283 - 3.1416
    ct, st = torch.cos(ang), torch.sin(ang)
    qw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    kw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    dm, counts = mh.cube_map(grid, n_dense=n_dense, video_row0=n_dense, dense_row0=0, device=dev)
    want = two_kernels(x, heads, grid, qw, kw, ct, st, rot, dm, True, "heads", 0, None)
    got = mh.heads_partial_pool(x, heads, grid, qw, kw, ct, st, rot=rot, map=dm)
    torch.cuda.synchronize()
    for name, a, b in zip(("q", "k", "v", "qc", "kc"), got, want):
        assert same(a, b), f"{name} differs at 768p"
    assert bool(torch.isfinite(got[3]).all()) and bool(torch.isfinite(got[4]).all())


GRID_CASES = [
    # grid, heads, rot, rows before the video rows, rows after them, layout
    ((8, 8, 12), 2, 96, 70, 0, "heads"),
    ((7, 9, 10), 3, 96, 0, 33, "heads"),
    ((5, 3, 6), 5, 128, 12, 7, "rows"),
    ((3, 5, 9), 40, 96, 19, 0, "heads"),
]


@pytest.mark.parametrize("grid,heads,rot,n_before,n_after,layout", GRID_CASES)
def test_heads_partial_pool_grid_layout(dev, grid, heads, rot, n_before, n_after, layout):
    """The grid layout: no map, the outputs in the model's order; the same bits as heads_partial then cube_pool with
    MH3_CUBES_GRID at the video rows' first row."""
    C = orc.cube_count(*grid)
    video = grid[0] * grid[1] * grid[2]
    rows = n_before + video + n_after
    x, qw, kw, ct, st = inputs(dev, rows, heads, rot, seed=7 * sum(grid) + heads)
    q, k, v = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot, layout=layout)
    hs, rs = (rows * 128, 128) if layout == "heads" else (128, heads * 128)
    counts_a = torch.full((C,), -7, dtype=torch.int32, device=dev)
    counts_b = torch.full((C,), -9, dtype=torch.int32, device=dev)
    qc, kc = mh.cube_pool(mh.cube_args(heads, grid, layout=mh.CUBES_GRID, row0=n_before, head_stride=hs,
                                       row_stride=rs), q, k, counts=counts_a)
    got = mh.heads_partial_pool(x, heads, grid, qw, kw, ct, st, rot=rot, layout=layout, row0=n_before,
                                cube_layout=mh.CUBES_GRID, counts=counts_b)
    torch.cuda.synchronize()
    for name, g_, w_ in zip(("q", "k", "v", "qc", "kc"), got, (q, k, v, qc, kc)):
        assert same(g_, w_), f"{name} differs for grid {grid} heads {heads} layout {layout}"
    assert torch.equal(counts_a, counts_b)


def test_heads_partial_pool_grid_layout_768p(dev):
    """768p in the model's order: 512 text rows, then the 32 x 48 x 84 grid; 40 heads."""
    grid, heads, rot, n_dense = (32, 48, 84), 40, 96, 512
    rows = n_dense + grid[0] * grid[1] * grid[2]
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((rows, 3 * heads * 128), generator=g, device=dev).to(torch.bfloat16)
    ang = torch.rand((rows, rot // 2), generator=g, device=dev) * 6.283 - 3.1416
    ct, st = torch.cos(ang), torch.sin(ang)
    q, k, v = mh.heads_partial(x, heads, None, None, ct, st, rot=rot)
    qc, kc = mh.cube_pool(mh.cube_args(heads, grid, layout=mh.CUBES_GRID, row0=n_dense, head_stride=rows * 128), q, k)
    got = mh.heads_partial_pool(x, heads, grid, None, None, ct, st, rot=rot, row0=n_dense, cube_layout=mh.CUBES_GRID)
    torch.cuda.synchronize()
    for name, a, b in zip(("q", "k", "v", "qc", "kc"), got, (q, k, v, qc, kc)):
        assert same(a, b), f"{name} differs at 768p (grid layout)"
