"""Parity of flash_attn_sparse_128 with the oracle (bf16 output; 1e-2 relative, checked per element against the
row's scale, and the reference's diff() pair: relative RMS error and the lowest row cosine)."""
import math

import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import (attn_sparse_f32, bits_to_f64, check_attn_f32, diff, from_bits, nan_filled, randn_bf16_bits,
                     to_bits)

pytestmark = pytest.mark.gpu


def check(got_bits, want_bits, what):
    g, w = bits_to_f64(got_bits).reshape(-1, 128), bits_to_f64(want_bits).reshape(-1, 128)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True)) + 1e-30              # a row's RMS
    err = np.abs(g - w)
    assert np.all(err <= 1e-2 * (np.abs(w) + scale)), f"{what}: worst {(err / (np.abs(w) + scale)).max():.3g}"
    rel, cos = diff(g, w, 128)
    assert rel < 5e-3 and cos > 0.9999, f"{what}: rel {rel:.3g} cos {cos:.6f}"


def run(dev, q, k, v, idx, cnt, grid, layout, row0, dense_row0, n_dense, out_init=None, order=None):
    heads, rows, _ = q.shape
    a = mh.cube_args(heads, grid, layout=layout, row0=row0, head_stride=rows * 128, out_stride=idx.shape[2])
    out = None if out_init is None else from_bits(out_init, dev)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    got = mh.flash_attn_sparse_128(a, from_bits(q, dev), from_bits(k, dev), from_bits(v, dev), t(idx), t(cnt),
                                   dense_row0=dense_row0, n_dense=n_dense, out=out,
                                   order=None if order is None else t(order))
    return to_bits(got)


def order_by_middle_entry(idx, cnt, cubes):
    """cube_order's result restated with numpy: each head's cubes by the middle entry of their pass lists (entries
    outside [0, cubes), and empty lists, as `cubes`), equal entries by cube index (a stable sort)."""
    n = np.clip(cnt, 0, idx.shape[2])
    mid = np.take_along_axis(idx, (n // 2)[..., None], axis=2)[..., 0]
    key = np.where((n > 0) & (mid >= 0) & (mid < cubes), mid, cubes)
    return np.argsort(key, axis=1, kind="stable").astype(np.int32)


CASES = [
    # grid, layout, row0, dense_row0, n_dense, k, local
    ((8, 8, 12), orc.CUBES_GRID, 0, 768, 40, 4, 1),
    ((7, 9, 10), orc.CUBES_GATHERED, 70, 0, 70, 5, 3),
    ((8, 8, 12), orc.CUBES_GRID, 5, 0, 0, 3, 0),
    ((4, 5, 4), orc.CUBES_GRID, 64, 0, 64, 1, 1),
    ((13, 10, 9), orc.CUBES_GRID, 0, 1170, 130, 6, 1),
    # 64 cubes and 4 dense tiles x 2 heads, both multiples of 8: the XCD-sliced order with rotated pass lists
    ((16, 16, 16), orc.CUBES_GRID, 0, 4096, 256, 6, 1),
    ((15, 16, 16), orc.CUBES_GATHERED, 256, 0, 200, 9, 3),
]


@pytest.mark.parametrize("grid,layout,row0,dense_row0,n_dense,k_sel,local", CASES)
def test_flash_attn_sparse_matches_oracle(dev, grid, layout, row0, dense_row0, n_dense, k_sel, local):
    rng = np.random.default_rng(sum(grid) + n_dense + layout)
    C = orc.cube_count(*grid)
    video = C * 64 if layout == orc.CUBES_GATHERED else grid[0] * grid[1] * grid[2]
    rows = max(row0 + video, dense_row0 + n_dense)
    q, k, v = [randn_bf16_bits(rng, (2, rows, 128)) for _ in range(3)]
    idx, cnt = orc.cube_topk(rng.standard_normal((2, C, C)), grid, k_sel, local, out_stride=k_sel + 3)
    want = orc.attn_sparse(q, k, v, idx, cnt, grid, dense_row0, n_dense, layout, row0)
    got = run(dev, q, k, v, idx, cnt, grid, layout, row0, dense_row0, n_dense)
    check(got, want, f"attn {grid} layout {layout}")
    # The float32 GPU restatement the whole-launch tests use agrees with the oracle (rounded to bf16) on every row.
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    ref = attn_sparse_f32(from_bits(q, dev), from_bits(k, dev), from_bits(v, dev), t(idx), t(cnt), grid, dense_row0,
                          n_dense, layout=layout, row0=row0)
    w64 = torch.from_numpy(bits_to_f64(want)).to(dev)
    for h, (rows, out) in ref.items():
        w = w64[h, rows]
        rms = w.pow(2).mean(1, keepdim=True).sqrt()
        # within the oracle's one bf16 rounding (half a unit in the last place: 2^-8 relative at most)
        assert bool(((out.double() - w).abs() <= (2 ** -8 + 1e-5) * w.abs() + 1e-4 * rms).all()), \
            f"f32 restatement head {h}"
    if layout == orc.CUBES_GATHERED:
        vrow = np.concatenate([orc.attn_tile_rows(grid, layout, row0, dense_row0, n_dense, (n_dense + 63) // 64 + c)
                               for c in range(C)])
        pad = np.setdiff1d(np.arange(row0, row0 + 64 * C), vrow)
        assert len(pad) and (got[:, pad] == 0).all()


@pytest.mark.parametrize("grid,layout,row0,dense_row0,n_dense,k_sel,local", CASES)
def test_flash_attn_sparse_ordered_matches_oracle(dev, grid, layout, row0, dense_row0, n_dense, k_sel, local):
    """The ordered form, with cube_order's order and with a random permutation of each head's cubes: every row the
    call writes against the oracle (the output NaN-filled first, so an unwritten row fails)."""
    rng = np.random.default_rng(7 * sum(grid) + n_dense + layout)
    C = orc.cube_count(*grid)
    video = C * 64 if layout == orc.CUBES_GATHERED else grid[0] * grid[1] * grid[2]
    rows = max(row0 + video, dense_row0 + n_dense)
    q, k, v = [randn_bf16_bits(rng, (2, rows, 128)) for _ in range(3)]
    idx, cnt = orc.cube_topk(rng.standard_normal((2, C, C)), grid, k_sel, local, out_stride=k_sel + 3)
    want = orc.attn_sparse(q, k, v, idx, cnt, grid, dense_row0, n_dense, layout, row0)
    a = mh.cube_args(2, grid, layout=layout, row0=row0, head_stride=rows * 128, out_stride=idx.shape[2])
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    order = mh.cube_order(a, t(idx), t(cnt)).cpu().numpy()
    assert (order == order_by_middle_entry(idx, cnt, C)).all()
    written = np.concatenate([orc.attn_tile_rows(grid, layout, row0, dense_row0, n_dense, t_)
                              for t_ in range((n_dense + 63) // 64 + C)])
    nan = np.full((2, rows, 128), 0x7FC0, np.uint16)
    for name, o in (("cube_order", order), ("random", np.stack([rng.permutation(C) for _ in range(2)]))):
        got = run(dev, q, k, v, idx, cnt, grid, layout, row0, dense_row0, n_dense, out_init=nan,
                  order=o.astype(np.int32))
        check(got[:, written], want[:, written], f"ordered ({name}) attn {grid} layout {layout}")


def test_cube_order_edge_cases(dev):
    """cube_order against its numpy restatement on pass lists with empty lists, counts above out_stride (clamped),
    negative counts, middle entries outside [0, cubes), unsorted lists and many equal middle entries; 3 heads of a
    padded grid (5 x 9 x 13: 2 x 3 x 4 = 24 cubes) and 40 heads of 768p's 2016 cubes."""
    for heads, grid, stride in ((3, (5, 9, 13), 7), (40, (32, 48, 84), 205)):
        rng = np.random.default_rng(heads)
        C = orc.cube_count(*grid)
        idx = rng.integers(-3, C + 3, (heads, C, stride)).astype(np.int32)
        idx[:, ::3] = rng.integers(0, 4, (heads, len(range(0, C, 3)), stride))   # many equal middle entries
        cnt = rng.integers(-2, stride + 4, (heads, C)).astype(np.int32)
        cnt[:, ::5] = 0
        a = mh.cube_args(heads, grid, out_stride=stride)
        t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
        got = mh.cube_order(a, t(idx), t(cnt)).cpu().numpy()
        want = order_by_middle_entry(idx, cnt, C)
        assert (got == want).all(), f"cube_order {heads} heads {grid}"
        assert (np.sort(got, axis=1) == np.arange(C)).all()


@pytest.mark.parametrize("grid,layout,row0,dense_row0,n_dense", [((7, 9, 10), orc.CUBES_GRID, 0, 630, 70),
                                                                   ((7, 9, 10), orc.CUBES_GATHERED, 70, 0, 70)])
def test_flash_attn_sparse_interleaved_rows(dev, grid, layout, row0, dense_row0, n_dense):
    """q, k, v (and out) as the model's rows, [rows][heads x 128] (head stride 128, row stride heads x 128): the K/V
    loads' row offsets then differ from the head tiles' 256 bytes."""
    heads = 3
    rng = np.random.default_rng(31 + layout)
    C = orc.cube_count(*grid)
    video = C * 64 if layout == orc.CUBES_GATHERED else grid[0] * grid[1] * grid[2]
    rows = max(row0 + video, dense_row0 + n_dense)
    q, k, v = [randn_bf16_bits(rng, (heads, rows, 128)) for _ in range(3)]
    idx, cnt = orc.cube_topk(rng.standard_normal((heads, C, C)), grid, 5, 1, out_stride=8)
    want = orc.attn_sparse(q, k, v, idx, cnt, grid, dense_row0, n_dense, layout, row0)
    a = mh.cube_args(heads, grid, layout=layout, row0=row0, head_stride=128, row_stride=heads * 128, out_stride=8)
    rowwise = lambda x: from_bits(np.ascontiguousarray(x.transpose(1, 0, 2)), dev)  # noqa: E731
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    got = mh.flash_attn_sparse_128(a, rowwise(q), rowwise(k), rowwise(v), t(idx), t(cnt), dense_row0=dense_row0,
                                   n_dense=n_dense)
    got = to_bits(got).reshape(rows, heads, 128).transpose(1, 0, 2)
    rows_written = np.concatenate([orc.attn_tile_rows(grid, layout, row0, dense_row0, n_dense, t_)
                                   for t_ in range((n_dense + 63) // 64 + C)])
    check(got[:, rows_written], want[:, rows_written], f"interleaved rows {grid} layout {layout}")


def test_flash_attn_sparse_every_cube_is_dense_attention(dev):
    """Every cube selected: each query attends every token, as torch's attention (float32 on the GPU) does."""
    rng = np.random.default_rng(21)
    grid = (8, 8, 8)
    C = orc.cube_count(*grid)
    q, k, v = [randn_bf16_bits(rng, (2, 542, 128)) for _ in range(3)]
    idx = np.tile(np.arange(C, dtype=np.int32), (2, C, 1))
    cnt = np.full((2, C), C, np.int32)
    got = run(dev, q, k, v, idx, cnt, grid, orc.CUBES_GRID, 0, 512, 30)
    f = lambda a: torch.from_numpy(bits_to_f64(a)).to(dev, torch.float32)  # noqa: E731
    want = torch.nn.functional.scaled_dot_product_attention(f(q), f(k), f(v)).to(torch.bfloat16)
    check(got, to_bits(want), "every cube")


def test_flash_attn_sparse_leaves_other_rows_and_skips_bad_entries(dev):
    """Rows that are neither tokens nor dense rows keep their contents; an idx entry outside the cubes is skipped."""
    rng = np.random.default_rng(22)
    grid, row0, dense_row0, n_dense = (8, 8, 12), 3, 800, 20
    C = orc.cube_count(*grid)
    rows = 830
    q, k, v = [randn_bf16_bits(rng, (1, rows, 128)) for _ in range(3)]
    idx, cnt = orc.cube_topk(rng.standard_normal((1, C, C)), grid, 4, 1, out_stride=8)
    bad_idx, bad_cnt = idx.copy(), cnt.copy()
    bad_idx[0, 5, cnt[0, 5]] = C + 7                                    # one entry past the cubes, counted
    bad_cnt[0, 5] += 1
    sentinel = np.full((1, rows, 128), 0x3F80, np.uint16)               # 1.0 in bf16
    got = run(dev, q, k, v, bad_idx, bad_cnt, grid, orc.CUBES_GRID, row0, dense_row0, n_dense, out_init=sentinel)
    want = orc.attn_sparse(q, k, v, idx, cnt, grid, dense_row0, n_dense, orc.CUBES_GRID, row0, out=sentinel.copy())
    check(got, want, "bad entry skipped")
    untouched = np.r_[0:row0, row0 + 768:dense_row0, dense_row0 + n_dense:rows]
    assert (got[0, untouched] == 0x3F80).all()


def test_flash_attn_sparse_768p_sampled(dev):
    """The 768p shape (grid 32 x 48 x 84: 2016 cubes; 512 text rows after the video rows), two heads, the pass lists
    from cube_select at ratio 0.1 (k = 202) and local 1 on structured q and k: a dense tile and eight cube tiles
    a head checked against the oracle."""
    grid, heads, n_dense = (32, 48, 84), 2, 512
    video = 32 * 48 * 84
    rows = video + n_dense
    g = torch.Generator(device=dev).manual_seed(5)
    q, k, v = [torch.randn((heads, rows, 128), generator=g, device=dev).to(torch.bfloat16) for _ in range(3)]
    t = torch.arange(video, device=dev)
    tt, yy, xx = (t // (48 * 84)).float() / 32, (t // 84 % 48).float() / 48, (t % 84).float() / 84
    for h in range(heads):                                              # low-frequency structure across cubes
        for f in range(3):
            u = torch.randn(128, generator=g, device=dev)
            wave = torch.cos(2 * math.pi * ((f + 1) * tt + (2 - f) * yy + f * xx))
            q[h, :video] += (0.5 * wave[:, None] * u[None, :]).to(torch.bfloat16)
            k[h, :video] += (0.5 * wave[:, None] * u[None, :]).to(torch.bfloat16)
    C = orc.cube_count(*grid)
    kk = mh.topk_k(0.1, C)
    a = mh.cube_args(heads, grid, head_stride=rows * 128, k=kk, local=1)
    qc, kc = mh.cube_pool(a, q, k)
    idx, cnt = mh.cube_select(a, qc, kc)
    out = mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense)
    qb, kb, vb, ob = (to_bits(x) for x in (q, k, v, out))
    idx_n, cnt_n = idx.cpu().numpy(), cnt.cpu().numpy()
    nd = n_dense // 64
    rng = np.random.default_rng(6)
    tiles = [(h, 0) for h in range(heads)] + [(h, nd + int(c)) for h in range(heads)
                                              for c in rng.choice(C, 8, replace=False)]
    want = orc.attn_sparse(qb, kb, vb, idx_n, cnt_n, grid, video, n_dense, tiles=tiles)
    for h, tile in tiles:
        r = orc.attn_tile_rows(grid, orc.CUBES_GRID, 0, video, n_dense, tile)
        check(ob[h, r], want[h, r], f"768p head {h} tile {tile}")


@pytest.mark.parametrize("ordered", [False, True])
def test_flash_attn_sparse_rotated_walk_every_tile(dev, ordered):
    """Enough cube tiles an XCD that most walk their pass lists from a rotated start: 160 heads of a 16 x 16 x 16 grid
    (64 cubes, one dense tile), so each XCD runs 1280 cube tiles in sequence, and tiles from the fourth round of the
    XCD's resident workgroups on (rank 512 and up at 4 workgroups a CU on 256 CUs) start a fraction of the way into
    their lists. Every output row against the float32 restatement, the output buffer NaN-filled first; a sample of
    rotated tiles against the oracle."""
    grid, heads, n_dense = (16, 16, 16), 160, 64
    video = 16 * 16 * 16
    rows = video + n_dense
    C = orc.cube_count(*grid)
    g = torch.Generator(device=dev).manual_seed(41)
    q, k, v = [torch.randn((heads, rows, 128), generator=g, device=dev).to(torch.bfloat16) for _ in range(3)]
    rng = np.random.default_rng(42)
    idx_n, cnt_n = orc.cube_topk(rng.standard_normal((heads, C, C)), grid, 6, 1, out_stride=8)
    idx, cnt = torch.from_numpy(idx_n).to(dev), torch.from_numpy(cnt_n).to(dev)
    a = mh.cube_args(heads, grid, head_stride=rows * 128, out_stride=8)
    order = mh.cube_order(a, idx, cnt) if ordered else None
    out = mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense,
                                   out=nan_filled((heads, rows, 128), dev), order=order)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "an output row left unwritten"
    worst = (0.0, 0.0)
    for h0 in range(0, heads, 40):
        ref = attn_sparse_f32(q, k, v, idx, cnt, grid, video, n_dense, heads=range(h0, h0 + 40), chunk=1024)
        e, r = check_attn_f32(out, ref, "rotated walk")
        worst = (max(worst[0], e), max(worst[1], r))
    print(f"rotated walk: worst element error {worst[0]:.3g}, worst row RMS error {worst[1]:.3g} of the row's RMS")
    # Oracle: two cube tiles of each of the last eight heads (XCD ranks well past 512), every XCD slice covered.
    hs = list(range(heads - 8, heads))
    tiles = [(j, 1 + ((j % 8) * C) // 8 + int(rng.integers(0, C // 8))) for j in range(8)]
    tiles += [(j, 1 + int(rng.integers(0, C))) for j in range(8)]
    sub = lambda x: to_bits(x[hs])  # noqa: E731
    qb, kb, vb, ob = sub(q), sub(k), sub(v), sub(out)
    want = orc.attn_sparse(qb, kb, vb, idx_n[hs], cnt_n[hs], grid, video, n_dense, tiles=tiles)
    for lh, tile in tiles:
        r = orc.attn_tile_rows(grid, orc.CUBES_GRID, 0, video, n_dense, tile)
        check(ob[lh, r], want[lh, r], f"rotated walk: head {hs[lh]} tile {tile}")


@pytest.mark.parametrize("ordered", [False, True])
def test_flash_attn_sparse_768p_40_heads(dev, ordered):
    """The launch bench.py times: 40 heads of the 768p shape (2016 cubes, 512 text rows after the video rows), whose
    tile count lets each XCD take a contiguous eighth of every head's query cubes with rotated pass lists, the pass
    lists from cube_select at ratio 0.1 (k = 202), local 1. The output buffer is NaN-filled first and every row is
    finite after; every dense tile and the cube tiles of three whole heads against the float32 restatement; tiles of
    every head -- one dense tile of each fifth head, cube tiles spread over all XCD slices -- against the oracle."""
    grid, heads, n_dense = (32, 48, 84), 40, 512
    video = 32 * 48 * 84
    rows = video + n_dense
    g = torch.Generator(device=dev).manual_seed(15)
    q, k, v = [torch.randn((heads, rows, 128), generator=g, device=dev).to(torch.bfloat16) for _ in range(3)]
    t = torch.arange(video, device=dev)
    tt, yy, xx = (t // (48 * 84)).float() / 32, (t // 84 % 48).float() / 48, (t % 84).float() / 84
    for h in range(heads):
        u = torch.randn(128, generator=g, device=dev)
        wave = torch.cos(2 * math.pi * ((h % 3) * tt + (h % 2 + 1) * yy + (h % 4) * xx))
        q[h, :video] += (0.5 * wave[:, None] * u[None, :]).to(torch.bfloat16)
        k[h, :video] += (0.5 * wave[:, None] * u[None, :]).to(torch.bfloat16)
    C = orc.cube_count(*grid)
    kk = mh.topk_k(0.1, C)
    a = mh.cube_args(heads, grid, head_stride=rows * 128, k=kk, local=1)
    qc, kc = mh.cube_pool(a, q, k)
    idx, cnt = mh.cube_select(a, qc, kc)
    order = mh.cube_order(a, idx, cnt) if ordered else None
    out = mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=n_dense,
                                   out=nan_filled((heads, rows, 128), dev), order=order)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "an output row left unwritten"
    # Every dense tile of every head, and every cube tile of three whole heads (head 0's tiles are among each XCD's
    # first, which walk their lists unrotated; heads 2 and 39 are past the fourth round and rotated), against the
    # float32 restatement.
    worst = (0.0, 0.0)
    for h0 in range(0, heads, 8):
        ref = attn_sparse_f32(q, k, v, idx, cnt, grid, video, n_dense, heads=range(h0, h0 + 8),
                              cubes=torch.empty(0, dtype=torch.long))
        e, r = check_attn_f32(out, ref, "768p dense tiles")
        worst = (max(worst[0], e), max(worst[1], r))
    for h in (0, 2, heads - 1):
        ref = attn_sparse_f32(q, k, v, idx, cnt, grid, video, n_dense, heads=[h], dense=False)
        e, r = check_attn_f32(out, ref, "768p cube tiles")
        worst = (max(worst[0], e), max(worst[1], r))
    print(f"768p 40 heads: worst element error {worst[0]:.3g}, worst row RMS error {worst[1]:.3g} of the row's RMS")
    nd = n_dense // 64
    rng = np.random.default_rng(16)
    # cube c of head h lands in XCD slice c * 8 // C; cover every slice across the heads
    tiles = [(h, int(rng.integers(0, nd))) for h in range(0, heads, 5)]
    tiles += [(h, nd + int(c)) for h in range(heads) for c in [((h % 8) * C) // 8 + int(rng.integers(0, C // 8))]]
    hs = sorted({h for h, _ in tiles})
    sub = lambda x: to_bits(x[hs])  # noqa: E731
    qb, kb, vb, ob = sub(q), sub(k), sub(v), sub(out)
    idx_n, cnt_n = idx[hs].cpu().numpy(), cnt[hs].cpu().numpy()
    local = [(hs.index(h), tile) for h, tile in tiles]
    want = orc.attn_sparse(qb, kb, vb, idx_n, cnt_n, grid, video, n_dense, tiles=local)
    for (h, tile), (lh, _) in zip(tiles, local):
        r = orc.attn_tile_rows(grid, orc.CUBES_GRID, 0, video, n_dense, tile)
        check(ob[lh, r], want[lh, r], f"768p 40 heads: head {h} tile {tile}")
