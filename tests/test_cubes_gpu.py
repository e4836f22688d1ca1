"""Parity of the cube selector (cube_pool, cube_scores, cube_topk, cube_select) with the CPU oracle.

- Pooled means are float: 1e-5 relative (plus 1e-6 absolute, means of 64 N(0,1) values being ~0.1).
- Scores: 1e-5 relative to the row's score scale against the oracle's float64 scores.
- The GPU's top-k over its own float scores must equal the oracle's top-k over the same scores exactly (same ranking
  rule, integer output); against the oracle's float64 scores the selected sets must be identical except where the
  swapped cubes' scores tie with the k-th within 1e-3 relative.
"""
import math

import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, check_selection, from_bits, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu


def make_qk(rng, heads, rows, row_stride=128):
    q = randn_bf16_bits(rng, (heads, rows, row_stride))
    k = randn_bf16_bits(rng, (heads, rows, row_stride))
    return q, k


def pooled(dev, a, q, k):
    qc, kc = mh.cube_pool(a, from_bits(q, dev), from_bits(k, dev))
    return qc.cpu().numpy(), kc.cpu().numpy()


@pytest.mark.parametrize("grid", [(8, 8, 12), (5, 7, 9), (4, 4, 4), (1, 1, 1), (9, 13, 6)])
@pytest.mark.parametrize("layout", [mh.CUBES_GRID, mh.CUBES_GATHERED])
def test_cube_pool(dev, grid, layout):
    rng = np.random.default_rng(sum(grid))
    heads, row0 = 3, 5
    cubes = mh.cube_count(*grid)
    rows = row0 + (cubes * 64 if layout == mh.CUBES_GATHERED else grid[0] * grid[1] * grid[2]) + 3
    q, k = make_qk(rng, heads, rows)
    a = mh.cube_args(heads, grid, layout=layout, row0=row0, head_stride=rows * 128)
    counts = torch.empty(cubes, dtype=torch.int32, device=dev)
    qc, kc = mh.cube_pool(a, from_bits(q, dev), from_bits(k, dev), counts=counts)
    wq, wk, wc = orc.cube_pool(q, k, heads, grid, layout=layout, row0=row0, head_stride=rows * 128)
    assert_close(qc.cpu().numpy(), wq, 1e-5, 1e-6, "qc")
    assert_close(kc.cpu().numpy(), wk, 1e-5, 1e-6, "kc")
    assert (counts.cpu().numpy() == wc).all()


def test_cube_pool_interleaved_heads(dev):
    """q and k as a QKV projection leaves them: row-major [rows][heads * 128] (row_stride = heads * 128)."""
    rng = np.random.default_rng(11)
    heads, grid = 4, (8, 4, 8)
    rows = grid[0] * grid[1] * grid[2]
    q = randn_bf16_bits(rng, (rows, heads * 128))
    k = randn_bf16_bits(rng, (rows, heads * 128))
    a = mh.cube_args(heads, grid, head_stride=128, row_stride=heads * 128)
    qc, kc = mh.cube_pool(a, from_bits(q, dev), from_bits(k, dev))
    wq, wk, _ = orc.cube_pool(q, k, heads, grid, head_stride=128, row_stride=heads * 128)
    assert_close(qc.cpu().numpy(), wq, 1e-5, 1e-6, "qc interleaved")
    assert_close(kc.cpu().numpy(), wk, 1e-5, 1e-6, "kc interleaved")


@pytest.mark.parametrize("cubes_grid", [(8, 8, 12), (5, 7, 9), (12, 24, 44)])
def test_cube_scores(dev, cubes_grid):
    rng = np.random.default_rng(3)
    heads = 2
    cubes = mh.cube_count(*cubes_grid)
    qc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    a = mh.cube_args(heads, cubes_grid)
    s = mh.cube_scores(a, torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)).cpu().numpy()
    want = orc.cube_scores(qc, kc)
    scale = np.abs(want).max(axis=2, keepdims=True)
    assert (np.abs(s - want) <= 1e-5 * scale).all()


def test_cube_scores_special_values(dev):
    """Scores are four bf16 products of split operands unless a 16 x 16 block has a non-finite score; such a block
    (an infinite or NaN operand, or one so large that its bf16 rounding overflows) is scored by float FMAs instead.
    Against float64: +inf in q gives +-inf by k's sign along that row, NaN in k gives a NaN column, 3.4e38 in q (whose
    bf16 rounding is infinite) against keys 1e-4 small in that dimension stays finite and within 1e-5; every block
    without such an operand is unchanged."""
    rng = np.random.default_rng(21)
    grid = (16, 16, 16)  # 64 cubes: 4 x 4 blocks a head, so most blocks keep the split products
    heads, cubes = 2, mh.cube_count(*grid)
    qc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    qc[0, 3, 5] = np.inf
    kc[0, 7, 9] = np.nan
    qc[1, 10, 0] = 3.4e38
    kc[1, :, 0] *= 1e-4
    a = mh.cube_args(heads, grid)
    tq, tk = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)
    s = mh.cube_scores(a, tq, tk).cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        want = orc.cube_scores(qc, kc)
    assert (np.isnan(s) == np.isnan(want)).all()
    assert np.isnan(s[0, :, 7]).all() and np.isnan(s).sum() == cubes
    inf = np.isinf(s)
    assert (inf == np.isinf(want)).all() and inf.sum() == cubes - 1
    assert (np.sign(s[inf]) == np.sign(want[inf])).all()
    fin = np.isfinite(want)
    scale = np.abs(np.where(fin, want, 0)).max(axis=2, keepdims=True)
    err = np.abs(np.where(fin, s, 0) - np.where(fin, want, 0))
    assert (err[fin] <= (1e-5 * np.broadcast_to(scale, s.shape))[fin]).all()
    assert np.isfinite(s[1, 10]).all() and np.abs(s[1, 10]).max() > 1e30
    # The selection over these scores (no NaN: head 0 without its NaN key) equals cube_scores + cube_topk.
    kc[0, 7, 9] = 0.0
    tk = torch.from_numpy(kc).to(dev)
    a = mh.cube_args(heads, grid, k=20, local=1, out_stride=23)
    s = mh.cube_scores(a, tq, tk)
    idx, cnt = mh.cube_topk(a, s)
    sidx, scnt = mh.cube_select(a, tq, tk)
    assert (scnt.cpu() == cnt.cpu()).all() and (sidx.cpu() == idx.cpu()).all()
    widx, wcnt = orc.cube_topk(s.cpu().numpy().astype(np.float64), grid, 20, 1, out_stride=23)
    assert (cnt.cpu().numpy() == wcnt).all() and (idx.cpu().numpy() == widx).all()


@pytest.mark.parametrize("grid", [(32, 32, 128), (4, 92, 356)])
def test_select_lane_boundaries_and_outlier_keys(dev, grid):
    """The float top-k at the edges of its lane layout (32 cubes a lane, 64 lanes): 2048 cubes fill every lane, 2047
    leave one NaN slot in the last lane. Head 1's key cube 5 has 1000 times the norm of the others, so its scores
    stretch every row's range and the histogram's first level leaves t's bin over 64 scores: the search narrows to
    deeper levels. cube_select equals cube_topk over cube_scores bit for bit, and the oracle's top-k over the same
    scores on sampled rows (all rows of the 2047-cube grid's last tile)."""
    rng = np.random.default_rng(29)
    heads, cubes = 2, mh.cube_count(*grid)
    assert cubes in (2048, 2047)
    qc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc[1, 5] *= 1000.0
    k = mh.topk_k(0.1, cubes)
    a = mh.cube_args(heads, grid, k=k, local=1)
    tq, tk = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)
    s = mh.cube_scores(a, tq, tk)
    idx, cnt = mh.cube_topk(a, s)
    sidx, scnt = mh.cube_select(a, tq, tk)
    assert torch.equal(scnt, cnt) and torch.equal(sidx, idx)
    sn = s.cpu().numpy().astype(np.float64)
    rows = np.unique(np.concatenate([np.arange(cubes - 16, cubes), np.arange(0, cubes, 97)]))
    for h in range(heads):
        for i in rows:
            oi, oc = orc.cube_topk_row(sn[h, i], int(i), grid, k, 1)
            assert int(cnt[h, i]) == oc and np.array_equal(idx[h, i].cpu().numpy()[:oc], oi[:oc]), f"head {h} row {i}"


def test_select_non_finite_rows_and_workspace_reuse(dev):
    """cube_select ranks a row whose scores include +-inf or NaN as order-preserving keys (the scoring waves flag
    such rows), every other row on its floats: the selection equals cube_topk over cube_scores' scores, which takes
    the same rule from the scores in HBM. NaN in kc[0, 7] makes a NaN column in every row of head 0; +inf in
    qc[1, 3] makes row 3 of head 1 +-inf; 3.4e38 in qc[1, 10] (bf16-overflowing, scored by float FMAs) leaves row 10
    finite. Then one workspace sized for the larger call serves a smaller one after it."""
    rng = np.random.default_rng(23)
    grid = (16, 16, 32)  # 128 cubes: 8 query tiles and 8 key blocks a head
    heads, cubes = 2, mh.cube_count(*grid)
    qc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc[0, 7, 9] = np.nan
    qc[1, 3, 5] = np.inf
    qc[1, 10, 0] = 3.4e38
    kc[1, :, 0] *= 1e-4
    a = mh.cube_args(heads, grid, k=13, local=1, out_stride=14)
    tq, tk = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)
    s = mh.cube_scores(a, tq, tk)
    sn = s.cpu().numpy()
    assert np.isnan(sn[0]).any(axis=1).all() and np.isinf(sn[1, 3]).any() and np.isfinite(sn[1, 10]).all()
    idx, cnt = mh.cube_topk(a, s)
    ws = torch.empty(mh.cube_select_workspace_bytes(a), dtype=torch.uint8, device=dev)
    sidx, scnt = mh.cube_select(a, tq, tk, workspace=ws)
    assert torch.equal(scnt, cnt) and torch.equal(sidx, idx)
    small = (8, 16, 16)  # 32 cubes, in the same workspace
    a2 = mh.cube_args(1, small, k=5, local=3, out_stride=8)
    n2 = mh.cube_count(*small)
    q2, k2 = tq[0, :n2].contiguous(), tk[1, :n2].contiguous()
    assert mh.cube_select_workspace_bytes(a2) < ws.numel()
    i2, c2 = mh.cube_select(a2, q2, k2, workspace=ws)
    w2, wc2 = mh.cube_topk(a2, mh.cube_scores(a2, q2, k2))
    assert torch.equal(c2, wc2) and torch.equal(i2, w2)


@pytest.mark.parametrize("grid", [(8, 8, 12), (5, 7, 9), (16, 16, 16)])
@pytest.mark.parametrize("local", [0, 1, 3])
@pytest.mark.parametrize("ratio", [0.0001, 0.1, 0.25, 0.9, 1.0])
def test_topk_and_select_match_oracle_on_gpu_scores(dev, grid, local, ratio):
    """The GPU's selection over its own float scores is the oracle's over the same scores, bit for bit; the fused
    cube_select equals cube_scores + cube_topk; and against float64 scores only near-ties may differ."""
    rng = np.random.default_rng(int(ratio * 1000) + local)
    heads = 2
    cubes = mh.cube_count(*grid)
    k = mh.topk_k(ratio, cubes)
    qc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    a = mh.cube_args(heads, grid, k=k, local=local, out_stride=k + local + 2)
    tq, tk = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)
    s = mh.cube_scores(a, tq, tk)
    idx, cnt = mh.cube_topk(a, s)
    sidx, scnt = mh.cube_select(a, tq, tk)
    s_np = s.cpu().numpy().astype(np.float64)
    widx, wcnt = orc.cube_topk(s_np, grid, k, local, out_stride=k + local + 2)
    assert (cnt.cpu().numpy() == wcnt).all()
    assert (idx.cpu().numpy() == widx).all()
    assert (scnt.cpu().numpy() == wcnt).all()
    assert (sidx.cpu().numpy() == widx).all()
    s64 = orc.cube_scores(qc, kc)
    oidx, ocnt = orc.cube_topk(s64, grid, k, local, out_stride=k + local + 2)
    check_selection(idx.cpu().numpy(), cnt.cpu().numpy(), s64, oidx, ocnt, k)
    if ratio == 1.0:
        assert (cnt.cpu().numpy() == cubes).all()
        assert (idx.cpu().numpy()[:, :, :cubes] == np.arange(cubes)).all()


@pytest.mark.parametrize("grid", [(32, 48, 84), (52, 52, 52)])
@pytest.mark.parametrize("k", [1, 202, 1500])
def test_topk_score_shapes(dev, grid, k):
    """cube_topk over crafted rows of scores against the oracle over the same scores, exactly: normal rows, a far
    outlier above a narrow bulk (the histogram's bracket bin holds nearly every key, so the binary search takes over),
    quarter-step ties, +-inf (no histogram), a constant row, signed zeros with scores near +-3e38 (a range that
    overflows float). 2016 cubes (32 a lane) and 2197 (64 a lane)."""
    cubes = mh.cube_count(*grid)
    rng = np.random.default_rng(k)
    s = rng.standard_normal((1, cubes, cubes))
    rows = np.arange(cubes)
    kind = rows % 6
    pick = rng.integers(0, cubes, (cubes, 4))
    s[0, kind == 1] *= 1e-3
    s[0, rows[kind == 1], pick[kind == 1, 0]] = 1e3
    s[0, kind == 2] = np.round(s[0, kind == 2] * 4) / 4
    s[0, rows[kind == 3], pick[kind == 3, 0]] = np.inf
    s[0, rows[kind == 3], pick[kind == 3, 1]] = -np.inf
    s[0, kind == 4] = 0.5
    z = s[0, kind == 5]
    z[:, ::7] = 0.0
    z[:, 3::7] = -0.0
    z[:, 0], z[:, 1] = -3e38, 3e38
    s[0, kind == 5] = z
    s32 = s.astype(np.float32)
    a = mh.cube_args(1, grid, k=k, local=1)
    idx, cnt = mh.cube_topk(a, torch.from_numpy(s32).to(dev))
    widx, wcnt = orc.cube_topk(s32.astype(np.float64), grid, k, 1, sorted_form=True)
    assert (cnt.cpu().numpy() == wcnt).all()
    assert (idx.cpu().numpy() == widx).all()


def test_select_constructed_ranking_and_ties(dev):
    """Cube-constant q and k with an analytic answer: every query cube's pooled q is e0 and cube j's pooled k is
    floor(j / 2) e0 / 16 (exact in bf16), so scores rise with j in equal pairs. The top k are the highest indices;
    at an odd k the boundary pair splits and the lower index of the pair is kept."""
    grid = (8, 8, 12)
    cubes = mh.cube_count(*grid)
    heads = 1
    rows = grid[0] * grid[1] * grid[2]
    q = np.zeros((heads, rows, 128), np.float32)
    k = np.zeros((heads, rows, 128), np.float32)
    t, y, x = np.meshgrid(np.arange(grid[0]), np.arange(grid[1]), np.arange(grid[2]), indexing="ij")
    cube = ((t // 4) * (grid[1] // 4) + y // 4) * (grid[2] // 4) + x // 4
    q[0, :, 0] = 1.0
    k[0, :, 0] = (cube.reshape(-1) // 2) / 16.0
    qb = torch.from_numpy(q).to(torch.bfloat16).to(dev)
    kb = torch.from_numpy(k).to(torch.bfloat16).to(dev)
    for kk in (1, 5, 6, 12):
        a = mh.cube_args(heads, grid, k=kk, local=0)
        qc, kc = mh.cube_pool(a, qb, kb)
        idx, cnt = mh.cube_select(a, qc, kc)
        top = cubes - 1 - np.arange(kk)               # descending score pairs (c-1, c-2), (c-3, c-4)...
        if kk % 2:                                     # the split pair keeps its lower index
            top[-1] = top[-1] - 1
        want = np.sort(top)
        assert (cnt.cpu().numpy() == kk).all()
        assert (idx.cpu().numpy()[0] == want).all(), f"k={kk}"


def smooth_qk(dev, heads, grid, alpha, seed):
    """Q, K ~ N(0,1) + alpha * sum_j u_{h,j} cos(2 pi f_j . (t/T, y/Y, x/X) + phi_j): per-head random unit u,
    low integer frequencies f_j in {0..2}^3, so cube means separate above the pooled noise."""
    T, Y, X = grid
    gen = torch.Generator(device=dev).manual_seed(seed)
    rng = np.random.default_rng(seed)
    tt = torch.arange(T, device=dev, dtype=torch.float32).view(T, 1, 1) / T
    yy = torch.arange(Y, device=dev, dtype=torch.float32).view(1, Y, 1) / Y
    xx = torch.arange(X, device=dev, dtype=torch.float32).view(1, 1, X) / X
    out = []
    for _ in range(2):
        t = torch.empty((heads, T * Y * X, 128), dtype=torch.bfloat16, device=dev)
        for h in range(heads):
            acc = torch.randn((T * Y * X, 128), generator=gen, device=dev)
            for _j in range(4):
                f = rng.integers(0, 3, 3)
                phi = rng.uniform(0, 2 * math.pi)
                u = rng.standard_normal(128)
                u = torch.from_numpy(u / np.linalg.norm(u)).float().to(dev)
                wave = torch.cos(2 * math.pi * (f[0] * tt + f[1] * yy + f[2] * xx) + phi).reshape(-1, 1)
                acc += alpha * wave * u
            t[h] = acc.to(torch.bfloat16)
        out.append(t)
    return out


def test_select_768p_every_head(dev):
    """Q, K bf16 [40, 129,024, 128] on the 32x48x84 grid with the smooth component (alpha 0.5), 2016 cubes, ratio 0.1
    (k = 202), local 1.
    - Every head's pooled means against a float64 reshape-mean on the GPU.
    - Every (head, query cube)'s selection against the top k of the float64 scores of those means, plus the local
      cube: identical except where a swapped cube's score ties with the k-th within 1e-3 relative (all 80,640 rows).
    - Every (head, query cube)'s selection against torch's stable descending sort of the GPU's own scores (higher
      score first, equal scores lower index first), united with the local cube: all 80,640 rows.
    - The oracle pools two whole heads (compared for every cube) and ranks 48 query cubes of each from its float64
      scores (ties within 1e-3 may differ)."""
    heads, grid = 40, (32, 48, 84)
    q, k = smooth_qk(dev, heads, grid, 0.5, seed=0)
    cubes = mh.cube_count(*grid)
    kk = mh.topk_k(0.1, cubes)
    assert cubes == 2016 and kk == 202
    a = mh.cube_args(heads, grid, k=kk, local=1)
    qc, kc = mh.cube_pool(a, q, k)
    idx, cnt = mh.cube_select(a, qc, kc)
    torch.cuda.synchronize()
    c = cnt.cpu().numpy()
    assert ((c == kk) | (c == kk + 1)).all()
    T, Y, X = grid
    ar = torch.arange(cubes, device=dev)
    got_all = torch.zeros((heads, cubes, cubes + 1), dtype=torch.bool, device=dev)
    got_all.scatter_(2, torch.where(idx >= 0, idx, cubes).long(), True)
    differ = 0
    for h in range(heads):
        means = []
        for got, src in ((qc[h], q[h]), (kc[h], k[h])):
            want = src.double().reshape(T // 4, 4, Y // 4, 4, X // 4, 4, 128).mean((1, 3, 5)).reshape(cubes, 128)
            assert bool(((got.double() - want).abs() <= 1e-5 * want.abs() + 1e-6).all()), f"pool head {h}"
            means.append(want)
        # Every (head, query cube)'s selection against the float64 scores of the exact means: the top k plus the local
        # cube, equal except where a swapped cube's score ties with the k-th within 1e-3 relative.
        s64 = means[0] @ means[1].t() / math.sqrt(128)
        top = torch.topk(s64, kk, dim=-1)
        kth = top.values[:, -1:]
        want_h = torch.zeros((cubes, cubes), dtype=torch.bool, device=dev)
        want_h.scatter_(1, top.indices, True)
        want_h[ar, ar] = True
        swapped = got_all[h, :, :cubes] ^ want_h
        outside = swapped & ((s64 - kth).abs() > 1e-3 * kth.abs())
        assert not bool(outside.any()), \
            f"head {h}: {int(outside.sum())} selected cubes differ from the float64 top-k beyond the 1e-3 tie band"
        differ += int(swapped.any(1).sum())
    print(f"768p selection: {differ} of {heads * cubes} rows differ from the float64 top-k, all within the tie band")
    del got_all
    s = mh.cube_scores(a, qc, kc)
    order = torch.sort(s, dim=-1, descending=True, stable=True).indices[..., :kk]
    want_sel = torch.zeros((heads, cubes, cubes), dtype=torch.bool, device=dev)
    want_sel.scatter_(2, order, True)
    want_sel[:, ar, ar] = True
    del order, s
    got_sel = torch.zeros((heads, cubes, cubes + 1), dtype=torch.bool, device=dev)
    got_sel.scatter_(2, torch.where(idx >= 0, idx, cubes).long(), True)
    assert torch.equal(got_sel[..., :cubes], want_sel), "selection differs from the sorted scores"
    assert torch.equal(cnt.long(), want_sel.sum(-1))
    pos = torch.arange(idx.shape[2], device=dev)
    valid = pos[None, None, :] < cnt[..., None]
    assert bool((idx[~valid] == -1).all())
    assert bool((idx[..., 1:] > idx[..., :-1])[valid[..., 1:]].all()), "indices not ascending"
    del want_sel, got_sel
    rng = np.random.default_rng(0)
    for h in (0, heads - 1):
        qh, kh = to_bits(q[h]).reshape(1, -1, 128), to_bits(k[h]).reshape(1, -1, 128)
        wq, wk, _ = orc.cube_pool(qh, kh, 1, grid)
        assert_close(qc[h].cpu().numpy(), wq[0], 1e-5, 1e-6, f"qc head {h}")
        assert_close(kc[h].cpu().numpy(), wk[0], 1e-5, 1e-6, f"kc head {h}")
        rows = np.unique(np.concatenate([[0, cubes - 1], rng.integers(0, cubes, 46)]))
        s64 = (wq[0][rows].astype(np.float64) @ wk[0].astype(np.float64).T) / math.sqrt(128)
        oidx = np.empty((len(rows), kk + 1), np.int32)
        ocnt = np.empty(len(rows), np.int32)
        for n, i in enumerate(rows):
            oidx[n], ocnt[n] = orc.cube_topk_row(s64[n], int(i), grid, kk, 1)
        gi = idx[h].cpu().numpy()[rows]
        gc = c[h][rows]
        check_selection(gi, gc, s64, oidx, ocnt, kk)


@pytest.mark.parametrize("local", [1, 3])
def test_topk_beyond_2048_cubes(dev, local):
    """52 x 52 x 52 grid: 13^3 = 2197 cubes, the 64-cubes-a-lane top-k. The GPU's selection over its own scores is the
    oracle's over the same scores; cube_select refuses more than 2048 cubes (its LDS tile holds 2048)."""
    rng = np.random.default_rng(31 + local)
    heads, grid = 1, (52, 52, 52)
    cubes = mh.cube_count(*grid)
    assert cubes == 2197
    kk = mh.topk_k(0.1, cubes)
    qc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    kc = rng.standard_normal((heads, cubes, 128)).astype(np.float32)
    a = mh.cube_args(heads, grid, k=kk, local=local)
    tq, tk = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)
    s = mh.cube_scores(a, tq, tk)
    idx, cnt = mh.cube_topk(a, s)
    widx, wcnt = orc.cube_topk(s.cpu().numpy().astype(np.float64), grid, kk, local)
    assert (cnt.cpu().numpy() == wcnt).all()
    assert (idx.cpu().numpy() == widx).all()
    with pytest.raises(RuntimeError):
        mh.cube_select(a, tq, tk)
