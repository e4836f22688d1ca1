"""The hot path at MiniMax-H3's own shapes (docs/architecture.md:23,31-33,61-65; docs/performance.md:17,40-43): width
5376, 56 heads of 128, fc1 5376 -> 2 x 14,336, fc2 14,336 -> 5376, the out projection 7168 -> 5376, QKV 5376 ->
21,504, and the 1344x768 video's 37 x 24 x 42 latent grid, padded to 40 x 24 x 44 = 660 cubes, with 512 dense rows.
Sampled rows and tiles against the oracle; every output finite; the selection's invariants on every row."""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import bits_to_f64, diff, to_bits

pytestmark = pytest.mark.gpu

D, HEADS, FFN = 5376, 56, 14336
GRID = (37, 24, 42)
N_DENSE = 512


def check(got_bits, want_bits, width, what, rtol=1e-2, row_frac=1e-3):
    """Each element within rtol of itself plus row_frac of its row's RMS (attention, whose bf16 probabilities round
    against a long sum, takes the 1e-2 of the row's scale test_attn_gpu.py uses), and the diff() pair."""
    g, w = bits_to_f64(got_bits).reshape(-1, width), bits_to_f64(want_bits).reshape(-1, width)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True)) + 1e-30
    err = np.abs(g - w)
    assert np.all(err <= rtol * np.abs(w) + row_frac * scale), f"{what}: worst {(err / (np.abs(w) + scale)).max():.3g}"
    rel, cos = diff(g, w, width)
    assert rel < 5e-3 and cos > 0.9999, f"{what}: rel {rel:.3g} cos {cos:.6f}"


def sample_rows(m, n=12, seed=0):
    return np.unique(np.concatenate([[0, 255, 256, m - 1], np.random.default_rng(seed).integers(0, m, n)]))


@pytest.mark.parametrize("which", ["fc1_w8a16", "fc1_w8a8", "qkv", "out", "fc2"])
def test_h3_projections(dev, which):
    m = 3000  # rows; the kernels' row tiling is independent of m beyond the 256-row tail
    g = torch.Generator(device=dev).manual_seed(21)
    k, n = {"fc1_w8a16": (D, FFN), "fc1_w8a8": (D, FFN), "qkv": (D, 3 * HEADS * 128), "out": (HEADS * 128, D),
            "fc2": (FFN, D)}[which]
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    wrows = 2 * n if which.startswith("fc1") else n
    w = torch.randint(-127, 128, (wrows, k), generator=g, device=dev, dtype=torch.int8)
    s = (torch.rand(wrows, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
    rows = sample_rows(m)
    ri = torch.from_numpy(rows).to(dev)
    wn, sn = w.cpu().numpy(), s.cpu().numpy()
    if which == "fc1_w8a16":
        out = mh.gemm_w8a16_swiglu(x, w, s)
        want = orc.gemm_w8a16_swiglu(to_bits(x[ri]), wn, sn)
    elif which == "fc1_w8a8":
        xq, xs = mh.quant_rows_i8(x)
        out = mh.gemm_i8_swiglu(xq, xs, w, s)
        want = orc.gemm_i8_swiglu(xq[ri].cpu().numpy(), xs[ri].cpu().numpy(), wn, sn)
    elif which == "qkv":
        out = mh.gemm(x, w, w_scale=s)
        want = orc.gemm(to_bits(x[ri]), wn, orc.GEMM_W8A16, None, sn)
    else:
        res = torch.randn((m, n), generator=g, device=dev).to(torch.bfloat16)
        res0 = to_bits(res[ri])
        gate = (0.1 * torch.randn(n, generator=g, device=dev)).float()
        out = mh.gemm_gate_add(x, w, res, gate, w_scale=s)
        want = orc.gemm_gate_add(to_bits(x[ri]), wn, orc.GEMM_W8A16, res0, gate.cpu().numpy(), None, sn)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    check(to_bits(out[ri]), want, out.shape[1], f"H3 {which}")


def test_h3_rows_width_5376(dev):
    """The fused modulated norm + gated residual and SwiGLU (fc1's fused [gate | up] row) at H3's widths."""
    g = torch.Generator(device=dev).manual_seed(22)
    m = 1031
    x = torch.randn((m, D), generator=g, device=dev).to(torch.bfloat16)
    r = torch.randn((m, D), generator=g, device=dev).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(D, generator=g, device=dev)).float()
    sh, sc, ga = [(0.1 * torch.randn((1, D), generator=g, device=dev)).float() for _ in range(3)]
    got = mh.rms_mod_gate_add_rows(x, r, w, sh, sc, ga)
    want = orc.rms_mod_gate_add_rows(to_bits(x), to_bits(r), w.cpu().numpy(), sh.cpu().numpy(), sc.cpu().numpy(),
                                     ga.cpu().numpy())
    check(to_bits(got), want, D, "H3 fused rows")
    gu = torch.randn((m, 2 * FFN), generator=g, device=dev).to(torch.bfloat16)
    check(to_bits(mh.swiglu_rows(gu)), orc.swiglu_rows(to_bits(gu)), FFN, "H3 swiglu")


def test_h3_sparse_path(dev):
    """heads_partial through the cube map of the padded grid, then the selector and the sparse attention, at 56 heads
    and 660 cubes (k = 66 at ratio 0.1, local 1): the gathered heads against the oracle on sampled rows, the pooled
    means on sampled cubes, the selection's invariants on every row, and sampled attention tiles against the oracle's
    attention over the same head tiles and pass lists."""
    g = torch.Generator(device=dev).manual_seed(23)
    gt, gh, gw = GRID
    video = gt * gh * gw
    model_rows = N_DENSE + video                     # the dense rows first, then the video grid
    C = orc.cube_count(*GRID)
    assert C == 660
    qkv = torch.randn((model_rows, 3 * HEADS * 128), generator=g, device=dev).to(torch.bfloat16)
    ang = torch.rand((model_rows, 48), generator=g, device=dev) * 6.2831853 - 3.1415927
    ct, st = torch.cos(ang), torch.sin(ang)
    qw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    kw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    # The cube map (the library's mh3_cube_map, checked against the oracle's): attention row 64 c + l is cube c's slot l
    # (-1 where the padded grid has no token), then the dense rows.
    dmap, dcounts = mh.cube_map((gt, gh, gw), n_dense=N_DENSE, video_row0=N_DENSE, dense_row0=0, device=dev)
    cmap, counts = orc.cube_map((gt, gh, gw), N_DENSE, N_DENSE, 0)
    assert np.array_equal(dmap.cpu().numpy(), cmap) and np.array_equal(dcounts.cpu().numpy(), counts)
    att_rows = cmap.size
    q, k, v = mh.heads_partial(qkv, HEADS, qw, kw, ct, st, map=dmap)
    rows = np.unique(np.concatenate([np.flatnonzero(cmap < 0)[:3], np.random.default_rng(1).integers(0, att_rows, 40),
                                     [att_rows - 1]]))
    ri = torch.from_numpy(rows).to(dev)
    src = cmap[rows]
    wq, wk, wv = orc.heads_partial(to_bits(qkv[torch.from_numpy(np.maximum(src, 0)).to(dev)]), HEADS,
                                   qw.cpu().numpy(), kw.cpu().numpy(), ct[torch.from_numpy(np.maximum(src, 0)).to(dev)]
                                   .cpu().numpy(), st[torch.from_numpy(np.maximum(src, 0)).to(dev)].cpu().numpy())
    for arr in (wq, wk, wv):
        arr[:, src < 0] = 0
    check(to_bits(q[:, ri]), wq, 128, "H3 heads q")
    check(to_bits(k[:, ri]), wk, 128, "H3 heads k")
    assert np.array_equal(to_bits(v[:, ri]), wv)

    kk = mh.topk_k(0.1, C)
    assert kk == 66
    a = mh.cube_args(HEADS, GRID, layout=mh.CUBES_GATHERED, row0=0, head_stride=att_rows * 128, k=kk, local=1)
    qc, kc = mh.cube_pool(a, q, k)
    idx, cnt = mh.cube_select(a, qc, kc)
    torch.cuda.synchronize()
    # Pooled means on sampled (head, cube) pairs, from the gathered tiles.
    ent = np.random.default_rng(2).integers(0, HEADS * C, 24)
    pq, pk = orc.cube_pool_some(to_bits(q), to_bits(k), ent, GRID, att_rows * 128, layout=orc.CUBES_GATHERED)
    qcn, kcn = qc.cpu().numpy().reshape(-1, 128), kc.cpu().numpy().reshape(-1, 128)
    assert np.allclose(qcn[ent], pq, rtol=1e-5, atol=1e-6) and np.allclose(kcn[ent], pk, rtol=1e-5, atol=1e-6)
    # Every row: k or k + 1 cubes (the local cube united), ascending, unique, the query cube present.
    ic, cc = idx.cpu().numpy().reshape(HEADS * C, -1), cnt.cpu().numpy().reshape(-1)
    assert np.all((cc == kk) | (cc == kk + 1))
    for r_ in range(HEADS * C):
        sel = ic[r_, : cc[r_]]
        assert np.all(np.diff(sel) > 0) and (r_ % C) in sel and np.all(ic[r_, cc[r_]:] == -1)
    # The selection against the oracle's top-k of the GPU's own scores on sampled rows.
    s = mh.cube_scores(a, qc, kc).cpu().numpy()
    for h, i in [(0, 0), (13, 331), (55, 659), (27, 100)]:
        want, n = orc.cube_topk_row(s[h, i].astype(np.float64), i, GRID, kk, 1, idx.shape[-1])
        assert n == cc[h * C + i] and np.array_equal(ic[h * C + i], want), (h, i)

    aa = mh.cube_args(HEADS, GRID, layout=mh.CUBES_GATHERED, row0=0, head_stride=att_rows * 128,
                      out_stride=idx.shape[-1])
    out = mh.flash_attn_sparse_128(aa, q, k, v, idx, cnt, dense_row0=64 * C, n_dense=N_DENSE)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    nd = N_DENSE // 64
    tiles = [(0, 0), (55, nd - 1), (3, nd + 0), (20, nd + 330), (55, nd + C - 1), (41, nd + 123)]
    qb, kb, vb = to_bits(q), to_bits(k), to_bits(v)
    for h, tile in tiles:
        trows = orc.attn_tile_rows(GRID, orc.CUBES_GATHERED, 0, 64 * C, N_DENSE, tile)
        want = orc.attn_sparse(qb[h:h + 1], kb[h:h + 1], vb[h:h + 1], ic.reshape(HEADS, C, -1)[h:h + 1],
                               cc.reshape(HEADS, C)[h:h + 1], GRID, 64 * C, N_DENSE, orc.CUBES_GATHERED, 0,
                               tiles=[(0, tile)])
        check(to_bits(out[h:h + 1, torch.from_numpy(trows).to(dev)]), want[0, trows], 128, f"H3 attention h{h} t{tile}",
              row_frac=1e-2)
