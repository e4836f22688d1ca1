"""Parity of heads_partial with the oracle (bf16 outputs within 1e-2 relative of the row's scale, v and padding rows
bit-exact), its gather through a cube map against cube_pool's grid layout, in-place use, and its error paths."""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import bits_to_f64, diff, from_bits, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu


def check(got_bits, want_bits, what):
    g, w = bits_to_f64(got_bits).reshape(-1, 128), bits_to_f64(want_bits).reshape(-1, 128)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True)) + 1e-30
    err = np.abs(g - w)
    assert np.all(err <= 1e-2 * (np.abs(w) + scale)), f"{what}: worst {(err / (np.abs(w) + scale)).max():.3g}"
    rel, cos = diff(g, w, 128)
    assert rel < 5e-3 and cos > 0.9999, f"{what}: rel {rel:.3g} cos {cos:.6f}"


def make(rng, rows, heads, rot, extra=0, weights=True):
    qkv = randn_bf16_bits(rng, (rows, 3 * heads * 128 + extra), 1.5)
    ang = rng.uniform(-np.pi, np.pi, (rows, rot // 2))
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    w = [(1 + 0.1 * rng.standard_normal(128)).astype(np.float32) if weights else None for _ in range(2)]
    return qkv, w[0], w[1], cos_t, sin_t


def dev_args(dev, qkv, q_w, k_w, cos_t, sin_t):
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return from_bits(qkv, dev), t(q_w), t(k_w), t(cos_t), t(sin_t)


CASES = [
    # rows, heads, rot, extra columns, weights, with v
    (1, 1, 96, 0, True, True),
    (37, 2, 96, 0, True, True),
    (130, 5, 128, 8, False, True),
    (64, 3, 16, 0, True, False),
    (45, 40, 96, 0, True, True),
    (9, 56, 96, 24, True, True),
    (200, 1, 0, 0, True, False),
]


@pytest.mark.parametrize("rows,heads,rot,extra,weights,with_v", CASES)
def test_heads_partial_matches_oracle(dev, rows, heads, rot, extra, weights, with_v):
    rng = np.random.default_rng(rows + 13 * heads + rot)
    qkv, q_w, k_w, cos_t, sin_t = make(rng, rows, heads, rot, extra, weights)
    want = orc.heads_partial(qkv, heads, q_w, k_w, cos_t, sin_t, rot=rot, with_v=with_v)
    got = mh.heads_partial(*dev_args(dev, qkv, q_w, k_w, cos_t, sin_t)[:1], heads,
                           *dev_args(dev, qkv, q_w, k_w, cos_t, sin_t)[1:], rot=rot, with_v=with_v)
    for name, g, w in zip("qk", got[:2], want[:2]):
        check(to_bits(g), w, f"{name} rows {rows} heads {heads} rot {rot}")
    if with_v:
        assert np.array_equal(to_bits(got[2]), want[2])
    else:
        assert got[2] is None


def test_heads_partial_rows_layout_and_in_place(dev):
    rng = np.random.default_rng(5)
    rows, heads, rot = 77, 4, 96
    qkv, q_w, k_w, cos_t, sin_t = make(rng, rows, heads, rot)
    x, qw, kw, ct, st = dev_args(dev, qkv, q_w, k_w, cos_t, sin_t)
    hq, hk, hv = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot)
    rq, rk, rv = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot, layout="rows")
    for h_, r_ in ((hq, rq), (hk, rk), (hv, rv)):
        assert torch.equal(h_.view(torch.int16), r_.view(rows, heads, 128).permute(1, 0, 2).view(torch.int16))
    # In place: q and k written over their own columns of qkv (v left where it is).
    y = x.clone()
    third = heads * 128
    a = mh.HeadsArgs()
    a.rows, a.model_rows, a.heads, a.head_dim, a.rot, a.eps = rows, rows, heads, 128, rot, 1e-6
    a.qkv_stride, a.out_head_stride, a.out_row_stride = 3 * third, 128, 3 * third
    p = y.data_ptr()
    rc = mh.lib.mh3_heads_partial(mh.C.byref(a), p, qw.data_ptr(), kw.data_ptr(), ct.data_ptr(), st.data_ptr(), None,
                                  p, p + 2 * third, None, mh._stream())
    assert rc == mh.OK
    torch.cuda.synchronize()
    assert torch.equal(y[:, :third].view(torch.int16), rq.view(torch.int16))
    assert torch.equal(y[:, third:2 * third].view(torch.int16), rk.view(torch.int16))
    assert torch.equal(y[:, 2 * third:].view(torch.int16), x[:, 2 * third:].view(torch.int16))


@pytest.mark.parametrize("grid", [(8, 8, 12), (7, 9, 10)])
def test_heads_partial_cube_map_feeds_pool_and_attention(dev, grid):
    rng = np.random.default_rng(sum(grid))
    heads, rot, n_dense = 2, 96, 70
    video = grid[0] * grid[1] * grid[2]
    rows = n_dense + video  # text rows first, then the video rows (row0 = n_dense)
    qkv, q_w, k_w, cos_t, sin_t = make(rng, rows, heads, rot)
    x, qw, kw, ct, st = dev_args(dev, qkv, q_w, k_w, cos_t, sin_t)
    dm, _ = mh.cube_map(grid, n_dense=n_dense, video_row0=n_dense, dense_row0=0, device=dev)
    m = dm.cpu().numpy()
    assert np.array_equal(m, orc.cube_map(grid, n_dense, n_dense, 0)[0])
    gq, gk, gv = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot, map=dm)
    fq, fk, fv = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot)
    C = orc.cube_count(*grid)
    for g, f in ((gq, fq), (gk, fk), (gv, fv)):
        valid = torch.from_numpy(m >= 0).to(dev)
        idx = torch.from_numpy(np.maximum(m, 0).astype(np.int64)).to(dev)
        assert torch.equal(g[:, valid].view(torch.int16), f[:, idx[valid]].view(torch.int16))
        assert (g[:, ~valid].view(torch.int16) == 0).all()
    # The gathered tiles pool to the same cube means as the model-order rows in the grid layout.
    ag = mh.cube_args(heads, grid, layout=mh.CUBES_GATHERED, row0=0, head_stride=(64 * C + n_dense) * 128)
    ar = mh.cube_args(heads, grid, layout=mh.CUBES_GRID, row0=n_dense, head_stride=rows * 128)
    qc_g, kc_g = mh.cube_pool(ag, gq, gk)
    qc_r, kc_r = mh.cube_pool(ar, fq, fk)
    assert torch.equal(qc_g, qc_r) and torch.equal(kc_g, kc_r)
    # Attention over the gathered tiles equals attention over the model-order rows, row for row.
    idx, cnt = mh.cube_select(mh.cube_args(heads, grid, k=4, local=1, layout=mh.CUBES_GRID, row0=n_dense,
                                           head_stride=rows * 128), qc_r, kc_r)
    out_g = mh.flash_attn_sparse_128(mh.cube_args(heads, grid, layout=mh.CUBES_GATHERED, row0=0,
                                                  head_stride=(64 * C + n_dense) * 128, out_stride=idx.shape[-1]),
                                     gq, gk, gv, idx, cnt, dense_row0=64 * C, n_dense=n_dense)
    out_r = mh.flash_attn_sparse_128(mh.cube_args(heads, grid, layout=mh.CUBES_GRID, row0=n_dense,
                                                  head_stride=rows * 128, out_stride=idx.shape[-1]),
                                     fq, fk, fv, idx, cnt, dense_row0=0, n_dense=n_dense)
    valid = np.flatnonzero(m >= 0)
    got = to_bits(out_g)[:, valid]
    want = to_bits(out_r)[:, m[valid]]
    check(got, want, f"gathered vs grid attention {grid}")


def test_heads_partial_768p_sampled(dev):
    """The 768p shape: 129,536 model rows (512 text + 32 x 48 x 84 video), 40 heads; sampled rows against the oracle,
    every output finite, v bit-exact on the sample."""
    rows, heads, rot = 512 + 32 * 48 * 84, 40, 96
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((rows, 3 * heads * 128), generator=g, device=dev).to(torch.bfloat16)
    ang = torch.rand((rows, rot // 2), generator=g, device=dev) * 6.283 - 3.1416
    ct, st = torch.cos(ang), torch.sin(ang)
    qw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    kw = 1 + 0.1 * torch.randn(128, generator=g, device=dev)
    q, k, v = mh.heads_partial(x, heads, qw, kw, ct, st, rot=rot)
    torch.cuda.synchronize()
    for t in (q, k):
        assert bool(torch.isfinite(t).all())
    sample = np.unique(np.concatenate([np.arange(4), np.arange(rows - 4, rows),
                                       np.random.default_rng(0).integers(0, rows, 60)]))
    si = torch.from_numpy(sample).to(dev)
    xs = to_bits(x[si])
    want = orc.heads_partial(xs, heads, qw.cpu().numpy(), kw.cpu().numpy(), ct[si].cpu().numpy(),
                             st[si].cpu().numpy(), rot=rot)
    check(to_bits(q[:, si]), want[0], "q 768p")
    check(to_bits(k[:, si]), want[1], "k 768p")
    assert np.array_equal(to_bits(v[:, si]), want[2])


def test_heads_partial_rejects_bad_calls(dev):
    x = torch.zeros((8, 3 * 2 * 128), dtype=torch.bfloat16, device=dev)
    ct = torch.zeros((8, 48), device=dev)
    q = torch.empty((2, 8, 128), dtype=torch.bfloat16, device=dev)

    def call(**kw):
        a = mh.HeadsArgs()
        a.rows, a.model_rows, a.heads, a.head_dim, a.rot, a.eps = 8, 8, 2, 128, 96, 1e-6
        a.qkv_stride, a.out_head_stride, a.out_row_stride = 768, 8 * 128, 128
        ptrs = dict(qkv=x.data_ptr(), cos=ct.data_ptr(), sin=ct.data_ptr(), q=q.data_ptr(), k=q.data_ptr() + 0)
        for key, val in kw.items():
            if hasattr(a, key):
                setattr(a, key, val)
            else:
                ptrs[key] = val
        return mh.lib.mh3_heads_partial(mh.C.byref(a), ptrs["qkv"], None, None, ptrs["cos"], ptrs["sin"], None,
                                        ptrs["q"], ptrs["k"], None, mh._stream())

    assert call(rot=24) == mh.ERR_PARAM
    assert call(rot=144) == mh.ERR_PARAM
    assert call(head_dim=64) == mh.ERR_UNSUPPORTED
    assert call(eps=0.0) == mh.ERR_PARAM
    assert call(qkv_stride=700) == mh.ERR_SHAPE
    assert call(model_rows=4) == mh.ERR_SHAPE
    assert call(cos=None) == mh.ERR_POINTER
    assert call(q=x.data_ptr() + 256) == mh.ERR_PARAM  # over qkv, not in place
    assert call(q=q.data_ptr() + 2) == mh.ERR_ALIGN
    with pytest.raises(RuntimeError):
        mh.heads_partial(x, 2, None, None, ct, ct, rot=40)
