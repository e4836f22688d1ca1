"""One H3 block through the library, every stage feeding the next on the GPU, in the order the reference's block
runs its kernels (docs/architecture.md:47-70,118-133): the modulation table from the time MLP and the AdaLN
projection; rms_mod_rows; the QKV GEMM (int8 weights); heads_partial gathered through H3::Cubes' map with cube_pool in
the same pass; cube_select; flash_attn_sparse_128; the out projection with gate_add_rows in its epilogue (after the
attention's rows go back to the model's order); rms_mod_rows; fc1 W8A16 with SwiGLU; fc2 with gate_add_rows.

Each stage is checked against the oracle run on that stage's GPU inputs (the unit tests' bars), so the chain pins
the hand-offs between the kernels: layouts, strides, the cube map, the modulation table's views. The whole block is
then checked against the oracle's own chain, run from the same inputs on the GPU's selection (a discrete choice
that float summation order may flip at near-ties), by the reference's comparison metric."""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, bits_to_f64, diff, from_bits, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu

D, HEADS, FFN, ROT = 256, 2, 512, 96
GRID, N_DENSE = (8, 8, 12), 64


def check_bits(got, want, width, what, rtol=1e-2, row_frac=1e-3):
    g, w = bits_to_f64(got).reshape(-1, width), bits_to_f64(want).reshape(-1, width)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True)) + 1e-30
    err = np.abs(g - w)
    assert np.all(err <= rtol * np.abs(w) + row_frac * scale), f"{what}: worst {(err / (np.abs(w) + scale)).max():.3g}"


def test_one_block_through_the_library(dev):
    rng = np.random.default_rng(41)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    video = GRID[0] * GRID[1] * GRID[2]
    rows = N_DENSE + video  # model rows: the text rows first, then the video grid
    # Weights: int8 projections with per-row scales (quantized from normals by the library, as at load), norms.
    def w8(n, k):
        q, s = mh.quant_rows_i8(t((0.05 * rng.standard_normal((n, k))).astype(np.float32)))
        return q, s
    wqkv, sqkv = w8(3 * HEADS * 128, D)
    wo, so = w8(D, HEADS * 128)
    w1, s1 = w8(2 * FFN, D)
    w2, s2 = w8(D, FFN)
    n1, n2 = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    qw, kw = [(1 + 0.1 * rng.standard_normal(128)).astype(np.float32) for _ in range(2)]
    ang = rng.uniform(-np.pi, np.pi, (rows, ROT // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x0 = randn_bf16_bits(rng, (rows, D))

    # The modulation table: time MLP (256 -> D -> D / 2), then the block's AdaLN projection (D / 2 -> 18 D), one level,
    # tag 0: shift, scale and gate of the attention half, then of the MLP half.
    w_in = (rng.standard_normal((D, 256)) / 16).astype(np.float32)
    w_out = (rng.standard_normal((D // 2, D)) / 16).astype(np.float32)
    b_in, b_out = np.zeros(D, np.float32), np.zeros(D // 2, np.float32)
    w_ada = orc.bf16_from_f64(0.05 * rng.standard_normal((18 * D, D // 2)))
    temb, cond = mh.time_embed(t(np.array([0.7], np.float32)), t(w_in), t(b_in), t(w_out), t(b_out))
    table = mh.adaln_mod(cond, from_bits(w_ada, dev))
    _, ocond = orc.time_embed(np.array([0.7], np.float32), w_in, b_in, w_out, b_out)
    gc, wc = bits_to_f64(to_bits(cond)), bits_to_f64(ocond)   # one bf16 step apart at most (independent roundings)
    assert np.all(np.abs(gc - wc) <= 2 ** -7 * np.abs(wc) + 1e-6 * np.abs(wc).max()), "cond"
    tab = table.view(3, 6, D)[0]                       # level 0, tag 0
    sh_a, sc_a, ga_a, sh_m, sc_m, ga_m = (tab[i].contiguous() for i in range(6))
    assert_close(table.cpu().numpy().reshape(-1), orc.adaln_mod(to_bits(cond), w_ada).reshape(-1), 1e-5,
                 1e-5 * float(np.abs(table.cpu().numpy()).max()), "modulation table")
    npv = lambda a: a.cpu().numpy()  # noqa: E731
    row = lambda a: npv(a).reshape(1, D)  # noqa: E731

    # 1. h = modulated norm of x (attention half)
    x = from_bits(x0, dev)
    h = mh.rms_mod_rows(x, t(n1), sh_a, sc_a)
    check_bits(to_bits(h), orc.rms_mod_rows(x0, n1, row(sh_a), row(sc_a)), D, "rms_mod_rows (attention)", 1e-2, 1e-5)
    # 2. QKV GEMM, int8 weights
    qkv = mh.gemm(h, wqkv, w_scale=sqkv)
    check_bits(to_bits(qkv), orc.gemm(to_bits(h), npv(wqkv), orc.GEMM_W8A16, w_scale=npv(sqkv)), 3 * HEADS * 128,
               "qkv projection", 1e-2, 1e-4)
    # 3. heads_partial through the cube map, cube_pool in the same pass
    cmap, counts = mh.cube_map(GRID, n_dense=N_DENSE, video_row0=N_DENSE, dense_row0=0, device=dev)
    cube_rows = cmap.numel()
    q, k, v, qc, kc = mh.heads_partial_pool(qkv, HEADS, GRID, t(qw), t(kw), t(cs), t(sn), rot=ROT, map=cmap)
    oq, ok, ov = orc.heads_partial(to_bits(qkv), HEADS, qw, kw, cs, sn, rot=ROT, map_=npv(cmap))
    check_bits(to_bits(q), oq, 128, "heads_partial q")
    check_bits(to_bits(k), ok, 128, "heads_partial k")
    assert np.array_equal(to_bits(v), ov), "heads_partial v"
    oqc, okc, _ = orc.cube_pool(to_bits(q), to_bits(k), HEADS, GRID, layout=orc.CUBES_GATHERED,
                                head_stride=cube_rows * 128)
    assert_close(npv(qc), oqc, 1e-5, 1e-6, "pooled q")
    assert_close(npv(kc), okc, 1e-5, 1e-6, "pooled k")
    # 4. the selection, identical to the oracle's top-k over the GPU's own scores
    kk = mh.topk_k(0.25, mh.cube_count(*GRID))
    a = mh.cube_args(HEADS, GRID, layout=mh.CUBES_GATHERED, head_stride=cube_rows * 128, k=kk, local=1)
    idx, cnt = mh.cube_select(a, qc, kc)
    widx, wcnt = orc.cube_topk(mh.cube_scores(a, qc, kc).cpu().numpy().astype(np.float64), GRID, kk, 1)
    assert np.array_equal(npv(idx), widx) and np.array_equal(npv(cnt), wcnt), "cube_select"
    # 5. sparse attention over the gathered tiles; the dense rows follow the cubes
    dense0 = cube_rows - N_DENSE
    att = mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=dense0, n_dense=N_DENSE)
    oatt = orc.attn_sparse(to_bits(q), to_bits(k), to_bits(v), npv(idx), npv(cnt), GRID, dense0, N_DENSE,
                           layout=orc.CUBES_GATHERED)
    check_bits(to_bits(att), oatt, 128, "flash_attn_sparse_128", 1e-2, 1e-2)
    # 6. back to the model's rows ([rows][heads x 128]), then the out projection with gate_add_rows
    m = npv(cmap)
    valid = np.flatnonzero(m >= 0)
    back = torch.empty((rows, HEADS, 128), dtype=torch.bfloat16, device=dev)
    back[torch.from_numpy(m[valid]).to(dev)] = att.permute(1, 0, 2)[torch.from_numpy(valid).to(dev)]
    att_rows = back.reshape(rows, HEADS * 128)
    x1_in = to_bits(x)
    x1 = mh.gemm_gate_add(att_rows, wo, x, ga_a, w_scale=so)
    check_bits(to_bits(x1), orc.gemm_gate_add(to_bits(att_rows), npv(wo), orc.GEMM_W8A16, x1_in, npv(ga_a),
                                              w_scale=npv(so)), D, "out projection + gate_add_rows", 1e-2, 1e-4)
    # 7. the MLP half: modulated norm, fc1 W8A16 + SwiGLU, fc2 + gate_add_rows
    h2 = mh.rms_mod_rows(x1, t(n2), sh_m, sc_m)
    check_bits(to_bits(h2), orc.rms_mod_rows(to_bits(x1), n2, row(sh_m), row(sc_m)), D, "rms_mod_rows (MLP)", 1e-2,
               1e-5)
    f = mh.gemm_w8a16_swiglu(h2, w1, s1)
    check_bits(to_bits(f), orc.gemm_w8a16_swiglu(to_bits(h2), npv(w1), npv(s1)), FFN, "fc1 + SwiGLU", 1e-2, 1e-4)
    x2_in = to_bits(x1)
    x2 = mh.gemm_gate_add(f, w2, x1, ga_m, w_scale=s2)
    check_bits(to_bits(x2), orc.gemm_gate_add(to_bits(f), npv(w2), orc.GEMM_W8A16, x2_in, npv(ga_m), w_scale=npv(s2)),
               D, "fc2 + gate_add_rows", 1e-2, 1e-4)

    # The whole block: the oracle's own chain from x0 (on the GPU's modulation table and selection).
    ox = x0
    oh = orc.rms_mod_rows(ox, n1, row(sh_a), row(sc_a))
    oqkv = orc.gemm(oh, npv(wqkv), orc.GEMM_W8A16, w_scale=npv(sqkv))
    oq, ok, ov = orc.heads_partial(oqkv, HEADS, qw, kw, cs, sn, rot=ROT, map_=m)
    oatt = orc.attn_sparse(oq, ok, ov, npv(idx), npv(cnt), GRID, dense0, N_DENSE, layout=orc.CUBES_GATHERED)
    oback = np.zeros((rows, HEADS, 128), np.uint16)
    oback[m[valid]] = oatt.transpose(1, 0, 2)[valid]
    ox1 = orc.gemm_gate_add(oback.reshape(rows, HEADS * 128), npv(wo), orc.GEMM_W8A16, ox, npv(ga_a), w_scale=npv(so))
    oh2 = orc.rms_mod_rows(ox1, n2, row(sh_m), row(sc_m))
    of = orc.gemm_w8a16_swiglu(oh2, npv(w1), npv(s1))
    ox2 = orc.gemm_gate_add(of, npv(w2), orc.GEMM_W8A16, ox1, npv(ga_m), w_scale=npv(s2))
    rel, cos = diff(bits_to_f64(to_bits(x2)), bits_to_f64(ox2), D)
    print(f"whole block against the oracle's chain: rel {rel:.3g}, min row cos {cos:.7f}")
    assert rel < 2e-3 and cos > 0.99999, f"whole block: rel {rel:.3g} cos {cos:.7f}"


def test_one_block_in_the_models_row_order(dev):
    """The same block with no gather or scatter, as bench.py's `block` leg runs it: heads_partial writes q, k and v as
    the model's rows ([rows][heads x 128]) with cube_pool in its pass over the grid layout, the selection and the
    attention read those rows where they lie (its query cubes in cube_order's order), and the attention's output rows
    are the out projection's input. The video grid's rows come first here and the dense rows after them."""
    rng = np.random.default_rng(43)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    npv = lambda a: a.cpu().numpy()  # noqa: E731
    video = GRID[0] * GRID[1] * GRID[2]
    rows = video + N_DENSE

    def w8(n, k):
        return mh.quant_rows_i8(t((0.05 * rng.standard_normal((n, k))).astype(np.float32)))
    wqkv, sqkv = w8(3 * HEADS * 128, D)
    wo, so = w8(D, HEADS * 128)
    w1, s1 = w8(2 * FFN, D)
    w2, s2 = w8(D, FFN)
    n1, n2 = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    sh_a, sc_a, ga_a, sh_m, sc_m, ga_m = [(0.1 * rng.standard_normal((1, D))).astype(np.float32) for _ in range(6)]
    qw, kw = [(1 + 0.1 * rng.standard_normal(128)).astype(np.float32) for _ in range(2)]
    ang = rng.uniform(-np.pi, np.pi, (rows, ROT // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x0 = randn_bf16_bits(rng, (rows, D))

    x = from_bits(x0, dev)
    h = mh.rms_mod_rows(x, t(n1), t(sh_a[0]), t(sc_a[0]))
    qkv = mh.gemm(h, wqkv, w_scale=sqkv)
    q, k, v, qc, kc = mh.heads_partial_pool(qkv, HEADS, GRID, t(qw), t(kw), t(cs), t(sn), rot=ROT, layout="rows",
                                            cube_layout=mh.CUBES_GRID)
    kk = mh.topk_k(0.25, mh.cube_count(*GRID))
    a = mh.cube_args(HEADS, GRID, head_stride=128, row_stride=HEADS * 128, k=kk, local=1)
    idx, cnt = mh.cube_select(a, qc, kc)
    order = mh.cube_order(a, idx, cnt)   # the query cubes scheduled as bench.py's block schedules them
    att = mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=N_DENSE, order=order)
    x1 = mh.gemm_gate_add(att, wo, x, t(ga_a[0]), w_scale=so)
    h2 = mh.rms_mod_rows(x1, t(n2), t(sh_m[0]), t(sc_m[0]))
    f = mh.gemm_w8a16_swiglu(h2, w1, s1)
    x2 = mh.gemm_gate_add(f, w2, x1, t(ga_m[0]), w_scale=s2)

    # The pooled means and the selection against the oracle on the GPU's own head rows.
    heads_of = lambda a_: to_bits(a_).reshape(rows, HEADS, 128).transpose(1, 0, 2)  # noqa: E731
    oqc, okc, _ = orc.cube_pool(np.ascontiguousarray(heads_of(q)), np.ascontiguousarray(heads_of(k)), HEADS, GRID,
                                layout=orc.CUBES_GRID, head_stride=rows * 128)
    assert_close(npv(qc), oqc, 1e-5, 1e-6, "pooled q (model's rows)")
    assert_close(npv(kc), okc, 1e-5, 1e-6, "pooled k (model's rows)")
    widx, wcnt = orc.cube_topk(mh.cube_scores(a, qc, kc).cpu().numpy().astype(np.float64), GRID, kk, 1)
    assert np.array_equal(npv(idx), widx) and np.array_equal(npv(cnt), wcnt), "cube_select (model's rows)"

    # The whole block against the oracle's own chain from x0, on the GPU's selection.
    row = lambda a_: a_.reshape(1, D)  # noqa: E731
    oh = orc.rms_mod_rows(x0, n1, row(sh_a), row(sc_a))
    oqkv = orc.gemm(oh, npv(wqkv), orc.GEMM_W8A16, w_scale=npv(sqkv))
    oq, ok, ov = orc.heads_partial(oqkv, HEADS, qw, kw, cs, sn, rot=ROT)
    oatt = orc.attn_sparse(oq, ok, ov, npv(idx), npv(cnt), GRID, video, N_DENSE, layout=orc.CUBES_GRID)
    oatt_rows = np.ascontiguousarray(oatt.transpose(1, 0, 2)).reshape(rows, HEADS * 128)
    check_bits(to_bits(att), oatt_rows, 128, "attention in the model's rows", 1e-2, 1e-2)
    ox1 = orc.gemm_gate_add(oatt_rows, npv(wo), orc.GEMM_W8A16, x0, ga_a, w_scale=npv(so))
    oh2 = orc.rms_mod_rows(ox1, n2, row(sh_m), row(sc_m))
    of = orc.gemm_w8a16_swiglu(oh2, npv(w1), npv(s1))
    ox2 = orc.gemm_gate_add(of, npv(w2), orc.GEMM_W8A16, ox1, ga_m, w_scale=npv(s2))
    rel, cos = diff(bits_to_f64(to_bits(x2)), bits_to_f64(ox2), D)
    print(f"whole block in the model's rows against the oracle's chain: rel {rel:.3g}, min row cos {cos:.7f}")
    assert rel < 2e-3 and cos > 0.99999, f"whole block (model's rows): rel {rel:.3g} cos {cos:.7f}"


@pytest.mark.parametrize("order", ["epilogue", "block_order"])
def test_one_block_on_the_float_residual_stream(dev, order):
    """The block in the reference's numerics (docs/architecture.md:69-70): the residual stream x stays float and only
    the GEMMs' inputs are bf16, with no cast pass. rms_mod_rows turns the float x into the bf16 row the QKV GEMM and
    fc1 take; the out projection and fc2 add gate * y into the float x in their epilogue ("epilogue"), or the out
    projection stores a bf16 y and gate_add_rms_mod_rows adds it into the float x and gives fc1's bf16 row in one pass
    ("block_order"). Rows in the model's order, as bench.py's block leg runs them. The whole block against the oracle's
    chain on the same float stream, by the reference's comparison metric."""
    rng = np.random.default_rng(47)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    npv = lambda a: a.cpu().numpy()  # noqa: E731
    video = GRID[0] * GRID[1] * GRID[2]
    rows = video + N_DENSE

    def w8(n, k):
        return mh.quant_rows_i8(t((0.05 * rng.standard_normal((n, k))).astype(np.float32)))
    wqkv, sqkv = w8(3 * HEADS * 128, D)
    wo, so = w8(D, HEADS * 128)
    w1, s1 = w8(2 * FFN, D)
    w2, s2 = w8(D, FFN)
    n1, n2 = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float32) for _ in range(2)]
    sh_a, sc_a, ga_a, sh_m, sc_m, ga_m = [(0.1 * rng.standard_normal((1, D))).astype(np.float32) for _ in range(6)]
    qw, kw = [(1 + 0.1 * rng.standard_normal(128)).astype(np.float32) for _ in range(2)]
    ang = rng.uniform(-np.pi, np.pi, (rows, ROT // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x0 = rng.standard_normal((rows, D)).astype(np.float32)

    x = t(x0)
    bf = torch.bfloat16
    h = mh.rms_mod_rows(x, t(n1), t(sh_a[0]), t(sc_a[0]), out_dtype=bf)
    qkv = mh.gemm(h, wqkv, w_scale=sqkv)
    q, k, v, qc, kc = mh.heads_partial_pool(qkv, HEADS, GRID, t(qw), t(kw), t(cs), t(sn), rot=ROT, layout="rows",
                                            cube_layout=mh.CUBES_GRID)
    kk = mh.topk_k(0.25, mh.cube_count(*GRID))
    a = mh.cube_args(HEADS, GRID, head_stride=128, row_stride=HEADS * 128, k=kk, local=1)
    idx, cnt = mh.cube_select(a, qc, kc)
    att = mh.flash_attn_sparse_128(a, q, k, v, idx, cnt, dense_row0=video, n_dense=N_DENSE)
    if order == "epilogue":
        mh.gemm_gate_add(att, wo, x, t(ga_a[0]), w_scale=so)
        h2 = mh.rms_mod_rows(x, t(n2), t(sh_m[0]), t(sc_m[0]), out_dtype=bf)
    else:
        y = mh.gemm(att, wo, w_scale=so)
        h2 = mh.gate_add_rms_mod_rows(x, y, t(ga_a[0]), t(n2), t(sh_m[0]), t(sc_m[0]), h_dtype=bf)
    assert x.dtype == torch.float32 and h2.dtype == bf
    f = mh.gemm_w8a16_swiglu(h2, w1, s1)
    mh.gemm_gate_add(f, w2, x, t(ga_m[0]), w_scale=s2)

    # The oracle's chain on the same float stream, on the GPU's selection.
    row = lambda a_: a_.reshape(1, D)  # noqa: E731
    oh = orc.rms_mod_rows(x0, n1, row(sh_a), row(sc_a), out_dtype=np.uint16)
    oqkv = orc.gemm(oh, npv(wqkv), orc.GEMM_W8A16, w_scale=npv(sqkv))
    oq, ok, ov = orc.heads_partial(oqkv, HEADS, qw, kw, cs, sn, rot=ROT)
    oatt = orc.attn_sparse(oq, ok, ov, npv(idx), npv(cnt), GRID, video, N_DENSE, layout=orc.CUBES_GRID)
    oatt_rows = np.ascontiguousarray(oatt.transpose(1, 0, 2)).reshape(rows, HEADS * 128)
    if order == "epilogue":
        ox1 = orc.gemm_gate_add(oatt_rows, npv(wo), orc.GEMM_W8A16, x0, ga_a, w_scale=npv(so))
    else:
        ox1 = orc.gate_add_rows(x0, orc.gemm(oatt_rows, npv(wo), orc.GEMM_W8A16, w_scale=npv(so)), ga_a)
    oh2 = orc.rms_mod_rows(ox1, n2, row(sh_m), row(sc_m), out_dtype=np.uint16)
    of = orc.gemm_w8a16_swiglu(oh2, npv(w1), npv(s1))
    ox2 = orc.gemm_gate_add(of, npv(w2), orc.GEMM_W8A16, ox1, ga_m, w_scale=npv(s2))
    assert ox2.dtype == np.float32
    rel, cos = diff(npv(x).astype(np.float64), ox2.astype(np.float64), D)
    print(f"whole block on the float stream ({order}) against the oracle's chain: rel {rel:.3g}, min row cos {cos:.7f}")
    assert rel < 2e-3 and cos > 0.99999, f"whole block, float stream ({order}): rel {rel:.3g} cos {cos:.7f}"
