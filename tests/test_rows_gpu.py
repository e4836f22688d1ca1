"""Parity of the row kernels (rms_mod_rows, gate_add_rows, fused rms_mod_gate_add_rows) with the CPU oracle.

Tolerances: float rows 1e-5 relative (plus 1e-6 absolute for outputs that cancel to ~0); bf16 rows 1e-2 relative
(plus 1e-5 absolute) -- both the kernel and the oracle round once, so they differ by at most one bf16 ulp (2^-8).
"""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import assert_close, bits_to_f64, check_rows_f64, diff, from_bits, nan_filled, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu

BF16_RTOL, BF16_ATOL = 1e-2, 1e-5
F32_RTOL, F32_ATOL = 1e-5, 1e-6


def mod_params(rng, dim, n_sets=1):
    shift = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    scale = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    gate = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    w = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    return w, shift, scale, gate


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_rms_mod_rows_f32_4096x1024(dev):
    """x[4096,1024] ~ N(0,1); shift, scale ~ N(0,0.1); w = 1 + N(0,0.02); eps 1e-6; seed 0; fp32 at 1e-5."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4096, 1024)).astype(np.float32)
    w, shift, scale, _ = mod_params(rng, 1024)
    want = orc.rms_mod_rows(x, w, shift, scale, 1e-6)
    got = mh.rms_mod_rows(dev_t(x, dev), dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev), eps=1e-6)
    got = got.cpu().numpy()
    assert_close(got, want, F32_RTOL, F32_ATOL, "rms_mod_rows f32")
    rel, cos = diff(got, want, 1024)
    assert rel < 1e-6 and cos > 1 - 1e-9


@pytest.mark.parametrize("dim", [8, 64, 520, 1024, 5120, 5376])
@pytest.mark.parametrize("rows", [1, 3, 67])
def test_fused_bf16(dev, dim, rows):
    rng = np.random.default_rng(dim * 1000 + rows)
    x = randn_bf16_bits(rng, (rows, dim))
    res = randn_bf16_bits(rng, (rows, dim))
    w, shift, scale, gate = mod_params(rng, dim)
    want = orc.rms_mod_gate_add_rows(x, res, w, shift, scale, gate, 1e-6)
    got = mh.rms_mod_gate_add_rows(from_bits(x, dev), from_bits(res, dev), dev_t(w, dev), dev_t(shift, dev),
                                   dev_t(scale, dev), dev_t(gate, dev))
    assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, f"fused {rows}x{dim}")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("n_sets,dim", [(3, 5376), (9, 5120)])
def test_fused_per_row_sets(dev, dtype, n_sets, dim):
    """Rows pick their (level, tag) set through set_of_row; 9 sets of 5120 exceed the LDS coefficient table and take
    the global-memory path."""
    rng = np.random.default_rng(n_sets)
    rows = 50
    if dtype == "bf16":
        x, res = randn_bf16_bits(rng, (rows, dim)), randn_bf16_bits(rng, (rows, dim))
        tx, tr = from_bits(x, dev), from_bits(res, dev)
    else:
        x = rng.standard_normal((rows, dim)).astype(np.float32)
        res = rng.standard_normal((rows, dim)).astype(np.float32)
        tx, tr = dev_t(x, dev), dev_t(res, dev)
    w, shift, scale, gate = mod_params(rng, dim, n_sets)
    sets = rng.integers(0, n_sets, rows).astype(np.uint8)
    want = orc.rms_mod_gate_add_rows(x, res, w, shift, scale, gate, 1e-6, sets)
    got = mh.rms_mod_gate_add_rows(tx, tr, dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev), dev_t(gate, dev),
                                   set_of_row=dev_t(sets, dev), n_sets=n_sets)
    if dtype == "bf16":
        assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, "fused sets bf16")
    else:
        assert_close(got.cpu().numpy(), want, F32_RTOL, F32_ATOL, "fused sets f32")


def test_fused_gate_zero_is_residual(dev):
    """gate = 0 leaves the residual bit-exact, whatever x is."""
    rng = np.random.default_rng(1)
    x, res = randn_bf16_bits(rng, (33, 5120), 7.0), randn_bf16_bits(rng, (33, 5120))
    w, shift, scale, _ = mod_params(rng, 5120)
    gate = np.zeros((1, 5120), np.float32)
    got = mh.rms_mod_gate_add_rows(from_bits(x, dev), from_bits(res, dev), dev_t(w, dev), dev_t(shift, dev),
                                   dev_t(scale, dev), dev_t(gate, dev))
    assert (to_bits(got) == res).all()


def test_fused_in_place(dev):
    """out may be the residual buffer itself."""
    rng = np.random.default_rng(2)
    x, res = randn_bf16_bits(rng, (40, 5120)), randn_bf16_bits(rng, (40, 5120))
    w, shift, scale, gate = mod_params(rng, 5120)
    want = orc.rms_mod_gate_add_rows(x, res, w, shift, scale, gate)
    tres = from_bits(res, dev)
    mh.rms_mod_gate_add_rows(from_bits(x, dev), tres, dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev),
                             dev_t(gate, dev), out=tres)
    assert_close(bits_to_f64(to_bits(tres)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, "fused in place")


@pytest.mark.parametrize("dim", [64, 5120, 5376])
def test_rms_mod_rows_bf16(dev, dim):
    rng = np.random.default_rng(dim)
    x = randn_bf16_bits(rng, (29, dim), 3.0)
    w, shift, scale, _ = mod_params(rng, dim)
    want = orc.rms_mod_rows(x, w, shift, scale)
    got = mh.rms_mod_rows(from_bits(x, dev), dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev))
    assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, "rms_mod bf16")


def test_rms_mod_rows_without_weight(dev):
    """w = NULL means a weight of ones."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    _, shift, scale, _ = mod_params(rng, 256)
    ones = np.ones(256, np.float32)
    want = orc.rms_mod_rows(x, ones, shift, scale)
    got = mh.rms_mod_rows(dev_t(x, dev), None, dev_t(shift, dev), dev_t(scale, dev)).cpu().numpy()
    assert_close(got, want, F32_RTOL, F32_ATOL, "rms_mod no weight")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_gate_add_rows(dev, dtype):
    rng = np.random.default_rng(3)
    rows, dim, n_sets = 45, 5376, 2
    sets = rng.integers(0, n_sets, rows).astype(np.uint8)
    gate = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    if dtype == "bf16":
        x, y = randn_bf16_bits(rng, (rows, dim)), randn_bf16_bits(rng, (rows, dim))
        tx, ty = from_bits(x, dev), from_bits(y, dev)
    else:
        x = rng.standard_normal((rows, dim)).astype(np.float32)
        y = rng.standard_normal((rows, dim)).astype(np.float32)
        tx, ty = dev_t(x, dev), dev_t(y, dev)
    want = orc.gate_add_rows(x, y, gate, sets)
    mh.gate_add_rows(tx, ty, dev_t(gate, dev), set_of_row=dev_t(sets, dev), n_sets=n_sets)
    if dtype == "bf16":
        assert_close(bits_to_f64(to_bits(tx)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, "gate_add bf16")
    else:
        assert_close(tx.cpu().numpy(), want, F32_RTOL, F32_ATOL, "gate_add f32")


def test_zero_rows_is_a_no_op(dev):
    x = torch.empty((0, 5120), dtype=torch.bfloat16, device=dev)
    p = torch.zeros(5120, dtype=torch.float32, device=dev)
    out = mh.rms_mod_gate_add_rows(x, x, p, p, p, p)
    assert out.shape == (0, 5120)


def test_fused_768p_every_row(dev):
    """The 768p-shaped workload: N = 32x48x84 + 512 = 129,536 rows x 5120, x and residual ~ N(0,1), shift, scale,
    gate ~ N(0,0.1), w = 1 + N(0,0.02), into a NaN-filled output. Every element is checked against a float64
    restatement on the GPU over the same operands (1e-2 relative plus 1e-5 of the row's RMS), so a row the kernel's
    row-to-wave mapping skips or writes from the wrong row fails; 384 rows spread over the whole range (both ends
    included) are also checked against the oracle."""
    rows, dim = 129536, 5120
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((rows, dim), generator=g, device=dev).to(torch.bfloat16)
    res = torch.randn((rows, dim), generator=g, device=dev).to(torch.bfloat16)
    rng = np.random.default_rng(0)
    w, shift, scale, gate = mod_params(rng, dim)
    out = mh.rms_mod_gate_add_rows(x, res, dev_t(w, dev), dev_t(shift, dev), dev_t(scale, dev), dev_t(gate, dev),
                                   out=nan_filled((rows, dim), dev))
    wd, shd, scd, gad = (dev_t(a, dev).double().reshape(1, dim) for a in (w, shift, scale, gate))
    for r0 in range(0, rows, 8192):
        xs = x[r0:r0 + 8192].double()
        y = xs * torch.rsqrt(xs.pow(2).mean(1, keepdim=True) + 1e-6) * wd * (1 + scd) + shd
        want = res[r0:r0 + 8192].double() + gad * y
        check_rows_f64(out[r0:r0 + 8192], want, f"fused 768p rows {r0}..", BF16_RTOL, BF16_ATOL)
    pick = np.unique(np.concatenate([[0, 1, rows - 1], rng.integers(0, rows, 381)]))
    ti = torch.from_numpy(pick).to(dev)
    xs, rs, os_ = to_bits(x[ti]), to_bits(res[ti]), to_bits(out[ti])
    want = orc.rms_mod_gate_add_rows(xs, rs, w, shift, scale, gate)
    assert_close(bits_to_f64(os_), bits_to_f64(want), BF16_RTOL, BF16_ATOL, "fused 768p rows")
    rel, cos = diff(bits_to_f64(os_), bits_to_f64(want), dim)
    assert rel < 3e-3 and cos > 0.9999


@pytest.mark.parametrize("dim", [20480, 32768])
def test_wide_rows_four_vectors_a_thread(dev, dim):
    """Rows of more than 16,384 bf16 (2048 vectors) take the workgroup-per-row kernel with 4 vectors a thread; the
    widest accepted row is 4096 vectors."""
    rng = np.random.default_rng(dim)
    rows = 5
    x, res = randn_bf16_bits(rng, (rows, dim)), randn_bf16_bits(rng, (rows, dim))
    w, shift, scale, gate = mod_params(rng, dim)
    want = orc.rms_mod_gate_add_rows(x, res, w, shift, scale, gate, 1e-6)
    got = mh.rms_mod_gate_add_rows(from_bits(x, dev), from_bits(res, dev), dev_t(w, dev), dev_t(shift, dev),
                                   dev_t(scale, dev), dev_t(gate, dev))
    assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, f"fused {rows}x{dim}")
    tx = from_bits(res, dev)
    h = mh.gate_add_rms_mod_rows(tx, from_bits(x, dev), dev_t(gate, dev), dev_t(w, dev), dev_t(shift, dev),
                                 dev_t(scale, dev))
    want_x = orc.gate_add_rows(res, x, gate)
    assert_close(bits_to_f64(to_bits(tx)), bits_to_f64(want_x), BF16_RTOL, BF16_ATOL, f"block order x {dim}")
    want_h = orc.rms_mod_rows(to_bits(tx), w, shift, scale, 1e-6)
    assert_close(bits_to_f64(to_bits(h)), bits_to_f64(want_h), BF16_RTOL, BF16_ATOL, f"block order h {dim}")


def test_row_wider_than_4096_vectors_is_unsupported(dev):
    x = torch.zeros((2, 32776), dtype=torch.bfloat16, device=dev)
    ones = torch.ones(32776, device=dev)
    with pytest.raises(RuntimeError):
        mh.rms_mod_rows(x, ones, ones.view(1, -1), ones.view(1, -1))


@pytest.mark.parametrize("dim", [1024, 5120])
def test_modulation_table_views(dev, dim):
    """shift, scale and gate read straight from a [U][3][6][D] modulation table (sets 6 D floats apart; slots 0-2
    the attention half's shift, scale, gate, 3-5 the MLP half's) give, bit for bit, what contiguous copies of the
    same vectors give, for all four row ops. 6 sets of 1024 use the LDS coefficient table, 6 of 5120 global memory."""
    rng = np.random.default_rng(dim + 6)
    U, rows = 2, 70
    table = torch.from_numpy((0.1 * rng.standard_normal((U, 3, 6, dim))).astype(np.float32)).to(dev)
    w = dev_t((1 + 0.02 * rng.standard_normal(dim)).astype(np.float32), dev)
    sets = dev_t(rng.integers(0, U * 3, rows).astype(np.uint8), dev)
    x = from_bits(randn_bf16_bits(rng, (rows, dim)), dev)
    y = from_bits(randn_bf16_bits(rng, (rows, dim)), dev)
    sh, sc, ga = table[:, :, 3], table[:, :, 4], table[:, :, 5]             # [U][3][D] views, 6 D floats apart
    c_sh, c_sc, c_ga = [t.reshape(U * 3, dim).contiguous() for t in (sh, sc, ga)]
    kw = dict(set_of_row=sets, n_sets=U * 3)
    same = lambda a, b: torch.equal(a.view(torch.int16), b.view(torch.int16))  # noqa: E731
    assert same(mh.rms_mod_rows(x, w, sh, sc, **kw), mh.rms_mod_rows(x, w, c_sh, c_sc, **kw))
    assert same(mh.rms_mod_gate_add_rows(x, y, w, sh, sc, ga, **kw), mh.rms_mod_gate_add_rows(x, y, w, c_sh, c_sc,
                                                                                              c_ga, **kw))
    x1, x2 = x.clone(), x.clone()
    mh.gate_add_rows(x1, y, ga, **kw)
    mh.gate_add_rows(x2, y, c_ga, **kw)
    assert same(x1, x2)
    x1, x2 = x.clone(), x.clone()
    h1 = mh.gate_add_rms_mod_rows(x1, y, ga, w, sh, sc, **kw)
    h2 = mh.gate_add_rms_mod_rows(x2, y, c_ga, w, c_sh, c_sc, **kw)
    assert same(x1, x2) and same(h1, h2)
    want = orc.rms_mod_gate_add_rows(to_bits(x), to_bits(y), w.cpu().numpy(), c_sh.cpu().numpy(), c_sc.cpu().numpy(),
                                     c_ga.cpu().numpy(), 1e-6, sets.cpu().numpy())
    got = mh.rms_mod_gate_add_rows(x, y, w, sh, sc, ga, **kw)
    assert_close(bits_to_f64(to_bits(got)), bits_to_f64(want), BF16_RTOL, BF16_ATOL, "table views vs oracle")


def test_modulation_table_views_refused_when_uneven(dev):
    """Vectors whose sets are not evenly spaced, or whose strides differ, are refused before any launch."""
    t = torch.zeros((2, 3, 6, 64), device=dev)
    x = torch.zeros((4, 64), device=dev)
    with pytest.raises(ValueError):
        mh.rms_mod_rows(x, None, t[:, :, 0, :].transpose(0, 1), t[:, :, 1, :].transpose(0, 1), n_sets=6)
    with pytest.raises(ValueError):
        mh.rms_mod_rows(x, None, t[:, :, 0, :], t.reshape(36, 64)[:6], n_sets=6)
