"""Pins the CPU oracle (oracle/mh3_oracle.c). The reference holds no vectors for these ops (their implementation is
in the absent mako-common submodule), so each oracle function is checked against a library routine or a brute force
written independently of it, and against closed forms and invariants chosen so that a plausible slip (a dropped
"1 +", gate and up swapped, a transposed operand, an off-by-one cube index, a wrong tie rule) fails one of them.
The committed fixtures under tests/golden/ are checked here too."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc
from helpers import bits_to_f64, randn_bf16_bits

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- bf16 rounding -----------------------------------------------------------------------------------------------

def test_bf16_from_float_matches_torch():
    """float -> bf16 nearest-even equals torch's conversion on every float pattern class."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    bits = bits[((bits >> 23) & 0xFF) != 0xFF]            # finite values
    f = bits.view(np.float32)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([orc.bf16_from_float(float(v)) for v in f[:20000]], np.uint16)
    assert (got == want[:20000]).all()


def test_bf16_from_double_is_nearest_even():
    """For random doubles (and exact halfway cases) the result is the nearest bf16, ties to the even significand."""
    rng = np.random.default_rng(1)
    d = rng.standard_normal(100000) * np.exp(rng.uniform(-20, 20, 100000))
    got = orc.bf16_from_f64(d)
    g = bits_to_f64(got)
    up = bits_to_f64(got + np.uint16(1))
    dn = bits_to_f64(got - np.uint16(1))
    err = np.abs(d - g)
    assert (err <= np.abs(d - up)).all() and (err <= np.abs(d - dn)).all()
    # halfway between two bf16 values: 1 + 2^-8 lies between 1 and 1 + 2^-7; even is 1.0
    half = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8)])
    assert list(orc.bf16_from_f64(half)) == [0x3F80, 0x3F82, 0xBF80]
    # a double just above the halfway point rounds up (a float path would round it to the halfway point first)
    assert orc.bf16_from_f64(np.array([1 + 2**-8 + 2**-40]))[0] == 0x3F81


# ---- rows --------------------------------------------------------------------------------------------------------

def params(rng, dim, n_sets=1):
    shift = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    scale = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    gate = (rng.standard_normal((n_sets, dim)) * 0.1).astype(np.float32)
    w = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    return w, shift, scale, gate


def torch_mod_rms(x64, w, shift, scale, eps):
    n = torch.nn.functional.rms_norm(torch.from_numpy(x64), (x64.shape[1],), torch.from_numpy(w.astype(np.float64)),
                                     eps=eps).numpy()
    return n * (1 + scale.astype(np.float64)) + shift.astype(np.float64)


def test_rms_mod_rows_matches_torch_rms_norm():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 1024)).astype(np.float32)
    w, shift, scale, _ = params(rng, 1024)
    got = orc.rms_mod_rows(x, w, shift, scale, 1e-6)
    want = torch_mod_rms(x.astype(np.float64), w, shift[0], scale[0], 1e-6)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_rms_mod_rows_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 512)).astype(np.float32) * 5
    zero = np.zeros((1, 512), np.float32)
    ones = np.ones(512, np.float32)
    y = orc.rms_mod_rows(x, ones, zero, zero, 1e-12).astype(np.float64)
    assert np.allclose(np.sqrt((y ** 2).mean(1)), 1.0, atol=1e-6)          # unit RMS
    y2 = orc.rms_mod_rows((x * 3).astype(np.float32), ones, zero, zero, 1e-12)
    assert np.allclose(y2, y, rtol=1e-6, atol=1e-6)                         # scale invariance
    sc = np.full((1, 512), -1.0, np.float32)
    sh = rng.standard_normal((1, 512)).astype(np.float32)
    assert (orc.rms_mod_rows(x, ones, sh, sc, 1e-6) == sh).all()            # scale -1 leaves the shift


def test_rms_mod_rows_bf16_is_rounded_float64():
    rng = np.random.default_rng(4)
    x = randn_bf16_bits(rng, (16, 256))
    w, shift, scale, _ = params(rng, 256)
    got = orc.rms_mod_rows(x, w, shift, scale, 1e-6)
    want = orc.bf16_from_f64(torch_mod_rms(bits_to_f64(x), w, shift[0], scale[0], 1e-6))
    assert (np.abs(got.astype(np.int32) - want.astype(np.int32)) <= 1).all()
    assert (got == want).mean() > 0.99


def test_fused_is_residual_plus_gate_times_mod_rms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((32, 768)).astype(np.float32)
    res = rng.standard_normal((32, 768)).astype(np.float32)
    w, shift, scale, gate = params(rng, 768, 2)
    sets = rng.integers(0, 2, 32).astype(np.uint8)
    got = orc.rms_mod_gate_add_rows(x, res, w, shift, scale, gate, 1e-6, sets)
    want = res.astype(np.float64) + gate[sets] * torch_mod_rms(x.astype(np.float64), w, shift[sets], scale[sets], 1e-6)
    assert np.abs(got - want).max() <= 1e-5
    zero_gate = np.zeros_like(gate)
    assert (orc.rms_mod_gate_add_rows(x, res, w, shift, scale, zero_gate, 1e-6, sets) == res).all()
    # gate_add alone: x + gate * y
    y = rng.standard_normal((32, 768)).astype(np.float32)
    ga = orc.gate_add_rows(res, y, gate, sets)
    assert np.abs(ga - (res.astype(np.float64) + gate[sets] * y)).max() <= 1e-6


# ---- swiglu ------------------------------------------------------------------------------------------------------

def test_swiglu_matches_torch_silu():
    rng = np.random.default_rng(6)
    g = (rng.standard_normal((16, 200)) * 4).astype(np.float32)
    u = rng.standard_normal((16, 200)).astype(np.float32)
    want = torch.nn.functional.silu(torch.from_numpy(g.astype(np.float64))).numpy() * u
    assert np.abs(orc.swiglu_rows(g, u) - want).max() <= 1e-6 * np.abs(want).max()
    fused = np.concatenate([g, u], axis=1)                  # [gate | up]
    assert (orc.swiglu_rows(fused) == orc.swiglu_rows(g, u)).all()
    assert not np.allclose(orc.swiglu_rows(u, g), orc.swiglu_rows(g, u))   # the halves are not interchangeable


def test_swiglu_special_values():
    g = np.array([[0.0, 50.0, -50.0, 1.0]], np.float32)
    u = np.array([[5.0, 2.0, 2.0, 0.0]], np.float32)
    out = orc.swiglu_rows(g, u)
    assert out[0, 0] == 0 and out[0, 1] == 100.0 and abs(out[0, 2]) < 1e-19 and out[0, 3] == 0


# ---- cubes -------------------------------------------------------------------------------------------------------

def numpy_pool(x, grid):
    """Mean over 4x4x4 cubes of a [rows][hd] tensor in grid order, by reshaping (grid dims multiples of 4)."""
    T, Y, X = grid
    v = x.astype(np.float64).reshape(T // 4, 4, Y // 4, 4, X // 4, 4, -1)
    return v.mean(axis=(1, 3, 5)).reshape(-1, x.shape[-1])


def test_cube_pool_matches_reshape_mean():
    rng = np.random.default_rng(7)
    grid, heads = (8, 12, 16), 2
    rows = grid[0] * grid[1] * grid[2]
    q, k = randn_bf16_bits(rng, (heads, rows, 128)), randn_bf16_bits(rng, (heads, rows, 128))
    qc, kc, counts = orc.cube_pool(q, k, heads, grid)
    for h in range(heads):
        assert np.abs(qc[h] - numpy_pool(bits_to_f64(q[h]), grid)).max() < 1e-6
        assert np.abs(kc[h] - numpy_pool(bits_to_f64(k[h]), grid)).max() < 1e-6
    assert (counts == 64).all()


def brute_pool(x, grid):
    """Cube means by visiting every grid position (pads included as absent), cube id (ct*ch + cy)*cw + cx."""
    T, Y, X = grid
    ch, cw = (Y + 3) // 4, (X + 3) // 4
    C = ((T + 3) // 4) * ch * cw
    acc = np.zeros((C, x.shape[-1]))
    n = np.zeros(C)
    for t in range(T):
        for y in range(Y):
            for xx in range(X):
                c = ((t // 4) * ch + y // 4) * cw + xx // 4
                acc[c] += x[(t * Y + y) * X + xx]
                n[c] += 1
    return acc / n[:, None], n


def test_cube_pool_padded_grid_brute_force():
    rng = np.random.default_rng(8)
    grid = (5, 7, 9)
    rows = 5 * 7 * 9
    q, k = randn_bf16_bits(rng, (1, rows, 128)), randn_bf16_bits(rng, (1, rows, 128))
    qc, kc, counts = orc.cube_pool(q, k, 1, grid)
    want, n = brute_pool(bits_to_f64(q[0]), grid)
    assert np.abs(qc[0] - want).max() < 1e-6
    assert (counts == n).all()


def gather_rows(x, grid):
    """Grid-order rows -> cube-order rows (64 per cube, (dt, dy, dx) inside), padding rows left as garbage (7.0)."""
    T, Y, X = grid
    ch, cw = (Y + 3) // 4, (X + 3) // 4
    C = ((T + 3) // 4) * ch * cw
    out = np.full((C * 64, x.shape[-1]), 0x40E0, np.uint16)   # bf16 7.0 in every padding row
    for t in range(T):
        for y in range(Y):
            for xx in range(X):
                c = ((t // 4) * ch + y // 4) * cw + xx // 4
                out[c * 64 + ((t % 4) * 4 + y % 4) * 4 + xx % 4] = x[(t * Y + y) * X + xx]
    return out


def test_cube_pool_gathered_equals_grid():
    """The cube-gathered layout pools to the same means as the grid layout; padding rows are skipped by position."""
    rng = np.random.default_rng(9)
    grid = (6, 5, 10)
    rows = 6 * 5 * 10
    q, k = randn_bf16_bits(rng, (1, rows, 128)), randn_bf16_bits(rng, (1, rows, 128))
    qa, ka, _ = orc.cube_pool(q, k, 1, grid)
    qg, kg = gather_rows(q[0], grid)[None], gather_rows(k[0], grid)[None]
    qb, kb, _ = orc.cube_pool(np.ascontiguousarray(qg), np.ascontiguousarray(kg), 1, grid, layout=orc.CUBES_GATHERED)
    assert (qa == qb).all() and (ka == kb).all()


def test_cube_pool_permutation_invariant_inside_a_cube():
    rng = np.random.default_rng(10)
    grid = (4, 4, 8)
    rows = 128
    q, k = randn_bf16_bits(rng, (1, rows, 128)), randn_bf16_bits(rng, (1, rows, 128))
    qa, _, _ = orc.cube_pool(q, k, 1, grid)
    # swap two rows of cube 0: (0,0,0) and (3,3,3)
    q2 = q.copy()
    a, b = 0, (3 * 4 + 3) * 8 + 3
    q2[0, [a, b]] = q2[0, [b, a]]
    qb, _, _ = orc.cube_pool(q2, k, 1, grid)
    assert np.abs(qa - qb).max() < 1e-6


def test_cube_scores_matches_matmul():
    rng = np.random.default_rng(11)
    qc = rng.standard_normal((2, 40, 128)).astype(np.float32)
    kc = rng.standard_normal((2, 40, 128)).astype(np.float32)
    s = orc.cube_scores(qc, kc)
    want = np.einsum("hid,hjd->hij", qc.astype(np.float64), kc.astype(np.float64)) / math.sqrt(128)
    assert np.abs(s - want).max() < 1e-12
    assert not np.allclose(s, np.swapaxes(s, 1, 2))        # q and k are not interchangeable


def numpy_topk(s, k, local, grid, i):
    order = np.lexsort((np.arange(s.size), -s))             # score descending, then index ascending
    sel = set(order[:k].tolist())
    T, Y, X = grid
    plane = ((Y + 3) // 4) * ((X + 3) // 4)
    cth = (T + 3) // 4
    if local >= 1:
        sel.add(i)
    if local == 3:
        if i // plane > 0:
            sel.add(i - plane)
        if i // plane + 1 < cth:
            sel.add(i + plane)
    return np.array(sorted(sel), np.int32)


@pytest.mark.parametrize("local", [0, 1, 3])
@pytest.mark.parametrize("k", [1, 3, 20, 48])
def test_cube_topk_matches_lexsort(local, k):
    rng = np.random.default_rng(12 + k + local)
    grid = (12, 16, 16)                                      # 3 x 4 x 4 = 48 cubes
    C = orc.cube_count(*grid)
    s = rng.integers(-5, 5, (2, C, C)).astype(np.float64)    # many exact ties
    idx, cnt = orc.cube_topk(s, grid, k, local, out_stride=k + 4)
    for h in range(2):
        for i in range(C):
            want = numpy_topk(s[h, i], k, local, grid, i)
            assert cnt[h, i] == len(want)
            assert (idx[h, i, : cnt[h, i]] == want).all()
            assert (idx[h, i, cnt[h, i]:] == -1).all()


@pytest.mark.parametrize("local,k", [(0, 1), (1, 7), (3, 12), (1, 48)])
def test_cube_topk_sorted_form_equals_count_form(local, k):
    """The sort-a-row selection the CPU baseline times selects exactly what the O(C^2) count does."""
    rng = np.random.default_rng(40 + k + local)
    grid = (12, 16, 16)
    for s in (rng.integers(-3, 3, (2, 48, 48)).astype(np.float64), rng.standard_normal((2, 48, 48))):
        a_idx, a_cnt = orc.cube_topk(s, grid, k, local, out_stride=k + 4)
        b_idx, b_cnt = orc.cube_topk(s, grid, k, local, out_stride=k + 4, sorted_form=True)
        assert (a_cnt == b_cnt).all() and (a_idx == b_idx).all()


def test_cube_topk_ratio_one_selects_everything():
    rng = np.random.default_rng(13)
    grid = (8, 8, 8)
    C = orc.cube_count(*grid)
    s = rng.standard_normal((1, C, C))
    idx, cnt = orc.cube_topk(s, grid, C, 1)
    assert (cnt == C).all() and (idx[:, :, :C] == np.arange(C)).all()


def test_cube_topk_analytic_ranking():
    """Scores rising with j in equal pairs: the top k are the highest indices, a split pair keeps its lower one."""
    grid = (8, 8, 12)
    C = orc.cube_count(*grid)
    s = np.tile((np.arange(C) // 2).astype(np.float64), (1, C, 1))
    idx, cnt = orc.cube_topk(s, grid, 5, 0)
    assert list(idx[0, 0, :5]) == [C - 6, C - 4, C - 3, C - 2, C - 1]


# ---- int8 --------------------------------------------------------------------------------------------------------

def test_quant_rows_i8_invariants():
    rng = np.random.default_rng(14)
    w = (rng.standard_normal((50, 320)) * 0.02).astype(np.float32)
    w[3] = 0
    q, s = orc.quant_rows_i8(w)
    assert np.abs(q.astype(np.int32)).max() <= 127
    nz = np.arange(50) != 3
    assert (np.abs(q[nz]).max(1) == 127).all()                       # the row maximum maps to +-127
    assert (np.abs(w - q * s[:, None]) <= s[:, None] / 2 * (1 + 1e-6)).all()
    assert s[3] == 0 and (q[3] == 0).all()
    want = np.clip(np.rint(w[nz] / s[nz, None].astype(np.float32)), -127, 127)
    assert (q[nz] == want).all()


def test_gemm_w8a16_swiglu_matches_torch_matmul():
    rng = np.random.default_rng(15)
    m, n, k = 9, 24, 80
    x = randn_bf16_bits(rng, (m, k))
    w = rng.integers(-127, 128, (2 * n, k), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, 2 * n).astype(np.float32)
    got = orc.gemm_w8a16_swiglu(x, w, s)
    y = torch.from_numpy(bits_to_f64(x)) @ (torch.from_numpy(w.astype(np.float64)).T * torch.from_numpy(
        s.astype(np.float64)))
    want = torch.nn.functional.silu(y[:, :n]) * y[:, n:]
    assert (got == orc.bf16_from_f64(want.numpy())).all()


def test_gemm_exact_integers():
    """x small integers, w in {-1, 0, 1}, s = 1: y is exact; with gate rows giving y_gate = 40 (silu(40) = 40 to
    within 2^-52 relative), out = bf16(40 * y_up) exactly."""
    rng = np.random.default_rng(16)
    m, n, k = 6, 8, 64
    xf = rng.integers(-2, 3, (m, k)).astype(np.float32)
    xf[:, 0] = 1.0
    x = torch.from_numpy(xf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    w = np.zeros((2 * n, k), np.int8)
    w[:n, 0] = 40                                  # gate: 40 * x[:, 0] = 40
    w[n:] = rng.integers(-1, 2, (n, k), dtype=np.int8)
    s = np.ones(2 * n, np.float32)
    got = bits_to_f64(orc.gemm_w8a16_swiglu(x, w, s))
    up = xf.astype(np.float64) @ w[n:].T.astype(np.float64)
    assert (got == 40 * up).all()


def test_gemm_bf16_swiglu_matches_torch_matmul():
    rng = np.random.default_rng(17)
    m, n, k = 7, 16, 96
    x = randn_bf16_bits(rng, (m, k))
    w = orc.bf16_from_f64(rng.standard_normal((2 * n, k)) * 0.05)
    got = orc.gemm_bf16_swiglu(x, w)
    y = torch.from_numpy(bits_to_f64(x)) @ torch.from_numpy(bits_to_f64(w)).T
    want = torch.nn.functional.silu(y[:, :n]) * y[:, n:]
    assert (got == orc.bf16_from_f64(want.numpy())).all()


def test_gemm_bf16_exact_integers():
    """As for the int8 GEMM: gate rows giving 40 and up rows in {-1, 0, 1} make out = bf16(40 * y_up) exactly; the
    gate and up halves must not be swapped (a swap gives silu(y_up) * 40)."""
    rng = np.random.default_rng(18)
    m, n, k = 5, 8, 64
    xf = rng.integers(-2, 3, (m, k)).astype(np.float32)
    xf[:, 0] = 1.0
    x = orc.bf16_from_f64(xf.astype(np.float64))
    wf = np.zeros((2 * n, k))
    wf[:n, 0] = 40.0
    wf[n:] = rng.integers(-1, 2, (n, k))
    got = bits_to_f64(orc.gemm_bf16_swiglu(x, orc.bf16_from_f64(wf)))
    up = xf.astype(np.float64) @ wf[n:].T
    assert (got == 40 * up).all()


def test_gemm_i8_swiglu_matches_torch_matmul():
    rng = np.random.default_rng(19)
    m, n, k = 6, 16, 96
    x = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (2 * n, k), dtype=np.int8)
    sx = rng.uniform(0.005, 0.05, m).astype(np.float32)
    sw = rng.uniform(0.5e-3, 2e-3, 2 * n).astype(np.float32)
    got = orc.gemm_i8_swiglu(x, sx, w, sw)
    y = (torch.from_numpy(x.astype(np.int64)) @ torch.from_numpy(w.astype(np.int64)).T).double()
    y = y * torch.from_numpy(sx.astype(np.float64))[:, None] * torch.from_numpy(sw.astype(np.float64))[None, :]
    want = torch.nn.functional.silu(y[:, :n]) * y[:, n:]
    assert (got == orc.bf16_from_f64(want.numpy())).all()


def test_gemm_i8_exact_integers():
    """Unit scales, gate rows giving 40, up rows in {-1, 0, 1}: out = bf16(40 * y_up) exactly."""
    rng = np.random.default_rng(20)
    m, n, k = 5, 8, 128
    x = rng.integers(-2, 3, (m, k), dtype=np.int8)
    x[:, 0] = 1
    w = np.zeros((2 * n, k), np.int8)
    w[:n, 0] = 40
    w[n:] = rng.integers(-1, 2, (n, k), dtype=np.int8)
    got = bits_to_f64(orc.gemm_i8_swiglu(x, np.ones(m, np.float32), w, np.ones(2 * n, np.float32)))
    up = x.astype(np.float64) @ w[n:].T.astype(np.float64)
    assert (got == 40 * up).all()


# ---- committed fixtures --------------------------------------------------------------------------------------------

def test_golden_fixtures_reproduce():
    """The fixtures under tests/golden/ (inputs and the oracle's outputs when they were written, by
    tests/golden/make_golden.py) still come out of the oracle unchanged."""
    import make_golden
    manifest = json.loads((GOLDEN / "manifest.json").read_text())
    assert manifest["cases"], "no fixtures"
    for case in manifest["cases"]:
        data = np.load(GOLDEN / case["file"])
        got = make_golden.run_case(case, data)
        for name, arr in got.items():
            assert (arr == data[name]).all(), f"{case['name']}: {name} changed"


# ---- the float residual stream with bf16 GEMM rows ------------------------------------------------------------------

def test_rms_mod_rows_float_to_bf16_is_rounded_float64():
    """A float x normed into the bf16 row a GEMM takes: torch's float64 rms_norm restatement, rounded once to bf16
    (within half a bf16 step of it, and equal to torch's own rounding nearly everywhere); set rows pick their sets."""
    rng = np.random.default_rng(40)
    x = rng.standard_normal((48, 768)).astype(np.float32)
    w, shift, scale, _ = params(rng, 768, 3)
    sets = rng.integers(0, 3, 48).astype(np.uint8)
    got = orc.rms_mod_rows(x, w, shift, scale, 1e-6, sets, out_dtype=np.uint16)
    assert got.dtype == np.uint16
    want = torch_mod_rms(x.astype(np.float64), w, shift[sets], scale[sets], 1e-6)
    g = bits_to_f64(got)
    assert np.all(np.abs(g - want) <= 2 ** -8 * np.abs(want) + 1e-30)
    tb = torch.from_numpy(want).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (got == tb).mean() > 0.999
    # the float output of the same rows, rounded to bf16, is the same row (one rounding either way, from double)
    f = orc.rms_mod_rows(x, w, shift, scale, 1e-6, sets)
    assert np.abs(bits_to_f64(got) - f.astype(np.float64)).max() <= 2 ** -8 * np.abs(f).max()


def test_gate_add_rows_float_x_bf16_y():
    """x (float) += gate * y (bf16): y's bf16 values decoded exactly (gate 1 and x 0 give y's values bit for bit),
    gate 0 leaves x bit-exact, and the sum matches float64 within half a float step."""
    rng = np.random.default_rng(41)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    y = randn_bf16_bits(rng, (16, 512))
    gate = (0.1 * rng.standard_normal((2, 512))).astype(np.float32)
    sets = rng.integers(0, 2, 16).astype(np.uint8)
    got = orc.gate_add_rows(x, y, gate, sets)
    assert got.dtype == np.float32
    want = x.astype(np.float64) + gate[sets].astype(np.float64) * bits_to_f64(y)
    assert np.all(np.abs(got - want) <= 2 ** -24 * np.abs(want))
    assert (orc.gate_add_rows(x, y, np.zeros_like(gate), sets) == x).all()
    ones = np.ones((1, 512), np.float32)
    assert (orc.gate_add_rows(np.zeros_like(x), y, ones) == bits_to_f64(y).astype(np.float32)).all()
