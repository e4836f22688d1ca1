"""TEST INFRASTRUCTURE ONLY: numpy binding of the CPU oracle (mh3_oracle.c), for tests/, the smoke check and
bench.py's CPU-baseline leg. The product never imports this module.

bf16 arrays are numpy uint16 (the raw bits). Each function mirrors one oracle entry point; see mh3_oracle.h for the
reference file each follows and how each is pinned.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmh3_oracle.so"
F32, BF16 = 0, 1
SWIGLU_SPLIT, SWIGLU_FUSED = 0, 1
CUBES_GRID, CUBES_GATHERED = 0, 1


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "libmh3_oracle.so"], check=True)
    return LIB_PATH


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    return C.CDLL(str(LIB_PATH))


_lib = _load()
_P = C.c_void_p
_lib.mh3o_bf16_from_double.restype = C.c_uint16
_lib.mh3o_bf16_from_double.argtypes = [C.c_double]
_lib.mh3o_bf16_from_float.restype = C.c_uint16
_lib.mh3o_bf16_from_float.argtypes = [C.c_float]
_lib.mh3o_cube_count.restype = C.c_int64
_lib.mh3o_cube_count.argtypes = [C.c_uint32] * 3
_lib.mh3o_cube_topk_row.restype = C.c_int32
_lib.mh3o_cube_topk_row.argtypes = [C.c_uint32] * 6 + [C.c_uint64, _P, _P]
_lib.mh3o_rms_mod_rows.argtypes = [C.c_uint32, C.c_uint32, C.c_float, C.c_int] + [_P] * 6
_lib.mh3o_gate_add_rows.argtypes = [C.c_uint32, C.c_uint32, C.c_int] + [_P] * 4
_lib.mh3o_rms_mod_gate_add_rows.argtypes = [C.c_uint32, C.c_uint32, C.c_float, C.c_int] + [_P] * 8
_lib.mh3o_swiglu_rows.argtypes = [C.c_uint32, C.c_uint32, C.c_int, C.c_int] + [_P] * 3
_lib.mh3o_cube_pool.argtypes = [C.c_uint32] * 5 + [C.c_int, C.c_uint64, C.c_uint64, C.c_uint64] + [_P] * 5
_lib.mh3o_cube_pool_some.argtypes = [C.c_uint32] * 4 + [C.c_int, C.c_uint64, C.c_uint64, C.c_uint64] + \
    [_P, _P, _P, C.c_uint64, _P, _P]
_lib.mh3o_cube_scores.argtypes = [C.c_uint32] * 3 + [_P] * 3
_lib.mh3o_cube_topk.argtypes = [C.c_uint32] * 7 + [_P] * 3
_lib.mh3o_cube_topk_sorted.argtypes = [C.c_uint32] * 7 + [_P] * 3
_ATTN_GEOM = [C.c_uint32] * 3 + [C.c_int, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, C.c_double]
_lib.mh3o_attn_sparse_tile.argtypes = _ATTN_GEOM + [_P] * 5 + [C.c_uint32, C.c_uint32, C.c_uint64, _P]
_lib.mh3o_attn_sparse.argtypes = [C.c_uint32] + _ATTN_GEOM + [_P] * 5 + [C.c_uint32, _P]
_lib.mh3o_heads_partial.argtypes = [C.c_uint32] * 4 + [C.c_float] + [C.c_uint64] * 3 + [_P] * 9
_lib.mh3o_quant_rows_i8.argtypes = [C.c_uint32, C.c_uint32, C.c_int] + [_P] * 3
_lib.mh3o_gemm_w8a16_swiglu.argtypes = [C.c_uint32] * 3 + [_P] * 4
_lib.mh3o_gemm_bf16_swiglu.argtypes = [C.c_uint32] * 3 + [_P] * 3
_lib.mh3o_gemm_i8_swiglu.argtypes = [C.c_uint32] * 3 + [_P] * 5
_lib.mh3o_gemm.argtypes = [C.c_uint32] * 3 + [C.c_int] * 2 + [_P] * 6 + [C.c_uint32, _P]
_lib.mh3o_rms_mod_rows2.argtypes = [C.c_uint32, C.c_uint32, C.c_float, C.c_int, C.c_int] + [_P] * 6
_lib.mh3o_gate_add_rows2.argtypes = [C.c_uint32, C.c_uint32, C.c_int, C.c_int] + [_P] * 4
_lib.mh3o_cube_map.restype = C.c_int64
_lib.mh3o_cube_map.argtypes = [C.c_uint32] * 4 + [C.c_uint64, C.c_uint64, _P, _P]
_lib.mh3o_time_embed.argtypes = [C.c_uint32] * 4 + [C.c_double] + [_P] * 7
_lib.mh3o_adaln_mod.argtypes = [C.c_uint32] * 3 + [_P] * 4
_lib.mh3o_curve_mods.argtypes = [C.c_uint32] * 4 + [_P] * 5
_lib.mh3o_bf16_to_float_n.argtypes = [_P, _P, C.c_uint64]
_lib.mh3o_bf16_from_double_n.argtypes = [_P, _P, C.c_uint64]


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.uint16:
        return BF16
    if a.dtype == np.float32:
        return F32
    raise ValueError(f"oracle rows are float32 or bf16 bits (uint16), not {a.dtype}")


# ---- bf16 ------------------------------------------------------------------------------------------------------------

def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    _lib.mh3o_bf16_to_float_n(_p(a), _p(out), a.size)
    return out


def bf16_from_f64(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float64)
    out = np.empty(a.shape, np.uint16)
    _lib.mh3o_bf16_from_double_n(_p(a), _p(out), a.size)
    return out


def bf16_from_float(f: float) -> int:
    return int(_lib.mh3o_bf16_from_float(C.c_float(f)))


# ---- rows ------------------------------------------------------------------------------------------------------------

def rms_mod_rows(x, w, shift, scale, eps=1e-6, set_of_row=None, out_dtype=None):
    """x float32 or bf16 bits; y of x's type, or of out_dtype (np.uint16: bf16 bits) for a float x."""
    rows, dim = x.shape
    y = np.empty(x.shape, out_dtype or x.dtype)
    _lib.mh3o_rms_mod_rows2(rows, dim, eps, _dtype_code(x), _dtype_code(y), _p(x), _p(w), _p(shift), _p(scale),
                            _p(set_of_row), _p(y))
    return y


def gate_add_rows(x, y, gate, set_of_row=None):
    """x + gate * y, in x's type (y may be bf16 bits with a float x)."""
    x = x.copy()
    rows, dim = x.shape
    _lib.mh3o_gate_add_rows2(rows, dim, _dtype_code(x), _dtype_code(y), _p(x), _p(np.ascontiguousarray(y)), _p(gate),
                             _p(set_of_row))
    return x


def rms_mod_gate_add_rows(x, residual, w, shift, scale, gate, eps=1e-6, set_of_row=None):
    rows, dim = x.shape
    out = np.empty_like(x)
    _lib.mh3o_rms_mod_gate_add_rows(rows, dim, eps, _dtype_code(x), _p(x), _p(residual), _p(w), _p(shift), _p(scale),
                                    _p(gate), _p(set_of_row), _p(out))
    return out


def swiglu_rows(gate, up=None):
    if up is None:
        rows, two = gate.shape
        dim, layout = two // 2, SWIGLU_FUSED
    else:
        rows, dim = gate.shape
        layout = SWIGLU_SPLIT
    out = np.empty((rows, dim), gate.dtype)
    _lib.mh3o_swiglu_rows(rows, dim, layout, _dtype_code(gate), _p(gate), _p(up), _p(out))
    return out


# ---- cubes -----------------------------------------------------------------------------------------------------------

def cube_count(gt, gh, gw) -> int:
    return int(_lib.mh3o_cube_count(gt, gh, gw))


def cube_pool(q, k, heads, grid, layout=CUBES_GRID, row0=0, head_stride=None, row_stride=128, head_dim=128):
    gt, gh, gw = grid
    C_ = cube_count(gt, gh, gw)
    if head_stride is None:
        rows = row0 + (C_ * 64 if layout == CUBES_GATHERED else gt * gh * gw)
        head_stride = rows * row_stride
    qc = np.empty((heads, C_, head_dim), np.float32)
    kc = np.empty((heads, C_, head_dim), np.float32)
    counts = np.empty(C_, np.int32)
    _lib.mh3o_cube_pool(heads, head_dim, gt, gh, gw, layout, row0, head_stride, row_stride, _p(q), _p(k), _p(qc),
                        _p(kc), _p(counts))
    return qc, kc, counts


def cube_pool_some(q, k, entries, grid, head_stride, layout=CUBES_GRID, row0=0, row_stride=128, head_dim=128):
    gt, gh, gw = grid
    entries = np.ascontiguousarray(entries, dtype=np.int64)
    qc = np.empty((len(entries), head_dim), np.float32)
    kc = np.empty((len(entries), head_dim), np.float32)
    _lib.mh3o_cube_pool_some(head_dim, gt, gh, gw, layout, row0, head_stride, row_stride, _p(q), _p(k), _p(entries),
                             len(entries), _p(qc), _p(kc))
    return qc, kc


def cube_scores(qc, kc):
    heads, cubes, hd = qc.shape
    s = np.empty((heads, cubes, cubes), np.float64)
    _lib.mh3o_cube_scores(heads, cubes, hd, _p(np.ascontiguousarray(qc)), _p(np.ascontiguousarray(kc)), _p(s))
    return s


def cube_topk(s, grid, k, local, out_stride=None, sorted_form=False):
    """sorted_form: the O(C log C) a row selection (mh3o_cube_topk_sorted) instead of the O(C^2) count."""
    heads, cubes, _ = s.shape
    out_stride = k + local if out_stride is None else out_stride
    idx = np.empty((heads, cubes, out_stride), np.int32)
    cnt = np.empty((heads, cubes), np.int32)
    fn = _lib.mh3o_cube_topk_sorted if sorted_form else _lib.mh3o_cube_topk
    fn(heads, *grid, k, local, out_stride, _p(np.ascontiguousarray(s, dtype=np.float64)), _p(idx), _p(cnt))
    return idx, cnt


def cube_topk_row(row_scores, i, grid, k, local, out_stride=None):
    out_stride = k + local if out_stride is None else out_stride
    row = np.ascontiguousarray(row_scores, dtype=np.float64)
    out = np.empty(out_stride, np.int32)
    n = _lib.mh3o_cube_topk_row(*grid, k, local, out_stride, i, _p(row), _p(out))
    return out, int(n)


# ---- heads_partial -----------------------------------------------------------------------------------------------------

def heads_partial(qkv, heads, q_w=None, k_w=None, cos_t=None, sin_t=None, rot=96, eps=1e-6, map_=None, with_v=True):
    """qkv bf16 bits [model_rows][>= 3 heads 128] -> (q, k, v) bf16 bits [heads][rows][128] (v None without with_v):
    per-head RMS norm and rotary on q and k, v copied, output row r from model row map_[r] (or r)."""
    model_rows, stride = qkv.shape
    rows = model_rows if map_ is None else len(map_)
    qkv = np.ascontiguousarray(qkv, dtype=np.uint16)
    m = None if map_ is None else np.ascontiguousarray(map_, dtype=np.int32)
    f = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
    q_w, k_w, cos_t, sin_t = f(q_w), f(k_w), f(cos_t), f(sin_t)
    outs = [np.empty((heads, rows, 128), np.uint16) for _ in range(3 if with_v else 2)] + ([] if with_v else [None])
    _lib.mh3o_heads_partial(rows, model_rows, heads, rot, eps, stride, rows * 128, 128, _p(qkv), _p(q_w), _p(k_w),
                            _p(cos_t), _p(sin_t), _p(m), *(_p(a) for a in outs))
    return tuple(outs)


# ---- int8 ------------------------------------------------------------------------------------------------------------

def quant_rows_i8(w):
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    _lib.mh3o_quant_rows_i8(rows, cols, _dtype_code(w), _p(w), _p(q), _p(s))
    return q, s


def gemm_bf16_swiglu(x, w):
    """x bf16 bits [m][k], w bf16 bits [2n][k] -> silu(x w_gate^T) * (x w_up^T), bf16 bits [m][n]."""
    m, k = x.shape
    n = w.shape[0] // 2
    out = np.empty((m, n), np.uint16)
    _lib.mh3o_gemm_bf16_swiglu(m, n, k, _p(np.ascontiguousarray(x)), _p(np.ascontiguousarray(w)), _p(out))
    return out


def gemm_i8_swiglu(x, x_scale, w, w_scale):
    """x int8 [m][k] with x_scale f32 [m], w int8 [2n][k] with w_scale f32 [2n] -> bf16 bits [m][n]."""
    m, k = x.shape
    n = w.shape[0] // 2
    out = np.empty((m, n), np.uint16)
    _lib.mh3o_gemm_i8_swiglu(m, n, k, _p(np.ascontiguousarray(x)), _p(np.ascontiguousarray(x_scale)),
                             _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(w_scale)), _p(out))
    return out


def gemm_w8a16_swiglu(x, w, scale):
    m, k = x.shape
    n = w.shape[0] // 2
    out = np.empty((m, n), np.uint16)
    _lib.mh3o_gemm_w8a16_swiglu(m, n, k, _p(np.ascontiguousarray(x)), _p(np.ascontiguousarray(w)),
                                _p(np.ascontiguousarray(scale)), _p(out))
    return out


GEMM_W8A16, GEMM_BF16, GEMM_W8A8 = 0, 1, 2


def gemm(x, w, form, x_scale=None, w_scale=None):
    """y = x w^T rounded to bf16 bits [m][n]: form GEMM_W8A16 (x bf16 bits, w int8, w_scale), GEMM_BF16 (both bf16
    bits) or GEMM_W8A8 (x int8 with x_scale, w int8 with w_scale)."""
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.uint16)
    c = np.ascontiguousarray
    _lib.mh3o_gemm(m, n, k, form, 0, _p(c(x)), _p(None if x_scale is None else c(x_scale, dtype=np.float32)),
                   _p(c(w)), _p(None if w_scale is None else c(w_scale, dtype=np.float32)), None, None, 0, _p(out))
    return out


def gemm_gate_add(x, w, form, residual, gate, x_scale=None, w_scale=None, set_of_row=None):
    """residual + gate[set(row)] * (x w^T), one rounding to bf16 bits (or to float for a float32 residual); gate f32
    [n_sets][n] (or [n])."""
    m, k = x.shape
    n = w.shape[0]
    f32 = np.asarray(residual).dtype == np.float32
    out = np.array(residual, dtype=np.float32 if f32 else np.uint16, copy=True, order="C")
    c = np.ascontiguousarray
    g = c(gate, dtype=np.float32).reshape(-1, n)
    _lib.mh3o_gemm(m, n, k, form, 2 if f32 else 1, _p(c(x)), _p(None if x_scale is None else c(x_scale, dtype=np.float32)),
                   _p(c(w)), _p(None if w_scale is None else c(w_scale, dtype=np.float32)), _p(g),
                   _p(None if set_of_row is None else c(set_of_row, dtype=np.uint8)), n, _p(out))
    return out


# ---- flash_attn_sparse_128 ---------------------------------------------------------------------------------------------

def attn_sparse(q, k, v, idx, cnt, grid, dense_row0, n_dense, layout=CUBES_GRID, row0=0, scale=None, tiles=None,
                out=None):
    """Sparse attention of q, k, v bf16 bits [heads][rows][128] over the pass lists idx / cnt ([heads][cubes][stride]
    and [heads][cubes], as cube_topk writes them) plus the dense rows [dense_row0, dense_row0 + n_dense). Every query
    tile when `tiles` is None, else only the (head, tile) pairs listed (tile numbering: dense runs of 64 first, then
    cube c as tile nd + c). Rows not written keep `out`'s values (zero when out is None)."""
    heads, rows, hd = q.shape
    assert hd == 128 and k.shape == q.shape and v.shape == q.shape
    scale = 1.0 / np.sqrt(128.0) if scale is None else scale
    out = np.zeros_like(q) if out is None else out
    q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
    idx, cnt = np.ascontiguousarray(idx, dtype=np.int32), np.ascontiguousarray(cnt, dtype=np.int32)
    geom = (*grid, layout, row0, rows * 128, 128, dense_row0, n_dense, scale)
    if tiles is None:
        _lib.mh3o_attn_sparse(heads, *geom, _p(q), _p(k), _p(v), _p(idx), _p(cnt), idx.shape[2], _p(out))
    else:
        for h, t in tiles:
            _lib.mh3o_attn_sparse_tile(*geom, _p(q), _p(k), _p(v), _p(idx), _p(cnt), idx.shape[2], h, t, _p(out))
    return out


def attn_tile_rows(grid, layout, row0, dense_row0, n_dense, tile):
    """The rows of attention tile `tile` that are tokens (dense runs of 64 first, then one tile per cube)."""
    gt, gh, gw = grid
    nd = (n_dense + 63) // 64
    if tile < nd:
        return np.arange(dense_row0 + 64 * tile, dense_row0 + min(n_dense, 64 * tile + 64))
    c = tile - nd
    ch, cw = (gh + 3) // 4, (gw + 3) // 4
    ct, cy, cx = c // (ch * cw), c // cw % ch, c % cw
    rows = []
    for l in range(64):
        dt, dy, dx = l // 16, l // 4 % 4, l % 4
        t, y, x = 4 * ct + dt, 4 * cy + dy, 4 * cx + dx
        if t < gt and y < gh and x < gw:
            rows.append(row0 + 64 * c + l if layout == CUBES_GATHERED else row0 + (t * gh + y) * gw + x)
    return np.array(rows, dtype=np.int64)


def cube_map(grid, n_dense=0, video_row0=None, dense_row0=0):
    """H3::Cubes' map -> (map int32 [cubes * 64 + n_dense], counts int32 [cubes]); the video grid's tokens at model
    rows video_row0 + (t * H + y) * W + x (default: right after the dense rows)."""
    gt, gh, gw = grid
    cubes = cube_count(gt, gh, gw)
    video_row0 = dense_row0 + n_dense if video_row0 is None else video_row0
    m = np.empty(cubes * 64 + n_dense, np.int32)
    counts = np.empty(cubes, np.int32)
    _lib.mh3o_cube_map(gt, gh, gw, n_dense, video_row0, dense_row0, _p(m), _p(counts))
    return m, counts


def time_embed(t, w_in, b_in, w_out, b_out, max_period=10000.0):
    """The sinusoidal embedding of each t (cos half first) through the time MLP -> (temb float32 [levels][out_dim],
    cond bf16 bits [levels][out_dim] = bf16(silu(temb)))."""
    t = np.ascontiguousarray(t, np.float32)
    hidden, freq_dim = w_in.shape
    out_dim = w_out.shape[0]
    temb = np.empty((t.size, out_dim), np.float32)
    cond = np.empty((t.size, out_dim), np.uint16)
    _lib.mh3o_time_embed(t.size, freq_dim, hidden, out_dim, max_period, _p(t), _p(w_in), _p(b_in), _p(w_out),
                         _p(b_out), _p(temb), _p(cond))
    return temb, cond


def adaln_mod(cond, w, bias=None):
    """mod[u][r] = w[r] . cond[u] + bias[r]: cond and w bf16 bits, double accumulation -> float32 [levels][n]."""
    levels, k = cond.shape
    n = w.shape[0]
    mod = np.empty((levels, n), np.float32)
    _lib.mh3o_adaln_mod(levels, n, k, _p(cond), _p(w), _p(bias), _p(mod))
    return mod


def curve_mods(t, table, w, bias=None):
    """The pruned checkpoints' curve: table [points][width] interpolated at t (points - 1), through w [n][width]."""
    t = np.ascontiguousarray(t, np.float32)
    points, width = table.shape
    n = w.shape[0]
    mod = np.empty((t.size, n), np.float32)
    _lib.mh3o_curve_mods(t.size, n, points, width, _p(t), _p(table), _p(w), _p(bias), _p(mod))
    return mod
