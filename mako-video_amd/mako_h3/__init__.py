"""Python binding of libmako_h3 (include/mako_h3.h) for torch device tensors.

The op names are the reference's kernel names (mako-common's `rms_mod_rows`, `gate_add_rows`, `swiglu_rows`,
`cube_pool`, `cube_scores`, `cube_topk`, `quant_rows_i8`; fc1's `gemm_i8` + `swiglu_rows` as `gemm_w8a16_swiglu`),
and errors raise RuntimeError as the reference's host code throws std::runtime_error on a bad call
(src/video/audio_vae.cpp:231-232). Every call checks the tensors against the sizes the kernel will touch before it
reaches the library, launches on torch's current stream, and returns without synchronizing.

torch is used here only for device memory and streams; the compute is the library's HIP kernels. There is no
fallback: if libmako_h3.so is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os
from pathlib import Path

import torch

_LIB_PATH = Path(os.environ.get("MAKO_H3_LIB", Path(__file__).resolve().parent.parent / "lib" / "libmako_h3.so"))

ABI_VERSION = 5  # MH3_ABI_VERSION of include/mako_h3.h, whose structs this module mirrors
OK, ERR_SHAPE, ERR_POINTER, ERR_ALIGN, ERR_PARAM, ERR_HIP, ERR_UNSUPPORTED = 0, -1, -2, -3, -4, -5, -6
F32, BF16 = 0, 1
ROWS_NORM_BF16, ROWS_Y_BF16 = 1, 2  # MH3RowsArgs.flags: the float stream's bf16 GEMM rows
SWIGLU_SPLIT, SWIGLU_FUSED = 0, 1
GEMM_W8A16, GEMM_BF16, GEMM_W8A8 = 0, 1, 2
CUBES_GRID, CUBES_GATHERED = 0, 1
INT8_QKV, INT8_OUT, INT8_FC1, INT8_FC2, INT8_ALL = 1, 2, 4, 8, 15


class RowsArgs(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("dim", C.c_uint32), ("n_sets", C.c_uint32), ("dtype", C.c_uint32),
                ("eps", C.c_float), ("set_stride", C.c_uint32), ("flags", C.c_uint32), ("reserved", C.c_uint32)]


class SwigluArgs(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("dim", C.c_uint32), ("layout", C.c_uint32), ("dtype", C.c_uint32)]


class CubeArgs(C.Structure):
    _fields_ = [("heads", C.c_uint32), ("head_dim", C.c_uint32), ("grid_t", C.c_uint32), ("grid_h", C.c_uint32),
                ("grid_w", C.c_uint32), ("layout", C.c_uint32), ("row0", C.c_uint64), ("head_stride", C.c_uint64),
                ("row_stride", C.c_uint64), ("k", C.c_uint32), ("local", C.c_uint32), ("out_stride", C.c_uint32),
                ("reserved", C.c_uint32)]


class AttnArgs(C.Structure):
    _fields_ = [("cubes", CubeArgs), ("dense_row0", C.c_uint64), ("n_dense", C.c_uint32), ("scale", C.c_float)]


class HeadsArgs(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("model_rows", C.c_uint32), ("heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("rot", C.c_uint32), ("eps", C.c_float), ("qkv_stride", C.c_uint64), ("out_head_stride", C.c_uint64),
                ("out_row_stride", C.c_uint64)]


class CubeMapArgs(C.Structure):
    _fields_ = [("grid_t", C.c_uint32), ("grid_h", C.c_uint32), ("grid_w", C.c_uint32), ("n_dense", C.c_uint32),
                ("video_row0", C.c_uint64), ("dense_row0", C.c_uint64)]


class TimeArgs(C.Structure):
    _fields_ = [("levels", C.c_uint32), ("freq_dim", C.c_uint32), ("hidden", C.c_uint32), ("out_dim", C.c_uint32),
                ("max_period", C.c_float), ("reserved", C.c_uint32 * 3)]


class CurveArgs(C.Structure):
    _fields_ = [("levels", C.c_uint32), ("n", C.c_uint32), ("points", C.c_uint32), ("width", C.c_uint32)]


class QuantArgs(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("dtype", C.c_uint32), ("reserved", C.c_uint32)]


class GemmArgs(C.Structure):
    _fields_ = [("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32), ("n_sets", C.c_uint32),
                ("gate_stride", C.c_uint32), ("reserved", C.c_uint32)]


def _load() -> C.CDLL:
    if not _LIB_PATH.exists():
        raise ImportError(f"{_LIB_PATH} is not built: run `python mako-video_amd/build.py`")
    lib = C.CDLL(str(_LIB_PATH))
    P, U32, I32, I64, F = C.c_void_p, C.c_uint32, C.c_int, C.c_int64, C.c_float
    sig = {
        "mh3_abi_version": (I32, []),
        "mh3_strerror": (C.c_char_p, [I32]),
        "mh3_last_hip_error": (C.c_char_p, []),
        "mh3_parse_int8": (I32, [C.c_char_p, C.POINTER(U32)]),
        "mh3_check_sparse": (I32, [F, U32]),
        "mh3_topk_k": (I64, [F, U32]),
        "mh3_cube_count": (I64, [U32, U32, U32]),
        "mh3_rms_mod_rows": (I32, [C.POINTER(RowsArgs), P, P, P, P, P, P, P]),
        "mh3_gate_add_rows": (I32, [C.POINTER(RowsArgs), P, P, P, P, P]),
        "mh3_rms_mod_gate_add_rows": (I32, [C.POINTER(RowsArgs), P, P, P, P, P, P, P, P, P]),
        "mh3_gate_add_rms_mod_rows": (I32, [C.POINTER(RowsArgs), P, P, P, P, P, P, P, P, P]),
        "mh3_swiglu_rows": (I32, [C.POINTER(SwigluArgs), P, P, P, P]),
        "mh3_cube_pool": (I32, [C.POINTER(CubeArgs), P, P, P, P, P, P]),
        "mh3_cube_scores": (I32, [C.POINTER(CubeArgs), P, P, P, P]),
        "mh3_cube_topk": (I32, [C.POINTER(CubeArgs), P, P, P, P]),
        "mh3_cube_select_workspace_bytes": (I64, [C.POINTER(CubeArgs)]),
        "mh3_cube_select": (I32, [C.POINTER(CubeArgs), P, P, P, C.c_uint64, P, P, P]),
        "mh3_cube_order": (I32, [C.POINTER(CubeArgs), P, P, P, P]),
        "mh3_cube_map": (I32, [C.POINTER(CubeMapArgs), P, P, P]),
        "mh3_time_embed_workspace_bytes": (I64, [C.POINTER(TimeArgs)]),
        "mh3_time_embed": (I32, [C.POINTER(TimeArgs), P, P, P, P, P, P, C.c_uint64, P, P, P]),
        "mh3_time_embed_noalloc": (I32, [C.POINTER(TimeArgs), P, P, P, P, P, P, P, P]),
        "mh3_adaln_mod": (I32, [C.POINTER(GemmArgs), P, P, P, P, P]),
        "mh3_curve_mods": (I32, [C.POINTER(CurveArgs), P, P, P, P, P, P]),
        "mh3_heads_partial": (I32, [C.POINTER(HeadsArgs), P, P, P, P, P, P, P, P, P, P]),
        "mh3_heads_partial_pool": (I32, [C.POINTER(HeadsArgs), C.POINTER(CubeArgs)] + [P] * 13),
        "mh3_flash_attn_sparse_128": (I32, [C.POINTER(AttnArgs), P, P, P, P, P, P, P]),
        "mh3_flash_attn_sparse_128_ordered": (I32, [C.POINTER(AttnArgs), P, P, P, P, P, P, P, P]),
        "mh3_quant_rows_i8": (I32, [C.POINTER(QuantArgs), P, P, P, P]),
        "mh3_gemm_w8a16_swiglu": (I32, [C.POINTER(GemmArgs), P, P, P, P, P]),
        "mh3_gemm_bf16_swiglu": (I32, [C.POINTER(GemmArgs), P, P, P, P]),
        "mh3_gemm_i8_swiglu": (I32, [C.POINTER(GemmArgs), P, P, P, P, P, P]),
        "mh3_gemm": (I32, [C.POINTER(GemmArgs), U32, P, P, P, P, P, P]),
        "mh3_gemm_gate_add": (I32, [C.POINTER(GemmArgs), U32, P, P, P, P, P, P, P, P]),
        "mh3_gemm_gate_add_f32": (I32, [C.POINTER(GemmArgs), U32, P, P, P, P, P, P, P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    if lib.mh3_abi_version() != ABI_VERSION:
        raise ImportError(f"{_LIB_PATH} has ABI version {lib.mh3_abi_version()}, this module mirrors {ABI_VERSION}")
    return lib


lib = _load()
LIB_PATH = _LIB_PATH


def strerror(code: int) -> str:
    return lib.mh3_strerror(code).decode()


def _check(rc: int, what: str) -> None:
    if rc != OK:
        extra = lib.mh3_last_hip_error().decode() if rc == ERR_HIP else ""
        raise RuntimeError(f"{what}: {strerror(rc)} ({rc}){': ' + extra if extra else ''}")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, numel: int) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be on the GPU")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements, the call touches {numel}")


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {t.dtype}")


# ---- H3 options (host only) ------------------------------------------------------------------------------------------

def parse_int8(text: str) -> int | None:
    """H3::parse_int8: "none", "all", or a comma list of qkv, out, fc1, fc2 -> mask; None for anything else."""
    m = C.c_uint32(0)
    rc = lib.mh3_parse_int8(text.encode(), C.byref(m))
    return int(m.value) if rc == OK else None


def check_sparse(ratio: float, local: int) -> bool:
    """H3::set_sparse's domain: ratio in [0, 1], local in {0, 1, 3}."""
    return lib.mh3_check_sparse(float(ratio), int(local)) == OK


def topk_k(ratio: float, cubes: int) -> int:
    k = int(lib.mh3_topk_k(float(ratio), int(cubes)))
    if k < 0:
        raise ValueError(f"ratio {ratio} outside [0, 1]")
    return k


def cube_count(grid_t: int, grid_h: int, grid_w: int) -> int:
    return int(lib.mh3_cube_count(grid_t, grid_h, grid_w))


# ---- rows ----------------------------------------------------------------------------------------------------------

def _rows_args(x: torch.Tensor, n_sets: int, eps: float) -> RowsArgs:
    if x.dim() != 2:
        raise ValueError("rows must be [rows][dim]")
    a = RowsArgs()
    a.rows, a.dim, a.n_sets, a.dtype, a.eps = x.shape[0], x.shape[1], n_sets, _dt(x), eps
    return a


def _set_stride(t: torch.Tensor, name: str, dim: int, n_sets: int) -> int:
    """Floats between consecutive sets of a modulation vector tensor [..., dim]: its leading dimensions must collapse
    to one stride (a contiguous [n_sets][dim] tensor, or a view into a table such as [U][3][6][D] with one of the six
    vectors selected) and cover n_sets sets."""
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda" or t.dtype != torch.float32:
        raise ValueError(f"{name}: expected a float32 tensor on the GPU")
    if t.shape[-1] != dim or t.stride(-1) != 1:
        raise ValueError(f"{name}: the last dimension must be dim ({dim}) and contiguous")
    lead = [(n, st) for n, st in zip(t.shape[:-1], t.stride()[:-1]) if n != 1]
    for (n0, s0), (n1, s1) in zip(lead, lead[1:]):
        if s0 != s1 * n1:
            raise ValueError(f"{name}: its sets are not evenly spaced")
    sets = 1
    for n, _ in lead:
        sets *= n
    if sets < n_sets:
        raise ValueError(f"{name}: {sets} sets, the call uses {n_sets}")
    return lead[-1][1] if lead else dim


def _mod_params(a, dim, n_sets, w, shift, scale, gate, set_of_row, rows):
    if w is not None:
        _need(w, "w", torch.float32, dim)
    strides = {_set_stride(t, name, dim, n_sets) for name, t in (("shift", shift), ("scale", scale), ("gate", gate))
               if t is not None}
    if len(strides) > 1:
        raise ValueError("shift, scale and gate must share one set stride")
    if n_sets > 1 and strides:
        a.set_stride = strides.pop()
    if set_of_row is not None:
        _need(set_of_row, "set_of_row", torch.uint8, rows)


def rms_mod_rows(x, w, shift, scale, *, eps=1e-6, set_of_row=None, n_sets=1, out=None, out_dtype=None):
    """y = x * rsqrt(mean(x^2) + eps) * w * (1 + scale[s]) + shift[s] per row (x: [rows][dim] f32 or bf16). With a
    float x and out_dtype bf16 (or a bf16 `out`), y is the bf16 row the next GEMM takes, rounded once."""
    a = _rows_args(x, n_sets, eps)
    _need(x, "x", x.dtype, x.numel())
    _mod_params(a, x.shape[1], n_sets, w, shift, scale, None, set_of_row, x.shape[0])
    odt = out.dtype if out is not None else (out_dtype or x.dtype)
    if odt != x.dtype:
        a.flags = ROWS_NORM_BF16
    out = torch.empty(x.shape, dtype=odt, device=x.device) if out is None else out
    _need(out, "out", odt, x.numel())
    _check(lib.mh3_rms_mod_rows(C.byref(a), _ptr(x), _ptr(w), _ptr(shift), _ptr(scale), _ptr(set_of_row), _ptr(out),
                                _stream()), "rms_mod_rows")
    return out


def gate_add_rows(x, y, gate, *, set_of_row=None, n_sets=1):
    """x += gate[s] * y per row, in place; returns x. A float x may take a bf16 y (a GEMM's output)."""
    a = _rows_args(x, n_sets, 1.0)
    _need(x, "x", x.dtype, x.numel())
    if y.dtype != x.dtype:
        a.flags = ROWS_Y_BF16
    _need(y, "y", y.dtype, x.numel())
    _mod_params(a, x.shape[1], n_sets, None, None, None, gate, set_of_row, x.shape[0])
    _check(lib.mh3_gate_add_rows(C.byref(a), _ptr(x), _ptr(y), _ptr(gate), _ptr(set_of_row), _stream()),
           "gate_add_rows")
    return x


def rms_mod_gate_add_rows(x, residual, w, shift, scale, gate, *, eps=1e-6, set_of_row=None, n_sets=1, out=None):
    """out = residual + gate[s] * (x * rsqrt(mean(x^2) + eps) * w * (1 + scale[s]) + shift[s]), one HBM pass."""
    a = _rows_args(x, n_sets, eps)
    _need(x, "x", x.dtype, x.numel())
    _need(residual, "residual", x.dtype, x.numel())
    _mod_params(a, x.shape[1], n_sets, w, shift, scale, gate, set_of_row, x.shape[0])
    out = torch.empty_like(x) if out is None else out
    _need(out, "out", x.dtype, x.numel())
    _check(lib.mh3_rms_mod_gate_add_rows(C.byref(a), _ptr(x), _ptr(residual), _ptr(w), _ptr(shift), _ptr(scale),
                                         _ptr(gate), _ptr(set_of_row), _ptr(out), _stream()), "rms_mod_gate_add_rows")
    return out


def gate_add_rms_mod_rows(x, y, gate, w, shift, scale, *, eps=1e-6, set_of_row=None, n_sets=1, h=None,
                          h_dtype=None):
    """The block's order: x += gate[s] * y in place, then h = x * rsqrt(mean(x^2) + eps) * w * (1 + scale[s]) +
    shift[s] of the updated x; one HBM pass. Returns h. With a float x (the reference's float residual stream), h may
    be bf16 (h_dtype, or a bf16 `h`: the next GEMM's input), and then y may be bf16 too (a GEMM's output)."""
    a = _rows_args(x, n_sets, eps)
    _need(x, "x", x.dtype, x.numel())
    _need(y, "y", y.dtype, x.numel())
    _mod_params(a, x.shape[1], n_sets, w, shift, scale, gate, set_of_row, x.shape[0])
    hdt = h.dtype if h is not None else (h_dtype or x.dtype)
    a.flags = (ROWS_NORM_BF16 if hdt != x.dtype else 0) | (ROWS_Y_BF16 if y.dtype != x.dtype else 0)
    h = torch.empty(x.shape, dtype=hdt, device=x.device) if h is None else h
    _need(h, "h", hdt, x.numel())
    _check(lib.mh3_gate_add_rms_mod_rows(C.byref(a), _ptr(x), _ptr(y), _ptr(gate), _ptr(w), _ptr(shift), _ptr(scale),
                                         _ptr(set_of_row), _ptr(h), _stream()), "gate_add_rms_mod_rows")
    return h


# ---- swiglu --------------------------------------------------------------------------------------------------------

def swiglu_rows(gate, up=None, *, out=None):
    """out = silu(gate) * up. With up None, gate is fc1's fused [rows][2 dim] row ([gate | up])."""
    a = SwigluArgs()
    if up is None:
        rows, two = gate.shape
        if two % 2:
            raise ValueError("a fused row has an even width")
        a.rows, a.dim, a.layout = rows, two // 2, SWIGLU_FUSED
    else:
        a.rows, a.dim, a.layout = gate.shape[0], gate.shape[1], SWIGLU_SPLIT
        _need(up, "up", gate.dtype, a.rows * a.dim)
    a.dtype = _dt(gate)
    _need(gate, "gate", gate.dtype, gate.numel())
    out = torch.empty((a.rows, a.dim), dtype=gate.dtype, device=gate.device) if out is None else out
    _need(out, "out", gate.dtype, a.rows * a.dim)
    _check(lib.mh3_swiglu_rows(C.byref(a), _ptr(gate), _ptr(up), _ptr(out), _stream()), "swiglu_rows")
    return out


# ---- cubes ---------------------------------------------------------------------------------------------------------

def cube_args(heads, grid, *, layout=CUBES_GRID, row0=0, head_stride=None, row_stride=128, k=0, local=1,
              out_stride=None, head_dim=128) -> CubeArgs:
    gt, gh, gw = grid
    a = CubeArgs()
    a.heads, a.head_dim, a.grid_t, a.grid_h, a.grid_w, a.layout = heads, head_dim, gt, gh, gw, layout
    cubes = cube_count(gt, gh, gw)
    rows = row0 + (cubes * 64 if layout == CUBES_GATHERED else gt * gh * gw)
    a.row0, a.row_stride = row0, row_stride
    a.head_stride = rows * row_stride if head_stride is None else head_stride
    a.k, a.local = k, local
    a.out_stride = (k + local) if out_stride is None else out_stride
    return a


def _rows_touched(a: CubeArgs) -> int:
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    last = a.row0 + (cubes * 64 - 1 if a.layout == CUBES_GATHERED else a.grid_t * a.grid_h * a.grid_w - 1)
    return (a.heads - 1) * a.head_stride + last * a.row_stride + a.head_dim


def cube_pool(a: CubeArgs, q, k, *, qc=None, kc=None, counts=None):
    """Per head, the mean of each 4x4x4 cube's q and k rows -> (qc, kc) float [heads][cubes][head_dim]."""
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    n = _rows_touched(a)
    _need(q, "q", torch.bfloat16, n)
    _need(k, "k", torch.bfloat16, n)
    shape = (a.heads, cubes, a.head_dim)
    qc = torch.empty(shape, dtype=torch.float32, device=q.device) if qc is None else qc
    kc = torch.empty(shape, dtype=torch.float32, device=q.device) if kc is None else kc
    _need(qc, "qc", torch.float32, a.heads * cubes * a.head_dim)
    _need(kc, "kc", torch.float32, a.heads * cubes * a.head_dim)
    if counts is not None:
        _need(counts, "counts", torch.int32, cubes)
    _check(lib.mh3_cube_pool(C.byref(a), _ptr(q), _ptr(k), _ptr(qc), _ptr(kc), _ptr(counts), _stream()), "cube_pool")
    return qc, kc


def cube_scores(a: CubeArgs, qc, kc, *, out=None):
    """s[h][i][j] = qc[h][i] . kc[h][j] / sqrt(head_dim), float [heads][cubes][cubes]."""
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    _need(qc, "qc", torch.float32, a.heads * cubes * a.head_dim)
    _need(kc, "kc", torch.float32, a.heads * cubes * a.head_dim)
    out = torch.empty((a.heads, cubes, cubes), dtype=torch.float32, device=qc.device) if out is None else out
    _need(out, "scores", torch.float32, a.heads * cubes * cubes)
    _check(lib.mh3_cube_scores(C.byref(a), _ptr(qc), _ptr(kc), _ptr(out), _stream()), "cube_scores")
    return out


def _topk_out(a: CubeArgs, device, idx, cnt):
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    idx = torch.empty((a.heads, cubes, a.out_stride), dtype=torch.int32, device=device) if idx is None else idx
    cnt = torch.empty((a.heads, cubes), dtype=torch.int32, device=device) if cnt is None else cnt
    _need(idx, "idx", torch.int32, a.heads * cubes * a.out_stride)
    _need(cnt, "cnt", torch.int32, a.heads * cubes)
    return idx, cnt


def cube_topk(a: CubeArgs, scores, *, idx=None, cnt=None):
    """Per (head, query cube): the top a.k cubes by score plus the local cubes, ascending, padded with -1."""
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    _need(scores, "scores", torch.float32, a.heads * cubes * cubes)
    idx, cnt = _topk_out(a, scores.device, idx, cnt)
    _check(lib.mh3_cube_topk(C.byref(a), _ptr(scores), _ptr(idx), _ptr(cnt), _stream()), "cube_topk")
    return idx, cnt


def cube_select_workspace_bytes(a: CubeArgs) -> int:
    n = int(lib.mh3_cube_select_workspace_bytes(C.byref(a)))
    _check(min(n, 0), "cube_select_workspace_bytes")
    return n


def cube_select(a: CubeArgs, qc, kc, *, workspace=None, idx=None, cnt=None):
    """cube_scores and cube_topk fused: the scores stay on chip. `workspace` (uint8, at least
    cube_select_workspace_bytes(a), allocated here when None) holds kc split for the matrix cores."""
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    _need(qc, "qc", torch.float32, a.heads * cubes * a.head_dim)
    _need(kc, "kc", torch.float32, a.heads * cubes * a.head_dim)
    nbytes = cube_select_workspace_bytes(a)
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=qc.device)
    _need(workspace, "workspace", torch.uint8, nbytes)
    idx, cnt = _topk_out(a, qc.device, idx, cnt)
    _check(lib.mh3_cube_select(C.byref(a), _ptr(qc), _ptr(kc), _ptr(workspace), workspace.numel(), _ptr(idx),
                               _ptr(cnt), _stream()), "cube_select")
    return idx, cnt


def cube_order(a: CubeArgs, idx, cnt, *, order=None):
    """The query-cube order for flash_attn_sparse_128(order=...): int32 [heads][cubes], each head's cubes sorted by
    the middle entry of their pass lists (idx[h][c][cnt / 2]), equal entries by cube index."""
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    _need(idx, "idx", torch.int32, a.heads * cubes * a.out_stride)
    _need(cnt, "cnt", torch.int32, a.heads * cubes)
    order = torch.empty((a.heads, cubes), dtype=torch.int32, device=idx.device) if order is None else order
    _need(order, "order", torch.int32, a.heads * cubes)
    _check(lib.mh3_cube_order(C.byref(a), _ptr(idx), _ptr(cnt), _ptr(order), _stream()), "cube_order")
    return order


def cube_map(grid, *, n_dense=0, video_row0=None, dense_row0=0, device=None, map=None, counts=None):
    """H3::Cubes' map: int32 [cubes * 64 + n_dense], attention row -> model row (-1 for a cube's padding slot), the
    video grid's tokens at model rows video_row0 + (t * H + y) * W + x (default: right after the dense rows) and the
    dense rows at dense_row0 ... Returns (map, counts), counts int32 [cubes] the cubes' token counts."""
    gt, gh, gw = grid
    a = CubeMapArgs()
    a.grid_t, a.grid_h, a.grid_w, a.n_dense = gt, gh, gw, n_dense
    a.video_row0 = dense_row0 + n_dense if video_row0 is None else video_row0
    a.dense_row0 = dense_row0
    cubes = cube_count(gt, gh, gw)
    device = device or torch.device("cuda", torch.cuda.current_device())
    map = torch.empty(cubes * 64 + n_dense, dtype=torch.int32, device=device) if map is None else map
    counts = torch.empty(cubes, dtype=torch.int32, device=device) if counts is None else counts
    _need(map, "map", torch.int32, cubes * 64 + n_dense)
    _need(counts, "counts", torch.int32, cubes)
    _check(lib.mh3_cube_map(C.byref(a), _ptr(map), _ptr(counts), _stream()), "cube_map")
    return map, counts


# ---- time conditioning -------------------------------------------------------------------------------------------------

def _time_args(levels, freq_dim, hidden, out_dim, max_period) -> TimeArgs:
    a = TimeArgs()
    a.levels, a.freq_dim, a.hidden, a.out_dim, a.max_period = levels, freq_dim, hidden, out_dim, max_period
    return a


def time_embed_workspace_bytes(levels, freq_dim, hidden, out_dim, max_period=10000.0) -> int:
    n = int(lib.mh3_time_embed_workspace_bytes(C.byref(_time_args(levels, freq_dim, hidden, out_dim, max_period))))
    _check(min(n, 0), "time_embed_workspace_bytes")
    return n


def time_embed(t, w_in, b_in, w_out, b_out, *, max_period=10000.0, workspace=None, temb=None, cond=None,
               with_cond=True):
    """The sinusoidal embedding of each level t[u] (freq_dim = w_in's width, cos half first) through the F32 time MLP
    (w_in [hidden][freq_dim], w_out [out_dim][hidden], biases may be None) -> (temb float [levels][out_dim],
    cond bf16 [levels][out_dim] = bf16(silu(temb)), or None without with_cond)."""
    levels = t.numel()
    hidden, freq_dim = w_in.shape
    out_dim = w_out.shape[0]
    if w_out.shape[1] != hidden:
        raise ValueError("w_out must be [out_dim][hidden]")
    _need(t, "t", torch.float32, levels)
    _need(w_in, "w_in", torch.float32, hidden * freq_dim)
    _need(w_out, "w_out", torch.float32, out_dim * hidden)
    if b_in is not None:
        _need(b_in, "b_in", torch.float32, hidden)
    if b_out is not None:
        _need(b_out, "b_out", torch.float32, out_dim)
    a = _time_args(levels, freq_dim, hidden, out_dim, max_period)
    nbytes = int(lib.mh3_time_embed_workspace_bytes(C.byref(a)))
    _check(min(nbytes, 0), "time_embed")
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=t.device)
    _need(workspace, "workspace", torch.uint8, nbytes)
    temb = torch.empty((levels, out_dim), dtype=torch.float32, device=t.device) if temb is None else temb
    _need(temb, "temb", torch.float32, levels * out_dim)
    if with_cond:
        cond = torch.empty((levels, out_dim), dtype=torch.bfloat16, device=t.device) if cond is None else cond
        _need(cond, "cond", torch.bfloat16, levels * out_dim)
    else:
        cond = None
    _check(lib.mh3_time_embed(C.byref(a), _ptr(t), _ptr(w_in), _ptr(b_in), _ptr(w_out), _ptr(b_out),
                              _ptr(workspace), workspace.numel(), _ptr(temb), _ptr(cond), _stream()), "time_embed")
    return temb, cond


def adaln_mod(cond, w, bias=None, *, out=None):
    """A block's AdaLN projection: mod[u][r] = w[r] . cond[u] + bias[r] (cond bf16 [levels][k], w bf16 [n][k], bias
    float [n] or None) -> float [levels][n]; with n = 18 D, view it as the [levels][3][6][D] table."""
    levels, k = cond.shape
    n = w.shape[0]
    if w.dim() != 2 or w.shape[1] != k:
        raise ValueError("w must be [n][k]")
    _need(cond, "cond", torch.bfloat16, levels * k)
    _need(w, "w", torch.bfloat16, n * k)
    if bias is not None:
        _need(bias, "bias", torch.float32, n)
    out = torch.empty((levels, n), dtype=torch.float32, device=cond.device) if out is None else out
    _need(out, "mod", torch.float32, levels * n)
    a = GemmArgs()
    a.m, a.n, a.k = levels, n, k
    _check(lib.mh3_adaln_mod(C.byref(a), _ptr(cond), _ptr(w), _ptr(bias), _ptr(out), _stream()), "adaln_mod")
    return out


def curve_mods(t, table, w, bias=None, *, out=None):
    """The pruned checkpoints' modulation: the curve table [points][width] interpolated at t[u] (points - 1), through
    w float [n][width] plus bias, no silu -> float [levels][n]."""
    levels = t.numel()
    points, width = table.shape
    n = w.shape[0]
    if w.dim() != 2 or w.shape[1] != width:
        raise ValueError("w must be [n][width]")
    _need(t, "t", torch.float32, levels)
    _need(table, "table", torch.float32, points * width)
    _need(w, "w", torch.float32, n * width)
    if bias is not None:
        _need(bias, "bias", torch.float32, n)
    out = torch.empty((levels, n), dtype=torch.float32, device=t.device) if out is None else out
    _need(out, "mod", torch.float32, levels * n)
    a = CurveArgs()
    a.levels, a.n, a.points, a.width = levels, n, points, width
    _check(lib.mh3_curve_mods(C.byref(a), _ptr(t), _ptr(table), _ptr(w), _ptr(bias), _ptr(out), _stream()),
           "curve_mods")
    return out


# ---- heads_partial ---------------------------------------------------------------------------------------------------

def _heads_setup(qkv, heads, q_w, k_w, cos_t, sin_t, rot, eps, map, with_v, layout, q, k, v):
    if qkv.dim() != 2:
        raise ValueError("qkv must be [rows][3 heads 128]")
    model_rows, stride = qkv.shape
    _need(qkv, "qkv", torch.bfloat16, qkv.numel())
    rows = model_rows if map is None else map.numel()
    if map is not None:
        _need(map, "map", torch.int32, rows)
    a = HeadsArgs()
    a.rows, a.model_rows, a.heads, a.head_dim, a.rot, a.eps, a.qkv_stride = rows, model_rows, heads, 128, rot, eps, stride
    if layout == "heads":
        shape, a.out_head_stride, a.out_row_stride = (heads, rows, 128), rows * 128, 128
    elif layout == "rows":
        shape, a.out_head_stride, a.out_row_stride = (rows, heads * 128), 128, heads * 128
    else:
        raise ValueError("layout is 'heads' or 'rows'")
    for name, t in (("q_w", q_w), ("k_w", k_w)):
        if t is not None:
            _need(t, name, torch.float32, 128)
    if rot:
        for name, t in (("cos_t", cos_t), ("sin_t", sin_t)):
            _need(t, name, torch.float32, model_rows * (rot // 2))
    outs = []
    for name, t, want in (("q", q, True), ("k", k, True), ("v", v, with_v)):
        if not want:
            outs.append(None)
            continue
        t = torch.empty(shape, dtype=torch.bfloat16, device=qkv.device) if t is None else t
        _need(t, name, torch.bfloat16, heads * rows * 128)
        outs.append(t)
    ptrs = (_ptr(qkv), _ptr(q_w), _ptr(k_w), _ptr(cos_t if rot else None), _ptr(sin_t if rot else None), _ptr(map))
    return a, outs, ptrs


def heads_partial(qkv, heads, q_w=None, k_w=None, cos_t=None, sin_t=None, *, rot=96, eps=1e-6, map=None,
                  with_v=True, layout="heads", q=None, k=None, v=None):
    """After the QKV GEMM: qkv bf16 [model_rows][>= 3 heads 128] ([q heads | k heads | v heads] a row) -> q and k
    with the per-head RMS norm (weights q_w, k_w f32 [128]; None: 1) and the rotary positions on the first `rot`
    values (cos_t, sin_t f32 [model_rows][rot / 2]), v copied (not written when with_v is False). Output row r is model
    row map[r] (int32 [rows]; entries outside [0, model_rows) give zeros), or row r without a map. layout "heads"
    gives [heads][rows][128] tensors, "rows" gives [rows][heads * 128]. Returns (q, k, v)."""
    a, outs, ptrs = _heads_setup(qkv, heads, q_w, k_w, cos_t, sin_t, rot, eps, map, with_v, layout, q, k, v)
    _check(lib.mh3_heads_partial(C.byref(a), *ptrs, *(_ptr(t) for t in outs), _stream()), "heads_partial")
    return tuple(outs)


def heads_partial_pool(qkv, heads, grid, q_w=None, k_w=None, cos_t=None, sin_t=None, *, rot=96, eps=1e-6, map=None,
                       with_v=True, layout="heads", row0=0, cube_layout=CUBES_GATHERED, q=None, k=None, v=None,
                       qc=None, kc=None, counts=None):
    """heads_partial followed by cube_pool over its output, in one pass. Gathered (the default): cube c of the video
    grid (T, H, W) = `grid` is output rows row0 + 64 c ... + 63. CUBES_GRID (no map): the outputs stay in the model's
    order, the grid's tokens at rows row0 + (t H + y) W + x. Returns (q, k, v, qc, kc), the same bits as
    heads_partial(...) then cube_pool(cube_args(heads, grid, layout=cube_layout, row0=row0, ...), q, k)."""
    a, outs, ptrs = _heads_setup(qkv, heads, q_w, k_w, cos_t, sin_t, rot, eps, map, with_v, layout, q, k, v)
    ca = cube_args(heads, grid, layout=cube_layout, row0=row0, head_stride=a.out_head_stride,
                   row_stride=a.out_row_stride)
    cubes = cube_count(*grid)
    shape = (heads, cubes, 128)
    qc = torch.empty(shape, dtype=torch.float32, device=qkv.device) if qc is None else qc
    kc = torch.empty(shape, dtype=torch.float32, device=qkv.device) if kc is None else kc
    _need(qc, "qc", torch.float32, heads * cubes * 128)
    _need(kc, "kc", torch.float32, heads * cubes * 128)
    if counts is not None:
        _need(counts, "counts", torch.int32, cubes)
    _check(lib.mh3_heads_partial_pool(C.byref(a), C.byref(ca), *ptrs, *(_ptr(t) for t in outs), _ptr(qc), _ptr(kc),
                                      _ptr(counts), _stream()), "heads_partial_pool")
    return (*outs, qc, kc)


# ---- flash_attn_sparse_128 -------------------------------------------------------------------------------------------

def flash_attn_sparse_128(a: CubeArgs, q, k, v, idx, cnt, *, dense_row0=0, n_dense=0, scale=0.0, out=None,
                          order=None):
    """Sparse attention over the pass lists idx / cnt (as cube_select writes them): the queries of cube i attend the
    tokens of its selected cubes and the dense rows [dense_row0, dense_row0 + n_dense); a dense row's query attends
    every token. q, k, v (and out) bf16 in the cube geometry `a` (grid or gathered layout); scale 0 is 1/sqrt(128).
    Rows that are not written keep `out`'s values (zero when out is None). With `order` (cube_order's int32
    [heads][cubes]) the query cubes are scheduled in that order (mh3_flash_attn_sparse_128_ordered)."""
    cubes = cube_count(a.grid_t, a.grid_h, a.grid_w)
    n = _rows_touched(a)
    if n_dense:
        n = max(n, (a.heads - 1) * a.head_stride + (dense_row0 + n_dense - 1) * a.row_stride + a.head_dim)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(t, name, torch.bfloat16, n)
    _need(idx, "idx", torch.int32, a.heads * cubes * a.out_stride)
    _need(cnt, "cnt", torch.int32, a.heads * cubes)
    out = torch.zeros_like(q) if out is None else out
    _need(out, "out", torch.bfloat16, n)
    args = AttnArgs()
    args.cubes, args.dense_row0, args.n_dense, args.scale = a, dense_row0, n_dense, scale
    if order is None:
        _check(lib.mh3_flash_attn_sparse_128(C.byref(args), _ptr(q), _ptr(k), _ptr(v), _ptr(idx), _ptr(cnt),
                                             _ptr(out), _stream()), "flash_attn_sparse_128")
    else:
        _need(order, "order", torch.int32, a.heads * cubes)
        _check(lib.mh3_flash_attn_sparse_128_ordered(C.byref(args), _ptr(q), _ptr(k), _ptr(v), _ptr(idx), _ptr(cnt),
                                                     _ptr(order), _ptr(out), _stream()), "flash_attn_sparse_128")
    return out


# ---- int8 ----------------------------------------------------------------------------------------------------------

def quant_rows_i8(w, *, q=None, scale=None):
    """Each [out][in] row to symmetric int8 with a float scale (max |row| -> 127)."""
    if w.dim() != 2:
        raise ValueError("w must be [rows][cols]")
    a = QuantArgs()
    a.rows, a.cols, a.dtype = w.shape[0], w.shape[1], _dt(w)
    _need(w, "w", w.dtype, w.numel())
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device) if q is None else q
    scale = torch.empty(w.shape[0], dtype=torch.float32, device=w.device) if scale is None else scale
    _need(q, "q", torch.int8, w.numel())
    _need(scale, "scale", torch.float32, w.shape[0])
    _check(lib.mh3_quant_rows_i8(C.byref(a), _ptr(w), _ptr(q), _ptr(scale), _stream()), "quant_rows_i8")
    return q, scale


def gemm_w8a16_swiglu(x, w, scale, *, out=None):
    """fc1 + SwiGLU: x bf16 [m][k], w int8 [2n][k] (gate rows then up rows), scale f32 [2n] -> bf16 [m][n]."""
    m, k = x.shape
    two_n = w.shape[0]
    if w.dim() != 2 or w.shape[1] != k or two_n % 2:
        raise ValueError("w must be [2n][k]")
    n = two_n // 2
    _need(x, "x", torch.bfloat16, m * k)
    _need(w, "w", torch.int8, two_n * k)
    _need(scale, "scale", torch.float32, two_n)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, m * n)
    a = GemmArgs()
    a.m, a.n, a.k = m, n, k
    _check(lib.mh3_gemm_w8a16_swiglu(C.byref(a), _ptr(x), _ptr(w), _ptr(scale), _ptr(out), _stream()),
           "gemm_w8a16_swiglu")
    return out


def gemm_bf16_swiglu(x, w, *, out=None):
    """The dense bf16 fc1 + SwiGLU: x bf16 [m][k], w bf16 [2n][k] (gate rows then up rows) -> bf16 [m][n]."""
    m, k = x.shape
    two_n = w.shape[0]
    if w.dim() != 2 or w.shape[1] != k or two_n % 2:
        raise ValueError("w must be [2n][k]")
    n = two_n // 2
    _need(x, "x", torch.bfloat16, m * k)
    _need(w, "w", torch.bfloat16, two_n * k)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, m * n)
    a = GemmArgs()
    a.m, a.n, a.k = m, n, k
    _check(lib.mh3_gemm_bf16_swiglu(C.byref(a), _ptr(x), _ptr(w), _ptr(out), _stream()), "gemm_bf16_swiglu")
    return out


def gemm_i8_swiglu(x, x_scale, w, w_scale, *, out=None):
    """The W8A8 fc1 + SwiGLU: x int8 [m][k] with x_scale f32 [m], w int8 [2n][k] with w_scale f32 [2n] -> bf16 [m][n].
    quant_rows_i8 of the bf16 activations gives x and x_scale."""
    m, k = x.shape
    two_n = w.shape[0]
    if w.dim() != 2 or w.shape[1] != k or two_n % 2:
        raise ValueError("w must be [2n][k]")
    n = two_n // 2
    _need(x, "x", torch.int8, m * k)
    _need(x_scale, "x_scale", torch.float32, m)
    _need(w, "w", torch.int8, two_n * k)
    _need(w_scale, "w_scale", torch.float32, two_n)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, m * n)
    a = GemmArgs()
    a.m, a.n, a.k = m, n, k
    _check(lib.mh3_gemm_i8_swiglu(C.byref(a), _ptr(x), _ptr(x_scale), _ptr(w), _ptr(w_scale), _ptr(out), _stream()),
           "gemm_i8_swiglu")
    return out


# ---- the qkv, out and fc2 projections -------------------------------------------------------------------------------

def _gemm_operands(x, w, x_scale, w_scale):
    """The form of a projection from its operand dtypes: bf16 x and w, bf16 x with int8 w (weight-only, w_scale), or
    int8 x (x_scale) with int8 w (w_scale)."""
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1]:
        raise ValueError("x must be [m][k] and w [n][k]")
    m, k = x.shape
    n = w.shape[0]
    if x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16:
        form = GEMM_BF16
    elif x.dtype == torch.bfloat16 and w.dtype == torch.int8:
        form = GEMM_W8A16
    elif x.dtype == torch.int8 and w.dtype == torch.int8:
        form = GEMM_W8A8
    else:
        raise ValueError(f"unsupported operand dtypes {x.dtype} x {w.dtype}")
    _need(x, "x", x.dtype, m * k)
    _need(w, "w", w.dtype, n * k)
    if form != GEMM_BF16:
        _need(w_scale, "w_scale", torch.float32, n)
    if form == GEMM_W8A8:
        _need(x_scale, "x_scale", torch.float32, m)
    a = GemmArgs()
    a.m, a.n, a.k = m, n, k
    return a, form


def gemm(x, w, *, x_scale=None, w_scale=None, out=None):
    """The qkv projection (the reference's Gemm::encode, or gemm_i8 under --int8): out = x w^T, bf16 [m][n], with w
    [n][k] output-channel rows; int8 w takes w_scale f32 [n], int8 x (quant_rows_i8) takes x_scale f32 [m]."""
    a, form = _gemm_operands(x, w, x_scale, w_scale)
    out = torch.empty((a.m, a.n), dtype=torch.bfloat16, device=x.device) if out is None else out
    _need(out, "out", torch.bfloat16, a.m * a.n)
    _check(lib.mh3_gemm(C.byref(a), form, _ptr(x), _ptr(x_scale if form == GEMM_W8A8 else None), _ptr(w),
                        _ptr(w_scale if form != GEMM_BF16 else None), _ptr(out), _stream()), "gemm")
    return out


def gemm_gate_add(x, w, residual, gate, *, x_scale=None, w_scale=None, set_of_row=None, n_sets=1):
    """The out projection and fc2 with gate_add_rows folded in: residual += gate[s] * (x w^T), [m][n] in place,
    s = set_of_row[row]; gate f32 [n_sets][n] (or a view with a set stride). residual is bf16, or float (the
    reference's float residual stream). Returns residual."""
    a, form = _gemm_operands(x, w, x_scale, w_scale)
    f32 = residual.dtype == torch.float32
    _need(residual, "residual", torch.float32 if f32 else torch.bfloat16, a.m * a.n)
    stride = _set_stride(gate, "gate", a.n, n_sets)
    a.n_sets, a.gate_stride = n_sets, stride
    if set_of_row is not None:
        _need(set_of_row, "set_of_row", torch.uint8, a.m)
    fn = lib.mh3_gemm_gate_add_f32 if f32 else lib.mh3_gemm_gate_add
    _check(fn(C.byref(a), form, _ptr(x), _ptr(x_scale if form == GEMM_W8A8 else None), _ptr(w),
              _ptr(w_scale if form != GEMM_BF16 else None), _ptr(gate), _ptr(set_of_row), _ptr(residual), _stream()),
           "gemm_gate_add")
    return residual
