"""The C-ABI without a GPU: libmako_h3.so loads, exports every entry point include/mako_h3.h declares, parses H3's
options as the reference does, and refuses invalid calls with the right code before launching anything (the calls
below never reach a kernel, so they run on a machine without a GPU)."""
import ctypes as C
import re
from pathlib import Path

import pytest

import mako_h3 as mh

HEADER = Path(__file__).resolve().parent.parent / "include" / "mako_h3.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mh3_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 17
    for n in names:
        assert hasattr(mh.lib, n), f"{n} declared in mako_h3.h but not exported"


def test_stream_probe_library_loads_and_refuses_bad_calls():
    """The measurement probe bench.py loads beside the library: both entry points exist, and a bad kind, a null
    pointer or a misaligned pointer is refused before any launch."""
    probe = C.CDLL(str(Path(mh.lib._name).parent / "libmh3_stream_probe.so"))
    probe.mh3_probe_stream.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_int, C.c_uint32,
                                       C.c_void_p]
    assert hasattr(probe, "mh3_probe_device")
    buf = C.create_string_buffer(64)
    a = (C.addressof(buf) + 15) // 16 * 16
    assert probe.mh3_probe_stream(8, a, a, a, 1, 4, 0, None) == -1
    assert probe.mh3_probe_stream(-1, a, a, a, 1, 4, 0, None) == -1
    assert probe.mh3_probe_stream(6, a, None, a, 1, 4, 0, None) == -1     # two read streams need b
    assert probe.mh3_probe_stream(7, a, None, a, 1, 4, 0, None) == -1
    assert probe.mh3_probe_stream(5, a, None, a, 1, 4, 8, None) == -1     # the buffer form has a flat grid only
    assert probe.mh3_probe_stream(4, a, None, a, 1 << 28, 4, 0, None) == -1  # beyond 32-bit byte offsets
    assert probe.mh3_probe_stream(2, a, None, a, 1, 4, 0, None) == -1
    assert probe.mh3_probe_stream(3, a, None, a, 1, 4, 0, None) == -1
    assert probe.mh3_probe_stream(1, a, None, a, 1, 3, 0, None) == -1
    assert probe.mh3_probe_stream(1, a + 4, None, a, 1, 4, 0, None) == -2
    assert probe.mh3_probe_stream(1, a, None, a, 0, 4, 0, None) == 0


def test_abi_version_and_strings():
    assert mh.lib.mh3_abi_version() == 5
    # The Python structs mirror the header: its MH3_ABI_VERSION is the module's (import refuses another library's).
    header = (Path(__file__).resolve().parent.parent / "include" / "mako_h3.h").read_text()
    assert re.search(r"#define MH3_ABI_VERSION (\d+)", header).group(1) == str(mh.ABI_VERSION) == "5"
    assert mh.strerror(mh.ERR_SHAPE) == "bad shape"
    assert mh.strerror(123) == "unknown error"


@pytest.mark.parametrize("text,mask", [("none", 0), ("all", 15), ("qkv", 1), ("out", 2), ("fc1", 4), ("fc2", 8),
                                       ("fc1,fc2", 12), ("qkv,out,fc1,fc2", 15), ("fc2,qkv", 9)])
def test_parse_int8_accepts(text, mask):
    assert mh.parse_int8(text) == mask


@pytest.mark.parametrize("text", ["", "None", "fc3", "fc1,", ",fc1", "fc1,,fc2", "all,fc1", "fc1 ", "qkv;out"])
def test_parse_int8_refuses(text):
    assert mh.parse_int8(text) is None


def test_sparse_domain():
    """src/server/video_models.cpp:117-126: ratio in [0, 1], local in {0, 1, 3}."""
    assert mh.check_sparse(0.0, 1) and mh.check_sparse(1.0, 3) and mh.check_sparse(0.1, 0)
    for r, l in ((-0.01, 1), (1.01, 1), (float("nan"), 1), (0.1, 2), (0.1, 4)):
        assert not mh.check_sparse(r, l)


def test_topk_k_and_cube_count():
    assert mh.cube_count(32, 48, 84) == 2016
    assert mh.cube_count(37, 24, 42) == 10 * 6 * 11          # padded to 40 x 24 x 44
    assert mh.topk_k(0.1, 2016) == 202
    assert mh.topk_k(1.0, 2016) == 2016 and mh.topk_k(0.0, 2016) == 0
    assert mh.topk_k(0.5, 2016) == 1008
    # The float ratio stands for its decimal: 0.1f * 660 = 66.000001 keeps 66 cubes, 0.3f * 10 keeps 3; a genuine
    # fraction still rounds up.
    assert mh.topk_k(0.1, 660) == 66 and mh.topk_k(0.3, 10) == 3 and mh.topk_k(0.7, 10) == 7
    assert mh.topk_k(0.1001, 660) == 67 and mh.topk_k(0.25, 7) == 2
    with pytest.raises(ValueError):
        mh.topk_k(1.5, 10)


FAKE = C.c_void_p(0x1000)        # aligned; never dereferenced: every call below fails validation first
ODD = C.c_void_p(0x1008)


def rows_args(**kw):
    a = mh.RowsArgs()
    a.rows, a.dim, a.n_sets, a.dtype, a.eps = 4, 5120, 1, mh.BF16, 1e-6
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [({"dtype": 7}, mh.ERR_PARAM), ({"eps": 0.0}, mh.ERR_PARAM),
                                     ({"dim": 5121}, mh.ERR_SHAPE), ({"dim": 0}, mh.ERR_SHAPE),
                                     ({"n_sets": 0}, mh.ERR_SHAPE), ({"dim": 16384 * 8}, mh.ERR_UNSUPPORTED),
                                     ({"set_stride": 5116}, mh.ERR_PARAM), ({"set_stride": 5122}, mh.ERR_PARAM)])
def test_rows_validation(kw, code):
    a = rows_args(**kw)
    rc = mh.lib.mh3_rms_mod_gate_add_rows(C.byref(a), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, None)
    assert rc == code


def test_rows_pointer_checks():
    a = rows_args()
    assert mh.lib.mh3_rms_mod_gate_add_rows(None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, None) == \
        mh.ERR_POINTER
    assert mh.lib.mh3_rms_mod_gate_add_rows(C.byref(a), None, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, None) == \
        mh.ERR_POINTER
    assert mh.lib.mh3_rms_mod_gate_add_rows(C.byref(a), ODD, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, None) == \
        mh.ERR_ALIGN
    z = rows_args(rows=0)
    assert mh.lib.mh3_rms_mod_gate_add_rows(C.byref(z), None, None, None, None, None, None, None, None, None) == mh.OK
    assert mh.lib.mh3_rms_mod_rows(C.byref(a), FAKE, None, None, FAKE, None, FAKE, None) == mh.ERR_POINTER
    assert mh.lib.mh3_gate_add_rows(C.byref(rows_args(eps=0.0)), FAKE, ODD, FAKE, None, None) == mh.ERR_ALIGN


def test_rows_refuse_partial_overlaps():
    """A row output may equal an input row array where documented; a shifted overlap (rows racing each other) or an
    overlap with the modulation vectors is refused."""
    a = rows_args(rows=64, dim=5120)                        # 64 rows x 10 KiB
    x, r, o = C.c_void_p(0x1000000), C.c_void_p(0x2000000), C.c_void_p(0x3000000)
    vec = C.c_void_p(0x4000000)
    lib = mh.lib
    shifted_x = C.c_void_p(0x1000000 + 10240)              # one row on
    assert lib.mh3_rms_mod_rows(C.byref(a), x, None, vec, vec, None, shifted_x, None) == mh.ERR_PARAM
    assert lib.mh3_rms_mod_rows(C.byref(a), x, None, vec, C.c_void_p(0x3000000 + 512), None, o, None) == mh.ERR_PARAM
    assert lib.mh3_gate_add_rows(C.byref(a), x, shifted_x, vec, None, None) == mh.ERR_PARAM
    assert lib.mh3_rms_mod_gate_add_rows(C.byref(a), x, r, None, vec, vec, vec, None, C.c_void_p(0x2000000 + 16),
                                         None) == mh.ERR_PARAM
    assert lib.mh3_rms_mod_gate_add_rows(C.byref(a), x, r, None, vec, vec, vec, o, o, None) == mh.ERR_PARAM   # sets
    assert lib.mh3_gate_add_rms_mod_rows(C.byref(a), x, r, vec, None, vec, vec, None, C.c_void_p(0x2000000 - 1024),
                                         None) == mh.ERR_PARAM                          # h's last row inside y
    s = mh.SwigluArgs()
    s.rows, s.dim, s.layout, s.dtype = 64, 5120, mh.SWIGLU_FUSED, mh.BF16
    assert lib.mh3_swiglu_rows(C.byref(s), x, None, x, None) == mh.ERR_PARAM           # fused rows are 2 dim wide
    s.layout = mh.SWIGLU_SPLIT
    assert lib.mh3_swiglu_rows(C.byref(s), x, r, C.c_void_p(0x2000000 + 10240), None) == mh.ERR_PARAM


def test_swiglu_validation():
    a = mh.SwigluArgs()
    a.rows, a.dim, a.layout, a.dtype = 4, 13824, mh.SWIGLU_FUSED, mh.BF16
    assert mh.lib.mh3_swiglu_rows(C.byref(a), FAKE, FAKE, FAKE, None) == mh.ERR_PARAM     # fused takes no `up`
    a.layout = 5
    assert mh.lib.mh3_swiglu_rows(C.byref(a), FAKE, None, FAKE, None) == mh.ERR_PARAM
    a.layout, a.dim = mh.SWIGLU_SPLIT, 13825
    assert mh.lib.mh3_swiglu_rows(C.byref(a), FAKE, FAKE, FAKE, None) == mh.ERR_SHAPE
    a.dim = 13824
    assert mh.lib.mh3_swiglu_rows(C.byref(a), FAKE, None, FAKE, None) == mh.ERR_POINTER
    assert mh.lib.mh3_swiglu_rows(C.byref(a), FAKE, ODD, FAKE, None) == mh.ERR_ALIGN
    a.rows = 2**31
    assert mh.lib.mh3_swiglu_rows(C.byref(a), FAKE, FAKE, FAKE, None) == mh.ERR_SHAPE


def test_cube_validation():
    a = mh.cube_args(40, (32, 48, 84), k=202, local=1)
    bad = mh.cube_args(40, (32, 48, 84), k=202, local=2)
    assert mh.lib.mh3_cube_select(C.byref(bad), FAKE, FAKE, FAKE, 1 << 30, FAKE, FAKE, None) == mh.ERR_PARAM
    bad = mh.cube_args(40, (32, 48, 84), k=0, local=1)
    assert mh.lib.mh3_cube_topk(C.byref(bad), FAKE, FAKE, FAKE, None) == mh.ERR_PARAM
    bad = mh.cube_args(40, (32, 48, 84), k=2017, local=1)
    assert mh.lib.mh3_cube_topk(C.byref(bad), FAKE, FAKE, FAKE, None) == mh.ERR_PARAM
    bad = mh.cube_args(40, (32, 48, 84), k=202, local=1, out_stride=202)
    assert mh.lib.mh3_cube_select(C.byref(bad), FAKE, FAKE, FAKE, 1 << 30, FAKE, FAKE, None) == mh.ERR_SHAPE
    bad = mh.cube_args(40, (32, 48, 84), head_dim=64)
    assert mh.lib.mh3_cube_pool(C.byref(bad), FAKE, FAKE, FAKE, FAKE, None, None) == mh.ERR_UNSUPPORTED
    bad = mh.cube_args(40, (0, 48, 84))
    assert mh.lib.mh3_cube_pool(C.byref(bad), FAKE, FAKE, FAKE, FAKE, None, None) == mh.ERR_SHAPE
    bad = mh.cube_args(40, (32, 48, 84), row_stride=100)
    assert mh.lib.mh3_cube_pool(C.byref(bad), FAKE, FAKE, FAKE, FAKE, None, None) == mh.ERR_ALIGN
    assert mh.lib.mh3_cube_pool(C.byref(a), FAKE, None, FAKE, FAKE, None, None) == mh.ERR_POINTER
    big = mh.cube_args(1, (400, 400, 400), k=10, local=1)                 # 10^6 cubes: top-k beyond 4096 cubes
    assert mh.lib.mh3_cube_topk(C.byref(big), FAKE, FAKE, FAKE, None) == mh.ERR_UNSUPPORTED


def test_cube_select_workspace():
    """cube_select's workspace: 8 KiB a (head, 16-key-cube block); refused when missing, misaligned, short, or
    overlapping an input or output (every check before any GPU call)."""
    lib = mh.lib
    a = mh.cube_args(40, (32, 48, 84), k=202, local=1)          # 2016 cubes: 126 key blocks a head
    need = lib.mh3_cube_select_workspace_bytes(C.byref(a))
    assert need == 40 * 126 * 8192
    assert lib.mh3_cube_select_workspace_bytes(C.byref(mh.cube_args(40, (0, 48, 84)))) == mh.ERR_SHAPE
    assert lib.mh3_cube_select_workspace_bytes(None) == mh.ERR_POINTER
    qc, kc, idx, cnt, ws = (C.c_void_p(b << 28) for b in (1, 2, 3, 4, 5))  # 256 MiB apart: disjoint
    sel = lambda w, n, **kw: lib.mh3_cube_select(C.byref(a), kw.get("qc", qc), kw.get("kc", kc), w, n,  # noqa: E731
                                                 kw.get("idx", idx), cnt, None)
    assert sel(None, need) == mh.ERR_POINTER
    assert sel(ODD, need) == mh.ERR_ALIGN
    assert sel(ws, need - 1) == mh.ERR_SHAPE
    assert sel(C.c_void_p((2 << 28) + 4096), need) == mh.ERR_PARAM     # inside kc
    assert sel(C.c_void_p((3 << 28) - 4096), need) == mh.ERR_PARAM     # runs into idx
    assert sel(ws, need, idx=C.c_void_p((5 << 28) + need - 16)) == mh.ERR_PARAM  # idx starts in its last unit


def test_quant_and_gemm_validation():
    q = mh.QuantArgs()
    q.rows, q.cols, q.dtype = 4, 100, mh.BF16
    assert mh.lib.mh3_quant_rows_i8(C.byref(q), FAKE, FAKE, FAKE, None) == mh.ERR_SHAPE
    q.cols, q.dtype = 128, 9
    assert mh.lib.mh3_quant_rows_i8(C.byref(q), FAKE, FAKE, FAKE, None) == mh.ERR_PARAM
    g = mh.GemmArgs()
    g.m, g.n, g.k = 100, 13824, 5120
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), FAKE, FAKE, None, FAKE, None) == mh.ERR_POINTER
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), ODD, FAKE, FAKE, FAKE, None) == mh.ERR_ALIGN
    g.k = 5000
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), FAKE, FAKE, FAKE, FAKE, None) == mh.ERR_SHAPE
    g.k, g.n = 5120, 100
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), FAKE, FAKE, FAKE, FAKE, None) == mh.ERR_SHAPE
    g.n, g.m = 128, 0
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), FAKE, FAKE, FAKE, FAKE, None) == mh.ERR_SHAPE


def test_python_wrapper_checks_sizes_before_the_library():
    import torch
    x = torch.zeros((4, 5120), dtype=torch.bfloat16)      # host tensor: refused before any call
    with pytest.raises(ValueError):
        mh.rms_mod_gate_add_rows(x, x, None, x, x, x)


def attn_args(**kw):
    a = mh.AttnArgs()
    a.cubes = mh.cube_args(2, (8, 8, 12), k=3, local=1)
    a.dense_row0, a.n_dense, a.scale = 768, 40, 0.0
    for key, val in kw.items():
        if hasattr(a.cubes, key) and key not in ("dense_row0", "n_dense", "scale"):
            setattr(a.cubes, key, val)
        else:
            setattr(a, key, val)
    return a


@pytest.mark.parametrize("kw,code", [({"layout": 2}, mh.ERR_PARAM), ({"heads": 0}, mh.ERR_SHAPE),
                                     ({"head_dim": 64}, mh.ERR_UNSUPPORTED), ({"out_stride": 0}, mh.ERR_SHAPE),
                                     ({"scale": -1.0}, mh.ERR_PARAM), ({"dense_row0": 700}, mh.ERR_PARAM),
                                     ({"row_stride": 100}, mh.ERR_ALIGN), ({"grid_w": 0}, mh.ERR_SHAPE)])
def test_flash_attn_sparse_validation(kw, code):
    """Bad geometry, a negative scale, dense rows overlapping the video rows and misaligned strides are refused."""
    a = attn_args(**kw)
    out = C.c_void_p(0x2000)
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), FAKE, FAKE, FAKE, FAKE, FAKE, out, None) == code


def test_flash_attn_sparse_pointer_checks():
    a = attn_args()
    assert mh.lib.mh3_flash_attn_sparse_128(None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None) == mh.ERR_POINTER
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), FAKE, FAKE, None, FAKE, FAKE, FAKE, None) == mh.ERR_POINTER
    out = C.c_void_p(0x2000)
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), ODD, FAKE, FAKE, FAKE, FAKE, out, None) == mh.ERR_ALIGN
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None) == mh.ERR_PARAM


def test_flash_attn_sparse_refuses_an_output_over_k_or_v():
    """out overlapping k or v (read by every other workgroup) is refused; separate arrays pass validation."""
    a = attn_args()                        # 2 heads; video rows 0 .. 767, dense rows 768 .. 807
    q, k, v = C.c_void_p(0x100000), C.c_void_p(0x200000), C.c_void_p(0x300000)
    span = (a.cubes.head_stride + 807 * a.cubes.row_stride + 128) * 2   # start to the last head's last row
    inside_v = C.c_void_p(0x300000 + span - 256)            # out's first row is v's last
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), q, k, v, FAKE, FAKE, inside_v, None) == mh.ERR_PARAM
    before_k = C.c_void_p(0x200000 - span + 256)            # out's last row is k's first
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), q, k, v, FAKE, FAKE, before_k, None) == mh.ERR_PARAM


def test_flash_attn_sparse_refuses_an_output_over_q_or_the_pass_lists():
    """out may not partially overlap q (each workgroup reads its own query tile when it starts) nor the pass lists."""
    a = attn_args()
    q, k, v = C.c_void_p(0x100000), C.c_void_p(0x200000), C.c_void_p(0x300000)
    idx, cnt = C.c_void_p(0x400000), C.c_void_p(0x500000)
    span = (a.cubes.head_stride + 807 * a.cubes.row_stride + 128) * 2
    inside_q = C.c_void_p(0x100000 + 256)                   # out one row after q's start
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), q, k, v, idx, cnt, inside_q, None) == mh.ERR_PARAM
    lists = 2 * 12 * a.cubes.out_stride * 4                 # heads x cubes x out_stride int32
    over_idx = C.c_void_p(0x400000 + lists - 16 - span + 16)  # out's last bytes on idx's last entries
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), q, k, v, idx, cnt, over_idx, None) == mh.ERR_PARAM
    over_cnt = C.c_void_p(0x500000 + 64)
    assert mh.lib.mh3_flash_attn_sparse_128(C.byref(a), q, k, v, idx, cnt, over_cnt, None) == mh.ERR_PARAM


def test_flash_attn_sparse_ordered_checks():
    """The ordered form makes the plain form's checks, needs its order (4-byte aligned) and refuses an out over it."""
    f = mh.lib.mh3_flash_attn_sparse_128_ordered
    a = attn_args()
    q, k, v = C.c_void_p(0x100000), C.c_void_p(0x200000), C.c_void_p(0x300000)
    idx, cnt, order, out = C.c_void_p(0x400000), C.c_void_p(0x500000), C.c_void_p(0x600000), C.c_void_p(0x700000)
    assert f(None, q, k, v, idx, cnt, order, out, None) == mh.ERR_POINTER
    assert f(C.byref(a), q, k, v, idx, cnt, None, out, None) == mh.ERR_POINTER
    assert f(C.byref(a), q, k, v, idx, cnt, C.c_void_p(0x600002), out, None) == mh.ERR_ALIGN
    assert f(C.byref(a), q, k, v, idx, cnt, order, C.c_void_p(0x600000 + 32), None) == mh.ERR_PARAM  # out over order
    assert f(C.byref(a), q, k, v, idx, cnt, order, q, None) == mh.ERR_PARAM
    for kw, code in [({"heads": 0}, mh.ERR_SHAPE), ({"head_dim": 64}, mh.ERR_UNSUPPORTED),
                     ({"row_stride": 100}, mh.ERR_ALIGN)]:
        assert f(C.byref(attn_args(**kw)), q, k, v, idx, cnt, order, out, None) == code


def test_cube_order_validation():
    """cube_order refuses bad geometry, null or misaligned pointers, an order over the pass lists and > 4096 cubes."""
    f = mh.lib.mh3_cube_order
    a = mh.cube_args(2, (8, 8, 12), k=3, local=1)
    idx, cnt, order = C.c_void_p(0x400000), C.c_void_p(0x500000), C.c_void_p(0x600000)
    assert f(None, idx, cnt, order, None) == mh.ERR_POINTER
    assert f(C.byref(a), None, cnt, order, None) == mh.ERR_POINTER
    assert f(C.byref(a), idx, cnt, None, None) == mh.ERR_POINTER
    assert f(C.byref(a), idx, cnt, C.c_void_p(0x600002), None) == mh.ERR_ALIGN
    assert f(C.byref(a), idx, cnt, C.c_void_p(0x500000 + 8), None) == mh.ERR_PARAM    # order over cnt
    assert f(C.byref(a), idx, cnt, C.c_void_p(0x400000 + 16), None) == mh.ERR_PARAM   # order over idx
    bad = mh.cube_args(2, (8, 8, 12), k=3, local=1)
    bad.out_stride = 0
    assert f(C.byref(bad), idx, cnt, order, None) == mh.ERR_SHAPE
    bad = mh.cube_args(1, (8, 8, 12), k=3, local=1)
    bad.head_dim = 64
    assert f(C.byref(bad), idx, cnt, order, None) == mh.ERR_UNSUPPORTED
    big = mh.cube_args(1, (64, 64, 68), k=3, local=1)   # 16 x 16 x 17 = 4352 cubes
    assert f(C.byref(big), idx, cnt, order, None) == mh.ERR_UNSUPPORTED


def test_quant_refuses_overlapping_outputs():
    a = mh.QuantArgs()
    a.rows, a.cols, a.dtype = 64, 128, mh.BF16             # w 16 KiB, q 8 KiB, scale 256 B
    w = C.c_void_p(0x100000)
    assert mh.lib.mh3_quant_rows_i8(C.byref(a), w, C.c_void_p(0x100000 + 8192), FAKE, None) == mh.ERR_PARAM
    assert mh.lib.mh3_quant_rows_i8(C.byref(a), w, C.c_void_p(0x200000), w, None) == mh.ERR_PARAM
    assert mh.lib.mh3_quant_rows_i8(C.byref(a), w, C.c_void_p(0x200000), C.c_void_p(0x200000 + 8188), None) == \
        mh.ERR_PARAM                                                                        # scale on q's last bytes


def test_gemm_refuses_an_output_that_overlaps_an_operand():
    """An out (or gate-add residual) range that overlaps x or w races with the tiles still reading them: refused."""
    g = mh.GemmArgs()
    g.m, g.n, g.k = 256, 256, 256
    x = C.c_void_p(0x100000)
    w = C.c_void_p(0x200000)
    gate = C.c_void_p(0x300000)
    inside_x = C.c_void_p(0x100000 + 256 * 256)             # out starts in the middle of x
    assert mh.lib.mh3_gemm_gate_add(C.byref(g), mh.GEMM_BF16, x, None, w, None, gate, None, inside_x, None) == \
        mh.ERR_PARAM
    assert mh.lib.mh3_gemm(C.byref(g), mh.GEMM_BF16, x, None, w, None, w, None) == mh.ERR_PARAM
    before_x = C.c_void_p(0x100000 - 256 * 256 * 2 + 16)    # out's last bytes reach into x
    assert mh.lib.mh3_gemm_gate_add(C.byref(g), mh.GEMM_W8A16, x, None, w, FAKE, gate, None, before_x, None) == \
        mh.ERR_PARAM
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), x, w, FAKE, x, None) == mh.ERR_PARAM
    out = C.c_void_p(0x400000)                              # clear of x and w, but not of the vectors below
    assert mh.lib.mh3_gemm_w8a16_swiglu(C.byref(g), x, w, C.c_void_p(0x400000 + 64), out, None) == mh.ERR_PARAM
    assert mh.lib.mh3_gemm_gate_add(C.byref(g), mh.GEMM_BF16, x, None, w, None, C.c_void_p(0x400000 + 256), None,
                                    out, None) == mh.ERR_PARAM                           # gate inside residual
    assert mh.lib.mh3_gemm_gate_add(C.byref(g), mh.GEMM_BF16, x, None, w, None, gate, C.c_void_p(0x400000), out,
                                    None) == mh.ERR_PARAM                                # set_of_row inside residual


def test_cube_map_validation():
    a = mh.CubeMapArgs()
    a.grid_t, a.grid_h, a.grid_w, a.n_dense, a.video_row0, a.dense_row0 = 32, 48, 84, 512, 512, 0
    assert mh.lib.mh3_cube_map(None, FAKE, None, None) == mh.ERR_POINTER
    assert mh.lib.mh3_cube_map(C.byref(a), None, None, None) == mh.ERR_POINTER
    a.dense_row0 = 600                                      # dense rows inside the video rows
    assert mh.lib.mh3_cube_map(C.byref(a), FAKE, None, None) == mh.ERR_PARAM
    a.dense_row0, a.grid_w = 0, 0
    assert mh.lib.mh3_cube_map(C.byref(a), FAKE, None, None) == mh.ERR_SHAPE
    a.grid_w, a.video_row0 = 84, 2**31 - 100                # model rows beyond int32
    assert mh.lib.mh3_cube_map(C.byref(a), FAKE, None, None) == mh.ERR_SHAPE


def test_selector_refuses_overlapping_outputs():
    """A selector output overlapping its inputs or another output races inside the launch: refused."""
    a = mh.CubeArgs()
    a.heads, a.head_dim, a.grid_t, a.grid_h, a.grid_w = 2, 128, 8, 8, 12
    a.layout, a.row0, a.head_stride, a.row_stride = mh.CUBES_GRID, 0, 768 * 128, 128
    a.k, a.local, a.out_stride = 4, 1, 5                     # 24 cubes
    q, k = C.c_void_p(0x100000), C.c_void_p(0x200000)      # each spans 2 * 768 * 256 bytes
    qc, kc = C.c_void_p(0x1000000), C.c_void_p(0x1010000)
    lib = mh.lib
    assert lib.mh3_cube_pool(C.byref(a), q, k, C.c_void_p(0x100000 + 768 * 256), kc, None, None) == mh.ERR_PARAM
    assert lib.mh3_cube_pool(C.byref(a), q, k, qc, qc, None, None) == mh.ERR_PARAM            # qc = kc
    assert lib.mh3_cube_pool(C.byref(a), q, k, qc, kc, C.c_void_p(0x1000000 + 16), None) == mh.ERR_PARAM
    assert lib.mh3_cube_scores(C.byref(a), qc, kc, kc, None) == mh.ERR_PARAM                  # s over kc
    s, idx, cnt = C.c_void_p(0x2000000), C.c_void_p(0x3000000), C.c_void_p(0x4000000)
    assert lib.mh3_cube_topk(C.byref(a), s, s, cnt, None) == mh.ERR_PARAM                     # idx = s
    assert lib.mh3_cube_topk(C.byref(a), s, idx, C.c_void_p(0x3000000 + 4), None) == mh.ERR_PARAM
    ws = C.c_void_p(0x5000000)
    assert lib.mh3_cube_select(C.byref(a), qc, kc, ws, 1 << 20, idx, qc, None) == mh.ERR_PARAM  # cnt = qc
    m = mh.CubeMapArgs()
    m.grid_t, m.grid_h, m.grid_w, m.n_dense, m.video_row0, m.dense_row0 = 8, 8, 12, 16, 0, 768
    assert lib.mh3_cube_map(C.byref(m), idx, C.c_void_p(0x3000000 + 64), None) == mh.ERR_PARAM


def time_args(**kw):
    a = mh.TimeArgs()
    a.levels, a.freq_dim, a.hidden, a.out_dim, a.max_period = 3, 256, 5376, 2688, 10000.0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [({"levels": 0}, mh.ERR_SHAPE), ({"levels": 65}, mh.ERR_SHAPE),
                                     ({"freq_dim": 100}, mh.ERR_SHAPE), ({"freq_dim": 2048}, mh.ERR_SHAPE),
                                     ({"hidden": 5378}, mh.ERR_SHAPE), ({"hidden": 8196}, mh.ERR_SHAPE),
                                     ({"out_dim": 0}, mh.ERR_SHAPE), ({"max_period": 1.0}, mh.ERR_PARAM)])
def test_time_embed_validation(kw, code):
    a = time_args(**kw)
    assert mh.lib.mh3_time_embed_workspace_bytes(C.byref(a)) == code
    assert mh.lib.mh3_time_embed(C.byref(a), FAKE, FAKE, None, FAKE, None, FAKE, 1 << 30, FAKE, None, None) == code


def test_time_embed_workspace_checks():
    a = time_args()
    need = mh.lib.mh3_time_embed_workspace_bytes(C.byref(a))
    assert need >= 3 * 5376 * 4 and need % 256 == 0
    assert mh.lib.mh3_time_embed(C.byref(a), FAKE, FAKE, None, FAKE, None, FAKE, need - 1, FAKE, None, None) == \
        mh.ERR_SHAPE
    assert mh.lib.mh3_time_embed(C.byref(a), FAKE, FAKE, None, FAKE, None, None, need, FAKE, None, None) == \
        mh.ERR_POINTER
    assert mh.lib.mh3_time_embed(C.byref(a), FAKE, FAKE, None, FAKE, None, ODD, need, FAKE, None, None) == \
        mh.ERR_ALIGN
    assert mh.lib.mh3_time_embed(C.byref(a), None, FAKE, None, FAKE, None, FAKE, need, FAKE, None, None) == \
        mh.ERR_POINTER


def test_time_embed_refuses_overlapping_outputs():
    """temb, cond and the workspace overlapping each other or an input would race inside the launch: refused."""
    a = time_args()
    need = mh.lib.mh3_time_embed_workspace_bytes(C.byref(a))
    t, w_in, w_out = C.c_void_p(0x1000), C.c_void_p(0x100000), C.c_void_p(0x1000000)
    ws, temb, cond = C.c_void_p(0x10000000), C.c_void_p(0x20000000), C.c_void_p(0x30000000)
    call = mh.lib.mh3_time_embed
    assert call(C.byref(a), t, w_in, None, w_out, None, ws, need, ws, None, None) == mh.ERR_PARAM      # temb = ws
    assert call(C.byref(a), t, w_in, None, w_out, None, ws, need, temb, temb, None) == mh.ERR_PARAM    # cond = temb
    inside_w_out = C.c_void_p(0x1000000 + 4096)
    assert call(C.byref(a), t, w_in, None, w_out, None, ws, need, inside_w_out, None, None) == mh.ERR_PARAM
    assert call(C.byref(a), t, w_in, None, w_out, None, C.c_void_p(0x1000 - 256), need, temb, cond, None) == \
        mh.ERR_PARAM                                                                       # ws runs into t
    assert mh.lib.mh3_time_embed_noalloc(C.byref(a), t, w_in, None, w_out, None, w_in, None, None) == mh.ERR_PARAM


def test_hip_error_text_is_recorded():
    """A valid call that fails in HIP itself returns MH3_ERR_HIP with HIP's own message in mh3_last_hip_error. Without
    a GPU the variant that allocates nothing fails at the device lookup for its scratch array, after every check of
    its arguments and before any launch."""
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a visible GPU would take the call past the device lookup to a launch on these stand-in pointers")
    a = time_args()
    t, w_in, w_out = C.c_void_p(0x1000), C.c_void_p(0x100000), C.c_void_p(0x1000000)
    temb, cond = C.c_void_p(0x20000000), C.c_void_p(0x30000000)
    assert mh.lib.mh3_time_embed_noalloc(C.byref(a), t, w_in, None, w_out, None, temb, cond, None) == mh.ERR_HIP
    text = mh.lib.mh3_last_hip_error().decode()
    assert text and text != "no error", text


def test_adaln_and_curve_refuse_overlapping_outputs():
    g = mh.GemmArgs()
    g.m, g.n, g.k = 3, 96768, 2688
    cond, w, mod = C.c_void_p(0x1000), C.c_void_p(0x100000), C.c_void_p(0x100000 + 2 * 2688 * 10)
    assert mh.lib.mh3_adaln_mod(C.byref(g), cond, w, None, mod, None) == mh.ERR_PARAM          # mod inside w
    assert mh.lib.mh3_adaln_mod(C.byref(g), cond, w, None, cond, None) == mh.ERR_PARAM         # mod = cond
    c = mh.CurveArgs()
    c.levels, c.n, c.points, c.width = 2, 96768, 1025, 8
    t, table, cw = C.c_void_p(0x1000), C.c_void_p(0x10000), C.c_void_p(0x100000)
    assert mh.lib.mh3_curve_mods(C.byref(c), t, table, cw, None, table, None) == mh.ERR_PARAM  # mod = table
    assert mh.lib.mh3_curve_mods(C.byref(c), t, table, cw, cw, C.c_void_p(0x100000 + 4 * 8 * 96768 - 4), None) == \
        mh.ERR_PARAM                                                                         # mod on w's last float


def test_adaln_and_curve_validation():
    g = mh.GemmArgs()
    g.m, g.n, g.k = 3, 96768, 2688
    assert mh.lib.mh3_adaln_mod(C.byref(g), FAKE, None, None, FAKE, None) == mh.ERR_POINTER
    assert mh.lib.mh3_adaln_mod(C.byref(g), FAKE, ODD, None, FAKE, None) == mh.ERR_ALIGN
    g.k = 2690
    assert mh.lib.mh3_adaln_mod(C.byref(g), FAKE, FAKE, None, FAKE, None) == mh.ERR_SHAPE
    g.k = 4104
    assert mh.lib.mh3_adaln_mod(C.byref(g), FAKE, FAKE, None, FAKE, None) == mh.ERR_UNSUPPORTED
    g.k, g.m = 2688, 65
    assert mh.lib.mh3_adaln_mod(C.byref(g), FAKE, FAKE, None, FAKE, None) == mh.ERR_SHAPE
    c = mh.CurveArgs()
    c.levels, c.n, c.points, c.width = 2, 96768, 1025, 8
    assert mh.lib.mh3_curve_mods(C.byref(c), FAKE, FAKE, None, None, FAKE, None) == mh.ERR_POINTER
    c.points = 1
    assert mh.lib.mh3_curve_mods(C.byref(c), FAKE, FAKE, FAKE, None, FAKE, None) == mh.ERR_SHAPE
    c.points, c.width = 1025, 33
    assert mh.lib.mh3_curve_mods(C.byref(c), FAKE, FAKE, FAKE, None, FAKE, None) == mh.ERR_SHAPE


def test_heads_partial_pool_validation():
    """The fused heads_partial + cube_pool takes only the gathered geometry of the tiles it writes."""
    grid, heads = (8, 8, 12), 2
    cubes = 2 * 2 * 3
    rows = cubes * 64 + 70
    h = mh.HeadsArgs()
    h.rows, h.model_rows, h.heads, h.head_dim, h.rot, h.eps = rows, rows, heads, 128, 96, 1e-6
    h.qkv_stride, h.out_head_stride, h.out_row_stride = 3 * heads * 128, rows * 128, 128

    base = 0x1000  # aligned; never dereferenced

    def call(cube_kw=None, qc=base + 2**38, hk=None, counts=None, **ptrs):
        ca = mh.cube_args(heads, grid, layout=mh.CUBES_GATHERED, head_stride=rows * 128)
        for key, val in (cube_kw or {}).items():
            setattr(ca, key, val)
        a = mh.HeadsArgs.from_buffer_copy(h)
        for key, val in (hk or {}).items():
            setattr(a, key, val)
        p = dict(qkv=base, cos=base, q=base + 2**34, k=base + 2**35, kc=base + 2**36)
        p.update(ptrs)
        return mh.lib.mh3_heads_partial_pool(C.byref(a), C.byref(ca), p["qkv"], None, None, p["cos"], p["cos"],
                                             p.get("map"), p["q"], p["k"], None, qc, p["kc"], counts, None)

    assert mh.lib.mh3_heads_partial_pool(None, None, *([None] * 13)) == mh.ERR_POINTER
    assert call({"layout": 2}) == mh.ERR_PARAM
    assert call({"layout": mh.CUBES_GRID}, map=base + 2**37) == mh.ERR_PARAM  # the grid layout keeps the model's order
    assert call({"layout": mh.CUBES_GRID, "row0": rows - 768 + 1}) == mh.ERR_SHAPE  # the grid's tokens past the rows
    assert call({"heads": 3}) == mh.ERR_PARAM
    assert call({"row_stride": 256}) == mh.ERR_PARAM
    assert call({"head_stride": rows * 128 + 8}) == mh.ERR_PARAM
    assert call({"row0": 71}) == mh.ERR_SHAPE                            # the cube rows run past the output rows
    assert call(hk={"rows": cubes * 64 - 1}) == mh.ERR_SHAPE
    assert call(hk={"rot": 24}) == mh.ERR_PARAM                          # heads_partial's own checks still apply
    assert call(qc=None) == mh.ERR_POINTER
    assert call(qc=base + 4) == mh.ERR_ALIGN
    assert call(kc=base + 2**36 + 8) == mh.ERR_ALIGN
    # The pooled outputs may not overlap an input, the head tiles the call writes, or each other.
    pooled = heads * cubes * 128 * 4
    assert call(qc=base) == mh.ERR_PARAM                                 # qc on qkv
    assert call(qc=base + 2**34 + 4096) == mh.ERR_PARAM                  # qc inside the q tiles
    assert call(kc=base + 2**38 + pooled - 16) == mh.ERR_PARAM          # kc runs into qc's last float4
    assert call(counts=base + 2**36 + 64) == mh.ERR_PARAM                # counts inside kc
    assert call(counts=base + 2**37, map=base + 2**37) == mh.ERR_PARAM   # counts on the map
    # heads_partial's outputs may not overlap the rotary tables or the map.
    assert call(q=base) == mh.ERR_PARAM                                  # q on qkv, not in place
    assert call(cos=base + 2**35 + 1024) == mh.ERR_PARAM                 # the cos table inside k
    assert call(map=base + 2**34 + 256) == mh.ERR_PARAM                  # the map inside q


@pytest.mark.parametrize("call,kw,code", [
    ("rms_mod", {"flags": mh.ROWS_NORM_BF16}, mh.ERR_PARAM),                       # a flag with a bf16 stream
    ("rms_mod", {"dtype": mh.F32, "flags": 4}, mh.ERR_PARAM),                      # an unknown flag
    ("rms_mod", {"dtype": mh.F32, "flags": mh.ROWS_Y_BF16}, mh.ERR_PARAM),         # no y to take
    ("gate_add", {"dtype": mh.F32, "flags": mh.ROWS_NORM_BF16}, mh.ERR_PARAM),     # no norm to give
    ("fused", {"dtype": mh.F32, "flags": mh.ROWS_NORM_BF16}, mh.ERR_PARAM),        # the fused op takes none
    ("order", {"dtype": mh.F32, "flags": mh.ROWS_Y_BF16}, mh.ERR_PARAM),           # a bf16 y needs a bf16 h
    ("rms_mod", {"dtype": mh.F32, "flags": mh.ROWS_NORM_BF16, "dim": 6152}, mh.ERR_UNSUPPORTED),
    ("rms_mod", {"dtype": mh.F32, "flags": mh.ROWS_NORM_BF16, "dim": 5124}, mh.ERR_SHAPE),
])
def test_float_stream_flags_validation(call, kw, code):
    """The float residual stream's flags: only with a float stream, only where the entry point takes them, and within
    the widths its kernel holds."""
    a = rows_args(**kw)
    if call == "rms_mod":
        rc = mh.lib.mh3_rms_mod_rows(C.byref(a), FAKE, FAKE, FAKE, FAKE, None, C.c_void_p(0x10000000), None)
    elif call == "gate_add":
        rc = mh.lib.mh3_gate_add_rows(C.byref(a), FAKE, C.c_void_p(0x10000000), FAKE, None, None)
    elif call == "fused":
        rc = mh.lib.mh3_rms_mod_gate_add_rows(C.byref(a), FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None,
                                              C.c_void_p(0x10000000), None)
    else:
        rc = mh.lib.mh3_gate_add_rms_mod_rows(C.byref(a), FAKE, C.c_void_p(0x10000000), FAKE, FAKE, FAKE, FAKE, None,
                                              C.c_void_p(0x20000000), None)
    assert rc == code


def test_float_stream_outputs_may_not_share_the_float_rows():
    """A bf16 output may not sit on the float x, not even at its start (its rows are half as long, so they race the
    float rows); the float residual of the GEMM epilogue may not overlap x."""
    a = rows_args(rows=64, dim=5120, dtype=mh.F32, flags=mh.ROWS_NORM_BF16)
    x, v = C.c_void_p(0x1000000), C.c_void_p(0x9000000)
    assert mh.lib.mh3_rms_mod_rows(C.byref(a), x, v, v, v, None, x, None) == mh.ERR_PARAM
    assert mh.lib.mh3_rms_mod_rows(C.byref(a), x, v, v, v, None, C.c_void_p(0x1000000 + 64 * 5120 * 4 - 16),
                                   None) == mh.ERR_PARAM
    g = mh.GemmArgs()
    g.m, g.n, g.k = 512, 256, 512
    xg, wg = C.c_void_p(0x1000000), C.c_void_p(0x2000000)
    inside_x = C.c_void_p(0x1000000 + 512 * 512 * 2 - 16)   # the residual's first float4 on x's last bytes
    assert mh.lib.mh3_gemm_gate_add_f32(C.byref(g), mh.GEMM_BF16, xg, None, wg, None, v, None, inside_x, None) == \
        mh.ERR_PARAM
