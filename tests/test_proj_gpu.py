"""Parity of the qkv / out / fc2 projections (mh3_gemm, mh3_gemm_gate_add) with the oracle, in each operand form:
bf16 outputs within 1e-2 relative plus 1e-4 of the row's RMS (products of a few thousand terms can cancel to near
zero, where the float32 accumulation error is a fixed fraction of the row's scale), the reference's diff() pair, the gate-add in place on the residual with per-row gate sets, and the error paths."""
import numpy as np
import pytest
import torch

import mako_h3 as mh
import oracle as orc
from helpers import bits_to_f64, check_gemm_full, diff, from_bits, nan_filled, randn_bf16_bits, to_bits

pytestmark = pytest.mark.gpu

FORMS = {"w8a16": orc.GEMM_W8A16, "bf16": orc.GEMM_BF16, "w8a8": orc.GEMM_W8A8}


def operands(rng, form, m, n, k):
    if form == orc.GEMM_W8A8:
        x = rng.integers(-127, 128, (m, k), dtype=np.int8)
        xs = rng.uniform(0.5e-2, 2e-2, m).astype(np.float32)
    else:
        x, xs = randn_bf16_bits(rng, (m, k)), None
    if form == orc.GEMM_BF16:
        w, ws = randn_bf16_bits(rng, (n, k), 0.02), None
    else:
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        ws = rng.uniform(0.5e-3, 2e-3, n).astype(np.float32)
    return x, xs, w, ws


def on_dev(dev, x, xs, w, ws):
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    tx = from_bits(x, dev) if x.dtype == np.uint16 else t(x)
    tw = from_bits(w, dev) if w.dtype == np.uint16 else t(w)
    return tx, t(xs), tw, t(ws)


def check(got_bits, want_bits, width, what):
    g, w = bits_to_f64(got_bits).reshape(-1, width), bits_to_f64(want_bits).reshape(-1, width)
    scale = np.sqrt((w ** 2).mean(1, keepdims=True)) + 1e-30
    err = np.abs(g - w)
    assert np.all(err <= 1e-2 * np.abs(w) + 1e-4 * scale), f"{what}: worst {(err / (np.abs(w) + scale)).max():.3g}"
    rel, cos = diff(g, w, width)
    assert rel < 5e-3 and cos > 0.9999, f"{what}: rel {rel:.3g} cos {cos:.6f}"


SHAPES = [(1, 256, 128), (37, 512, 256), (300, 256, 384), (513, 768, 640)]


@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_store(dev, form, m, n, k):
    f = FORMS[form]
    rng = np.random.default_rng(m + n + k + f)
    x, xs, w, ws = operands(rng, f, m, n, k)
    tx, txs, tw, tws = on_dev(dev, x, xs, w, ws)
    got = to_bits(mh.gemm(tx, tw, x_scale=txs, w_scale=tws))
    check(got, orc.gemm(x, w, f, xs, ws), n, f"gemm {form} {m}x{k}->{n}")


@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_gate_add(dev, form, m, n, k):
    f = FORMS[form]
    rng = np.random.default_rng(7 * m + n + k + f)
    x, xs, w, ws = operands(rng, f, m, n, k)
    res = randn_bf16_bits(rng, (m, n))
    gate = (0.5 * rng.standard_normal((3, n))).astype(np.float32)
    sets = rng.integers(0, 3, m).astype(np.uint8)
    tx, txs, tw, tws = on_dev(dev, x, xs, w, ws)
    tres = from_bits(res, dev)
    out = mh.gemm_gate_add(tx, tw, tres, torch.from_numpy(gate).to(dev), x_scale=txs, w_scale=tws,
                           set_of_row=torch.from_numpy(sets).to(dev), n_sets=3)
    assert out.data_ptr() == tres.data_ptr()
    want = orc.gemm_gate_add(x, w, f, res, gate, xs, ws, sets)
    check(to_bits(tres), want, n, f"gemm_gate_add {form} {m}x{k}->{n}")


def test_gemm_gate_add_zero_gate_leaves_residual(dev):
    rng = np.random.default_rng(3)
    x, xs, w, ws = operands(rng, orc.GEMM_BF16, 100, 256, 128)
    res = randn_bf16_bits(rng, (100, 256))
    tx, _, tw, _ = on_dev(dev, x, xs, w, ws)
    tres = from_bits(res, dev)
    mh.gemm_gate_add(tx, tw, tres, torch.zeros(256, device=dev))
    assert np.array_equal(to_bits(tres), res)


def test_gemm_store_equals_fc1_halves(dev):
    """The qkv kernel's plain store equals the fc1 kernel's products: with w the stacked [gate; up] rows and SwiGLU
    taken on the host from the stored y, the result matches gemm_bf16_swiglu within one bf16 rounding of y."""
    rng = np.random.default_rng(4)
    m, n, k = 64, 256, 256
    x = randn_bf16_bits(rng, (m, k))
    w = randn_bf16_bits(rng, (2 * n, k), 0.05)
    tx, tw = from_bits(x, dev), from_bits(w, dev)
    y = mh.gemm(tx, tw).float()
    sw = (torch.nn.functional.silu(y[:, :n]) * y[:, n:]).double().cpu().numpy()
    fused = bits_to_f64(to_bits(mh.gemm_bf16_swiglu(tx, tw)))
    assert np.allclose(fused, sw, rtol=2e-2, atol=2e-2 * np.abs(sw).mean())


@pytest.mark.parametrize("which,form", [("qkv", "bf16"), ("qkv", "w8a8"), ("out", "w8a16"), ("fc2", "w8a16"),
                                        ("fc2", "bf16")])
def test_gemm_768p_every_row(dev, which, form):
    """The 768p projections at full size (129,536 rows): qkv 5120 -> 15,360, the out projection 5120 -> 5120 and fc2
    13,824 -> 5120 with the gate-add (three gate sets, a set a row), in the weight forms the reference runs them in.
    qkv writes into a NaN-filled output; every element of every projection is checked against float64 products on
    the GPU over the same operands, and 16 sampled rows against the oracle."""
    m = 129536
    k, n = {"qkv": (5120, 15360), "out": (5120, 5120), "fc2": (13824, 5120)}[which]
    f = FORMS[form]
    g = torch.Generator(device=dev).manual_seed(5 + f)
    if f == orc.GEMM_W8A8:
        x = torch.randint(-127, 128, (m, k), generator=g, device=dev, dtype=torch.int8)
        xs = (torch.rand(m, generator=g, device=dev) * 0.01 + 0.005).float()
    else:
        x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
        xs = None
    if f == orc.GEMM_BF16:
        w = (0.02 * torch.randn((n, k), generator=g, device=dev)).to(torch.bfloat16)
        ws = None
    else:
        w = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
        ws = (torch.rand(n, generator=g, device=dev) * 1.5e-3 + 0.5e-3).float()
    if which == "qkv":
        out = mh.gemm(x, w, x_scale=xs, w_scale=ws, out=nan_filled((m, n), dev))
        rel, cos = check_gemm_full(out, x, w, f"{which} {form} 768p", x_scale=xs, w_scale=ws)
    else:
        res = torch.randn((m, n), generator=g, device=dev).to(torch.bfloat16)
        res0 = res.clone()
        gate = (0.1 * torch.randn((3, n), generator=g, device=dev)).float()
        sets = torch.randint(0, 3, (m,), generator=g, device=dev, dtype=torch.uint8)
        out = mh.gemm_gate_add(x, w, res, gate, x_scale=xs, w_scale=ws, set_of_row=sets, n_sets=3)
        rel, cos = check_gemm_full(out, x, w, f"{which} {form} 768p", x_scale=xs, w_scale=ws, epi="gate_add",
                                   residual0=res0, gate=gate, set_of_row=sets)
    assert rel < 5e-3 and cos > 0.9999, (rel, cos)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, m - 1], np.random.default_rng(0).integers(0, m, 11)]))
    ri = torch.from_numpy(rows).to(dev)
    xb = to_bits(x[ri]) if f != orc.GEMM_W8A8 else x[ri].cpu().numpy()
    wb = to_bits(w) if f == orc.GEMM_BF16 else w.cpu().numpy()
    xsb = None if xs is None else xs[ri].cpu().numpy()
    wsb = None if ws is None else ws.cpu().numpy()
    if which == "qkv":
        want = orc.gemm(xb, wb, f, xsb, wsb)
    else:
        want = orc.gemm_gate_add(xb, wb, f, to_bits(res0[ri]), gate.cpu().numpy(), xsb, wsb,
                                 sets[ri].cpu().numpy())
    check(to_bits(out[ri]), want, n, f"{which} {form} 768p oracle rows")


def test_gemm_rejects_bad_calls(dev):
    x = torch.zeros((8, 128), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((256, 128), dtype=torch.bfloat16, device=dev)
    out = torch.empty((8, 256), dtype=torch.bfloat16, device=dev)

    def call(form=mh.GEMM_BF16, n=256, k=128, gate=True, **kw):
        a = mh.GemmArgs()
        a.m, a.n, a.k = 8, n, k
        for key, val in kw.items():
            setattr(a, key, val)
        g = torch.zeros(n, device=dev) if gate else None
        return mh.lib.mh3_gemm_gate_add(mh.C.byref(a), form, x.data_ptr(), None, w.data_ptr(), None,
                                        None if g is None else g.data_ptr(), None, out.data_ptr(), mh._stream())

    assert call(n=128) == mh.ERR_SHAPE          # n a multiple of 256
    assert call(k=96) == mh.ERR_SHAPE           # k a multiple of 64
    assert call(form=7) == mh.ERR_PARAM
    assert call(gate=False) == mh.ERR_POINTER
    assert call(gate_stride=100) == mh.ERR_PARAM
    assert call(form=mh.GEMM_W8A16) == mh.ERR_POINTER   # int8 weights need their scale
    torch.cuda.synchronize()
    with pytest.raises(ValueError):
        mh.gemm(x, torch.zeros((256, 64), dtype=torch.bfloat16, device=dev))
