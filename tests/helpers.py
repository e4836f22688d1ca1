"""Comparison helpers shared by the parity tests."""
from __future__ import annotations

import numpy as np
import torch


def to_bits(t: torch.Tensor) -> np.ndarray:
    """A bf16 tensor's raw bits as numpy uint16 (host copy)."""
    assert t.dtype == torch.bfloat16
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def from_bits(a: np.ndarray, device) -> torch.Tensor:
    """numpy uint16 bf16 bits -> a bf16 tensor on `device`."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)


def bits_to_f64(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def randn_bf16_bits(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    """N(0, scale^2) samples rounded to bf16 (nearest even), as uint16 bits."""
    f = (rng.standard_normal(shape) * scale).astype(np.float32)
    return torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def diff(got: np.ndarray, want: np.ndarray, width: int) -> tuple[float, float]:
    """The reference's comparison metric (tests/h3_ref_test.cpp:67-90): relative RMS error over everything, and the
    lowest cosine similarity of a row of `width`."""
    g = got.astype(np.float64).reshape(-1, width)
    w = want.astype(np.float64).reshape(-1, width)
    rel = float(np.sqrt(((g - w) ** 2).sum() / (w ** 2).sum()))
    gw, gg, ww = (g * w).sum(1), (g * g).sum(1), (w * w).sum(1)
    ok = (gg > 0) & (ww > 0)
    cos = np.ones(len(g))
    cos[ok] = gw[ok] / np.sqrt(gg[ok] * ww[ok])
    return rel, float(cos.min())


def assert_close(got, want, rtol, atol, what=""):
    """Elementwise |got - want| <= atol + rtol |want| (finite values), NaN where and only where want is NaN."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    assert g.shape == w.shape, f"{what}: shape {g.shape} vs {w.shape}"
    nan_g, nan_w = np.isnan(g), np.isnan(w)
    assert (nan_g == nan_w).all(), f"{what}: NaN mismatch at {np.argwhere(nan_g != nan_w)[:5]}"
    fin = ~nan_w
    inf_w = np.isinf(w) & fin
    assert (g[inf_w] == w[inf_w]).all(), f"{what}: infinity mismatch"
    m = fin & ~inf_w
    err = np.abs(g[m] - w[m])
    bound = atol + rtol * np.abs(w[m])
    bad = err > bound
    if bad.any():
        i = np.argmax(err - bound)
        raise AssertionError(f"{what}: {int(bad.sum())} of {m.sum()} beyond tolerance (rtol {rtol}, atol {atol}); "
                             f"worst got {g[m][i]!r} want {w[m][i]!r}")


def check_selection(gpu_idx, gpu_cnt, scores64, oracle_idx, oracle_cnt, k, rel_tie=1e-3):
    """Selected cube sets equal the oracle's except at the k-th boundary, where the oracle's float64 scores of every
    swapped cube tie with the k-th score within `rel_tie` relative. Returns the number of rows that differed."""
    rows = gpu_cnt.size
    g_idx = gpu_idx.reshape(rows, -1)
    o_idx = oracle_idx.reshape(rows, -1)
    s = scores64.reshape(rows, -1)
    g_cnt, o_cnt = gpu_cnt.reshape(-1), oracle_cnt.reshape(-1)
    differ = 0
    for r in range(rows):
        gs = g_idx[r, : g_cnt[r]]
        os_ = o_idx[r, : o_cnt[r]]
        assert (g_idx[r, g_cnt[r]:] == -1).all(), f"row {r}: padding is not -1"
        assert (np.diff(gs) > 0).all(), f"row {r}: not strictly ascending"
        if gs.size == os_.size and (gs == os_).all():
            continue
        differ += 1
        kth = np.sort(s[r])[::-1][k - 1]
        swapped = np.setxor1d(gs, os_)
        tol = rel_tie * max(abs(kth), 1e-30)
        assert (np.abs(s[r][swapped] - kth) <= tol).all(), \
            f"row {r}: cubes {swapped} differ beyond the tie band (k-th score {kth}, theirs {s[r][swapped]})"
    return differ
