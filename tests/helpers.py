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


BF16_NAN = -1  # 0xffff as int16: a bf16 NaN, the fill that shows any output element a kernel leaves unwritten


def nan_filled(shape, device):
    """A bf16 output buffer every element of which is NaN until written."""
    return torch.full(shape, BF16_NAN, dtype=torch.int16, device=device).view(torch.bfloat16)


def check_rows_f64(got: torch.Tensor, want: torch.Tensor, what: str, rtol=1e-2, row_frac=1e-4):
    """Every element of a bf16 (or float) result against a float64 restatement on the GPU: finite, and
    |got - want| <= rtol |want| + row_frac rms(want's row). The row term covers results that cancel to near zero (a dot
    product of 5120 terms whose float32 accumulation error is a fixed fraction of its row's scale); rtol is the bf16
    bar. Returns the reference's diff() pair over the block."""
    g = got.double()
    assert bool(torch.isfinite(g).all()), f"{what}: non-finite outputs (an unwritten or corrupted element)"
    rms = want.pow(2).mean(1, keepdim=True).sqrt()
    err = (g - want).abs()
    bound = rtol * want.abs() + row_frac * rms
    bad = err > bound
    if bool(bad.any()):
        i = int(torch.argmax((err - bound).flatten()))
        r, c = divmod(i, want.shape[1])
        raise AssertionError(f"{what}: {int(bad.sum())} elements beyond tolerance; worst at ({r}, {c}) got "
                             f"{float(g[r, c])!r} want {float(want[r, c])!r}")
    e2, w2 = float(((g - want) ** 2).sum()), float((want ** 2).sum())
    gw = (g * want).sum(1)
    cos = gw / (g.pow(2).sum(1).sqrt() * want.pow(2).sum(1).sqrt()).clamp_min(1e-300)
    return (e2 / max(w2, 1e-300)) ** 0.5, float(cos.min())


def check_gemm_full(out: torch.Tensor, x: torch.Tensor, w: torch.Tensor, what: str, *, x_scale=None, w_scale=None,
                    epi: str = "store", residual0=None, gate=None, set_of_row=None, chunk: int = 4096,
                    rtol: float = 1e-2, row_frac: float = 1e-4):
    """Every element of a GEMM's output against float64 products on the GPU over the same operands, row chunk by row
    chunk: y = (x * x_scale[row]) (w * w_scale[col])^T, then epi "store" (out = y), "swiglu" (out = silu(y[:, :n]) *
    y[:, n:], n = out's width) or "gate_add" (out = residual0 + gate[set_of_row[row]] * y)."""
    m, n = out.shape
    wd = w.double()
    if w_scale is not None:
        wd = wd * w_scale.double()[:, None]
    wt = wd.t().contiguous()
    del wd
    if gate is not None:
        gate2 = gate.double().reshape(-1, gate.shape[-1])[:, :n]
    worst_rel, worst_cos = 0.0, 1.0
    for r0 in range(0, m, chunk):
        r1 = min(m, r0 + chunk)
        xs = x[r0:r1].double()
        if x_scale is not None:
            xs = xs * x_scale[r0:r1].double()[:, None]
        y = xs @ wt
        if epi == "swiglu":
            g, u = y[:, :n], y[:, n:]
            want = g * torch.sigmoid(g) * u
        elif epi == "gate_add":
            gr = gate2[set_of_row[r0:r1].long()] if set_of_row is not None else gate2[:1]
            want = residual0[r0:r1].double() + gr * y
        else:
            want = y
        rel, cos = check_rows_f64(out[r0:r1], want, f"{what} rows {r0}..{r1 - 1}", rtol, row_frac)
        worst_rel, worst_cos = max(worst_rel, rel), min(worst_cos, cos)
    return worst_rel, worst_cos


# ---- sparse attention on the GPU, in float32 -------------------------------------------------------------------------

def cube_rows_table(grid, layout: int, row0: int, device) -> torch.Tensor:
    """int64 [cubes][64]: the row of cube c's slot l = (dt * 4 + dy) * 4 + dx, or -1 where (4 ct + dt, 4 cy + dy,
    4 cx + dx) lies in the padding past the grid. layout 0 (grid): the token's row in the model's frame-major order;
    layout 1 (gathered): row0 + 64 c + l."""
    gt, gh, gw = grid
    ct_n, ch, cw = (gt + 3) // 4, (gh + 3) // 4, (gw + 3) // 4
    c = torch.arange(ct_n * ch * cw, device=device)[:, None]
    slot = torch.arange(64, device=device)[None, :]
    t = 4 * (c // (ch * cw)) + slot // 16
    y = 4 * (c // cw % ch) + slot // 4 % 4
    x = 4 * (c % cw) + slot % 4
    inside = (t < gt) & (y < gh) & (x < gw)
    row = row0 + 64 * c + slot if layout == 1 else row0 + (t * gh + y) * gw + x
    return torch.where(inside, row, torch.full_like(row, -1))


def attn_sparse_f32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, idx: torch.Tensor, cnt: torch.Tensor, grid,
                    dense_row0: int, n_dense: int, *, layout: int = 0, row0: int = 0, heads=None, cubes=None,
                    dense: bool = True, scale: float | None = None, chunk: int = 64) -> dict:
    """flash_attn_sparse_128's semantics restated with torch in float32 on the GPU, for checking whole launches.
    q, k, v: bf16 [heads][rows][128]; idx int32 [heads][cubes][stride], cnt int32 [heads][cubes] (entries past cnt,
    and entries outside [0, cubes), are skipped). The queries of cube c attend the tokens of its listed cubes and the
    dense rows; a dense row's query attends every token and every dense row. Returns {h: (rows, out)} for each head
    of `heads` (default all): the rows computed (the dense rows when `dense`, then the tokens of the query cubes
    `cubes`, default all) and float32 [len(rows)][128] results."""
    scale = 1.0 / 128 ** 0.5 if scale is None else scale
    dev = q.device
    table = cube_rows_table(grid, layout, row0, dev)
    n_cubes = table.shape[0]
    tokens = table[table >= 0]
    drows = torch.arange(dense_row0, dense_row0 + n_dense, device=dev)
    every_key = torch.cat([tokens, drows])
    cubes = torch.arange(n_cubes, device=dev) if cubes is None else torch.as_tensor(cubes, device=dev).long()
    res = {}
    for h in (range(q.shape[0]) if heads is None else heads):
        Q, K, V = q[h].float(), k[h].float(), v[h].float()
        rows_out, outs = [], []
        if dense and n_dense:
            s = (Q[drows] @ K[every_key].t().contiguous()) * scale
            outs.append(torch.softmax(s, -1) @ V[every_key])
            rows_out.append(drows)
        stride = idx.shape[2]
        for c0 in range(0, len(cubes), chunk):
            cs = cubes[c0:c0 + chunk]
            lists = idx[h, cs].long()                                        # [B][stride]
            live = (torch.arange(stride, device=dev)[None, :] < cnt[h, cs].long().clamp(0, stride)[:, None]) & \
                (lists >= 0) & (lists < n_cubes)
            kr = table[lists.clamp(0, n_cubes - 1)]                          # [B][stride][64]
            key_ok = (live[..., None] & (kr >= 0)).flatten(1)
            kr = kr.flatten(1)
            if n_dense:
                kr = torch.cat([kr, drows[None, :].expand(len(cs), -1)], 1)
                key_ok = torch.cat([key_ok, torch.ones((len(cs), n_dense), dtype=torch.bool, device=dev)], 1)
            kr = kr.clamp_min(0)
            qr = table[cs]                                                   # [B][64]
            qv = Q[qr.clamp_min(0)]                                          # [B][64][128]
            s = torch.bmm(qv, K[kr].transpose(1, 2).contiguous()) * scale    # [B][64][L]
            s = s.masked_fill(~key_ok[:, None, :], float("-inf"))
            o = torch.bmm(torch.softmax(s, -1), V[kr])                       # [B][64][128]
            tok = qr >= 0
            rows_out.append(qr[tok])
            outs.append(o[tok])
        res[h] = (torch.cat(rows_out), torch.cat(outs))
    return res


def check_attn_f32(got: torch.Tensor, ref: dict, what: str, elem_row=1e-2, row_rms=6e-3):
    """Sparse-attention outputs (bf16 [heads][rows][128]) against attn_sparse_f32's results, every listed row:
    finite; each element within 1e-2 of itself plus `elem_row` of its row's RMS; each row's RMS error within `row_rms`
    of the row's RMS. The bf16 P operand of the P V product rounds each probability by up to 2^-9 relative, and the
    output's own bf16 rounding adds as much: together about 3e-3 of a row's RMS, spread over its 128 values.
    Returns (worst element error / row RMS, worst row RMS error / row RMS)."""
    worst_e, worst_r = 0.0, 0.0
    for h, (rows, want) in ref.items():
        g = got[h, rows].float()
        assert bool(torch.isfinite(g).all()), f"{what} head {h}: non-finite outputs (an unwritten element)"
        rms = want.pow(2).mean(1, keepdim=True).sqrt().clamp_min(1e-30)
        err = (g - want).abs()
        bad = err > 1e-2 * want.abs() + elem_row * rms
        assert not bool(bad.any()), \
            f"{what} head {h}: {int(bad.sum())} elements beyond tolerance, worst {float((err / rms).max()):.3g} of rms"
        rerr = err.pow(2).mean(1, keepdim=True).sqrt() / rms
        assert bool((rerr <= row_rms).all()), f"{what} head {h}: row RMS error {float(rerr.max()):.3g} of the row's RMS"
        worst_e, worst_r = max(worst_e, float((err / rms).max())), max(worst_r, float(rerr.max()))
    return worst_e, worst_r
