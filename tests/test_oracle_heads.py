"""Pins the oracle's heads_partial (CPU): the per-head RMS norm against torch.nn.functional.rms_norm in float64, the
rotary positions against a complex product written independently (the (i, i + rot/2) pairs as complex numbers times
e^(i angle), torch.polar), plus invariants: angle 0 is the plain norm, angle pi/2 maps (a, b) to (-b, a), a rotation
keeps each pair's length, v is a copy, map entries outside the rows give zeros, and a gather through a map equals
indexing the ungathered result."""
import numpy as np
import pytest
import torch

import oracle as orc
from helpers import bits_to_f64, randn_bf16_bits


def torch_heads(qkv_bits, heads, q_w, k_w, cos_t, sin_t, rot, eps):
    """The same op in float64 torch, written from the definition: F.rms_norm over each head, then the rotation as a
    complex product; rounded to bf16 by the oracle's double -> bf16 (its nearest-even rounding is pinned separately)."""
    rows = qkv_bits.shape[0]
    x = torch.from_numpy(bits_to_f64(qkv_bits)[:, : 3 * heads * 128].reshape(rows, 3, heads, 128))
    outs = []
    for kind, w in ((0, q_w), (1, k_w)):
        wt = None if w is None else torch.from_numpy(w.astype(np.float64))
        y = torch.nn.functional.rms_norm(x[:, kind], (128,), weight=wt, eps=eps)  # [rows][heads][128]
        if rot:
            half = rot // 2
            z = torch.complex(y[..., :half], y[..., half:rot])
            ang = torch.atan2(torch.from_numpy(sin_t.astype(np.float64)), torch.from_numpy(cos_t.astype(np.float64)))
            mag = torch.from_numpy(np.hypot(cos_t.astype(np.float64), sin_t.astype(np.float64)))
            z = z * torch.polar(mag, ang)[:, None, :]
            y = torch.cat([z.real, z.imag, y[..., rot:]], dim=-1)
        outs.append(orc.bf16_from_f64(y.permute(1, 0, 2).contiguous().numpy()))
    v = np.ascontiguousarray(qkv_bits[:, 2 * heads * 128: 3 * heads * 128].reshape(rows, heads, 128).transpose(1, 0, 2))
    return outs[0], outs[1], v


def inputs(rng, rows, heads, rot, extra_cols=0, weights=True):
    qkv = randn_bf16_bits(rng, (rows, 3 * heads * 128 + extra_cols), 1.5)
    ang = rng.uniform(-np.pi, np.pi, (rows, rot // 2))
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q_w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32) if weights else None
    k_w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32) if weights else None
    return qkv, q_w, k_w, cos_t, sin_t


@pytest.mark.parametrize("rows,heads,rot,extra,weights", [(7, 1, 96, 0, True), (33, 3, 128, 16, False),
                                                          (20, 2, 16, 0, True), (9, 4, 0, 8, True)])
def test_heads_partial_matches_torch(rows, heads, rot, extra, weights):
    rng = np.random.default_rng(rows * 7 + heads + rot)
    qkv, q_w, k_w, cos_t, sin_t = inputs(rng, rows, heads, rot, extra, weights)
    got = orc.heads_partial(qkv, heads, q_w, k_w, cos_t, sin_t, rot=rot, eps=1e-6)
    want = torch_heads(qkv, heads, q_w, k_w, cos_t, sin_t, rot, 1e-6)
    for name, g, w in zip("qkv", got, want):
        gf, wf = bits_to_f64(g), bits_to_f64(w)
        # Both are float64 computations rounded once; they may differ only where a value sits on a rounding tie.
        assert (g == w).mean() > 0.999, name
        assert np.allclose(gf, wf, rtol=2 ** -7, atol=1e-30), name
    assert np.array_equal(got[2], want[2])


def test_heads_partial_angle_zero_is_plain_norm_and_quarter_turn_swaps():
    rng = np.random.default_rng(1)
    rows, heads, rot = 5, 2, 96
    qkv, q_w, k_w, _, _ = inputs(rng, rows, heads, rot)
    ones, zeros = np.ones((rows, rot // 2), np.float32), np.zeros((rows, rot // 2), np.float32)
    q0, k0, _ = orc.heads_partial(qkv, heads, q_w, k_w, ones, zeros, rot=rot)
    qn, kn, _ = orc.heads_partial(qkv, heads, q_w, k_w, None, None, rot=0)
    assert np.array_equal(q0, qn) and np.array_equal(k0, kn)
    x = torch.from_numpy(bits_to_f64(qkv).reshape(rows, 3, heads, 128))
    plain = torch.nn.functional.rms_norm(x[:, 0], (128,), weight=torch.from_numpy(q_w.astype(np.float64)), eps=1e-6)
    assert np.array_equal(qn, orc.bf16_from_f64(plain.permute(1, 0, 2).contiguous().numpy()))
    q90, _, _ = orc.heads_partial(qkv, heads, q_w, k_w, zeros, ones, rot=rot)
    h = rot // 2
    a, b = bits_to_f64(qn)[..., :h], bits_to_f64(qn)[..., h:rot]
    assert np.array_equal(bits_to_f64(q90)[..., :h], -b) and np.array_equal(bits_to_f64(q90)[..., h:rot], a)
    assert np.array_equal(q90[..., rot:], qn[..., rot:])


def test_heads_partial_rotation_keeps_pair_length():
    rng = np.random.default_rng(2)
    rows, heads, rot = 16, 2, 96
    qkv, q_w, k_w, cos_t, sin_t = inputs(rng, rows, heads, rot)
    qr, _, _ = orc.heads_partial(qkv, heads, q_w, k_w, cos_t, sin_t, rot=rot)
    qn, _, _ = orc.heads_partial(qkv, heads, q_w, k_w, None, None, rot=0)
    h = rot // 2
    lr = np.hypot(bits_to_f64(qr)[..., :h], bits_to_f64(qr)[..., h:rot])
    ln = np.hypot(bits_to_f64(qn)[..., :h], bits_to_f64(qn)[..., h:rot])
    assert np.allclose(lr, ln, rtol=2 ** -6, atol=1e-3)


def test_heads_partial_map_gathers_and_pads():
    rng = np.random.default_rng(3)
    rows, heads, rot = 12, 3, 96
    qkv, q_w, k_w, cos_t, sin_t = inputs(rng, rows, heads, rot)
    full = orc.heads_partial(qkv, heads, q_w, k_w, cos_t, sin_t, rot=rot)
    m = np.array([5, -1, 0, 11, 11, 12, 3, -7, 2], np.int32)  # 12 and -7 are outside the rows: padding
    got = orc.heads_partial(qkv, heads, q_w, k_w, cos_t, sin_t, rot=rot, map_=m)
    valid = (m >= 0) & (m < rows)
    for g, f in zip(got, full):
        assert np.array_equal(g[:, valid], f[:, m[valid]])
        assert (g[:, ~valid] == 0).all()
    _, _, nov = orc.heads_partial(qkv, heads, q_w, k_w, cos_t, sin_t, rot=rot, with_v=False)
    assert nov is None
