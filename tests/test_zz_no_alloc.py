"""mh3_time_embed_noalloc, the time embedding with its hidden layer in the library's own per-GPU array instead of a
caller's workspace, called through the C-ABI: bit-identical to mh3_time_embed on two calls in a row, the second
smaller than the first (fewer levels and a narrower hidden layer, so it reads only what it wrote itself), and sizes
beyond the array refused before any launch."""
import ctypes as C
import math

import pytest
import torch

import mako_h3 as mh

pytestmark = pytest.mark.gpu


def weights(dev, freq_dim, hidden, out_dim, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn((hidden, freq_dim), generator=g, device=dev) / math.sqrt(freq_dim),
            0.1 * torch.randn(hidden, generator=g, device=dev),
            torch.randn((out_dim, hidden), generator=g, device=dev) / math.sqrt(hidden),
            0.1 * torch.randn(out_dim, generator=g, device=dev))


def noalloc(t, w_in, b_in, w_out, b_out):
    levels = t.numel()
    hidden, freq_dim = w_in.shape
    out_dim = w_out.shape[0]
    a = mh.TimeArgs()
    a.levels, a.freq_dim, a.hidden, a.out_dim, a.max_period = levels, freq_dim, hidden, out_dim, 10000.0
    temb = torch.full((levels, out_dim), float("nan"), device=t.device)
    cond = torch.full((levels, out_dim), -1, dtype=torch.int16, device=t.device).view(torch.bfloat16)
    rc = mh.lib.mh3_time_embed_noalloc(C.byref(a), t.data_ptr(), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(),
                                       b_out.data_ptr(), temb.data_ptr(), cond.data_ptr(), mh._stream())
    assert rc == mh.OK, mh.strerror(rc)
    return temb, cond


def test_noalloc_equals_the_workspace_entry_point(dev):
    # first call: H3's shape, 3 levels (16,128 floats of the array)
    big = weights(dev, 256, 5376, 2688, 1)
    t3 = torch.tensor([0.9230769, 0.5, 0.999], device=dev)
    temb, cond = noalloc(t3, *big)
    want_t, want_c = mh.time_embed(t3, *big)
    torch.cuda.synchronize()
    assert torch.equal(temb, want_t)
    assert torch.equal(cond.view(torch.int16), want_c.view(torch.int16))
    # second call, smaller: 2 levels of a 1024-wide hidden layer; the array still holds the first call's values
    small = weights(dev, 128, 1024, 300, 2)
    t2 = torch.tensor([0.1, 0.75], device=dev)
    temb2, cond2 = noalloc(t2, *small)
    want_t2, want_c2 = mh.time_embed(t2, *small)
    torch.cuda.synchronize()
    assert torch.equal(temb2, want_t2)
    assert torch.equal(cond2.view(torch.int16), want_c2.view(torch.int16))


def test_noalloc_refuses_sizes_beyond_its_array(dev):
    a = mh.TimeArgs()
    a.levels, a.freq_dim, a.hidden, a.out_dim, a.max_period = 13, 256, 5376, 2688, 10000.0  # 69,888 floats
    fake = C.c_void_p(0x1000)
    assert mh.lib.mh3_time_embed_noalloc(C.byref(a), fake, fake, None, fake, None, fake, None, None) == \
        mh.ERR_UNSUPPORTED
    a.levels = 12                                                                          # 64,512 floats: fits
    a.max_period = 0.5
    assert mh.lib.mh3_time_embed_noalloc(C.byref(a), fake, fake, None, fake, None, fake, None, None) == mh.ERR_PARAM
