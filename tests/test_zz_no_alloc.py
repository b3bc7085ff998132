"""vgx_logits_argmax_rms_noalloc (key slots in the library's static device
array) against vgx_logits_argmax_rms (the group's own slots), through the
C-ABI: identical logits and token, bit for bit, on two calls in a row, the
second over a smaller group, whose launch has fewer workgroups and so leaves
slots of the first call in the array unread."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as o
from vgx import lib as vl
from vgx import mmcf

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _head(gpu, rng, rows, scale):
    """A q8 LM head of rows x 1024 in 1536-row tiles (the logits grid), full-range bytes."""
    mats, tiles = [], []
    for st in range(0, rows, 1536):
        n = min(1536, rows - st)
        body = rng.integers(0, 256, (n, 1024), dtype=np.uint8)
        m = mmcf.Matrix("q8", n, 1024, body.ravel(), float(scale), True,
                        rng.uniform(0.2, 1.0, n).astype(np.float32))
        mats.append(m)
        tiles.append(gpu.upload(m))
    return mats, tiles, gpu.group(tiles)


def test_noalloc_argmax_equals_group_slots(gpu):
    L = vl.load()
    rng = np.random.default_rng(7)
    eps = 1e-5
    x = torch.from_numpy(o.quantize_act(rng.standard_normal(1024).astype(np.float32))).cuda()
    w = torch.from_numpy(o.quantize_act(rng.uniform(0.5, 1.5, 1024).astype(np.float32))).cuda()
    # the first head's largest logits sit far above anything the second can
    # give, so a stale slot of the first call would win the second's argmax
    for rows, scale in ((64402, 2e-3), (3000, 1e-5)):
        mats, tiles, G = _head(gpu, rng, rows, scale)
        assert G.rows == rows
        la = torch.empty(rows, dtype=torch.int16, device="cuda")
        lb = torch.empty(rows, dtype=torch.int16, device="cuda")
        ta = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        tb = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        vl.check(L.vgx_logits_argmax_rms(gpu.ctx, G.h, _p(x), _p(w), ctypes.c_float(eps), _p(la), _p(ta)))
        vl.check(L.vgx_logits_argmax_rms_noalloc(gpu.ctx, G.h, _p(x), _p(w), ctypes.c_float(eps), _p(lb), _p(tb)))
        torch.cuda.synchronize()
        a, b = la.cpu().numpy(), lb.cpu().numpy()
        assert np.array_equal(a, b), rows
        assert int(ta.item()) == int(tb.item()) == o.argmax_i16(a), rows
        # and the logits are the oracle's
        xb = o.rmsnorm(x.cpu().numpy(), w.cpu().numpy(), eps)
        want = np.concatenate([o.store(o.rowval_q8(m.body, 1, m.rows, m.cols, o.row_scales(m.rows, m.scale, m.plane),
                                                   xb)) for m in mats])
        assert np.array_equal(b, want), rows
        G.free()
        for t in tiles:
            t.free()


def test_noalloc_argmax_refusals(gpu):
    """Each refusal with every other argument valid, so the check named is
    the one that fires: NULL outputs, a NULL norm weight, no context, no
    group; nothing is launched."""
    L = vl.load()
    z = ctypes.c_void_p(0)
    rng = np.random.default_rng(3)
    mats, tiles, G = _head(gpu, rng, 2000, 1e-3)
    x = torch.zeros(1024, dtype=torch.int16, device="cuda")
    w = torch.ones(1024, dtype=torch.int16, device="cuda")
    lg = torch.empty(2000, dtype=torch.int16, device="cuda")
    tk = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    eps = ctypes.c_float(1e-5)

    def refused(ctx, g, xp, wp, lp, tp, what):
        assert L.vgx_logits_argmax_rms_noalloc(ctx, g, xp, wp, eps, lp, tp) == vl.VGX_EINVAL
        assert what in L.vgx_last_error().decode()

    refused(gpu.ctx, G.h, _p(x), _p(w), z, _p(tk), "NULL output")
    refused(gpu.ctx, G.h, _p(x), _p(w), _p(lg), z, "NULL output")
    refused(gpu.ctx, G.h, _p(x), z, _p(lg), _p(tk), "NULL RMSNorm weight")
    refused(z, G.h, _p(x), _p(w), _p(lg), _p(tk), "no context")
    refused(gpu.ctx, z, _p(x), _p(w), _p(lg), _p(tk), "NULL argument")
    torch.cuda.synchronize()
    assert int(tk.item()) == -7  # nothing ran
    G.free()
    for t in tiles:
        t.free()
