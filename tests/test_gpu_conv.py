"""The LFM2 conv block kernel (csrc/vgx_conv.hip) against the oracle's
vgxo_conv_step, bit for bit: single positions, batches of positions, the state
export/import and reset."""
import numpy as np
import pytest

import oracle as o
from test_gpu_kernels import dev, host

pytestmark = pytest.mark.gpu


def _case(rng, layers, dim, T, scale=6000):
    w = (rng.standard_normal((layers, dim, 3)) * 0.8).astype(np.float32)
    bcx = np.clip(rng.standard_normal((T, 3 * dim)) * scale, -32768, 32767).astype(np.int16)
    return w, bcx


@pytest.mark.parametrize("dim", [64, 1024, 1000])
def test_conv_steps_match_oracle(gpu, dim):
    rng = np.random.default_rng(dim)
    T = 12
    w, bcx = _case(rng, 2, dim, T)
    C = gpu.conv(w)
    for layer in (0, 1):
        taps = o.conv_taps(w[layer])
        st = np.zeros((2, dim), np.int16)
        for t in range(T):
            want = o.conv_step(bcx[t], taps, st)
            got = host(C.step(layer, dev(bcx[t])))
            assert np.array_equal(got, want), (layer, t)
        assert np.array_equal(C.state(layer), st)
    C.free()


def test_conv_batch_equals_steps_and_state(gpu):
    rng = np.random.default_rng(7)
    dim, T = 1024, 37
    w, bcx = _case(rng, 1, dim, T, scale=20000)  # gates and conv hit the int16 rail
    taps = o.conv_taps(w[0])
    st = np.zeros((2, dim), np.int16)
    want = np.stack([o.conv_step(bcx[t], taps, st) for t in range(T)])
    C = gpu.conv(w)
    got = np.concatenate([host(C.step(0, dev(bcx[:5]))), host(C.step(0, dev(bcx[5:6]))),
                          host(C.step(0, dev(bcx[6:])))])
    assert np.array_equal(got, want)
    assert np.array_equal(C.state(0), st)
    # export / import (the prefix cache's conv history) and reset
    saved = C.state(0)
    C.reset()
    assert not C.state(0).any()
    C.set_state(0, saved)
    more = np.clip(rng.standard_normal((4, 3 * dim)) * 5000, -32768, 32767).astype(np.int16)
    w4 = np.stack([o.conv_step(more[t], taps, st) for t in range(4)])
    assert np.array_equal(host(C.step(0, dev(more))), w4)
    C.free()


def test_conv_refusals(gpu):
    from vgx.lib import VgxError
    w = np.zeros((2, 64, 3), np.float32)
    C = gpu.conv(w, layer_is_conv=[1, 0])
    with pytest.raises(VgxError):
        C.step(1, dev(np.zeros(192, np.int16)))  # an attention layer has no conv block
    with pytest.raises(VgxError):
        gpu.conv(np.zeros((1, 64, 4), np.float32))  # only the 3-tap kernel
    C.free()
