"""The reference's default q4 path reads the weights through a 4-bit texture
view (Model::apply_q4_fmt, engine/src/model.cpp:337-400: on for every chunked
FFN model unless Q4_FMT=0), whose fp32 arithmetic differs from the packed
view's.  libvgx computes the packed form exactly (integer dot products); the
oracle's rowval_q4_view4 restates the 4-bit view.  These tests pin that
restatement against the exact value it approximates, with an fp32 error
bound tight enough that plausible mistakes fall outside it, and bound the
view's gap to the packed form on the MiniMind3 q4 shapes.  CPU only.

Parity with the 4-bit view itself stays unpinned: how the driver converts
UNORM texels and whether its compiler fuses multiply-adds is not in the
reference's sources, and no reference output of the view exists to check."""
import numpy as np
import pytest

import oracle as o
from model import QModel, QModelView4, _Mat4, rowval_q4_view4
from vgx import synth

U = 2.0 ** -24


def _gamma(k):
    return k * U / (1 - k * U)


def _exact(nib, s16, m16, ps, rows, cols, x):
    """sum_g ps*(s*D + m*X) in float64 (every term is exact there), and the
    fp32 error bound of the 4-bit view's evaluation of it."""
    G = cols // 32
    b = nib.reshape(rows, cols // 2)
    n = np.empty((rows, cols), np.int64)
    n[:, 0::2], n[:, 1::2] = b & 15, b >> 4
    xi = x.astype(np.int64)
    D = (n * xi).reshape(rows, G, 32).sum(axis=2)
    A = (n * np.abs(xi)).reshape(rows, G, 32).sum(axis=2)
    X = xi.reshape(G, 32).sum(axis=1)
    s = s16.reshape(rows, G).astype(np.int64) & 0xFFFF
    m = m16.reshape(rows, G).astype(np.int64)
    ps = float(np.float32(ps))
    val = (ps * (s * D + m * X)).sum(axis=1)
    # weight conversion, 2 product roundings, 7 + 3 adds (d); 5 roundings in
    # the scale; 1 in sc*d; 5 in the minimum (against |m| <= 65536); 1 in the
    # group sum; G - 1 adds across groups -- one gamma over all of them
    mag = (ps * (s * A + 65536 * np.abs(X))).sum(axis=1)
    return val, 2 * _gamma(G + 30) * mag


def _random_q4(rng, rows, cols, xscale):
    body = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    s16 = rng.integers(1, 32768, rows * cols // 32).astype(np.int16)
    m16 = rng.integers(-32768, 32768, rows * cols // 32).astype(np.int16)
    x = np.clip(rng.normal(0, xscale, cols), -32768, 32767).astype(np.int16)
    return body, s16, m16, float(np.float32(rng.uniform(1e-7, 1e-5))), x


@pytest.mark.parametrize("cols", [768, 1216, 2432])
def test_view4_within_fp32_bound_of_exact(cols):
    rng = np.random.default_rng(cols)
    rows = 64
    for xscale in (200, 6000, 30000):
        body, s16, m16, ps, x = _random_q4(rng, rows, cols, xscale)
        got = rowval_q4_view4(body, s16, m16, ps, rows, cols, x).astype(np.float64)
        want, bound = _exact(body, s16, m16, ps, rows, cols, x)
        assert np.all(np.abs(got - want) <= bound)


def test_planted_mistakes_leave_the_bound():
    # a restatement that swaps the nibbles of a byte, the bytes of the scale,
    # or drops the minimum's term is outside the bound on most rows
    rng = np.random.default_rng(7)
    rows, cols = 64, 768
    body, s16, m16, ps, x = _random_q4(rng, rows, cols, 6000)
    want, bound = _exact(body, s16, m16, ps, rows, cols, x)
    swapped = ((body << 4) | (body >> 4)).astype(np.uint8)
    bswap = s16.view(np.uint16).byteswap().view(np.int16)
    for args in ((swapped, s16, m16), (body, bswap, m16), (body, s16, np.zeros_like(m16))):
        got = rowval_q4_view4(*args, ps, rows, cols, x).astype(np.float64)
        assert (np.abs(got - want) > bound).mean() > 0.9


def test_view4_equals_scalar_shader_order():
    # the vectorised restatement performs the shader's operations in its
    # order: a scalar fp32 loop written from matvec_i4_add_4x4's text
    # (engine/src/shaders.cpp:1765-1780) gives the same bits
    rng = np.random.default_rng(3)
    rows, cols = 3, 64
    body, s16, m16, ps, x = _random_q4(rng, rows, cols, 9000)
    f = np.float32
    got = rowval_q4_view4(body, s16, m16, ps, rows, cols, x)
    b = body.reshape(rows, cols // 2)
    for r in range(rows):
        s = f(0)
        for g in range(cols // 32):
            su = int(s16[r * (cols // 32) + g]) & 0xFFFF
            mu = int(m16[r * (cols // 32) + g]) & 0xFFFF
            u, v = f(f(979200) * f(ps)), f(f(3825) * f(ps))
            sc = f(f(f(su >> 8) / f(255)) * u) + f(f(f(su & 255) / f(255)) * v)
            raw = f(f(f(mu >> 8) / f(255)) * f(65280)) + f(f(f(mu & 255) / f(255)) * f(255))
            if raw >= f(32767.5):
                raw = f(raw - f(65536))
            mn = f(raw * f(ps))
            xsum, d = f(0), f(0)
            for t in range(4):
                c = g * 32 + t * 8
                xs = [f(int(x[c + j])) for j in range(8)]
                e = xs[0]
                for j in range(1, 8):
                    e = f(e + xs[j])
                xsum = f(xsum + e)
                acc = None
                for j in range(8):
                    byte = int(b[r, (c + j) // 2])
                    nib = byte & 15 if (c + j) % 2 == 0 else byte >> 4
                    p = f(f(f(nib) / f(15)) * xs[j])
                    acc = p if acc is None else f(acc + p)
                d = f(d + acc)
            s = f(s + f(f(sc * d) + f(mn * xsum)))
        assert s == got[r]


@pytest.fixture(scope="module")
def c3_models():
    spec = synth.minimind3_spec(seq=32)
    blob = synth.container(spec, "q4", seed=3)
    return spec, QModel(blob, kv_bits=8), QModelView4(blob, kv_bits=8)


def test_c3_scales_are_unsigned_safe(c3_models):
    # the 4-bit view reads a group scale as unsigned 16 bits, the packed view
    # as signed: they agree because the packer's scales are below 2^15
    _, q, _ = c3_models
    for L in q.mats:
        for m in L.values():
            if m.kind == "q4":
                assert m.s16.min() >= 0


def test_c3_matvec_gap_at_most_one_lsb(c3_models):
    # on the model's own matrices, the same q16 input stored through the two
    # views differs by at most one q16 step, and only where the row value is
    # within fp32 rounding of a half-step
    _, q, _ = c3_models
    rng = np.random.default_rng(11)
    L = q.mats[0]
    for name in ("qkv", "wo", "w1", "w3"):
        m = L[name]
        for xscale in (300, 3000, 20000):
            x = np.clip(rng.normal(0, xscale, m.cols), -32768, 32767).astype(np.int16)
            a, b = m.rowval(x), _Mat4.of(m).rowval(x)
            d = np.abs(o.store(a).astype(np.int32) - o.store(b).astype(np.int32))
            assert d.max() <= 1
            a64 = a.astype(np.float64)
            to_half = 0.5 - np.abs(a64 - np.floor(a64 + 0.5))
            assert np.all(to_half[d > 0] < 0.05)
    for a, b in q.w2ab[:1]:
        for half in (a, b):
            x = np.clip(rng.normal(0, 3000, half.cols), -32768, 32767).astype(np.int16)
            d = np.abs(o.store(half.rowval(x)).astype(np.int32) - o.store(_Mat4.of(half).rowval(x)).astype(np.int32))
            assert d.max() <= 1


def test_c3_decode_gap(c3_models):
    # eight layers compound the per-matvec steps: over six decode steps the
    # logits of the two views stay within 16 q16 steps and pick the same
    # token wherever the packed view's top-1 margin exceeds that
    spec, q, v = c3_models
    prompt = synth.prompt(6, spec.vocab, seed=3)
    for pos in range(6):
        lq, lv = q.step(int(prompt[pos]), pos), v.step(int(prompt[pos]), pos)
        assert np.abs(lq.astype(np.int32) - lv.astype(np.int32)).max() <= 16
        top = np.sort(lq.astype(np.int32))[::-1]
        if top[0] - top[1] > 32:
            assert int(np.argmax(lq)) == int(np.argmax(lv))
