"""Pins of the oracle (oracle/vgx_oracle.c) against the reference's own golden
vectors and against what the mathematics fixes.  CPU only.

Each check is chosen so that a plausible slip in the oracle -- a dropped term,
a wrong sign, rounding half-up where the reference rounds half-even, a swapped
byte or operand -- fails it.
"""
import math

import numpy as np
import pytest

import oracle as o


# ---- activation pack: engine/tests/test_xformat.cpp:53-107 (golden bytes) ----
def test_x_pack_goldens():
    assert list(o.x_pack([0.0, 1.0, -1.0, -128.0, 127.99609375, 1000.0], o.I16_1)) == [
        0x00, 0x00, 0x00, 0xFF, 0x01, 0x00, 0x00, 0xFF, 0xFF, 0x00, 0x00, 0xFF,
        0x80, 0x00, 0x00, 0xFF, 0x7F, 0xFF, 0x00, 0xFF, 0x7F, 0xFF, 0x00, 0xFF]
    assert list(o.x_pack([1.0, -1.0, 2.0], o.I16_2)) == [0x01, 0x00, 0xFF, 0x00, 0x02, 0x00, 0x00, 0x00]
    assert list(o.x_pack([0.0, 1.0, -1.0, 8.0, -8.0], o.I8_4)) == [128, 144, 112, 255, 1, 128, 128, 128]
    assert list(o.x_pack([0.0, 1.0, -1.0], o.I24_1)) == [
        0x00, 0x80, 0x00, 0x00, 0x00, 0x80, 0x01, 0x00, 0x00, 0x7F, 0xFF, 0x00]
    assert list(o.x_pack([1.0, -2.0], o.F32)) == [0x3F, 0x80, 0x00, 0x00, 0xC0, 0x00, 0x00, 0x00]
    assert list(o.x_pack([1.0, -2.0, 1.00390625], o.BF16)) == [0x3F, 0x80, 0xC0, 0x00, 0x3F, 0x80, 0x00, 0x00]
    assert list(o.x_pack([1.01171875], o.BF16)) == [0x3F, 0x82, 0x00, 0x00]
    assert o.x_pack([], o.I16_2).size == 0 and o.x_pack([], o.I8_4).size == 0


def test_q16_rounding_rules():
    # host grid: lrintf, half to even (common.h:188-195); shader grid: floor(x+0.5)
    half = np.array([0.5, 1.5, 2.5, -0.5, -1.5], np.float32) / 256.0
    assert list(o.quantize_act(half)) == [0, 2, 2, 0, -2]
    assert [o.lib.vgxo_q16_store(float(v)) for v in half] == [1, 2, 3, 0, -1]
    assert o.lib.vgxo_q16_store(200.0) == 32767 and o.lib.vgxo_q16_store(-200.0) == -32768
    v = np.random.default_rng(0).standard_normal(4096).astype(np.float32) * 40
    want = np.clip(np.floor(v.astype(np.float64) * 256 + 0.5), -32768, 32767)
    got = np.array([o.lib.vgxo_q16_store(float(x)) for x in v])
    assert np.array_equal(got, want)


# ---- unpack / dequantise (closed forms) ----------------------------------------
def test_row_scales_plane_grid():
    # gpu_upload.cpp:46-50: lrint(plane*65536) clamped to [0, 65535]; a plane of
    # 1.0 becomes 65535/65536 of the unit.
    plane = np.array([1.0, 0.5, 0.25 + 1.0 / 131072, 0.0, 3e-6], np.float32)
    ws = np.float32(0.0123)
    got = o.row_scales(5, float(ws), plane)
    p16 = np.clip(np.rint(plane.astype(np.float64) * 65536), 0, 65535).astype(np.float32)
    want = (p16 * ws) * np.float32(1 / 65536)
    assert np.array_equal(got, want)
    assert got[0] == np.float32(np.float32(65535 * ws) / 65536)
    assert np.array_equal(o.row_scales(3, 0.5), np.full(3, 0.5, np.float32))


def test_q8_decode_closed_form():
    rng = np.random.default_rng(1)
    body = rng.integers(0, 256, (5, 32), dtype=np.uint8)
    wsr = rng.uniform(0.001, 0.01, 5).astype(np.float32)
    # biased q8u8: level = byte - 128 (shaders.cpp:392); q8i8: the signed byte
    assert np.array_equal(o.dequant_q8(body, 1, 5, 32, wsr), (body.astype(np.float32) - 128) * wsr[:, None])
    assert np.array_equal(o.dequant_q8(body, 0, 5, 32, wsr), body.view(np.int8).astype(np.float32) * wsr[:, None])
    # the container bias is an XOR: both readings agree on the same level
    assert np.array_equal(o.dequant_q8(body ^ 0x80, 1, 5, 32, wsr), o.dequant_q8(body, 0, 5, 32, wsr))


def test_t3_codes_all_bytes():
    # brute force over every byte value in every position of a texel: the
    # decode reads row 2t / 2t+1, column group 8c..8c+3 / 8c+4..8c+7, weight k
    # at bits 2k (docs/checkpoint-container.md "The t3 body").
    for pos in range(4):
        body = np.zeros((256, 4), np.uint8)
        body[:, pos] = np.arange(256)
        codes = o.t3_codes(body.ravel(), 2 * 256, 8)
        for b in range(256):
            rr, cc = 2 * b + pos // 2, 4 * (pos % 2)
            assert list(codes[rr, cc:cc + 4]) == [(b >> (2 * k)) & 3 for k in range(4)]
            other = np.delete(codes[2 * b:2 * b + 2].ravel(), [(pos // 2) * 8 + cc + k for k in range(4)])
            assert not other.any()


def test_t3_pack_unpack_identity():
    rng = np.random.default_rng(2)
    for rows, cols in ((6, 64), (7, 40), (1, 8), (2, 16)):
        lev = rng.integers(-1, 2, (rows, cols)).astype(np.float32)
        s = rng.uniform(0.01, 0.05, (rows, 1)).astype(np.float32)
        w = lev * s
        packed, unit, plane = o.t3mat(w)
        codes = o.t3_codes(packed, rows, cols)
        level = (codes & 1).astype(np.int8) * (1 - 2 * ((codes >> 1) & 1).astype(np.int8))
        assert np.array_equal(level, np.sign(w).astype(np.int8))
        # the two scales reconstruct each row's magnitude: unit*plane*127 = s_row
        back = level.astype(np.float32) * (plane * np.float32(unit))[:, None] * np.float32(127)
        np.testing.assert_allclose(back, w, rtol=2e-7, atol=0)
    with pytest.raises(ValueError):
        o.t3mat(np.array([[0.1, 0.2, 0.0, -0.1, 0, 0, 0, 0]], np.float32))


def test_q4_dequant_closed_form():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((4, 64)).astype(np.float32)
    packed, s16, m16, ps = o.q4mat(w)
    n = np.empty((4, 64), np.int64)
    n[:, 0::2] = packed & 15
    n[:, 1::2] = packed >> 4
    sa = (s16.astype(np.float32) * np.float32(ps)).repeat(32, axis=1)
    ma = (m16.astype(np.float32) * np.float32(ps)).repeat(32, axis=1)
    got = o.dequant_q4(packed, s16, m16, np.float32(ps), 4, 64)
    assert np.array_equal(got, n.astype(np.float32) * sa + ma)
    # it is a 4-bit quantisation of w: error at most half a step (+ the planes' rounding)
    assert np.all(np.abs(got - w) <= 0.5 * sa + 4 * abs(ps) * 32767 * 2 ** -15 + 1e-6)


# ---- GEMV ------------------------------------------------------------------------
def _rand_q8(rng, rows, cols):
    body = rng.integers(1, 256, (rows, cols), dtype=np.uint8)  # levels -127..127
    x = rng.integers(-32768, 32768, cols).astype(np.int16)
    return body, x


def test_q8_rowsum_exact_and_ref32():
    rng = np.random.default_rng(4)
    body, x = _rand_q8(rng, 33, 768)
    exact = (body.astype(np.int64) - 128) @ x.astype(np.int64)
    assert np.array_equal(o.rowsum_q8(body, 1, 33, 768, x), exact)
    assert np.array_equal(o.rowsum_q8(body ^ 0x80, 0, 33, 768, x), exact)
    # realistic magnitudes keep every fp32 partial sum below 2^24: the literal
    # fp32 order of the shader then gives the same row values
    x2 = np.clip(rng.standard_normal(768) * 256, -32768, 32767).astype(np.int16)
    b2 = np.clip(rng.standard_normal((64, 768)) * 40, -127, 127).astype(np.int64) + 128
    b2 = b2.astype(np.uint8)
    wsr = o.row_scales(64, 3e-4)
    assert np.array_equal(o.rowval_q8(b2, 1, 64, 768, wsr, x2), o.rowval_q8(b2, 1, 64, 768, wsr, x2, ref32=True))


def test_q8_probe_rule():
    # engine/probes/wrow_probe.cpp:356-372: double accumulation, lrint; the
    # shader's form may differ from it by at most one q16 step
    rng = np.random.default_rng(5)
    rows, cols = 96, 768
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    q, unit, plane = o.q8_per_row(w)
    xq = o.quantize_act(rng.standard_normal(cols).astype(np.float32))
    res = o.quantize_act(rng.standard_normal(rows).astype(np.float32))
    body = (q.view(np.uint8) ^ 0x80)
    wsr = o.row_scales(rows, unit, plane)
    got = o.store(o.rowval_q8(body, 1, rows, cols, wsr, xq), res)
    p16 = np.clip(np.rint(plane.astype(np.float64) * 65536), 0, 65535) / 65536
    want = o.probe_q8(q, p16.astype(np.float32), unit, xq, res)
    assert np.max(np.abs(got.astype(np.int32) - want)) <= 1


def test_q4_rowval_against_dequant():
    rng = np.random.default_rng(6)
    rows, cols = 40, 256
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    packed, s16, m16, ps = o.q4mat(w)
    x = o.quantize_act(rng.standard_normal(cols).astype(np.float32))
    v = o.rowval_q4(packed, s16, m16, np.float32(ps), rows, cols, x)
    deq = o.dequant_q4(packed, s16, m16, np.float32(ps), rows, cols).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    np.testing.assert_allclose(v, ref, rtol=1e-5, atol=1e-2)
    v32 = o.rowval_q4(packed, s16, m16, np.float32(ps), rows, cols, x, ref32=True)
    assert np.max(np.abs(o.store(v).astype(int) - o.store(v32).astype(int))) <= 1


def q4_adversarial(rng, rows, cols):
    """q4 rows whose groups mix scales of 1-3 with scales near 2^15, minima at
    the int16 rails, all-0 / all-15 nibble groups, and a full-mantissa ps:
    per-group float terms then span ~2^39, beyond what a double sum of fp32
    terms holds exactly."""
    G = cols // 32
    nib = rng.integers(0, 16, (rows, cols))
    pat = rng.random((rows, G))
    nib = np.where(np.repeat(pat < 0.2, 32, axis=1), 15, np.where(np.repeat(pat > 0.85, 32, axis=1), 0, nib))
    body = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8).ravel()
    s16 = np.where(rng.random((rows, G)) < 0.5, rng.integers(1, 4, (rows, G)),
                   rng.integers(32000, 32768, (rows, G))).astype(np.int16)
    m16 = rng.choice(np.array([-32768, -1, 0, 1, 32767]), (rows, G)).astype(np.int16)
    ps = float(np.float32(2.0 ** -32 / 3))
    return body, s16.ravel(), m16.ravel(), ps, q4_adversarial_x(rng, cols)


def q4_adversarial_x(rng, cols):
    """Full-range activations with rail groups and near-empty groups."""
    x = rng.integers(-32768, 32768, cols).astype(np.int16)
    xg = x.reshape(cols // 32, 32)
    for g in range(cols // 32):
        r = rng.random()
        if r < 0.25:
            xg[g] = 32767 if rng.random() < 0.5 else -32767
        elif r < 0.4:
            xg[g] = 0
            xg[g, rng.integers(32)] = rng.integers(1, 4)
    return x


def _q4_exact_int(body, s16, m16, rows, cols, x):
    """sum_g s16*D + m16*X per row with Python integers."""
    G = cols // 32
    out = []
    for r in range(rows):
        I = 0
        for g in range(G):
            D = X = 0
            for k in range(16):
                b = int(body[r * cols // 2 + g * 16 + k])
                x0, x1 = int(x[g * 32 + 2 * k]), int(x[g * 32 + 2 * k + 1])
                D += (b & 15) * x0 + (b >> 4) * x1
                X += x0 + x1
            I += int(s16[r * G + g]) * D + int(m16[r * G + g]) * X
        out.append(I)
    return out


def test_q4_rowval_exact_and_order_free():
    # the row value is (float)I * ps of the exact integer I: Python integers
    # pin it, and any permutation of the groups gives the same bits
    rng = np.random.default_rng(17)
    rows, cols = 24, 384
    G = cols // 32
    body, s16, m16, ps, x = q4_adversarial(rng, rows, cols)
    got = o.rowval_q4(body, s16, m16, ps, rows, cols, x)
    ints = _q4_exact_int(body, s16, m16, rows, cols, x)
    assert max(abs(I) for I in ints) < 2 ** 47
    # |I| < 2^53: float(I) is exact, and its fp32 conversion rounds once, as (float)I
    want = np.array([np.float32(float(I)) * np.float32(ps) for I in ints], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    perm = rng.permutation(G)
    bp = body.reshape(rows, G, 16)[:, perm].ravel()
    sp, mp = s16.reshape(rows, G)[:, perm].ravel(), m16.reshape(rows, G)[:, perm].ravel()
    xp = x.reshape(G, 32)[perm].ravel()
    assert np.array_equal(o.rowval_q4(bp, sp, mp, ps, rows, cols, xp).view(np.uint32), got.view(np.uint32))


def test_t3_rowval_exact():
    rng = np.random.default_rng(7)
    rows, cols = 9, 64
    lev = rng.integers(-1, 2, (rows, cols)).astype(np.float32)
    w = lev * rng.uniform(0.01, 0.05, (rows, 1)).astype(np.float32)
    packed, unit, plane = o.t3mat(w)
    x = rng.integers(-32768, 32768, cols).astype(np.int16)
    wsr = o.row_scales(rows, np.float32(np.float32(unit) * np.float32(127)), plane)
    v = o.rowval_t3(packed, rows, cols, wsr, x)
    exact = lev.astype(np.int64) @ x.astype(np.int64)
    assert np.array_equal(v, exact.astype(np.float32) * wsr)


def test_store_and_gate():
    v = np.array([0.5, -0.5, 1.49, 40000.0, -40000.0, 10.25], np.float32)
    assert list(o.store(v)) == [1, 0, 1, 32767, -32768, 10]
    assert list(o.store(v, np.array([1, 1, 1, 0, 0, -10], np.int16))) == [2, 1, 2, 32767, -32768, 0]
    rng = np.random.default_rng(8)
    v1 = rng.standard_normal(2000).astype(np.float32) * 600
    v3 = rng.standard_normal(2000).astype(np.float32) * 600
    for hs in (0, 2):
        h = o.gate(v1, v3, hs)
        g = np.clip(np.floor(v1.astype(np.float64) + 0.5), -32768, 32767) / 256
        u = np.clip(np.floor(v3.astype(np.float64) + 0.5), -32768, 32767) / 256
        want = g / (1 + np.exp(-g)) * u * 2.0 ** -hs * 256
        assert np.max(np.abs(h - np.clip(want, -32768, 32767))) <= 1.0
    assert o.gate(np.zeros(1, np.float32), np.full(1, 500.0, np.float32))[0] == 0


# ---- RMSNorm ---------------------------------------------------------------------
def test_rmsnorm_grid_and_value():
    rng = np.random.default_rng(9)
    for dim in (768, 1024, 100):
        x = np.clip(rng.standard_normal(dim) * 300, -32768, 32767).astype(np.int16)
        parts, tot = o.rmsnorm_stats(x)
        per = (dim + 31) // 32
        P = [int(np.sum(x[p * per:(p + 1) * per].astype(np.int64) ** 2)) for p in range(32)]
        assert list(parts) == [(p + 8) // 16 for p in P] and tot == sum((p + 8) // 16 for p in P)
        w = o.quantize_act(rng.uniform(0.5, 1.5, dim).astype(np.float32))
        y = o.rmsnorm(x, w, 1e-5)
        xf = x / 256.0
        want = xf / np.sqrt(np.mean(xf * xf) + 1e-5) * (w / 256.0) * 256
        assert np.max(np.abs(y - np.clip(want, -32768, 32767))) <= 1.0


# ---- attention -------------------------------------------------------------------
def _attn_setup(kv_bits, seq=40, qk=1, heads=4, kv_heads=2, hd=32, seed=10):
    rng = np.random.default_rng(seed)
    dim = heads * hd
    cfg = o.attn_cfg(dim, heads, kv_heads, hd, seq, kv_bits, 1, qk)
    rc, rs = o.rope_cos_sin(10000.0, hd, seq)
    rtab = o.rope_table(rc, rs)
    qn = o.quantize_act(rng.uniform(0.5, 1.5, hd).astype(np.float32)) if qk else None
    kn = o.quantize_act(rng.uniform(0.5, 1.5, hd).astype(np.float32)) if qk else None
    return rng, cfg, rtab, qn, kn


def test_rope_table_grid():
    rc, rs = o.rope_cos_sin(1e6, 96, 16)
    half = np.arange(48, dtype=np.float32)
    freq = (1.0 / np.float32(1e6) ** ((2.0 * half) / 96)).astype(np.float32)
    np.testing.assert_allclose(rc, np.cos(np.arange(16)[:, None] * freq), atol=2e-6)
    np.testing.assert_allclose(rs, np.sin(np.arange(16)[:, None] * freq), atol=2e-6)
    tab = o.rope_table(rc, rs)
    assert np.array_equal(tab[..., 0], np.rint(rc * 4096).astype(np.int32))
    assert tab[0, :, 0].tolist() == [4096] * 48 and tab[0, :, 1].tolist() == [0] * 48


@pytest.mark.parametrize("kv_bits", [16, 8])
def test_kv_write_closed_forms(kv_bits):
    rng, cfg, rtab, qn, kn = _attn_setup(kv_bits, qk=0)
    kv_dim = cfg.kv_heads * cfg.head_dim
    qkv = np.clip(rng.standard_normal(cfg.dim + 2 * kv_dim) * 256, -32768, 32767).astype(np.int16)
    kv = np.zeros(cfg.seq * o.kv_row_bytes(cfg), np.uint8)
    row = o.kv_write(cfg, qkv, None, rtab, 0, kv)
    vals = o.kv_decode(cfg, row)
    scale = 2048 if kv_bits == 16 else 16
    # position 0: cos 1, sin 0 -> K is the q16 value re-gridded; V likewise
    src = qkv[cfg.dim:].astype(np.float64) / 256
    want = np.clip(np.floor(src * scale + 0.5), -32768 if kv_bits == 16 else -128,
                   32767 if kv_bits == 16 else 127) / scale
    assert np.array_equal(vals, want)
    # q16 rows are big-endian pairs (encKV, shaders_attn.cpp:133-135)
    if kv_bits == 16:
        q = int(np.clip(np.floor(src[0] * 2048 + 0.5), -32768, 32767)) & 0xFFFF
        assert (row[0], row[1]) == (q >> 8, q & 255)


def test_attention_integer_equations():
    """check_att.py's recomputation (engine/scripts/check_att.py:86-121), in the
    linear sum domain: scores from the exact dot, max/sum of the stored grid,
    out from p = exp(s - max)/sum over the decoded V."""
    # pos 29 sums one chunk of positions, pos 70 three (the chunked order)
    for kv_bits, pos in ((16, 29), (8, 29), (16, 70), (8, 70)):
        rng, cfg, rtab, qn, kn = _attn_setup(kv_bits, seq=80)
        kv_dim = cfg.kv_heads * cfg.head_dim
        rb = o.kv_row_bytes(cfg)
        kv = np.zeros(cfg.seq * rb, np.uint8)
        for t in range(pos + 1):
            qkv = np.clip(rng.standard_normal(cfg.dim + 2 * kv_dim) * 200, -32768, 32767).astype(np.int16)
            out = o.attn_block(cfg, qkv, qn, kn, rtab, t, kv)
        qrot = o.q_rot(cfg, qkv, qn, rtab, pos)
        sc, st, out2 = o.attn_parts(cfg, qrot, kv, pos)
        assert np.array_equal(out, out2)
        hd, G = cfg.head_dim, cfg.heads // cfg.kv_heads
        dec = np.array([o.kv_decode(cfg, kv[t * rb:(t + 1) * rb]) for t in range(pos + 1)])
        for h in range(cfg.heads):
            kvh = h // G
            k = dec[:, kvh * hd:(kvh + 1) * hd]
            v = dec[:, kv_dim + kvh * hd:kv_dim + (kvh + 1) * hd]
            q = qrot[h * hd:(h + 1) * hd] / 256.0
            s = np.clip(np.floor(np.float32(k @ q) * np.float32(1 / math.sqrt(hd)) * 1024 + 0.5), -32768, 32767)
            assert np.max(np.abs(sc[h, :pos + 1] - s)) <= 1
            m = sc[h, :pos + 1].max()
            assert st[h, 0] == m
            e = np.exp(sc[h, :pos + 1] / 1024.0 - m / 1024.0)
            assert abs(st[h, 1] - np.floor(e.sum() * 32 + 0.5)) <= 1
            p = e / (st[h, 1] / 32.0)
            want = np.clip(np.floor((p @ v) * 256 + 0.5), -32768, 32767)
            assert np.max(np.abs(out[h * hd:(h + 1) * hd] - want)) <= 1


def test_attention_relative_position_invariance():
    # RoPE makes a score depend on the position difference only: the same q/k
    # written d positions later scores the same (up to the 1/4096 table grid)
    rng, cfg, rtab, qn, kn = _attn_setup(16, seq=64, qk=1)
    kv_dim = cfg.kv_heads * cfg.head_dim
    rb = o.kv_row_bytes(cfg)
    a = np.clip(rng.standard_normal(cfg.dim + 2 * kv_dim) * 200, -32768, 32767).astype(np.int16)
    base = None
    for shift in (0, 7, 30):
        kv = np.zeros(cfg.seq * rb, np.uint8)
        o.kv_write(cfg, a, kn, rtab, 3 + shift, kv)
        qrot = o.q_rot(cfg, a, qn, rtab, 9 + shift)
        sc, _, _ = o.attn_parts(cfg, qrot, kv, 9 + shift)
        s = sc[:, 3 + shift].astype(int)
        base = s if base is None else base
        assert np.max(np.abs(s - base)) <= 3


def test_conv_taps_grid():
    # set_conv_kernel (engine/src/gpu_conv.cpp:84-101): lrintf(w*256), the
    # int16 rail, tap-major from the channel-major f32 kernel
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((40, 3)) * 0.7).astype(np.float32)
    w[0, 0], w[1, 1], w[2, 2], w[3, 0] = 200.0, 2.5 / 256, 3.5 / 256, -200.0
    taps = o.conv_taps(w)
    assert taps.shape == (3, 40)
    want = np.clip(np.rint(w.T * np.float32(256)), -32768, 32767)
    assert np.array_equal(taps, want)
    assert (taps[0, 0], taps[1, 1], taps[2, 2], taps[0, 3]) == (32767, 2, 4, -32768)  # half-even ties


def _conv_run(taps, xs, b=256, c=256):
    dim = taps.shape[1]
    state = np.zeros((2, dim), np.int16)
    ys = []
    for x in xs:
        bcx = np.concatenate([np.full(dim, b), np.full(dim, c), x]).astype(np.int16)
        ys.append(o.conv_step(bcx, taps, state))
    return np.array(ys, np.int64), state


def test_conv_step_closed_forms():
    # With B = C = 1.0 the two gates pass x and cv through unchanged, so the
    # block is the causal depthwise convolution itself: taps (0, 0, 1) give
    # y_t = x_t, (0, 1, 0) y_t = x_{t-1}, (1, 0, 0) y_t = x_{t-2} (zero
    # history), and integer taps give the exact integer convolution
    # (conv3_act's operand order: tap 0 on pos-2, tap 2 on pos; Session's CPU
    # form engine/src/session.cpp:394-401 has the same order).
    rng = np.random.default_rng(13)
    dim, T = 64, 9
    xs = [rng.integers(-3000, 3001, dim).astype(np.int16) for _ in range(T)]
    X = np.array(xs, np.int64)
    Z = np.zeros((2, dim), np.int64)
    Xp = np.concatenate([Z, X])  # Xp[t + 2] = x_t
    for tap, shift in ((2, 0), (1, 1), (0, 2)):
        taps = np.zeros((3, dim), np.int16)
        taps[tap] = 256
        y, st = _conv_run(taps, xs)
        assert np.array_equal(y, Xp[2 - shift:2 - shift + T]), tap
        assert np.array_equal(st, X[-2:])  # the state holds the last two gated values
    a = rng.integers(-2, 3, (3, dim))
    y, _ = _conv_run((a * 256).astype(np.int16), xs)
    want = a[0] * Xp[0:T] + a[1] * Xp[1:T + 1] + a[2] * Xp[2:T + 2]
    assert np.array_equal(y, np.clip(want, -32768, 32767))
    # B = 2.0 doubles the gated value up to the int16 rail
    taps = np.zeros((3, dim), np.int16)
    taps[2] = 256
    big = [np.full(dim, 20000, np.int16), np.full(dim, -100, np.int16)]
    y, _ = _conv_run(taps, big, b=512)
    assert (y[0] == 32767).all() and (y[1] == -200).all()


def test_embed_and_argmax():
    rng = np.random.default_rng(11)
    emb = rng.integers(-127, 128, (10, 16)).astype(np.int8)
    es = rng.uniform(0.001, 0.01, 10).astype(np.float32)
    x = o.embed_q8(emb, es, 7)
    want = np.clip(np.rint((emb[7].astype(np.float32) * es[7]) * np.float32(256)), -32768, 32767)
    assert np.array_equal(x, want)
    assert o.argmax_i16(np.array([3, 9, -2, 9, 1], np.int16)) == 1
