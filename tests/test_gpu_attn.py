"""KV pack/unpack and decode attention against the oracle, through the C-ABI.

Bar: bit-exact -- the packed KV rows (in the reference's texel byte layout,
as MMKV1 persists them) and the q16 attention output at every position."""
import zlib

import numpy as np
import pytest
import torch

import oracle as o

pytestmark = pytest.mark.gpu

CONFIGS = [
    # name, dim, heads, kv_heads, hd, seq, kv_bits, rope_half, qk_norm, theta, steps
    ("minimind3-q16", 768, 8, 4, 96, 256, 16, 1, 1, 1e6, 255),
    ("minimind3-q8", 768, 8, 4, 96, 768, 8, 1, 1, 1e6, 40),
    ("lfm2", 1024, 16, 8, 64, 256, 16, 1, 1, 1e6, 24),
    ("bitcpm", 1024, 16, 2, 64, 512, 16, 1, 0, 10000.0, 24),
    ("interleaved", 256, 4, 2, 64, 64, 16, 0, 1, 10000.0, 20),
    ("interleaved-q8", 256, 4, 4, 64, 64, 8, 0, 0, 10000.0, 20),
]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("cfg", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_attention_matches_oracle(gpu, cfg):
    name, dim, heads, kvh, hd, seq, bits, half, qk, theta, steps = cfg
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layers = 2
    rc, rs = o.rope_cos_sin(theta, hd, seq)
    rtab = o.rope_table(rc, rs)
    qn = rng.uniform(0.5, 1.5, (layers, hd)).astype(np.float32) if qk else None
    kn = rng.uniform(0.5, 1.5, (layers, hd)).astype(np.float32) if qk else None
    A = gpu.attention(dim=dim, heads=heads, kv_heads=kvh, head_dim=hd, seq=seq, layers=layers, kv_bits=bits,
                      rope_half=half, qk_norm=qk, rope_cos=rc, rope_sin=rs, q_norm=qn, k_norm=kn)
    c = o.attn_cfg(dim, heads, kvh, hd, seq, bits, half, qk)
    rb = o.kv_row_bytes(c)
    assert A.row_bytes == rb
    kv = [np.zeros(seq * rb, np.uint8) for _ in range(layers)]
    kv_dim = kvh * hd
    layer = 1
    qnq = o.quantize_act(qn[layer]) if qk else None
    knq = o.quantize_act(kn[layer]) if qk else None
    scale = 600 if bits == 16 else 300
    for pos in range(steps):
        qkv = np.clip(rng.standard_normal(dim + 2 * kv_dim) * scale, -32768, 32767).astype(np.int16)
        want = o.attn_block(c, qkv, qnq, knq, rtab, pos, kv[layer])
        if pos % 2 == 0:
            got = A.block(layer, pos, dev(qkv))
        else:  # the unfused pair: pack, then attend
            q = dev(qkv)
            A.kv_append(layer, pos, q)
            got = A.decode(layer, pos, q)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), want), (name, pos)
    rows = A.read_rows(layer, 0, steps)
    assert np.array_equal(rows, kv[layer][:steps * rb])
    # the import path writes the same bytes back; attention over them agrees
    A.write_rows(layer, 0, rows)
    qkv = np.clip(rng.standard_normal(dim + 2 * kv_dim) * scale, -32768, 32767).astype(np.int16)
    want = o.attn_block(c, qkv, qnq, knq, rtab, steps, kv[layer])
    got = A.block(layer, steps, dev(qkv))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)
    A.free()


def test_attention_range_errors(gpu):
    rc, rs = o.rope_cos_sin(10000.0, 64, 8)
    A = gpu.attention(dim=128, heads=2, kv_heads=1, head_dim=64, seq=8, layers=1, kv_bits=16, rope_half=1,
                      qk_norm=0, rope_cos=rc, rope_sin=rs)
    from vgx import lib as vl
    qkv = dev(np.zeros(256, np.int16))
    with pytest.raises(vl.VgxError):
        A.block(0, 8, qkv)  # pos beyond seq
    with pytest.raises(vl.VgxError):
        A.block(1, 0, qkv)  # no such layer
    A.free()


@pytest.mark.parametrize("bits,hd", [(16, 256), (16, 64), (8, 256), (8, 96)])
def test_attention_rails(gpu, bits, hd):
    """Scores at the int16 / int8 rails: every cached K value at the grid's
    minimum or maximum and the rotated query saturated, with head_dim up to
    256 -- the widest exact integer sums the score dot product forms."""
    heads, kvh, seq = 2, 1, 40
    dim = heads * hd
    rng = np.random.default_rng(bits * 1000 + hd)
    rc, rs = o.rope_cos_sin(10000.0, hd, seq)
    rtab = o.rope_table(rc, rs)
    A = gpu.attention(dim=dim, heads=heads, kv_heads=kvh, head_dim=hd, seq=seq, layers=1, kv_bits=bits,
                      rope_half=1, qk_norm=0, rope_cos=rc, rope_sin=rs)
    c = o.attn_cfg(dim, heads, kvh, hd, seq, bits, 1, 0)
    rb = o.kv_row_bytes(c)
    n = 33
    vals = rng.choice([-32768, 32767] if bits == 16 else [-128, 127], size=(n, rb // (bits // 8)))
    if bits == 16:  # the texel layout: big-endian int16
        rows = vals.astype(">i2").view(np.uint8).reshape(-1)
    else:
        rows = vals.astype(np.int8).view(np.uint8).reshape(-1)
    kv = np.zeros(seq * rb, np.uint8)
    kv[:n * rb] = rows
    A.write_rows(0, 0, rows)
    for pos in (n, n + 1):
        qkv = rng.choice([-32768, 32767], size=dim + 2 * kvh * hd).astype(np.int16)
        want = o.attn_block(c, qkv, None, None, rtab, pos, kv)
        got = A.block(0, pos, dev(qkv))
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), want), pos
    A.free()


LONG = [(8, 96, 4, 2, 320, (32, 129, 200, 257, 319)), (16, 128, 4, 2, 320, (32, 129, 200, 257, 319)),
        (8, 128, 4, 2, 320, (32, 129, 200, 257, 319)), (16, 256, 4, 2, 320, (32, 129, 200, 257, 319)),
        (8, 256, 4, 2, 320, (32, 129, 200, 257, 319)),
        # KV q8 at head_dim 64 and 32, KV q16 at 64 and 32: one round of the
        # one-element plan up to 256 positions, the two-chunks-a-wave plan past it
        (8, 64, 4, 2, 320, (32, 255, 257, 319)), (8, 32, 4, 2, 320, (255, 257, 319)),
        (16, 64, 4, 2, 320, (32, 255, 257, 319)), (16, 32, 4, 2, 320, (255, 257, 319)),
        # MiniMind3 q4 / KV q8 at SEQ 768: 8 Q / 4 KV heads of 96, to the last row
        (8, 96, 8, 4, 768, (383, 511, 640, 767)),
        # MiniMind3 q8 / KV q16 at SEQ 768
        (16, 96, 8, 4, 768, (300, 767))]


@pytest.mark.parametrize("bits,hd,heads,kvh,seq,positions", LONG)
def test_attention_long_contexts(gpu, bits, hd, heads, kvh, seq, positions):
    """Contexts of several rounds of the weighted-V pass (and the plans it
    switches to there: two elements a lane above head_dim 64; up to 32 fields
    of 32 bits a head -- head_dim 128 at q8, 64 at q16 -- two chunks a wave of
    one field a lane), over
    random cached rows, through both the appending and the reading entry
    points."""
    dim = heads * hd
    rng = np.random.default_rng(bits * 7 + hd)
    rc, rs = o.rope_cos_sin(10000.0, hd, seq)
    rtab = o.rope_table(rc, rs)
    qn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    A = gpu.attention(dim=dim, heads=heads, kv_heads=kvh, head_dim=hd, seq=seq, layers=1, kv_bits=bits,
                      rope_half=1, qk_norm=1, rope_cos=rc, rope_sin=rs, q_norm=qn, k_norm=kn)
    c = o.attn_cfg(dim, heads, kvh, hd, seq, bits, 1, 1)
    qnq, knq = o.quantize_act(qn[0]), o.quantize_act(kn[0])
    rb = o.kv_row_bytes(c)
    n = seq - 1
    if bits == 16:  # the texel layout: big-endian int16, values within the q16 KV grid's usual range
        rows = rng.integers(-6000, 6000, size=(n, rb // 2)).astype(">i2").view(np.uint8).reshape(-1)
    else:
        rows = rng.integers(-128, 128, size=(n, rb)).astype(np.int8).view(np.uint8).reshape(-1)
    for pos in positions:
        print("long context bits=%d hd=%d pos=%d" % (bits, hd, pos), flush=True)
        kv = np.zeros(seq * rb, np.uint8)
        kv[:pos * rb] = rows[:pos * rb]
        A.write_rows(0, 0, rows[:pos * rb].copy())
        qkv = np.clip(rng.standard_normal(dim + 2 * kvh * hd) * 600, -32768, 32767).astype(np.int16)
        want = o.attn_block(c, qkv, qnq, knq, rtab, pos, kv)
        got = A.block(0, pos, dev(qkv))
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), want), pos
        # the reading entry point, over the row the append wrote, agrees
        assert np.array_equal(A.decode(0, pos, dev(qkv)).cpu().numpy(), want), pos
    A.free()


@pytest.mark.parametrize("bits", [16, 8])
def test_attention_sequences_in_lockstep(gpu, bits):
    """vgx_attn_block_seqs: nseq sequences at the same position, each on its
    own cache, equal the oracle run on each sequence alone; a view of one
    sequence takes the single-sequence entry points (batched append and
    decode, row export)."""
    dim, heads, kvh, hd, seq, nseq = 256, 4, 2, 64, 48, 3
    rng = np.random.default_rng(11 + bits)
    rc, rs = o.rope_cos_sin(10000.0, hd, seq)
    rtab = o.rope_table(rc, rs)
    qn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    A = gpu.attention(dim=dim, heads=heads, kv_heads=kvh, head_dim=hd, seq=seq, layers=1, kv_bits=bits,
                      rope_half=1, qk_norm=1, rope_cos=rc, rope_sin=rs, q_norm=qn, k_norm=kn, nseq=nseq)
    c = o.attn_cfg(dim, heads, kvh, hd, seq, bits, 1, 1)
    rb = o.kv_row_bytes(c)
    qnq, knq = o.quantize_act(qn[0]), o.quantize_act(kn[0])
    kv = [np.zeros(seq * rb, np.uint8) for _ in range(nseq)]
    width = dim + 2 * kvh * hd
    # sequence 1's first 9 positions through a view: one batched append + decode
    v1 = A.view(1)
    pre = np.clip(rng.standard_normal((9, width)) * 500, -32768, 32767).astype(np.int16)
    got = v1.block_batch(0, 0, dev(pre))
    torch.cuda.synchronize()
    for p in range(9):
        want = o.attn_block(c, pre[p], qnq, knq, rtab, p, kv[1])
        assert np.array_equal(got[p].cpu().numpy(), want), p
    # then all three in lockstep from position 9 (sequences 0 and 2 start
    # from caches of zeros, which the oracle mirrors)
    for pos in range(9, 30):
        q = np.clip(rng.standard_normal((nseq, width)) * 500, -32768, 32767).astype(np.int16)
        out = A.block_seqs(0, pos, dev(q))
        torch.cuda.synchronize()
        for s in range(nseq):
            want = o.attn_block(c, q[s], qnq, knq, rtab, pos, kv[s])
            assert np.array_equal(out[s].cpu().numpy(), want), (s, pos)
    for s in range(nseq):
        assert np.array_equal(A.view(s).read_rows(0, 0, 30), kv[s][:30 * rb]), s
    from vgx import lib as vl
    with pytest.raises(vl.VgxError):
        A.block_seqs(0, 30, dev(np.zeros((nseq + 1, width), np.int16)))  # more sequences than caches
    with pytest.raises(vl.VgxError):
        A.view(nseq)
    A.free()


def _attn_setup(gpu, rng, bits, heads, kvh, hd, seq, nseq=1, qk_norm=1):
    dim = heads * hd
    rc, rs = o.rope_cos_sin(10000.0, hd, seq)
    qn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    A = gpu.attention(dim=dim, heads=heads, kv_heads=kvh, head_dim=hd, seq=seq, layers=1, kv_bits=bits,
                      rope_half=1, qk_norm=qk_norm, rope_cos=rc, rope_sin=rs, q_norm=qn, k_norm=kn, nseq=nseq)
    c = o.attn_cfg(dim, heads, kvh, hd, seq, bits, 1, qk_norm)
    ref = (c, o.quantize_act(qn[0]) if qk_norm else None, o.quantize_act(kn[0]) if qk_norm else None,
           o.rope_table(rc, rs))
    return A, ref, dim + 2 * kvh * hd


# Batches of positions through the query-block kernel (a workgroup per KV head
# and block of 16/G positions): query heads per KV head 1, 2, 4, 8 and 32,
# head_dim 32..256, both KV widths, blocks cut short at the batch's end, and
# contexts of up to 24 chunks
QBLOCK = [  # bits, heads, kv_heads, head_dim, seq, batch sizes in order from position 0
    (8, 8, 4, 96, 768, (256, 37, 300)),
    (16, 8, 4, 96, 320, (5, 131, 64)),
    (16, 16, 2, 64, 512, (128, 3, 200)),
    (8, 16, 16, 64, 96, (17, 40)),
    (16, 4, 1, 256, 160, (33, 100)),
    (16, 32, 1, 32, 80, (30, 20)),
]


@pytest.mark.parametrize("bits,heads,kvh,hd,seq,batches", QBLOCK)
def test_query_block_batches(gpu, bits, heads, kvh, hd, seq, batches):
    rng = np.random.default_rng(heads * 31 + hd + bits)
    A, (c, qnq, knq, rtab), width = _attn_setup(gpu, rng, bits, heads, kvh, hd, seq)
    kv = np.zeros(seq * o.kv_row_bytes(c), np.uint8)
    pos = 0
    for n in batches:
        print("query block bits=%d heads=%d kvh=%d hd=%d rows %d..%d" % (bits, heads, kvh, hd, pos, pos + n - 1),
              flush=True)
        q = np.clip(rng.standard_normal((n, width)) * 700, -32768, 32767).astype(np.int16)
        got = A.block_batch(0, pos, dev(q)).cpu().numpy()
        for r in range(n):
            want = o.attn_block(c, q[r], qnq, knq, rtab, pos + r, kv)
            assert np.array_equal(got[r], want), pos + r
        pos += n
    assert np.array_equal(A.read_rows(0, 0, pos), kv[:pos * o.kv_row_bytes(c)])
    A.free()


@pytest.mark.parametrize("bits,heads,kvh,hd,seq", [(16, 16, 2, 64, 512), (8, 8, 4, 96, 768), (16, 8, 1, 128, 96)])
def test_query_block_sequences(gpu, bits, heads, kvh, hd, seq):
    # sequences in lockstep (each workgroup packs its KV head's row of the
    # position, then its G query heads attend), against the oracle per sequence
    nseq = 5
    rng = np.random.default_rng(heads + hd + bits)
    A, (c, qnq, knq, rtab), width = _attn_setup(gpu, rng, bits, heads, kvh, hd, seq, nseq=nseq)
    rb = o.kv_row_bytes(c)
    kv = [np.zeros(seq * rb, np.uint8) for _ in range(nseq)]
    pre = min(seq - 40, 300)
    for s in range(nseq):
        q = np.clip(rng.standard_normal((pre, width)) * 700, -32768, 32767).astype(np.int16)
        A.view(s).block_batch(0, 0, dev(q))
        for r in range(pre):
            o.attn_block(c, q[r], qnq, knq, rtab, r, kv[s])
    for pos in list(range(pre, pre + 3)) + [seq - 2, seq - 1]:
        print("query block sequences bits=%d hd=%d pos=%d" % (bits, hd, pos), flush=True)
        q = np.clip(rng.standard_normal((nseq, width)) * 700, -32768, 32767).astype(np.int16)
        out = A.block_seqs(0, pos, dev(q)).cpu().numpy()
        for s in range(nseq):
            assert np.array_equal(out[s], o.attn_block(c, q[s], qnq, knq, rtab, pos, kv[s])), (s, pos)
    for s in range(nseq):
        assert np.array_equal(A.view(s).read_rows(0, 0, seq), kv[s]), s
    A.free()
