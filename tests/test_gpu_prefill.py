"""Batched prefill (int8 matrix cores) against the batch-1 path: every row of
every batched op must equal the oracle's batch-1 result on that token, bit
for bit -- the reference's acceptance rule for a batched path
(docs/prefill-batching.md:98-113)."""
import numpy as np
import pytest
import torch

import oracle as o
from test_gpu_kernels import dev, host, oracle_rowval, q4_matrix, q8_matrix, rand_x, t3_matrix

pytestmark = pytest.mark.gpu

MK = {"q8": q8_matrix, "q4": q4_matrix, "t3": t3_matrix}


def x_rows(rng, ntok, cols, full=False):
    if full:
        return rng.integers(-32768, 32768, (ntok, cols)).astype(np.int16)
    return np.stack([rand_x(rng, cols) for _ in range(ntok)])


@pytest.mark.parametrize("kind,rows,cols", [("q8", 1536, 768), ("q8", 768, 2432), ("q8", 33, 96), ("q8", 7, 48),
                                            ("q4", 1536, 768), ("q4", 768, 2432), ("q4", 33, 96),
                                            ("t3", 1280, 1024), ("t3", 33, 96)])
@pytest.mark.parametrize("ntok", [1, 5, 37, 64])
def test_gemm_rows_equal_gemv(gpu, kind, rows, cols, ntok):
    rng = np.random.default_rng(rows + 7 * cols + ntok)
    m = MK[kind](rng, rows, cols)
    W = gpu.upload(m)
    x = x_rows(rng, ntok, cols)
    res = x_rows(rng, ntok, rows)
    got = host(gpu.gemm(W, dev(x)))
    got_r = host(gpu.gemm(W, dev(x), res=dev(res)))
    for t in range(ntok):
        v = oracle_rowval(m, x[t])
        assert np.array_equal(got[t], o.store(v)), t
        assert np.array_equal(got_r[t], o.store(v, res[t])), t


@pytest.mark.parametrize("kind,rows,cols", [("q8", 1536, 768), ("q4", 1536, 768), ("t3", 1280, 1024),
                                            ("q4", 768, 2432), ("q8", 2432, 768)])
def test_gemm_256_tokens(gpu, kind, rows, cols):
    """The prefill launches of 256 tokens: four waves a workgroup over many
    tiles (eight over the 2432-column rows' few), each wave's k-steps in
    rounds of eight, the last token tile ragged at 250 tokens; every row
    equals the batch-1 oracle."""
    rng = np.random.default_rng(rows * 3 + cols)
    m = MK[kind](rng, rows, cols)
    W = gpu.upload(m)
    for ntok in (256, 250):
        x = x_rows(rng, ntok, cols)
        res = x_rows(rng, ntok, rows)
        got = host(gpu.gemm(W, dev(x), res=dev(res)))
        for t in range(ntok):
            assert np.array_equal(got[t], o.store(oracle_rowval(m, x[t]), res[t])), (ntok, t)


@pytest.mark.parametrize("kind", ["q8", "t3"])
def test_gemm_full_range(gpu, kind):
    # int16 extremes and every weight byte: the byte-plane split and its
    # -128 offset stay exact
    rng = np.random.default_rng(3)
    m = q8_matrix(rng, 96, 512, full=True) if kind == "q8" else t3_matrix(rng, 96, 512)
    W = gpu.upload(m)
    x = x_rows(rng, 40, 512, full=True)
    x[0, :] = -32768
    x[1, :] = 32767
    got = host(gpu.gemm(W, dev(x)))
    for t in range(40):
        assert np.array_equal(got[t], o.store(oracle_rowval(m, x[t]))), t


@pytest.mark.parametrize("kind,rows,cols,split", [("q8", 768, 2432, 1216), ("q8", 40, 96, 48),
                                                  ("q4", 768, 2432, 1216), ("t3", 256, 1024, 512)])
def test_gemm_add_split(gpu, kind, rows, cols, split):
    # split 48 of 96 falls in the middle of a 32-column matrix-core step
    rng = np.random.default_rng(cols + split)
    m = MK[kind](rng, rows, cols)
    m.scale_mul = 4.0
    W = gpu.upload(m)
    ntok = 33
    x = x_rows(rng, ntok, cols)
    res = x_rows(rng, ntok, rows)
    got = host(gpu.gemm_add_split(W, split, dev(x), dev(res)))
    a, b = m.slice_cols(0, split), m.slice_cols(split, cols)
    for t in range(ntok):
        y1 = o.store(oracle_rowval(a, x[t, :split]), res[t])
        assert np.array_equal(got[t], o.store(oracle_rowval(b, x[t, split:]), y1)), t


@pytest.mark.parametrize("kind,rows,cols", [("q8", 2432, 768), ("q4", 1216, 768), ("t3", 512, 1024)])
def test_ffn_gate_batch(gpu, kind, rows, cols):
    rng = np.random.default_rng(rows)
    m1, m3 = MK[kind](rng, rows, cols), MK[kind](rng, rows, cols)
    W1, W3 = gpu.upload(m1), gpu.upload(m3)
    x = x_rows(rng, 37, cols)
    for hs in (0, 2):
        got = host(gpu.ffn_gate_batch(W1, W3, dev(x), hs))
        for t in range(37):
            want = o.gate(oracle_rowval(m1, x[t]), oracle_rowval(m3, x[t]), hs)
            assert np.array_equal(got[t], want), (hs, t)


@pytest.mark.parametrize("kind,rows,cols,ntok", [("t3", 1280, 1024, 32), ("q8", 1536, 768, 256), ("q4", 1536, 768, 37),
                                                 ("q8", 3072, 1024, 5), ("t3", 33, 96, 32), ("q8", 73, 64, 40)])
def test_gemm_rms(gpu, kind, rows, cols, ntok):
    """RMSNorm fused into the GEMM: per token the oracle's rmsnorm then its
    batch-1 row values, bit for bit, with and without a residual."""
    rng = np.random.default_rng(rows + cols + ntok)
    m = MK[kind](rng, rows, cols)
    W = gpu.upload(m)
    x = np.clip(rng.standard_normal((ntok, cols)) * 900, -32768, 32767).astype(np.int16)
    x[0, :] = 32767  # a row at the rail
    w = o.quantize_act(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    res = x_rows(rng, ntok, rows)
    got = host(gpu.gemm_rms(W, dev(x), dev(w), 1e-5))
    got_r = host(gpu.gemm_rms(W, dev(x), dev(w), 1e-5, res=dev(res)))
    for t in range(ntok):
        v = oracle_rowval(m, o.rmsnorm(x[t], w, 1e-5))
        assert np.array_equal(got[t], o.store(v)), t
        assert np.array_equal(got_r[t], o.store(v, res[t])), t


@pytest.mark.parametrize("kind,rows,cols,ntok", [("t3", 4096, 1024, 32), ("q4", 1216, 768, 64), ("q8", 2432, 768, 9)])
def test_ffn_gate_batch_rms(gpu, kind, rows, cols, ntok):
    rng = np.random.default_rng(rows + ntok)
    m1, m3 = MK[kind](rng, rows, cols), MK[kind](rng, rows, cols)
    W1, W3 = gpu.upload(m1), gpu.upload(m3)
    x = np.clip(rng.standard_normal((ntok, cols)) * 700, -32768, 32767).astype(np.int16)
    w = o.quantize_act(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    got = host(gpu.ffn_gate_batch_rms(W1, W3, dev(x), dev(w), 1e-5, 1))
    for t in range(ntok):
        xn = o.rmsnorm(x[t], w, 1e-5)
        assert np.array_equal(got[t], o.gate(oracle_rowval(m1, xn), oracle_rowval(m3, xn), 1)), t


def test_rmsnorm_and_embed_batch(gpu):
    rng = np.random.default_rng(5)
    x = np.clip(rng.standard_normal((19, 768)) * 900, -32768, 32767).astype(np.int16)
    w = o.quantize_act(rng.uniform(0.5, 1.5, 768).astype(np.float32))
    got = host(gpu.rmsnorm_batch(dev(x), dev(w), 1e-5))
    for t in range(19):
        assert np.array_equal(got[t], o.rmsnorm(x[t], w, 1e-5)), t
    emb = rng.integers(-127, 128, (6400, 768)).astype(np.int8)
    es = rng.uniform(1e-4, 1e-2, 6400).astype(np.float32)
    toks = np.array([0, 17, 6399, 17, 5], np.int32)
    got = host(gpu.embed_q8_batch(dev(emb), dev(es), dev(toks)))
    for t, tk in enumerate(toks):
        assert np.array_equal(got[t], o.embed_q8(emb, es, int(tk))), t


@pytest.mark.parametrize("dim", [768, 1024, 100, 2304])
def test_embed_rms_batch(gpu, dim):
    # the embedding rows and their RMSNorm in one launch (dim up to 2048; 2304
    # takes the two launches): the oracle's embedding, then its rmsnorm
    rng = np.random.default_rng(dim)
    emb = rng.integers(-127, 128, (500, dim)).astype(np.int8)
    es = rng.uniform(1e-4, 1.05, 500).astype(np.float32)  # the largest values clamp at the int16 rail
    w = o.quantize_act(rng.uniform(0.5, 1.5, dim).astype(np.float32))
    toks = np.array([0, 499, 17, 17, 250, 3, 0], np.int32)
    x, y = gpu.embed_q8_rms_batch(dev(emb), dev(es), dev(toks), dev(w), 1e-5)
    x, y = host(x), host(y)
    for t, tk in enumerate(toks):
        e = o.embed_q8(emb, es, int(tk))
        assert np.array_equal(x[t], e), t
        assert np.array_equal(y[t], o.rmsnorm(e, w, 1e-5)), t


@pytest.mark.parametrize("kv_bits", [16, 8])
def test_attention_batch_equals_serial(gpu, kv_bits):
    # MiniMind3 heads: 20 positions one at a time against batches of 7 and 13
    dim, heads, kvh, hd, seq = 768, 8, 4, 96, 64
    rc, rs = o.rope_cos_sin(1e6, hd, seq)
    rng = np.random.default_rng(kv_bits)
    qn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, (1, hd)).astype(np.float32)

    def make():
        return gpu.attention(dim=dim, heads=heads, kv_heads=kvh, head_dim=hd, seq=seq, layers=1, kv_bits=kv_bits,
                             rope_half=1, qk_norm=1, rope_cos=rc, rope_sin=rs, q_norm=qn, k_norm=kn)

    A1, A2 = make(), make()
    qkv = np.clip(rng.standard_normal((20, dim + 2 * kvh * hd)) * 300, -32768, 32767).astype(np.int16)
    serial = np.stack([host(A1.block(0, p, dev(qkv[p]))) for p in range(20)])
    b1 = host(A2.block_batch(0, 0, dev(qkv[:7])))
    b2 = host(A2.block_batch(0, 7, dev(qkv[7:])))
    assert np.array_equal(np.concatenate([b1, b2]), serial)
    assert np.array_equal(A1.read_rows(0, 0, 20), A2.read_rows(0, 0, 20))
    A1.free()
    A2.free()


def test_batch_refusals(gpu):
    from vgx.lib import VgxError
    rng = np.random.default_rng(9)
    W = gpu.upload(q8_matrix(rng, 64, 64))
    with pytest.raises(VgxError):
        gpu.gemm(W, torch.empty((0, 64), dtype=torch.int16, device="cuda"))
    with pytest.raises(VgxError):
        gpu.gemm_add_split(W, 40, dev(x_rows(rng, 3, 64)), dev(x_rows(rng, 3, 64)))  # not a multiple of 16
    rc, rs = o.rope_cos_sin(1e6, 64, 8)
    A = gpu.attention(dim=128, heads=2, kv_heads=1, head_dim=64, seq=8, layers=1, kv_bits=16, rope_half=1,
                      qk_norm=0, rope_cos=rc, rope_sin=rs)
    with pytest.raises(VgxError):
        A.block_batch(0, 5, dev(np.zeros((4, 256), np.int16)))  # positions 5..8 past the cache
    A.free()


def test_gemm_q4_adversarial_groups(gpu):
    # the q4 group terms of test_q4_adversarial_groups through the batched
    # GEMM: plain, split and gate epilogues, bit-exact per token
    from test_gpu_kernels import q4_adversarial_matrix
    from test_oracle_pins import q4_adversarial_x
    rng = np.random.default_rng(77)
    rows, cols, ntok = 256, 768, 37
    m, m3 = q4_adversarial_matrix(rng, rows, cols), q4_adversarial_matrix(rng, rows, cols)
    W, W3 = gpu.upload(m), gpu.upload(m3)
    x = np.stack([q4_adversarial_x(rng, cols) for _ in range(ntok)])
    res = x_rows(rng, ntok, rows, full=True)
    got = host(gpu.gemm(W, dev(x), res=dev(res)))
    gate = host(gpu.ffn_gate_batch(W, W3, dev(x), 0))
    split = 384
    got_s = host(gpu.gemm_add_split(W, split, dev(x), dev(res)))
    a, b = m.slice_cols(0, split), m.slice_cols(split, cols)
    for t in range(ntok):
        v = oracle_rowval(m, x[t])
        assert np.array_equal(got[t], o.store(v, res[t])), t
        assert np.array_equal(gate[t], o.gate(v, oracle_rowval(m3, x[t]), 0)), t
        y1 = o.store(oracle_rowval(a, x[t, :split]), res[t])
        assert np.array_equal(got_s[t], o.store(oracle_rowval(b, x[t, split:]), y1)), t


# Launches of one token tile whose row tiles leave most CUs idle (the decode
# batch) split K across workgroups: each stores its exact integer sums and an
# epilogue kernel adds them and applies the fp32 epilogue -- every row still
# equals the oracle's batch-1 result
@pytest.mark.parametrize("kind,rows,cols", [("q8", 768, 2432), ("q4", 768, 2432), ("t3", 1024, 4096),
                                            ("t3", 1280, 1024), ("q4", 1536, 768)])
@pytest.mark.parametrize("ntok", [1, 7, 32])
def test_split_k_decode_batch(gpu, kind, rows, cols, ntok):
    rng = np.random.default_rng(rows + cols + ntok)
    m = MK[kind](rng, rows, cols)
    W = gpu.upload(m)
    x = x_rows(rng, ntok, cols, full=True)
    res = x_rows(rng, ntok, rows)
    got = host(gpu.gemm(W, dev(x), res=dev(res)))
    split = cols // 2 // 32 * 32
    got_s = host(gpu.gemm_add_split(W, split, dev(x), dev(res)))
    a, b = m.slice_cols(0, split), m.slice_cols(split, cols)
    m3 = MK[kind](rng, rows, cols)
    gate = host(gpu.ffn_gate_batch(W, gpu.upload(m3), dev(x), 2))
    rw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    rwq = o.quantize_act(rw)
    got_r = host(gpu.gemm_rms(W, dev(x), dev(rwq), 1e-5))
    for t in range(ntok):
        v = oracle_rowval(m, x[t])
        assert np.array_equal(got[t], o.store(v, res[t])), t
        y1 = o.store(oracle_rowval(a, x[t, :split]), res[t])
        assert np.array_equal(got_s[t], o.store(oracle_rowval(b, x[t, split:]), y1)), t
        assert np.array_equal(gate[t], o.gate(v, oracle_rowval(m3, x[t]), 2)), t
        xn = o.rmsnorm(x[t], rwq, 1e-5)
        assert np.array_equal(got_r[t], o.store(oracle_rowval(m, xn))), t


@pytest.mark.parametrize("kind,rows,cols", [("t3", 1024, 1024), ("q8", 768, 2432), ("q4", 768, 768),
                                            ("t3", 1024, 4096), ("q8", 1040, 2432)])
@pytest.mark.parametrize("ntok", [1, 32, 40])
def test_gemm_norm_equals_gemm_then_rmsnorm(gpu, kind, rows, cols, ntok):
    # the GEMM that writes the residual stream and the RMSNorm of its rows:
    # in the split-K epilogue launch (32 rows or fewer and rows longer than 32
    # k-steps: norm slices of 24, 32 and 33 values) or as a launch of its own
    # (40 rows, or K = 1024), the same bytes as vgx_gemm / vgx_gemm_add_split
    # then vgx_rmsnorm_batch, and the oracle's rows
    rng = np.random.default_rng(rows + ntok)
    m = MK[kind](rng, rows, cols)
    W = gpu.upload(m)
    x = x_rows(rng, ntok, cols, full=True)
    res = x_rows(rng, ntok, rows)
    nw = o.quantize_act(rng.uniform(0.5, 1.5, rows).astype(np.float32))
    split = cols // 2 // 32 * 32
    for sp in (0, split):
        y, yn = gpu.gemm_norm(W, dev(x), dev(res), dev(nw), 1e-5, split=sp)
        y, yn = host(y), host(yn)
        if sp:
            want_y = host(gpu.gemm_add_split(W, sp, dev(x), dev(res)))
        else:
            want_y = host(gpu.gemm(W, dev(x), res=dev(res)))
        assert np.array_equal(y, want_y), sp
        assert np.array_equal(yn, host(gpu.rmsnorm_batch(dev(y), dev(nw), 1e-5))), sp
        for t in range(min(ntok, 4)):
            assert np.array_equal(yn[t], o.rmsnorm(y[t], nw, 1e-5)), (sp, t)
