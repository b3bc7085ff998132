"""The decode engine (libvgx_engine over libvgx) against the whole-model oracle.

Bars:
- bit-exact q16 logits at every step and identical greedy tokens against
  oracle/model.py's QModel (the reference's GPU-loop numerics);
- against the reference's float CPU path (FModel, ref_forward.py semantics on
  the dequantised container): max |logit difference| <= 0.4 and top-1
  agreement >= 75% over the greedy decode.  The gap is the reference's own
  q16 activation grid: N(0, 0.02) embeddings (max |x| ~ 0.07) sit on a 1/256
  grid with ~2.5% relative error that every layer carries forward."""
import numpy as np
import pytest

from model import CFModel, FModel, QModel
from vgx import synth
from vgx.engine import Engine

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("scheme,q8_row", [("q8", True), ("q8", False), ("q4", False), ("t3", False)])
def test_tiny_engine_bit_exact(gpu, scheme, q8_row):
    spec = synth.tiny_spec(seq=48, hidden=2112 if scheme != "t3" else 96)
    blob = synth.container(spec, scheme, seed=3, q8_row=q8_row)
    ref = QModel(blob)
    eng = Engine(blob)
    prompt = synth.prompt(6, spec.vocab, seed=1)
    tok = None
    for pos in range(14):
        t = int(prompt[pos]) if pos < len(prompt) else tok
        want = ref.step(t, pos)
        got, nxt = eng.step(t, pos)
        assert np.array_equal(got, want), (scheme, pos)
        tok = int(np.argmax(want))
        assert nxt == tok
    eng.close()
    # greedy generate from a fresh KV matches the stepwise greedy sequence
    ref2, eng2 = QModel(blob), Engine(blob)
    out, _, _ = eng2.generate(prompt, 8)
    want, tok = [], None
    for pos in range(len(prompt) + 7):
        t = int(prompt[pos]) if pos < len(prompt) else tok
        lg = ref2.step(t, pos, want_logits=pos >= len(prompt) - 1)
        if lg is not None:
            tok = int(np.argmax(lg))
            want.append(tok)
    assert list(out) == want
    eng2.close()


def test_minimind3_q8_decode_c1(gpu):
    """MiniMind3-64M q8 per-row, KV q16, SEQ 256: 32 prompt tokens and 64
    greedy tokens, bit-exact logits and tokens against the oracle."""
    spec = synth.minimind3_spec(seq=256)
    blob = synth.container(spec, "q8", seed=0, q8_row=True)
    prompt = synth.prompt(32, spec.vocab, seed=0)
    eng = Engine(blob, kv_bits=16)
    out, pf, dc = eng.generate(prompt, 64)
    eng.close()
    ref, f = QModel(blob), FModel(blob)
    eng = Engine(blob, kv_bits=16)
    want, tok, diffs, agree = [], None, [], 0
    for pos in range(32 + 63):
        t = int(prompt[pos]) if pos < 32 else tok
        lq = ref.step(t, pos)
        if pos < 4 or pos % 16 == 0:
            got, _ = eng.step(t, pos)
            assert np.array_equal(got, lq), pos
        else:
            eng.step(t, pos, logits=False)
        lf = f.step(t, pos)
        if pos >= 31:
            tok = int(np.argmax(lq))
            want.append(tok)
            diffs.append(np.abs(lq / 256.0 - lf).max())
            agree += int(tok == int(np.argmax(lf)))
    assert list(out) == want
    assert max(diffs) <= 0.4, max(diffs)
    assert agree >= 0.75 * len(want), agree
    eng.close()


def test_minimind3_q4_kv8(gpu):
    """q4 weights with the KV cache packed q8 (the C3 layout), SEQ 768."""
    spec = synth.minimind3_spec(seq=768)
    blob = synth.container(spec, "q4", seed=0)
    prompt = synth.prompt(12, spec.vocab, seed=2)
    ref, eng = QModel(blob, kv_bits=8), Engine(blob, kv_bits=8)
    tok = None
    for pos in range(20):
        t = int(prompt[pos]) if pos < 12 else tok
        want = ref.step(t, pos)
        got, nxt = eng.step(t, pos)
        assert np.array_equal(got, want), pos
        tok = nxt
    eng.close()


@pytest.mark.parametrize("scheme", ["q8", "q4", "t3"])
def test_prefill_batches_equal_serial(gpu, scheme):
    """The reference's acceptance for a batched prefill: the logits after the
    prompt are byte-identical to the serial loop's (docs/prefill-batching.md:
    98-113), for one batch, uneven batches, and a prompt continued at pos0 > 0."""
    spec = synth.tiny_spec(seq=48, hidden=2112 if scheme != "t3" else 96)
    blob = synth.container(spec, scheme, seed=4)
    prompt = synth.prompt(29, spec.vocab, seed=3)
    ser = Engine(blob)
    ser.set_prefill_batch(0)
    want, wn = ser.prefill(prompt)
    ref = QModel(blob)
    for pos in range(len(prompt)):
        lq = ref.step(int(prompt[pos]), pos, want_logits=pos == len(prompt) - 1)
    assert np.array_equal(want, lq)
    for batch in (48, 8, 5):
        eng = Engine(blob)
        eng.set_prefill_batch(batch)
        got, gn = eng.prefill(prompt)
        assert np.array_equal(got, want), batch
        assert gn == wn
        if batch == 48:
            # decode continues identically from the batched KV
            a, _ = eng.step(gn, len(prompt))
            b, _ = ser.step(wn, len(prompt))
            assert np.array_equal(a, b)
        eng.close()
    # prompt split over two calls: positions 0..11, then 12..28
    eng = Engine(blob)
    eng.prefill(prompt[:12], 0, logits=False)
    got, _ = eng.prefill(prompt[12:], 12)
    assert np.array_equal(got, want)
    eng.close()
    ser.close()


def test_minimind3_q4_kv8_float_tolerance(gpu):
    """The C3 run against the float path: MiniMind3 q4, KV q8, SEQ 768, a
    256-token prompt in one batch, then 512 greedy steps (positions 256..767,
    so every per-head attention plan runs, the pair V plan past one round).

    Bars, at every greedy step (the engine's logits against CFModel, the float
    forward of engine/tools/ref_forward.py:47-115 on the dequantised weights,
    fed the engine's tokens):
    - max |logit difference| <= 0.6 and mean <= 0.12 (float logits' std
      0.55); measured on seed 0: max 0.465, mean <= 0.086;
    - top-1 agreement >= 70% of the steps (measured 412 of 512), the greedy
      token within the float top 5 at >= 95% (506 of 512) and always within
      its top 32 (worst rank 16).
    The KV cache's q8 grid (1/16, clamped to [-128, 127]:
    engine/src/shaders_attn.cpp:141-156) adds to the activation grid's gap.
    Its share is isolated by a second engine with a q16 cache fed the same
    tokens: |logits(KV q8) - logits(KV q16)| <= 0.4 (measured 0.289, mean
    0.053).  The clamp itself never engages on this workload: no cached value
    sits on a rail (the largest |q| is 70 of 128, i.e. |k|, |v| <= 4.4), which
    the oracle's cache shows at the end.  q16 logits equal the oracle's (QModel,
    KV q8) bit for bit at the prompt's last position and at every 64th step."""
    import oracle as o
    spec = synth.minimind3_spec(seq=768)
    blob = synth.container(spec, "q4", seed=0)
    prompt = synth.prompt(256, spec.vocab, seed=0)
    eng8, eng16 = Engine(blob, kv_bits=8), Engine(blob, kv_bits=16)
    ref, f = QModel(blob, kv_bits=8), CFModel(blob)
    got, tok = eng8.prefill(prompt)
    eng16.prefill(prompt, logits=False)
    for pos in range(256):
        lq = ref.step(int(prompt[pos]), pos, want_logits=pos == 255)
        lf = f.step(int(prompt[pos]), pos, logits=pos == 255)
    assert np.array_equal(got, lq)
    assert tok == int(np.argmax(lq))
    stats, grid = [], []
    for pos in range(256, 768):
        d = np.abs(got / 256.0 - lf)
        stats.append((d.max(), d.mean(), int((lf > lf[tok]).sum())))
        if pos == 767:
            break
        got, nxt = eng8.step(tok, pos)
        g16, _ = eng16.step(tok, pos)
        grid.append(np.abs(got.astype(np.int64) - g16).max() / 256.0)
        lq = ref.step(tok, pos, want_logits=pos % 64 == 0)
        if lq is not None:
            assert np.array_equal(got, lq), pos
        assert nxt == int(np.argmax(got)), pos
        lf = f.step(tok, pos)
        tok = nxt
    eng8.close()
    eng16.close()
    n = len(stats)
    assert n == 512
    assert max(s[0] for s in stats) <= 0.6, max(s[0] for s in stats)
    assert max(s[1] for s in stats) <= 0.12, max(s[1] for s in stats)
    assert sum(s[2] == 0 for s in stats) >= 0.70 * n, sum(s[2] == 0 for s in stats)
    assert sum(s[2] < 5 for s in stats) >= 0.95 * n, sum(s[2] < 5 for s in stats)
    assert max(s[2] for s in stats) < 32, max(s[2] for s in stats)
    assert max(grid) <= 0.4, max(grid)
    rb = o.kv_row_bytes(ref.cfg)
    for l in range(spec.layers):
        kv = ref.kv[l][:767 * rb].view(np.int8)
        assert not ((kv == -128) | (kv == 127)).any(), l


def test_minimind3_q4_prefill_256_kv8(gpu):
    """The C3 shape: MiniMind3 q4, KV q8, SEQ 768, a 256-token prompt in one
    batch against the serial loop, then greedy decode from both."""
    spec = synth.minimind3_spec(seq=768)
    blob = synth.container(spec, "q4", seed=0)
    prompt = synth.prompt(256, spec.vocab, seed=0)
    a, b = Engine(blob, kv_bits=8), Engine(blob, kv_bits=8)
    b.set_prefill_batch(0)
    la, ta = a.prefill(prompt)
    lb, tb = b.prefill(prompt)
    assert np.array_equal(la, lb) and ta == tb
    for pos in range(256, 264):
        la, ta = a.step(ta, pos)
        lb, tb = b.step(tb, pos)
        assert np.array_equal(la, lb) and ta == tb, pos
    a.close()
    b.close()


@pytest.mark.parametrize("scheme", ["q8", "q4", "t3"])
def test_hybrid_engine_bit_exact(gpu, scheme):
    """An LFM2-structured hybrid (conv, attn, conv): every step's logits equal
    the oracle's, and a batched prompt equals the serial loop."""
    spec = synth.tiny_hybrid_spec(seq=48, hidden=2112 if scheme != "t3" else 96)
    w = (synth.ternary_weights if scheme == "t3" else synth.dense_weights)(spec, seed=6)
    if scheme == "t3":
        rng = np.random.default_rng(6)
        w["conv_w"] = [rng.standard_normal((spec.dim, 3)).astype(np.float32) * np.float32(0.5)
                       if t == "conv" else None for t in spec.layer_types]
        w["conv_in"] = [synth.ternary_matrix(rng, 3 * spec.dim, spec.dim) if t == "conv" else None
                        for t in spec.layer_types]
        w["conv_out"] = [synth.ternary_matrix(rng, spec.dim, spec.dim) if t == "conv" else None
                         for t in spec.layer_types]
    else:
        w = synth.dense_weights(spec, seed=6, std=0.05, conv_std=0.5)
    blob = synth.container(spec, scheme, weights=w)
    ref, eng = QModel(blob), Engine(blob)
    prompt = synth.prompt(7, spec.vocab, seed=2)
    tok = None
    for pos in range(16):
        t = int(prompt[pos]) if pos < len(prompt) else tok
        want = ref.step(t, pos)
        got, nxt = eng.step(t, pos)
        assert np.array_equal(got, want), (scheme, pos)
        tok = nxt
    # a new sequence at position 0 starts from an empty conv history
    got, _ = eng.step(int(prompt[0]), 0)
    assert np.array_equal(got, QModel(blob).step(int(prompt[0]), 0))
    eng.close()
    a, b = Engine(blob), Engine(blob)
    b.set_prefill_batch(0)
    la, ta = a.prefill(prompt)
    lb, tb = b.prefill(prompt)
    assert np.array_equal(la, lb) and ta == tb
    la, _ = a.step(ta, len(prompt))
    lb, _ = b.step(tb, len(prompt))
    assert np.array_equal(la, lb)
    a.close()
    b.close()


def test_lfm2_230m_shape(gpu):
    """The C4 run (LFM2.5-230M-shaped q8: 8 conv + 6 attention layers, dim
    1024, vocab 64402; a 64-token prompt in one batch, 128 greedy steps, KV
    q16, SEQ 256): bit-exact against the oracle at the prompt's end and at
    every 16th step, and within the stated tolerance of the float path at
    every step.

    The gap is the reference's own q16 activation grid on a residual of order
    0.02 over 14 layers, which the reference documents for LFM2.5 (2-3
    significant bits per component after the embedding,
    engine/src/session.cpp:328-333).  Measured on seed 0 (prompt seed 4): max
    |logit difference| 1.38, mean <= 0.24, against float logits of std 0.64.
    Random N(0, 0.02) weights give a flat top: at 49 of the 128 steps the
    float path's two largest logits lie within 0.1 of each other, well inside
    the grid's mean gap, so top-1 agreement (measured 45 of 128) and rank
    (worst 364 of 64402) measure that flatness more than the error.  The
    bound that follows from the error is the float-path regret of the greedy
    token, max(lf) - lf[token] <= 2 max |lq - lf|: measured <= 1.07, mean 0.23.
    Bars: max <= 1.6, mean <= 0.3, regret <= 1.3 and its mean <= 0.3, top-1
    >= 25% and top-5 >= 50% (measured 78 of 128)."""
    spec = synth.lfm2_spec(seq=256)
    blob = synth.container(spec, "q8", seed=0, q8_row=True)
    prompt = synth.prompt(64, spec.vocab, seed=4)
    eng = Engine(blob)
    ref, f = QModel(blob), CFModel(blob)
    got, tok = eng.prefill(prompt)
    for pos in range(len(prompt)):
        lq = ref.step(int(prompt[pos]), pos, want_logits=pos == len(prompt) - 1)
        lf = f.step(int(prompt[pos]), pos, logits=pos == len(prompt) - 1)
    assert np.array_equal(got, lq)

    def gap(lq, lf, tok):
        d = np.abs(lq / 256.0 - lf)
        return d.max(), d.mean(), int((lf > lf[tok]).sum()), float(lf.max() - lf[tok])

    gaps = []
    for pos in range(len(prompt), len(prompt) + 128):
        gaps.append(gap(got, lf, tok))
        if pos == len(prompt) + 127:
            break
        got, nxt = eng.step(tok, pos)
        lq = ref.step(tok, pos, want_logits=pos < len(prompt) + 4 or pos % 16 == 0)
        if lq is not None:
            assert np.array_equal(got, lq), pos
        assert nxt == int(np.argmax(got)), pos
        lf = f.step(tok, pos)
        tok = nxt
    eng.close()
    n = len(gaps)
    assert n == 128
    assert max(g[0] for g in gaps) <= 1.6, max(g[0] for g in gaps)
    assert max(g[1] for g in gaps) <= 0.3, max(g[1] for g in gaps)
    assert max(g[3] for g in gaps) <= 1.3, max(g[3] for g in gaps)
    assert np.mean([g[3] for g in gaps]) <= 0.3, np.mean([g[3] for g in gaps])
    assert all(g[3] <= 2 * g[0] + 1e-6 for g in gaps)
    assert sum(g[2] == 0 for g in gaps) >= 0.25 * n, sum(g[2] == 0 for g in gaps)
    assert sum(g[2] < 5 for g in gaps) >= 0.5 * n, sum(g[2] < 5 for g in gaps)


def test_engine_refusals(gpu):
    from vgx import lib as vl
    spec = synth.tiny_spec(seq=8)
    blob = synth.container(spec, "q8", seed=0)
    eng = Engine(blob)
    with pytest.raises(vl.VgxError):
        eng.step(0, 8)  # position beyond the KV length
    with pytest.raises(vl.VgxError):
        eng.step(spec.vocab, 0)  # token outside the vocabulary
    with pytest.raises(vl.VgxError):
        eng.generate(np.zeros(6, np.int32), 4)  # 6 + 4 - 1 > 8
    eng.close()
    bad = bytearray(blob)
    bad[-3] ^= 1
    with pytest.raises(vl.VgxError):
        Engine(bytes(bad))  # body crc
    with pytest.raises(vl.VgxError):
        Engine(blob[:-16])  # truncated
    w = synth.dense_weights(spec, seed=0)
    w["wcls"] = np.concatenate([w["emb"], w["emb"][:16]])
    with pytest.raises(vl.VgxError, match="logits tiles"):
        Engine(synth.container(spec, "q8", weights=w))  # head tiles beyond the vocabulary


@pytest.mark.parametrize("scheme", ["q8", "t3", "q4"])
def test_generate_batch_equals_single(gpu, scheme):
    """Sequences decoded in lockstep (GEMMs over the sequences, one attention
    launch for all of them) give exactly the tokens each prompt gives alone."""
    spec = synth.tiny_spec(seq=48, hidden=2112 if scheme != "t3" else 96)
    blob = synth.container(spec, scheme, seed=8)
    prompts = np.stack([synth.prompt(7, spec.vocab, seed=s) for s in range(5)])
    eng = Engine(blob)
    got, pf, dc = eng.generate_batch(prompts, 12)
    assert got.shape == (5, 12)
    for s in range(5):
        want, _, _ = eng.generate(prompts[s], 12)
        assert list(got[s]) == list(want), s
    # a second call with fewer sequences reuses the caches
    got2, _, _ = eng.generate_batch(prompts[3:], 12)
    assert np.array_equal(got2, got[3:])
    eng.close()


def test_generate_batch_minimind3_shape(gpu):
    """The C1 model shape with 8 sequences: every row equals its own single
    generation (q8 per-row, KV q16)."""
    spec = synth.minimind3_spec(seq=96)
    blob = synth.container(spec, "q8", seed=0, q8_row=True)
    prompts = np.stack([synth.prompt(16, spec.vocab, seed=s) for s in range(8)])
    eng = Engine(blob)
    got, _, _ = eng.generate_batch(prompts, 24)
    for s in (0, 5, 7):
        want, _, _ = eng.generate(prompts[s], 24)
        assert list(got[s]) == list(want), s
    eng.close()


def test_generate_batch_refusals(gpu):
    from vgx import lib as vl
    spec = synth.tiny_hybrid_spec(seq=16)
    eng = Engine(synth.container(spec, "q8", seed=0))
    with pytest.raises(vl.VgxError):
        eng.generate_batch(np.zeros((2, 4), np.int32), 3)  # conv models decode one sequence
    eng.close()
    spec = synth.tiny_spec(seq=16)
    eng = Engine(synth.container(spec, "q8", seed=0))
    with pytest.raises(vl.VgxError):
        eng.generate_batch(np.zeros((2, 10), np.int32), 8)  # 10 + 8 - 1 > 16
    with pytest.raises(vl.VgxError):
        eng.generate_batch(np.zeros((17, 4), np.int32), 2)  # more sequences than min(seq, 512)
    eng.close()


def _mmkv_header(raw):
    """The MMKV1 header fields (engine/src/prefix_cache.cpp:33-56)."""
    import struct
    assert raw[:5] == b"MMKV1"
    ver, size, mtime = struct.unpack_from("<IQQ", raw, 8)
    dims = struct.unpack_from("<8I", raw, 28)
    theta, flags, n, width = struct.unpack_from("<fIII", raw, 60)
    off = 76
    vsw = None
    if ver >= 3:
        vsw, = struct.unpack_from("<I", raw, off)
        off += 4
    kscale, = struct.unpack_from("<f", raw, off)
    off += 4
    toks = np.frombuffer(raw, np.uint32, n, off)
    return dict(version=ver, size=size, mtime=mtime, dims=dims, theta=theta, flags=flags, n=n, width=width,
                vsw=vsw, kscale=kscale, toks=toks, body=off + 4 * n)


@pytest.mark.parametrize("kv_bits", [16, 8])
def test_prefix_cache_round_trip(gpu, tmp_path, kv_bits):
    """MMKV1: a cache saved after a prompt, loaded into a fresh engine, resumes
    to exactly the tokens the uncached run gives; the file holds the reference
    header and the KV rows in the texel byte layout."""
    import json
    spec = synth.tiny_spec(seq=48)
    blob = synth.container(spec, "q8", seed=5)
    prompt = synth.prompt(20, spec.vocab, seed=4)
    full, _, _ = Engine(blob, kv_bits=kv_bits).generate(prompt, 10)
    a = Engine(blob, kv_bits=kv_bits)
    a.prefill(prompt[:14], logits=False)
    path = tmp_path / "p.mmkv"
    a.save_prefix(path, prompt[:14], system_fnv=0x1234, tools_fnv=5)
    raw = path.read_bytes()
    h = _mmkv_header(raw)
    kv_dim = spec.kv_heads * spec.head_dim
    assert h["version"] == 2 and h["size"] == len(blob) and h["mtime"] == 0
    assert h["dims"] == (spec.dim, spec.hidden, spec.layers, spec.heads, spec.kv_heads, spec.vocab, 48,
                         spec.head_dim)
    assert h["flags"] == 1 | 2 | (4 if kv_bits == 16 else 8) and h["n"] == 14
    assert h["width"] == (kv_dim if kv_bits == 16 else kv_dim // 2)
    assert h["kscale"] == (2048.0 if kv_bits == 16 else 16.0)
    assert list(h["toks"]) == list(prompt[:14])
    rb = h["width"] * 4
    assert len(raw) == h["body"] + spec.layers * 14 * rb
    side = json.loads((tmp_path / "p.mmkv.json").read_text())
    assert side["format"] == "mmkv" and side["n_tokens"] == 14 and side["system_fnv64"] == "%016x" % 0x1234
    fnv = 1469598103934665603
    for t in prompt[:14]:
        for b in range(4):
            fnv = ((fnv ^ ((int(t) >> (8 * b)) & 0xFF)) * 1099511628211) & ((1 << 64) - 1)
    assert side["tokens_fnv64"] == "%016x" % fnv
    a.close()
    b = Engine(blob, kv_bits=kv_bits)
    assert list(b.load_prefix(path)) == list(prompt[:14])
    got, _, _ = b.generate_from(prompt, 14, 10)
    assert list(got) == list(full)
    b.close()
    # refusals: another KV packing, another container, a damaged header
    from vgx import lib as vl
    c = Engine(blob, kv_bits=8 if kv_bits == 16 else 16)
    with pytest.raises(vl.VgxError):
        c.load_prefix(path)
    c.close()
    other = synth.container(synth.tiny_spec(seq=48), "q8", seed=6, q8_row=True)
    if len(other) != len(blob):
        d = Engine(other, kv_bits=kv_bits)
        with pytest.raises(vl.VgxError):
            d.load_prefix(path)
        d.close()
    bad = bytearray(raw)
    bad[28] ^= 1  # dim
    (tmp_path / "bad.mmkv").write_bytes(bytes(bad))
    e = Engine(blob, kv_bits=kv_bits)
    with pytest.raises(vl.VgxError):
        e.load_prefix(tmp_path / "bad.mmkv")
    e.close()


def test_prefix_cache_hybrid_conv_history(gpu, tmp_path):
    """A hybrid's cache (version 4) carries the conv history, so a reload
    resumes the conv layers exactly."""
    spec = synth.tiny_hybrid_spec(seq=48, hidden=2112)
    w = synth.dense_weights(spec, seed=6, std=0.05, conv_std=0.5)
    blob = synth.container(spec, "q8", weights=w)
    prompt = synth.prompt(17, spec.vocab, seed=2)
    full, _, _ = Engine(blob).generate(prompt, 9)
    a = Engine(blob)
    a.prefill(prompt[:11], logits=False)
    path = tmp_path / "h.mmkv"
    a.save_prefix(path, prompt[:11])
    a.close()
    h = _mmkv_header(path.read_bytes())
    assert h["version"] == 4 and h["vsw"] == 0 and h["flags"] & 32
    nconv = sum(1 for t in spec.layer_types if t == "conv")
    assert len(path.read_bytes()) == h["body"] + spec.layers * 11 * h["width"] * 4 + nconv * 2 * 2 * spec.dim
    b = Engine(blob)
    b.load_prefix(path)
    got, _, _ = b.generate_from(prompt, 11, 9)
    assert list(got) == list(full)
    b.close()


@pytest.mark.parametrize("scheme", ["q8", "t3"])
def test_decode_graph_equals_launches(gpu, scheme):
    """The decode step replayed as one captured graph (the position and token
    in device memory) gives the tokens of the step-by-step launches, replay
    after replay, with other engine work and syncs in between."""
    spec = synth.tiny_spec(seq=64, hidden=2112 if scheme != "t3" else 96)
    blob = synth.container(spec, scheme, seed=21)
    a, b = Engine(blob), Engine(blob)
    b.set_graphs(False)
    for k in range(4):
        prompt = synth.prompt(5 + 3 * k, spec.vocab, seed=30 + k)
        ga, _, _ = a.generate(prompt, 20)
        gb, _, _ = b.generate(prompt, 20)
        assert list(ga) == list(gb), k
        # eager work on the graph engine between replays: a step and a prefill
        la, _ = a.step(int(prompt[0]), 0)
        lb, _ = b.step(int(prompt[0]), 0)
        assert np.array_equal(la, lb)
    a.close()
    b.close()


def test_decode_multi_step_graph_counts(gpu):
    """Greedy generation replays a graph of four decode steps for each run of
    four tokens and the one-step graph for the rest (a step of this tiny model
    has far fewer than 100 launches): every token count around the multiples
    of four -- no replay, only one-step replays, exactly one four-step replay,
    one with a remainder, several -- gives the step-by-step launches' tokens."""
    spec = synth.tiny_spec(seq=64, hidden=2112)
    blob = synth.container(spec, "q8", seed=23)
    a, b = Engine(blob), Engine(blob)
    b.set_graphs(False)
    prompt = synth.prompt(6, spec.vocab, seed=41)
    for n in (1, 2, 4, 5, 6, 9, 13):
        ga, _, _ = a.generate(prompt, n)
        gb, _, _ = b.generate(prompt, n)
        assert list(ga) == list(gb), n
    a.close()
    b.close()


def test_decode_graph_hybrid_and_cache(gpu, tmp_path):
    """The graph on a hybrid (conv state advancing inside the replay) and
    resuming from a loaded prefix cache."""
    spec = synth.tiny_hybrid_spec(seq=48, hidden=2112)
    blob = synth.container(spec, "q8", weights=synth.dense_weights(spec, seed=7, std=0.05, conv_std=0.5))
    prompt = synth.prompt(9, spec.vocab, seed=5)
    a, b = Engine(blob), Engine(blob)
    b.set_graphs(False)
    ga, _, _ = a.generate(prompt, 16)
    gb, _, _ = b.generate(prompt, 16)
    assert list(ga) == list(gb)
    a.prefill(prompt[:6], logits=False)
    a.save_prefix(tmp_path / "g.mmkv", prompt[:6])
    c = Engine(blob)
    c.load_prefix(tmp_path / "g.mmkv")
    gc, _, _ = c.generate_from(prompt, 6, 16)
    assert list(gc) == list(gb)
    for e in (a, b, c):
        e.close()


@pytest.fixture(scope="module")
def c5_model():
    """The C5 model: 0.5B Llama-shaped per-row ternary body (hidden 1024, 24
    layers, FFN 4096, 16 Q / 2 KV heads of 64, vocab 73448), KV q16, SEQ 512."""
    spec = synth.bitcpm_spec(seq=512)
    return spec, synth.container(spec, "t3", seed=0, q8_row=True)


def test_c5_ternary_decode(gpu, c5_model):
    """C5 at batch 1: a batched prompt then greedy decode, bit-exact q16
    logits and tokens against the oracle at every position, and within the
    stated tolerance of the float path (CFModel: the float forward on the
    dequantised weights).  Tolerance for this shape: max |logit difference|
    <= 0.8 and mean <= 0.15 (float logits' std 0.64), top-1 agreement >= 60%,
    the greedy token within the float top 8; measured on seed 0 over 14
    positions: max 0.33-0.57, mean 0.06-0.09, top-1 11 of 14, ranks 0-3."""
    spec, blob = c5_model
    prompt = synth.prompt(6, spec.vocab, seed=0)
    eng = Engine(blob, kv_bits=16)
    ref, f = QModel(blob), CFModel(blob)
    got, tok = eng.prefill(prompt)
    for pos in range(len(prompt)):
        lq = ref.step(int(prompt[pos]), pos)
        lf = f.step(int(prompt[pos]), pos)
    assert np.array_equal(got, lq)
    stats, toks = [], [tok]
    for pos in range(len(prompt), len(prompt) + 10):
        d = np.abs(lq / 256.0 - lf)
        stats.append((d.max(), d.mean(), int((lf > lf[int(np.argmax(lq))]).sum())))
        got, nxt = eng.step(tok, pos)
        lq, lf = ref.step(tok, pos), f.step(tok, pos)
        assert np.array_equal(got, lq), pos
        assert nxt == int(np.argmax(lq)), pos
        tok = nxt
        toks.append(tok)
    assert max(s[0] for s in stats) <= 0.8, stats
    assert max(s[1] for s in stats) <= 0.15, stats
    assert sum(s[2] == 0 for s in stats) >= 0.6 * len(stats), stats
    assert max(s[2] for s in stats) < 8, stats
    # greedy generation (prompt batched, decode replayed as a graph) = the steps
    out, _, _ = eng.generate(prompt, len(toks))
    assert list(out) == toks
    eng.close()


def test_c5_ternary_batch32(gpu, c5_model):
    """C5 at batch 32: 32 sequences in lockstep (the int8-MFMA GEMMs over the
    sequences, one attention launch, the concatenated q8 head) give exactly
    the tokens each prompt gives alone."""
    spec, blob = c5_model
    prompts = np.stack([synth.prompt(12, spec.vocab, seed=s) for s in range(32)])
    eng = Engine(blob, kv_bits=16)
    got, _, _ = eng.generate_batch(prompts, 10)
    assert got.shape == (32, 10)
    for s in range(32):
        want, _, _ = eng.generate(prompts[s], 10)
        assert list(got[s]) == list(want), s
    eng.close()
