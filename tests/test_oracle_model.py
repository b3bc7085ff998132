"""The whole-model oracle (oracle/model.py) against the float path and against
its own per-op pieces.  CPU only."""
import numpy as np

import oracle as o
from model import FModel, QModel, parse
from vgx import synth


def test_qmodel_tracks_float_path():
    # the q16-grid decode follows the float CPU path on the same container;
    # the tiny model's activations are well above the grid step
    spec = synth.tiny_spec(seq=32)
    blob = synth.container(spec, "q8", seed=5)
    q, f = QModel(blob), FModel(blob)
    prompt = synth.prompt(6, spec.vocab, seed=5)
    tok, agree = None, 0
    for pos in range(12):
        t = int(prompt[pos]) if pos < 6 else tok
        lq, lf = q.step(t, pos) / 256.0, f.step(t, pos)
        assert np.abs(lq - lf).max() < 0.12
        tok = int(np.argmax(lq))
        agree += tok == int(np.argmax(lf))
    assert agree >= 10


def test_qmodel_layer0_equals_its_pieces():
    # a one-layer container's step is exactly the composition of the per-op
    # oracle functions in the reference's order (Session::forward_gpu_hidden)
    spec = synth.tiny_spec(seq=8)
    spec.layers = 1
    blob = synth.container(spec, "q4", seed=2)
    q = QModel(blob)
    got = q.step(7, 0)
    _, recs = parse(blob)
    h = o.embed_q8(recs[1][4].view(np.int8).reshape(spec.vocab, spec.dim), recs[2][4].view(np.float32), 7)
    L = q.mats[0]
    xb = o.rmsnorm(h, o.quantize_act(recs[3][4].view(np.float32)), 1e-5)
    qkv = o.store(L["qkv"].rowval(xb))
    kv = np.zeros(8 * o.kv_row_bytes(q.cfg), np.uint8)
    att = o.attn_block(q.cfg, qkv, q.qnq[0], q.knq[0], q.rtab, 0, kv)
    # at position 0 the attention output is V on the q16 grid (p = 1)
    v = qkv[spec.dim + spec.kv_dim:]
    rep = spec.heads // spec.kv_heads
    want_att = np.repeat(v.reshape(spec.kv_heads, -1), rep, axis=0).reshape(-1)
    assert np.array_equal(att, want_att)
    x1 = o.store(L["wo"].rowval(att), h)
    xb = o.rmsnorm(x1, o.quantize_act(recs[4][4].view(np.float32)), 1e-5)
    hb = o.gate(L["w1"].rowval(xb), L["w3"].rowval(xb))
    h = o.store(L["w2"].rowval(hb), x1)
    xf = o.rmsnorm(h, o.quantize_act(recs[5][4].view(np.float32)), 1e-5)
    want = np.concatenate([o.store(t.rowval(xf)) for t in q.tiles])
    assert np.array_equal(got, want)


def test_c_float_path_equals_numpy_float_path():
    # the C/OpenMP float path (the decode benchmarks' CPU baseline) runs the
    # numpy float forward: dense, hybrid-conv and ternary containers, one
    # thread and all, differ only in fp32 summation order
    from model import CFModel, float_lib
    lib = float_lib()
    cores = lib.vgxf_threads()
    for spec, scheme in ((synth.tiny_spec(seq=32), "q8"), (synth.tiny_hybrid_spec(seq=32), "q4"),
                         (synth.tiny_spec(seq=32, qk_norm=False), "t3")):
        blob = synth.container(spec, scheme, seed=8)
        for th in (1, cores):
            lib.vgxf_set_threads(th)
            f, c = FModel(blob), CFModel(blob)
            for pos, t in enumerate(synth.prompt(24, spec.vocab, seed=2)):
                lf, lc = f.step(int(t), pos), c.step(int(t), pos)
                assert np.abs(lf - lc).max() <= 1e-5 * np.abs(lf).max()
    lib.vgxf_set_threads(cores)
