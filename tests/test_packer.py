"""The container toolchain (vgx.mmcf, the product's packer and reader) and the
oracle's C restatement of the quantizers, against vectors the reference
packer itself produced (tests/golden/packer_golden.npz, written by
tests/golden/make_packer_vectors.py from engine/tools/mmcf_hf.py and
engine/tools/mmcf_pack.py).  CPU only."""
import hashlib
import os
import struct
import zlib

import numpy as np
import pytest

import oracle as o
from inputs import tiny_model
from vgx import mmcf

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "packer_golden.npz"))


@pytest.mark.parametrize("name", ["a", "b", "c"])
def test_module_quantizers_match_reference(name):
    w = G["in_" + name]
    for impl in (mmcf, o):
        q, s = impl.qmat(w)
        assert np.array_equal(q, G["qmat_%s_q" % name]) and s == G["qmat_%s_s" % name]
        q, s = impl.q8mat(w)
        assert np.array_equal(q, G["q8mat_%s_q" % name]) and s == G["q8mat_%s_s" % name]
        r = impl.q4mat(w)
        assert np.array_equal(r[0], G["q4_%s_packed" % name])
        assert np.array_equal(r[1], G["q4_%s_s16" % name]) and np.array_equal(r[2], G["q4_%s_m16" % name])
        assert r[3] == G["q4_%s_ps" % name]


def test_t3mat_matches_reference():
    t = G["in_t"]
    packed, unit, plane = mmcf.t3mat(t)
    assert np.array_equal(np.frombuffer(packed, np.uint8), G["t3_packed"])
    assert unit == G["t3_unit"] and np.array_equal(plane, G["t3_plane"])
    packed2, unit2, plane2 = o.t3mat(t)
    assert np.array_equal(packed2, G["t3_packed"]) and np.float32(unit2) == np.float32(G["t3_unit"])
    assert np.array_equal(plane2, G["t3_plane"])


def _spec_from(m):
    return mmcf.ModelSpec(dim=m["dim"], hidden=m["hidden"], layers=m["layers"], heads=m["heads"],
                          kv_heads=m["kv"], vocab=m["vocab"], seq=m["seq"], theta=m["theta"],
                          rope_half=m["half"], qk_norm=bool(m["qk_norm"]))


@pytest.mark.parametrize("tag,scheme,q8_row,ternary,dedup", [
    ("q8row", "q8", True, False, False), ("q8", "q8", False, False, False),
    ("q4", "q4", False, False, False), ("t3", "t3", False, True, True)])
def test_container_bytes_match_reference(tag, scheme, q8_row, ternary, dedup):
    m = tiny_model(11, ternary)
    h = hashlib.sha256()
    for k in ("emb", "wq", "wk", "wv", "wo", "w1", "w3", "w2"):
        h.update(np.ascontiguousarray(m[k], np.float32).tobytes())
    assert np.array_equal(np.frombuffer(h.digest(), np.uint8), G["ct_%s_in_sha256" % tag]), \
        "the seeded inputs changed: regenerate the fixture"
    spec = _spec_from(m)
    w = {k: m[k] for k in ("emb", "wq", "wk", "wv", "wo", "w1", "w3", "w2", "rms_att", "rms_ffn",
                           "rms_final", "q_norm", "k_norm")}
    T = mmcf.tensors_from_float(spec, w, scheme, q8_row=q8_row, head_dedup=dedup)
    blob = mmcf.build(spec, T, scheme)
    assert blob == G["ct_" + tag].tobytes()


def test_oracle_q8_per_row_and_from_i16_match_container():
    # the nested packer functions are pinned through the golden container
    m = tiny_model(11, False)
    c = mmcf.Container(G["ct_q8row"].tobytes())
    mat = c.matrix(mmcf.T_WO, 0)
    q, unit, plane = o.q8_per_row(m["wo"][0])
    assert np.array_equal(q.view(np.uint8) ^ 0x80, mat.body.reshape(q.shape)) and np.float32(unit) == mat.scale
    assert np.array_equal(plane, mat.plane)
    c2 = mmcf.Container(G["ct_q8"].tobytes())
    mat2 = c2.matrix(mmcf.T_WO, 0)
    q2, s2 = o.q8_from_i16(m["wo"][0])
    assert np.array_equal(q2.view(np.uint8) ^ 0x80, mat2.body.reshape(q2.shape))
    assert np.float32(s2) == mat2.scale


def test_reader_round_trip_and_refusals():
    c = mmcf.Container(G["ct_q4"].tobytes())
    assert c.scheme == "q4" and c.spec.dim == 32 and c.spec.qk_norm
    mats = c.layer_mats(0)
    assert mats["w1"].rows == 64 and mats["w3"].rows == 64  # fused w13 split at its middle
    tiles = c.logits_tiles()
    assert len(tiles) == 1 and tiles[0].rows == 24 and tiles[0].kind == "q8"
    ct = mmcf.Container(G["ct_t3"].tobytes())
    t = ct.logits_tiles()  # head dedup: tiles rendered from the embedding
    emb, es = ct.embedding()
    assert not t[0].prebiased and np.array_equal(t[0].body, emb.view(np.uint8).ravel())
    assert t[0].scale == es.max() and np.array_equal(t[0].plane, es / es.max())
    raw = bytearray(G["ct_q8"].tobytes())
    with pytest.raises(ValueError):
        mmcf.Container(bytes(raw[:-1]))  # truncated: the size field catches it
    bad = bytearray(raw)
    bad[-1] ^= 0xFF
    with pytest.raises(ValueError):
        mmcf.Container(bytes(bad))  # body crc
    bad = bytearray(raw)
    bad[8] ^= 1
    with pytest.raises(ValueError):
        mmcf.Container(bytes(bad))  # header crc
