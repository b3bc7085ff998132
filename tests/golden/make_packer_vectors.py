#!/usr/bin/env python3
"""Write tests/golden/packer_golden.npz from the reference packer.

Run in the build container only (it reads /root/reference, which does not exist
on the GPU hosts):  python tests/golden/make_packer_vectors.py

The reference's quantizers (engine/tools/mmcf_hf.py: qmat, q8mat, q4mat,
t3mat and the nested q8_per_row / q8_from_i16 reached through
tensors_from_hf) and its container writer (engine/tools/mmcf_pack.py build)
run on small seeded float32 inputs; the fixture keeps the inputs and the
outputs (packed bytes, scales, planes, whole container bytes) as data.  Nothing
of the reference's code is stored.
"""
import os
import sys
import types

import hashlib

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from inputs import tiny_model  # noqa: E402

REF_TOOLS = "/root/reference/engine/tools"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "packer_golden.npz")


def main():
    if not os.path.isdir(REF_TOOLS):
        raise SystemExit("the reference tree is not here; the fixture is already committed")
    sys.path.insert(0, REF_TOOLS)
    import mmcf_hf
    import mmcf_pack

    rng = np.random.default_rng(20261201)
    out = {}
    a = rng.standard_normal((8, 64), dtype=np.float32) * np.float32(0.02)
    b = rng.standard_normal((16, 96), dtype=np.float32) * np.float32(0.5)
    b[3] = 0.0  # an all-zero row
    c = (rng.standard_normal((6, 64), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    out["in_a"], out["in_b"], out["in_c"] = a, b, c
    for name, w in (("a", a), ("b", b), ("c", c)):
        q, s = mmcf_hf.qmat(w)
        out["qmat_%s_q" % name], out["qmat_%s_s" % name] = q, np.float64(s)
        q, s = mmcf_hf.q8mat(w)
        out["q8mat_%s_q" % name], out["q8mat_%s_s" % name] = q, np.float64(s)
        packed, s16, m16, ps, groups = mmcf_hf.q4mat(w)
        out["q4_%s_packed" % name], out["q4_%s_s16" % name] = packed, s16
        out["q4_%s_m16" % name], out["q4_%s_ps" % name] = m16, np.float64(ps)
    # t3 on per-row ternary input, including an odd row count and a zero row
    tr = np.random.default_rng(7)
    lev = np.where(tr.random((7, 40)) < 0.4, 0, np.where(tr.random((7, 40)) < 0.5, 1, -1)).astype(np.float32)
    s = tr.uniform(0.01, 0.05, size=(7, 1)).astype(np.float32)
    t = lev * s
    t[2] = 0.0
    out["in_t"] = t
    packed, unit, plane = mmcf_hf.t3mat(t)
    out["t3_packed"] = np.frombuffer(packed, np.uint8).copy()
    out["t3_unit"], out["t3_plane"] = np.float64(unit), plane
    # whole containers: q8 per-row, q8 per-matrix (i16 first), q4, t3 (head dedup)
    args = types.SimpleNamespace(template="chatml", system="You are a helpful assistant.", chat=False,
                                 tools=False, vision=False, name="model", res="q16", rms_eps=None,
                                 add_bos=None, add_eos=None, _chat_templates=[])
    for tag, scheme, q8_row, ternary, dedup in (("q8row", "q8", True, False, False),
                                                ("q8", "q8", False, False, False),
                                                ("q4", "q4", False, False, False),
                                                ("t3", "t3", False, True, True)):
        m = tiny_model(11, ternary)
        meta, T = mmcf_hf.tensors_from_hf(None, scheme, 32, m=m, rail_check=False, q8_row=q8_row,
                                          head_dedup=dedup)
        blob = mmcf_pack.build(meta, T, None, args)
        out["ct_%s" % tag] = np.frombuffer(blob, np.uint8).copy()
        h = hashlib.sha256()
        for k in ("emb", "wq", "wk", "wv", "wo", "w1", "w3", "w2"):
            h.update(np.ascontiguousarray(m[k], np.float32).tobytes())
        out["ct_%s_in_sha256" % tag] = np.frombuffer(h.digest(), np.uint8).copy()
    np.savez_compressed(OUT, **out)
    print("wrote %s (%d arrays, %d bytes)" % (OUT, len(out), os.path.getsize(OUT)))


if __name__ == "__main__":
    main()
