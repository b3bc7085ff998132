#!/usr/bin/env python3
"""Write tests/golden/float_golden.npz from the reference's float CPU path.

Run in the build container only (it reads /root/reference, which does not exist
on the GPU hosts):  python tests/golden/make_float_vectors.py

For each seeded container of float_cases.py the dequantised weights (exactly
what oracle/model.py FModel multiplies by: emb * es, and each q8 / q4 / t3
matrix's level times its row or group scale) are written as a float32 HF
checkpoint (model.safetensors + config.json) into a temporary directory, and
the reference's numpy tools run on it:

  * engine/tools/ref_generate.py Model.forward: the prompt one token at a time
    over its K/V cache (logits at every position), and the whole prompt as one
    prefill (logits of the last position);
  * engine/tools/ref_forward.py main: the whole-sequence forward (rotate-half
    models only; it has no interleaved RoPE);
  * engine/tools/mmcf_hf.py residual_peaks_lfm2: the hybrid conv/attention
    forward, max |residual| per layer over its three vocabulary runs.

The fixture keeps inputs (case name, seed, token ids, the container's sha256)
and outputs (logits, peaks) as data; nothing of the reference's code is stored.
"""
import json
import os
import struct
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (HERE, os.path.join(ROOT, "vc4-gles2-inference_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)

import float_cases as fc  # noqa: E402
from model import FModel  # noqa: E402
from vgx import synth  # noqa: E402

REF_TOOLS = "/root/reference/engine/tools"
OUT = os.path.join(HERE, "float_golden.npz")


def write_safetensors(path, tensors):
    hdr, off, blobs = {}, 0, []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, np.float32)
        hdr[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def hf_checkpoint(d, f, spec):
    """The float weights FModel multiplies by, under the HF Llama/Qwen3 names."""
    t = {"model.embed_tokens.weight": f.emb.astype(np.float32) * f.es[:, None],
         "model.norm.weight": f.rms_final}
    for l, W in enumerate(f.W):
        p = "model.layers.%d." % l
        t[p + "input_layernorm.weight"] = f.rms_att[l]
        t[p + "post_attention_layernorm.weight"] = f.rms_ffn[l]
        q, kv = f.dim, f.kv_dim
        t[p + "self_attn.q_proj.weight"] = W["qkv"][:q]
        t[p + "self_attn.k_proj.weight"] = W["qkv"][q:q + kv]
        t[p + "self_attn.v_proj.weight"] = W["qkv"][q + kv:]
        t[p + "self_attn.o_proj.weight"] = W["wo"]
        if f.qk_norm:
            t[p + "self_attn.q_norm.weight"] = f.qn[l]
            t[p + "self_attn.k_norm.weight"] = f.kn[l]
        t[p + "mlp.gate_proj.weight"] = W["w1"]
        t[p + "mlp.up_proj.weight"] = W["w3"]
        t[p + "mlp.down_proj.weight"] = W["w2"]
    write_safetensors(os.path.join(d, "model.safetensors"), t)
    cfg = {"hidden_size": spec.dim, "num_attention_heads": spec.heads, "num_key_value_heads": spec.kv_heads,
           "num_hidden_layers": spec.layers, "rope_theta": float(spec.theta), "rms_norm_eps": float(f.eps),
           "rope_interleaved": not spec.rope_half}
    with open(os.path.join(d, "config.json"), "w") as fh:
        json.dump(cfg, fh)


def hybrid_model_dict(f, spec):
    """The model dict residual_peaks_lfm2 reads (mmcf_hf.py:1253-1311), from
    FModel's dequantised weights."""
    L = spec.layers
    m = dict(dim=spec.dim, heads=spec.heads, kv=spec.kv_heads, layers=L, vocab=spec.vocab,
             theta=float(spec.theta), rms_eps=float(f.eps), layer_types=list(spec.layer_types),
             emb=f.emb.astype(np.float32) * f.es[:, None], rms_att=f.rms_att, rms_ffn=f.rms_ffn,
             q_norm=f.qn, k_norm=f.kn)
    for k in ("conv_in", "conv_out", "wq", "wk", "wv", "wo", "conv_w"):
        m[k] = [None] * L
    for k in ("w1", "w3", "w2"):
        m[k] = [W[k] for W in f.W]
    for l, W in enumerate(f.W):
        if f.is_conv[l]:
            m["conv_in"][l], m["conv_out"][l] = W["conv_in"], W["conv_out"]
            m["conv_w"][l] = np.asarray(f.conv_w[l], np.float32)
        else:
            q, kv = f.dim, f.kv_dim
            m["wq"][l], m["wk"][l], m["wv"][l] = W["qkv"][:q], W["qkv"][q:q + kv], W["qkv"][q + kv:]
            m["wo"][l] = W["wo"]
    return m


def main():
    if not os.path.isdir(REF_TOOLS):
        raise SystemExit("the reference tree is not here; the fixture is already committed")
    sys.path.insert(0, REF_TOOLS)
    import mmcf_hf
    import ref_forward
    import ref_generate

    out = {}
    for i, case in enumerate(fc.ATTN_CASES):
        name, n = case[0], case[5]
        seed = 31 + i
        spec, blob = fc.attn_container(case, seed)
        f = FModel(blob, qk_eps=None, tied_head=True)
        ids = synth.prompt(n, spec.vocab, seed=seed)
        with tempfile.TemporaryDirectory() as d:
            hf_checkpoint(d, f, spec)
            M = ref_generate.Model(d)
            cache = [[np.zeros((0, M.KV, M.hd), np.float32), np.zeros((0, M.KV, M.hd), np.float32)]
                     for _ in range(M.L)]
            inc = [M.forward([int(ids[0])], cache, 0)]
            for t in range(1, n):
                inc.append(M.forward([int(ids[t])], cache, t))
            cache = [[np.zeros((0, M.KV, M.hd), np.float32), np.zeros((0, M.KV, M.hd), np.float32)]
                     for _ in range(M.L)]
            pre = M.forward([int(v) for v in ids], cache, 0)
            out["%s_seed" % name] = np.int64(seed)
            out["%s_ids" % name] = ids
            out["%s_sha256" % name] = fc.sha(blob)
            out["%s_inc" % name] = np.stack(inc).astype(np.float32)
            out["%s_prefill" % name] = np.asarray(pre, np.float32)
            if spec.rope_half:
                lg = ref_forward.main(d, [int(v) for v in ids], float(spec.theta), float(f.eps))
                out["%s_fwd" % name] = np.asarray(lg, np.float32)
    for seed in fc.HYBRID_SEEDS:
        spec, blob = fc.hybrid_container(seed)
        f = FModel(blob, qk_eps=None, tied_head=True)
        m = hybrid_model_dict(f, spec)
        out["hybrid%d_sha256" % seed] = fc.sha(blob)
        out["hybrid%d_peaks" % seed] = np.array([mmcf_hf.residual_peaks_lfm2(m, seq=s) for s in fc.HYBRID_RUNS],
                                                np.float64)
    np.savez_compressed(OUT, **out)
    print("wrote %s (%d arrays, %d bytes)" % (OUT, len(out), os.path.getsize(OUT)))


if __name__ == "__main__":
    main()
