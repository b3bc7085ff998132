"""Seeded containers whose float forward the reference's own numpy tools
computed (tests/golden/float_golden.npz, written by make_float_vectors.py).

Shared by the fixture writer and the test that reads the fixture: each case
is rebuilt here from its seed, and the fixture keeps the container's sha256,
so a change in the generator fails loudly instead of comparing other weights.
"""
import hashlib

import numpy as np

from vgx import mmcf, synth

# name, scheme, spec, weight std (None: ternary), q8 per-row, prompt length
ATTN_CASES = (
    # GQA 4/2, per-head q/k RMSNorm, rotate-half, q8 per-row scales
    ("q8_gqa_qknorm", "q8", dict(dim=64, hidden=96, layers=2, heads=4, kv_heads=2, vocab=80, seq=32,
                                 theta=10000.0, rope_half=True, qk_norm=True), 0.02, True, 12),
    # MQA 4/1, no q/k norm (weights large enough that the scores are not flat), q4 g32
    ("q4_mqa", "q4", dict(dim=64, hidden=128, layers=2, heads=4, kv_heads=1, vocab=96, seq=32,
                          theta=10000.0, rope_half=True, qk_norm=False), 0.15, False, 12),
    # per-row ternary projections, GQA with q/k norm, tied head from the embedding
    ("t3_gqa_qknorm", "t3", dict(dim=64, hidden=96, layers=2, heads=4, kv_heads=2, vocab=80, seq=32,
                                 theta=10000.0, rope_half=True, qk_norm=True), None, True, 12),
    # interleaved (2i, 2i+1) RoPE pairs, per-matrix q8, no q/k norm
    ("q8_interleaved", "q8", dict(dim=64, hidden=96, layers=2, heads=2, kv_heads=1, vocab=80, seq=32,
                                  theta=500.0, rope_half=False, qk_norm=False), 0.15, False, 12),
)

# LFM2-shaped hybrid (conv, attn, conv); conv_in / conv_out scaled up so that
# the short convolution, not the embedding, sets the residual
HYBRID_SPEC = dict(dim=64, hidden=96, layers=3, heads=4, kv_heads=2, vocab=80, seq=32, theta=10000.0,
                   rope_half=True, qk_norm=True, layer_types=["conv", "attn", "conv"])
HYBRID_SEEDS = (41, 42)
HYBRID_RUNS = (1, 2, 3, 4, 6, 8)  # residual_peaks_lfm2's seq


def attn_case(name):
    for c in ATTN_CASES:
        if c[0] == name:
            return c
    raise KeyError(name)


def attn_container(case, seed):
    _name, scheme, sp, std, q8_row, _n = case
    spec = mmcf.ModelSpec(**sp)
    w = synth.ternary_weights(spec, seed) if std is None else synth.dense_weights(spec, seed, std=std)
    return spec, synth.container(spec, scheme, weights=w, q8_row=q8_row)


def hybrid_container(seed):
    spec = mmcf.ModelSpec(**HYBRID_SPEC)
    w = synth.dense_weights(spec, seed, std=0.02, conv_std=1.0)
    for l, t in enumerate(spec.layer_types):
        if t == "conv":
            w["conv_in"][l] = w["conv_in"][l] * np.float32(15.0)
            w["conv_out"][l] = w["conv_out"][l] * np.float32(15.0)
    return spec, synth.container(spec, "q8", weights=w, q8_row=True, head_dedup=False)


def sha(blob):
    return np.frombuffer(hashlib.sha256(bytes(blob)).digest(), np.uint8).copy()
