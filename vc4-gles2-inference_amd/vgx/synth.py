"""Seeded synthetic models in the shapes the benchmarks name.

There are no checkpoints to download: weights are random with the stated
distribution from numpy's PCG64 (`default_rng(seed)`), float32, generated in a
fixed order (embedding, then per layer wq, wk, wv, wo -- or conv_in, the conv
kernel, conv_out for a conv layer -- then w1, w3, w2), and packed by vgx.mmcf
exactly as the reference packer would pack real float weights.
"""
import numpy as np

from . import mmcf


def minimind3_spec(seq=256):
    """MiniMind3-64M: 8 layers, hidden 768, SwiGLU 2432, 8 Q / 4 KV heads of
    96, vocab 6400, RoPE theta 1e6 (rotate-half), per-head q/k RMSNorm."""
    return mmcf.ModelSpec(dim=768, hidden=2432, layers=8, heads=8, kv_heads=4, vocab=6400, seq=seq,
                          theta=1e6, rope_half=True, qk_norm=True)


def bitcpm_spec(seq=512):
    """0.5B Llama-shaped ternary body: hidden 1024, 24 layers, FFN 4096,
    16 Q / 2 KV heads of 64, vocab 73448."""
    return mmcf.ModelSpec(dim=1024, hidden=4096, layers=24, heads=16, kv_heads=2, vocab=73448, seq=seq,
                          theta=10000.0, rope_half=True, qk_norm=False)


def tiny_spec(seq=64, qk_norm=True, hidden=96):
    """A small decoder with the same structure, for fast parity tests."""
    return mmcf.ModelSpec(dim=64, hidden=hidden, layers=2, heads=4, kv_heads=2, vocab=80, seq=seq,
                          theta=10000.0, rope_half=True, qk_norm=qk_norm)


LFM2_LAYERS = ["conv", "conv", "attn", "conv", "conv", "attn", "conv", "attn",
               "conv", "attn", "conv", "attn", "conv", "attn"]


def lfm2_spec(seq=256):
    """LFM2.5-230M-shaped hybrid: dim 1024, 8 gated short-conv layers (kernel 3)
    interleaved with 6 GQA attention layers (16 Q / 8 KV heads of 64, per-head
    q/k RMSNorm), SwiGLU 4608, vocab 64402, tied head, RoPE theta 1e6."""
    return mmcf.ModelSpec(dim=1024, hidden=4608, layers=14, heads=16, kv_heads=8, vocab=64402, seq=seq,
                          theta=1e6, rope_half=True, qk_norm=True, layer_types=list(LFM2_LAYERS))


def tiny_hybrid_spec(seq=48, hidden=96):
    """A small hybrid (conv, attn, conv) for fast parity tests."""
    return mmcf.ModelSpec(dim=64, hidden=hidden, layers=3, heads=4, kv_heads=2, vocab=80, seq=seq,
                          theta=10000.0, rope_half=True, qk_norm=True, layer_types=["conv", "attn", "conv"])


def dense_weights(spec, seed=0, std=0.02, conv_std=None):
    """N(0, std) projections and embedding, unit norm weights, tied head.
    Per layer, in this order: wq, wk, wv, wo for an attention layer, or
    conv_in (3*dim x dim), the depthwise kernel (dim x 3, N(0, conv_std),
    default std) and conv_out for a conv layer; then w1, w3, w2."""
    rng = np.random.default_rng(seed)

    def n(*shape, s=std):
        return rng.standard_normal(shape, dtype=np.float32) * np.float32(s)

    w = {"emb": n(spec.vocab, spec.dim)}
    for k in ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "conv_in", "conv_w", "conv_out"):
        w[k] = []
    types = spec.layer_types or ["attn"] * spec.layers
    for l in range(spec.layers):
        if types[l] == "conv":
            for k in ("wq", "wk", "wv", "wo"):
                w[k].append(None)
            w["conv_in"].append(n(3 * spec.dim, spec.dim))
            w["conv_w"].append(n(spec.dim, 3, s=std if conv_std is None else conv_std))
            w["conv_out"].append(n(spec.dim, spec.dim))
        else:
            for k in ("conv_in", "conv_w", "conv_out"):
                w[k].append(None)
            w["wq"].append(n(spec.dim, spec.dim))
            w["wk"].append(n(spec.kv_dim, spec.dim))
            w["wv"].append(n(spec.kv_dim, spec.dim))
            w["wo"].append(n(spec.dim, spec.dim))
        w["w1"].append(n(spec.hidden, spec.dim))
        w["w3"].append(n(spec.hidden, spec.dim))
        w["w2"].append(n(spec.dim, spec.hidden))
    w["rms_att"] = np.ones((spec.layers, spec.dim), np.float32)
    w["rms_ffn"] = np.ones((spec.layers, spec.dim), np.float32)
    w["rms_final"] = np.ones(spec.dim, np.float32)
    if spec.qk_norm:
        w["q_norm"] = np.ones((spec.layers, spec.head_dim), np.float32)
        w["k_norm"] = np.ones((spec.layers, spec.head_dim), np.float32)
    return w


def ternary_matrix(rng, rows, cols, p0=0.4, smin=0.01, smax=0.05):
    """Per-row {0, +-s}: entries i.i.d. P(0)=p0, P(+1)=P(-1)=(1-p0)/2, s ~ U(smin, smax)."""
    u = rng.random((rows, cols), dtype=np.float32)
    lev = np.where(u < p0, 0, np.where(u < p0 + (1 - p0) / 2, 1, -1)).astype(np.float32)
    s = rng.uniform(smin, smax, size=(rows, 1)).astype(np.float32)
    return lev * s


def ternary_weights(spec, seed=0, std=0.02):
    """Every projection per-row ternary; embedding N(0, std), unit norms."""
    rng = np.random.default_rng(seed)
    w = {"emb": rng.standard_normal((spec.vocab, spec.dim), dtype=np.float32) * np.float32(std)}
    for k in ("wq", "wk", "wv", "wo", "w1", "w3", "w2"):
        w[k] = []
    for _ in range(spec.layers):
        w["wq"].append(ternary_matrix(rng, spec.dim, spec.dim))
        w["wk"].append(ternary_matrix(rng, spec.kv_dim, spec.dim))
        w["wv"].append(ternary_matrix(rng, spec.kv_dim, spec.dim))
        w["wo"].append(ternary_matrix(rng, spec.dim, spec.dim))
        w["w1"].append(ternary_matrix(rng, spec.hidden, spec.dim))
        w["w3"].append(ternary_matrix(rng, spec.hidden, spec.dim))
        w["w2"].append(ternary_matrix(rng, spec.dim, spec.hidden))
    w["rms_att"] = np.ones((spec.layers, spec.dim), np.float32)
    w["rms_ffn"] = np.ones((spec.layers, spec.dim), np.float32)
    w["rms_final"] = np.ones(spec.dim, np.float32)
    if spec.qk_norm:
        w["q_norm"] = np.ones((spec.layers, spec.head_dim), np.float32)
        w["k_norm"] = np.ones((spec.layers, spec.head_dim), np.float32)
    return w


def container(spec, scheme, seed=0, q8_row=True, weights=None, head_dedup=None):
    """The MMCF bytes of a seeded synthetic model."""
    if weights is None:
        weights = ternary_weights(spec, seed) if scheme == "t3" else dense_weights(spec, seed)
    if head_dedup is None:
        head_dedup = scheme == "t3"
    T = mmcf.tensors_from_float(spec, weights, scheme, q8_row=q8_row, head_dedup=head_dedup)
    return mmcf.build(spec, T, scheme)


def prompt(n, vocab, seed=0):
    """n token ids uniform in [0, vocab)."""
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)
