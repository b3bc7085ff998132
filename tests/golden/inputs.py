"""Seeded float inputs shared by the fixture writer and the tests that read
the fixture (the fixture keeps a digest of them, so a change in numpy's
random streams fails loudly instead of comparing different inputs)."""
import numpy as np


def tiny_model(seed, ternary):
    """A 1-layer model dict in the shape of the reference's load_minimind
    result (engine/tools/mmcf_hf.py:1031-1043)."""
    rng = np.random.default_rng(seed)
    dim, hidden, heads, kv, vocab, layers = 32, 64, 2, 1, 24, 1
    hd = dim // heads

    def n(*s):
        return rng.standard_normal(s, dtype=np.float32) * np.float32(0.02)

    def t(r, c):
        u = rng.random((r, c), dtype=np.float32)
        lev = np.where(u < 0.4, 0, np.where(u < 0.7, 1, -1)).astype(np.float32)
        return lev * rng.uniform(0.01, 0.05, size=(r, 1)).astype(np.float32)

    mk = t if ternary else n
    emb = n(vocab, dim)
    return dict(dim=dim, hidden=hidden, layers=layers, heads=heads, kv=kv, vocab=vocab, seq=32,
                emb=emb, rms_att=np.ones((layers, dim), np.float32) * np.float32(1.25),
                rms_ffn=np.ones((layers, dim), np.float32), rms_final=np.ones(dim, np.float32),
                wq=np.stack([mk(dim, dim)]), wk=np.stack([mk(kv * hd, dim)]), wv=np.stack([mk(kv * hd, dim)]),
                wo=np.stack([mk(dim, dim)]), w1=np.stack([mk(hidden, dim)]), w3=np.stack([mk(hidden, dim)]),
                w2=np.stack([mk(dim, hidden)]), wcls=emb, theta=10000.0, half=True, rope_factors=None,
                qk_norm=1, q_norm=np.ones((layers, hd), np.float32), k_norm=np.ones((layers, hd), np.float32),
                untied=False, moe=None, sp_prefix=0)
