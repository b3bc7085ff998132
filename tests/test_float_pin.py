"""The float CPU path (oracle/model.py FModel) against the reference's own
numpy float tools, on the vectors tests/golden/make_float_vectors.py wrote with
them: engine/tools/ref_generate.py (K/V-cached forward, both RoPE layouts),
engine/tools/ref_forward.py (whole-sequence forward) and
engine/tools/mmcf_hf.py residual_peaks_lfm2 (the LFM2 conv/attention hybrid).

FModel runs here with the tools' conventions (q/k RMSNorm at the block eps,
logits against the float embedding); the engine's own conventions differ only
in those two settings.  Tolerance: fp32 summation order, 1e-5 of the largest
reference value (measured: at most 4e-7).  The planted mistakes below (in the
oracle, on the CPU) show that the tolerance fails each plausible slip.
CPU only.
"""
import os

import numpy as np
import pytest

import float_cases as fc
from model import FModel

GOLD = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "float_golden.npz"))
RTOL = 1e-5


def _attn_errors(cls, name):
    """Largest |FModel - reference| / max|reference| over the per-position
    logits, the prefill logits and (rotate-half) the whole-sequence logits."""
    case = fc.attn_case(name)
    spec, blob = fc.attn_container(case, int(GOLD[name + "_seed"]))
    assert np.array_equal(fc.sha(blob), GOLD[name + "_sha256"]), "the seeded container changed"
    f = cls(blob, qk_eps=None, tied_head=True)
    inc = GOLD[name + "_inc"]
    scale = float(np.abs(inc).max())
    err = 0.0
    for t, tok in enumerate(GOLD[name + "_ids"]):
        lg = f.step(int(tok), t)
        err = max(err, float(np.abs(lg - inc[t]).max()) / scale)
    err = max(err, float(np.abs(lg - GOLD[name + "_prefill"]).max()) / scale)
    if name + "_fwd" in GOLD:
        err = max(err, float(np.abs(lg - GOLD[name + "_fwd"]).max()) / scale)
    return err


def _hybrid_errors(cls, seed):
    """max |FModel peak - reference peak| / max peak over the runs of
    residual_peaks_lfm2 (mmcf_hf.py:1253-1311: three runs of consecutive ids
    starting at 0, vocab/2 - seq/2 and vocab - seq; the largest |residual| after
    each layer), and whether some run's peak sits at position 2 or later, so
    that the conv tap on position pos-2 is part of what is compared."""
    spec, blob = fc.hybrid_container(seed)
    assert np.array_equal(fc.sha(blob), GOLD["hybrid%d_sha256" % seed]), "the seeded container changed"
    want = GOLD["hybrid%d_peaks" % seed]
    err, late = 0.0, False
    for i, s in enumerate(fc.HYBRID_RUNS):
        pk = np.zeros(spec.layers)
        at = np.zeros(spec.layers, int)
        for st in (0, max(0, spec.vocab // 2 - s // 2), max(0, spec.vocab - s)):
            f = cls(blob, qk_eps=None, tied_head=True)
            for t in range(s):
                tr = []
                f.step(st + t, t, trace=tr)
                for l in range(spec.layers):
                    m = float(np.abs(tr[l]).max())
                    if m > pk[l]:
                        pk[l], at[l] = m, t
        err = max(err, float(np.abs(pk - want[i]).max() / want[i].max()))
        late = late or bool((at >= 2).any())
    return err, late


@pytest.mark.parametrize("name", [c[0] for c in fc.ATTN_CASES])
def test_float_path_equals_reference_tools(name):
    assert _attn_errors(FModel, name) <= RTOL


@pytest.mark.parametrize("seed", fc.HYBRID_SEEDS)
def test_hybrid_float_path_equals_reference_peaks(seed):
    err, late = _hybrid_errors(FModel, seed)
    assert err <= RTOL
    assert late


class _RopeSign(FModel):
    def _rope(self, x, pos):
        c, s = self.rcos[pos], -self.rsin[pos]
        if self.rope_half:
            x1, x2 = x[..., :self.hd // 2], x[..., self.hd // 2:]
            return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
        out = np.empty_like(x)
        out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
        out[..., 1::2] = x[..., 1::2] * c + x[..., 0::2] * s
        return out


class _GqaTiled(FModel):
    def _per_q_head(self, kv):
        return np.tile(kv, (1, self.heads // self.kv_heads, 1))


class _NoQkNorm(FModel):
    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self.qk_norm = 0


class _ConvTapsReversed(FModel):
    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self.conv_w = [None if w is None else np.ascontiguousarray(w[:, ::-1]) for w in self.conv_w]


@pytest.mark.parametrize("cls,name", [(_RopeSign, "q8_gqa_qknorm"), (_RopeSign, "q4_mqa"),
                                      (_RopeSign, "q8_interleaved"), (_GqaTiled, "q8_gqa_qknorm"),
                                      (_GqaTiled, "t3_gqa_qknorm"), (_NoQkNorm, "q8_gqa_qknorm")])
def test_planted_mistake_fails_the_pin(cls, name):
    assert _attn_errors(cls, name) > 100 * RTOL


def test_planted_conv_mistake_fails_the_pin():
    assert _hybrid_errors(_ConvTapsReversed, fc.HYBRID_SEEDS[0])[0] > 100 * RTOL
