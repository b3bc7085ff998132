"""The candidate pass and the host sampler: the numpy oracle pinned by known
answers, brute force and closed forms, then the library's host sampler
(pure host code in libvgx_engine, callable without a GPU) checked against it.
The reference ships no sampling tests or vectors (engine/tests holds none), so
the pins come from the C++ standard and the mathematics."""
import numpy as np
import pytest

import sampling as S  # oracle/sampling.py

F = np.float32


def test_mt19937_known_answer():
    # [rand.predef]: the 10000th invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995
    g = S.MT19937(5489)
    for _ in range(9999):
        g.next_u32()
    assert g.next_u32() == 4123659995


def test_uniform01_is_canonical():
    # generate_canonical<float, 24> of one 32-bit draw: float(u) / 2^32, in [0, 1)
    g1, g2 = S.MT19937(7), S.MT19937(7)
    for _ in range(2000):
        u = g2.next_u32()
        r = g1.uniform01()
        assert r == min(F(F(u) / F(2.0 ** 32)), np.nextafter(F(1), F(0)))
        assert F(0) <= r < F(1)


def _brute_top2(seg):
    """All index pairs: the first maximum, then the first maximum of the rest."""
    best = None
    for i in range(len(seg)):
        if best is None or seg[i] > seg[best]:
            best = i
    second = None
    for j in range(len(seg)):
        if j != best and (second is None or seg[j] > seg[second]):
            second = j
    return best, second


@pytest.mark.parametrize("n", [1, 15, 16, 17, 100, 257])
def test_chunks_top2_and_sum_pinned(n):
    rng = np.random.default_rng(n)
    # a narrow range forces ties (the first-index rules), the rails included
    q = rng.integers(-4, 5, n).astype(np.int16) * 256
    q[rng.integers(0, n)] = 32767
    if n > 3:
        q[rng.integers(0, n)] = -32768
    for temp in (0.0, 0.7, 1.0, 2.5):
        ch = S.chunks(q, temp)
        assert ch.shape == ((n + 15) // 16, 6)
        T = max(1e-4, temp)
        for c in range(ch.shape[0]):
            seg = q[16 * c: 16 * c + 16].astype(np.int64)
            b, s2 = _brute_top2(list(seg))
            assert (ch[c, 0], ch[c, 1]) == (seg[b], 16 * c + b)
            if s2 is None:
                assert ch[c, 3] == -1
            else:
                assert (ch[c, 2], ch[c, 3]) == (seg[s2], 16 * c + s2)
            assert ch[c, 4] == seg.max()
            closed = np.sum(np.exp((seg - seg.max()) / 256.0 / T))
            assert abs(ch[c, 5] - np.floor(closed * 2048 + 0.5)) <= 1


def test_assemble_pinned_by_closed_forms():
    rng = np.random.default_rng(3)
    q = np.clip(np.round(rng.normal(0, 3, 1000) * 256), -32768, 32767).astype(np.int16)
    temp, topk = 0.8, 40
    vals, toks, lse, gmax, denom, complete = S.assemble(S.chunks(q, temp), topk, temp, 0.9)
    # the kept candidates: the topk largest of the chunks' top-2 values
    ch = S.chunks(q, temp)
    pool = sorted(list(ch[:, 0]) + [v for v, i in zip(ch[:, 2], ch[:, 3]) if i >= 0], reverse=True)
    assert [int(round(v * 256)) for v in vals] == pool[:topk]
    assert all(q[t] == int(round(v * 256)) for v, t in zip(vals, toks))
    assert gmax == q.max() / 256.0
    # the denominator: sum over all logits of exp((v - max) / T), up to the 1/2048 grid
    exact = np.sum(np.exp((q.astype(np.float64) - q.max()) / 256.0 / temp))
    assert abs(denom - exact) <= ch.shape[0] * 0.5 / 2048 + 1e-4 * exact
    assert abs(lse - (np.log(exact) + q.max() / 256.0 / temp)) < 1e-3
    mass = sum(np.exp((v - gmax) / temp) for v in vals) / exact
    assert complete == (mass + 1e-6 >= 0.9) or abs(mass - 0.9) < 1e-3


def _freq_check(draw, probs, n):
    """Empirical frequencies of n draws against probs (dict token -> p):
    nothing outside, each within 5 sigma."""
    counts = {}
    for _ in range(n):
        t = draw()
        counts[t] = counts.get(t, 0) + 1
    assert set(counts) <= set(probs)
    for t, p in probs.items():
        f = counts.get(t, 0) / n
        assert abs(f - p) <= 5 * np.sqrt(p * (1 - p) / n) + 1e-9, (t, f, p)


def test_sample_token_distribution_pinned():
    logits = np.array([2.0, 1.0, 0.5, 3.0, -1.0, 2.5], np.float32)
    temp, top_p, top_k = 0.9, 0.8, 4
    # closed form: softmax at T, top 4, renormalise, shortest prefix reaching 0.8
    e = np.exp(logits.astype(np.float64) / temp)
    p = e / e.sum()
    order = np.argsort(-p, kind="stable")[:top_k]
    pk = p[order] / p[order].sum()
    cut = int(np.searchsorted(np.cumsum(pk), top_p) + 1)
    kept = {int(order[i]): pk[i] / pk[:cut].sum() for i in range(cut)}
    d, c = S.keep_distribution(logits, temp, top_p, top_k)
    assert [t for _, t in d] == [int(o) for o in order[:cut]]
    assert abs(c - pk[:cut].sum()) < 1e-6
    g = S.MT19937(11)
    _freq_check(lambda: S.sample_token(logits, temp, top_p, top_k, g)[0], kept, 4000)
    # temperature 0 is the first maximum
    assert S.sample_token(np.array([1, 5, 5], np.float32), 0.0, 0.9, 0, g)[0] == 1


def test_sample_candidates_distribution_pinned():
    values = np.array([1.5, 1.0, 0.25, 2.0], np.float32)
    tokens = [10, 20, 30, 40]
    temp = 0.7
    lse = float(np.log(np.sum(np.exp(values.astype(np.float64) / temp))))
    p = np.exp(values / temp - lse)
    kept = {t: pi / p.sum() for t, pi in zip(tokens, p)}
    g = S.MT19937(5)
    _freq_check(lambda: S.sample_candidates(values, tokens, True, lse, temp, 1.0, 4, g), kept, 4000)
    assert S.sample_candidates([], [], True, 0.0, temp, 1.0, 4, g) == 2


def test_penalties_closed_forms():
    x = np.array([2.0, -1.0, 0.5, 3.0, 1.0], np.float32)
    y = S.apply_penalties(x, [0, 1, 1], repetition=2.0)
    assert y[0] == 1.0 and y[1] == -2.0 and y[2] == 0.5
    y = S.apply_penalties(x, [3, 3, 2], frequency=0.5, presence=0.25)
    assert y[3] == F(3.0 - 1.0 - 0.25) and y[2] == F(0.5 - 0.5 - 0.25) and y[0] == 2.0
    # bigram ban: "4 2" occurred, the last token is 4: 2 is banned
    y = S.apply_penalties(x, [4, 2, 1, 4], no_repeat_ngram=2)
    assert y[2] == F(-1e30) and y[1] == -1.0
    y = S.apply_penalties(x, [], min_p=0.2)
    keep = x >= x.max() + np.log(np.float32(0.2))
    assert np.all(y[keep] == x[keep]) and np.all(y[~keep] == F(-1e30))


# ---- the library's host sampler against the oracle

def _engine():
    from vgx import engine as E
    E.load()
    return E


@pytest.mark.parametrize("seed", [0, 1, 12345, 2 ** 32 - 1])
def test_library_sampler_matches_oracle(seed):
    E = _engine()
    rng = np.random.default_rng(seed % 1000)
    for temp, top_p, top_k in ((1.0, 0.9, 0), (0.7, 0.95, 40), (1.3, 0.5, 5), (0.0, 0.9, 0), (2.0, 1.0, 1)):
        logits = rng.normal(0, 2, 300).astype(np.float32)
        s = E.Sampler(seed)
        g = S.MT19937(seed)
        for _ in range(20):
            t, lp = s.sample_logits(logits, temp, top_p, top_k)
            to, lpo = S.sample_token(logits, temp, top_p, top_k, g)
            assert t == to
            assert abs(lp - lpo) < 1e-5
        s.close()


def test_library_candidate_sampler_and_reports_match_oracle():
    E = _engine()
    rng = np.random.default_rng(9)
    for strict in (True, False):
        values = np.sort(rng.normal(0, 1, 30).astype(np.float32))[::-1].copy()
        tokens = rng.permutation(1000)[:30].astype(np.int32)
        lse = float(np.log(np.sum(np.exp(values.astype(np.float64) / 0.8))) + 0.1)
        s, g = E.Sampler(77), S.MT19937(77)
        for top_k in (0, 5, 30):
            for _ in range(10):
                a = s.sample_candidates(values, tokens, strict, lse, 0.8, 0.9, top_k)
                b = S.sample_candidates(values, tokens, strict, lse, 0.8, 0.9, top_k, g)
                assert a == b
    x = rng.normal(0, 1, 500).astype(np.float32)
    t, lp = E.argmax_report(x)
    to, lpo = S.argmax_report(x)
    assert t == to and abs(lp - lpo) < 1e-6
    for kw in (dict(repetition=1.3), dict(frequency=0.4, presence=-0.2), dict(no_repeat_ngram=3),
               dict(min_p=0.05), dict(repetition=0.7, min_p=0.3)):
        recent = [int(v) for v in rng.integers(0, 500, 40)] + [7, 8, 9, 7, 8]
        assert np.array_equal(E.apply_penalties(x, recent, **kw), S.apply_penalties(x, recent, **kw))
