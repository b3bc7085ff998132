"""numpy restatement of the reference's logits candidate pass and host sampler.

TEST INFRASTRUCTURE ONLY: tests/ import this module as the checker; the
product never does.  Each function names the reference file:line it restates
(paths relative to the reference repository root).  Float work is done in
float32 with numpy scalars (IEEE, no contraction), exponentials as the
float64 exp rounded to float32.

Pins (tests/test_sampling_oracle.py): the generator against the C++
standard's known answer for std::mt19937; the chunk top-2 against a brute
force over all index pairs; the chunk sum against the closed form
sum(exp((v - max) / T)); the draws' empirical distribution against the kept
distribution; the penalties against their closed forms.
"""
import numpy as np

F = np.float32


def _expf(x):
    return F(np.exp(np.float64(F(x))))


class MT19937:
    """std::mt19937(seed): numpy's legacy RandomState seeds the same
    Mersenne Twister state (init_genrand) and returns its raw 32-bit outputs
    for the full uint32 range."""

    def __init__(self, seed):
        self._rs = np.random.RandomState(int(seed) & 0xFFFFFFFF)

    def next_u32(self):
        return int(self._rs.randint(0, 2 ** 32, dtype=np.uint64))

    def uniform01(self):
        """uniform_real_distribution<float>(0, 1) of libstdc++: one 32-bit draw
        u, generate_canonical = float(u) / 2^32, kept below 1."""
        r = F(F(self.next_u32()) / F(2.0 ** 32))
        if r >= F(1.0):
            r = np.nextafter(F(1.0), F(0.0))
        return F(r)


# ---------------------------------------------------------------------------
# The candidate pass (engine/src/shaders_attn.cpp:477-494, 574-594) and its
# host side (engine/src/gpu_matvec.cpp:152-229).

def chunks(logits_q16, temp):
    """Per 16-logit chunk: (v1, i1, v2, i2, lm, sum_q).  v1/i1 the first
    maximum, v2/i2 the first maximum of the rest (i2 = -1 when the chunk has
    one logit), lm the maximum, sum_q = floor(2048 * S + 1/2) with S the
    shader's streaming sum of exp((v - max) * invt)."""
    q = np.asarray(logits_q16, dtype=np.int64)
    n = q.size
    invt = F(F(1.0) / max(F(0.0001), F(temp)))
    out = np.zeros(((n + 15) // 16, 6), dtype=np.int64)
    for c in range(out.shape[0]):
        seg = q[16 * c: min(16 * c + 16, n)]
        i1 = int(np.argmax(seg))
        rest = np.delete(np.arange(seg.size), i1)
        if rest.size:
            j = rest[int(np.argmax(seg[rest]))]
            v2, i2 = int(seg[j]), 16 * c + int(j)
        else:
            v2, i2 = 0, -1
        lm = F(F(seg[0]) / F(256.0))
        ls = F(1.0)
        for k in range(1, seg.size):
            v = F(F(seg[k]) / F(256.0))
            if v > lm:
                ls = F(ls * _expf(F((lm - v) * invt)) + F(1.0))
                lm = v
            else:
                ls = F(ls + _expf(F((v - lm) * invt)))
        out[c] = (int(seg[i1]), 16 * c + i1, v2, i2, int(round(float(lm) * 256.0)),
                  int(np.floor(F(ls * F(2048.0)) + F(0.5))))
    return out


def assemble(ch, topk, temp, top_p):
    """The candidate result from chunk records: (values, tokens) of the kept
    candidates sorted by value descending (ties by token, a stable order the
    reference's std::sort need not keep), logsumexp, max logit, denominator,
    complete."""
    cand = []
    cmax = np.full(ch.shape[0], F(-1e30), dtype=np.float32)
    csum = np.zeros(ch.shape[0], dtype=np.float32)
    gmax = F(-1e30)
    for g, (v1, i1, v2, i2, lm, sq) in enumerate(ch):
        for v, i in ((v1, i1), (v2, i2)):
            if i < 0:
                continue
            fv = F(F(v) / F(256.0))
            cand.append((fv, int(i)))
            cmax[g] = max(cmax[g], fv)
            gmax = max(gmax, fv)
        mx = F(F(lm) / F(256.0))
        cmax[g] = max(cmax[g], mx)
        csum[g] = F(F(sq) / F(2048.0))
        gmax = max(gmax, mx)
    cand.sort(key=lambda t: (-float(t[0]), t[1]))
    T = max(F(0.0001), F(temp))
    denom = F(0.0)
    for g in range(ch.shape[0]):
        denom = F(denom + F(csum[g] * _expf(F(F(cmax[g] - gmax) / T))))
    cand = cand[:topk]
    cum = F(0.0)
    for v, _ in cand:
        cum = F(cum + F(_expf(F(F(v - gmax) / T)) / denom))
    lse = F(F(np.log(np.float64(denom))) + F(gmax / T))
    return ([c[0] for c in cand], [c[1] for c in cand], lse, gmax, denom,
            bool(F(cum + F(1e-6)) >= F(top_p)))


# ---------------------------------------------------------------------------
# The host sampler (engine/src/sampling.cpp).

def keep_distribution(logits, temp, top_p, top_k):
    """engine/src/sampling.cpp:66-117: [(p, token)] descending and the kept
    mass.  Ties in p keep token order (the reference's sort may not)."""
    x = np.asarray(logits, dtype=np.float32)
    if temp <= 0:
        return [(F(1.0), int(np.argmax(x)))], F(1.0)
    t = F(temp)
    mx = F(-1e30)
    for v in x:
        mx = max(mx, F(v / t))
    e = np.array([_expf(F(F(v / t) - mx)) for v in x], dtype=np.float32)
    total = F(0.0)
    for v in e:
        total = F(total + v)
    p = [(F(v / total), i) for i, v in enumerate(e)]
    p.sort(key=lambda a: (-float(a[0]), a[1]))
    if 0 < top_k < len(p):
        p = p[:top_k]
        m = F(0.0)
        for v, _ in p:
            m = F(m + v)
        if m > 0:
            p = [(F(v / m), i) for v, i in p]
    c, cut = F(0.0), 0
    while cut < len(p):
        c = F(c + p[cut][0])
        cut += 1
        if c >= F(top_p):
            break
    return p[:cut], c


def sample_token(logits, temp, top_p, top_k, gen):
    """engine/src/sampling.cpp:119-142: (token, log-probability within the
    kept set)."""
    d, c = keep_distribution(logits, temp, top_p, top_k)
    r = F(gen.uniform01() * c)
    acc, pick = F(0.0), d[-1]
    for x in d:
        acc = F(acc + x[0])
        if r <= acc:
            pick = x
            break
    lp = np.log(np.float64(F(pick[0] / c) if c > 0 else pick[0]))
    return pick[1], F(lp)


def argmax_report(logits):
    """engine/src/sampling.cpp:144-155."""
    x = np.asarray(logits, dtype=np.float32)
    mx = np.float64(x.max())
    total = float(np.sum(np.exp(x.astype(np.float64) - mx)))
    i = int(np.argmax(x))
    return i, F((np.float64(x[i]) - mx) - np.log(total))


def sample_candidates(values, tokens, strict, logsumexp, temp, top_p, top_k, gen):
    """engine/src/sampling.cpp:164-199."""
    if len(values) == 0:
        return 2
    v = np.asarray(values, dtype=np.float32)
    if temp <= 0:
        return int(tokens[int(np.argmax(v))])
    t = F(temp)
    if strict:
        c = [(_expf(F(F(a / t) - F(logsumexp))), int(k)) for a, k in zip(v, tokens)]
    else:
        mx = F(-1e30)
        for a in v:
            mx = max(mx, F(a / t))
        c = [(_expf(F(F(a / t) - mx)), int(k)) for a, k in zip(v, tokens)]
        total = F(0.0)
        for a, _ in c:
            total = F(total + a)
        c = [(F(a / total), k) for a, k in c]
    c.sort(key=lambda a: (-float(a[0]), a[1]))
    kmax = top_k if 0 < top_k < len(c) else len(c)
    if top_k > 0:
        m = F(0.0)
        for a, _ in c[:kmax]:
            m = F(m + a)
        if m > 0:
            c = [(F(a / m), k) if i < kmax else (a, k) for i, (a, k) in enumerate(c)]
    cdf, cut = F(0.0), 0
    while cut < kmax:
        cdf = F(cdf + c[cut][0])
        cut += 1
        if cdf >= F(top_p):
            break
    x = F(gen.uniform01() * cdf)
    acc = F(0.0)
    for i in range(cut):
        acc = F(acc + c[i][0])
        if x <= acc:
            return c[i][1]
    return c[cut - 1][1]


def apply_penalties(logits, recent, repetition=1.0, frequency=0.0, presence=0.0, no_repeat_ngram=0,
                    min_p=0.0):
    """engine/src/sampling.cpp:16-56, on a copy."""
    x = np.array(logits, dtype=np.float32)
    recent = list(recent)
    if not recent and min_p <= 0:
        return x
    counts = {}
    for t in recent:
        counts[t] = counts.get(t, 0) + 1
    if repetition != 1.0:
        for t in counts:
            if 0 <= t < x.size:
                x[t] = F(x[t] / F(repetition)) if x[t] > 0 else F(x[t] * F(repetition))
    if frequency != 0.0 or presence != 0.0:
        for t, k in counts.items():
            if 0 <= t < x.size:
                x[t] = F(x[t] - F(F(frequency) * F(k)))
                x[t] = F(x[t] - F(presence))
    g = no_repeat_ngram
    if g > 1 and len(recent) >= g:
        tail = recent[len(recent) - (g - 1):]
        for i in range(len(recent) - g):
            if recent[i:i + g - 1] == tail:
                b = recent[i + g - 1]
                if 0 <= b < x.size:
                    x[b] = F(-1e30)
    if min_p > 0:
        cutoff = F(F(x.max()) + F(np.log(np.float64(F(min_p)))))
        x[x < cutoff] = F(-1e30)
    return x
