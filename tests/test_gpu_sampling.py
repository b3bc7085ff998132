"""The logits candidate pass on the GPU and the sampled worker requests.

vgx_logits_chunks against the oracle (oracle/sampling.py, pinned in
tests/test_sampling_oracle.py) bit for bit: the top-2 scan is integer work,
and the chunk sums use the same IEEE float operations as the oracle.  The
engine's candidate result (Session::step_candidates) against the oracle's
assembly of the same logits; the worker's sampled tokens against a replay of
the worker loop through the library's step and sampler calls."""
import base64
import json
import os
import subprocess

import numpy as np
import pytest
import torch

import sampling as S  # oracle/sampling.py
from vgx import mmcf, synth
from vgx.engine import Engine, Sampler, apply_penalties, argmax_report

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(__file__), "..", "vc4-gles2-inference_amd", "bin", "engine_mm3")


@pytest.mark.parametrize("n", [1, 17, 1000, 6401])
def test_logits_chunks_kernel_matches_oracle(gpu, n):
    rng = np.random.default_rng(n)
    q = np.clip(np.round(rng.normal(0, 600, n)), -32768, 32767).astype(np.int16)
    q[:n // 3] = (q[:n // 3] // 256) * 256  # runs of equal values: the first-index rules
    q[rng.integers(0, n)] = 32767
    q[rng.integers(0, n)] = -32768
    dev = torch.from_numpy(q).to("cuda")
    for temp in (0.0, 0.7, 1.0, 2.5):
        print("chunks n=%d temp=%g" % (n, temp), flush=True)
        got = gpu.logits_chunks(dev, temp).cpu().numpy().astype(np.int64)
        assert np.array_equal(got, S.chunks(q, temp))


def _spec(vocab):
    # two LM-head tiles (1536 + the rest) for a vocabulary above 1536
    return mmcf.ModelSpec(dim=64, hidden=96, layers=2, heads=4, kv_heads=2, vocab=vocab, seq=64,
                          theta=10000.0, rope_half=True, qk_norm=True)


def _check_candidates(res, q, temp, topk, top_p):
    want_v, want_t, lse, gmax, denom, complete = S.assemble(S.chunks(q, temp), topk, temp, top_p)
    v, t = res["values"], res["tokens"]
    # the same values in the same (descending) order; each token carries its value
    assert np.array_equal(np.round(v * 256).astype(int), np.round(np.array(want_v) * 256).astype(int))
    assert all(int(q[k]) == int(round(x * 256)) for x, k in zip(v, t))
    assert len(set(int(k) for k in t)) == len(t)
    # ties may be cut anywhere at the last kept value, never above it
    b = want_v[-1]
    assert {int(k) for x, k in zip(v, t) if x > b} == {int(k) for x, k in zip(want_v, want_t) if x > b}
    assert res["max_logit"] == gmax
    assert abs(res["denom"] - denom) <= 1e-6 * denom
    assert abs(res["logsumexp"] - lse) <= 1e-5 * max(1.0, abs(lse))
    assert res["complete"] == complete
    if not complete:
        assert np.array_equal(res["full"], q.astype(np.float32) / 256)


@pytest.mark.parametrize("vocab,scheme", [(80, "q8"), (3000, "q8"), (3000, "q4")])
def test_engine_step_candidates_match_oracle(gpu, vocab, scheme):
    spec = _spec(vocab)
    blob = synth.container(spec, scheme, seed=21)
    prompt = synth.prompt(6, vocab, seed=2)
    for temp, topk, top_p in ((1.0, 8, 0.5), (0.6, 40, 0.9), (1.5, 3, 1.0), (0.0, 10, 0.9)):
        print("candidates vocab=%d %s temp=%g topk=%d top_p=%g" % (vocab, scheme, temp, topk, top_p), flush=True)
        e = Engine(blob)
        e.prefill(prompt[:-1], 0, logits=False)
        res = e.step_candidates(int(prompt[-1]), len(prompt) - 1, topk, temp, top_p)
        q, _ = e.step(int(prompt[-1]), len(prompt) - 1)  # the same position again: the same logits
        _check_candidates(res, q, temp, topk, top_p)
        e.close()


def test_step_candidates_refusals(gpu):
    e = Engine(synth.container(synth.tiny_spec(), "q8", seed=1))
    for bad in (dict(topk=0), dict(token=999), dict(pos=64)):
        kw = dict(token=3, pos=0, topk=4, temp=1.0, top_p=0.9)
        kw.update(bad)
        with pytest.raises(Exception):
            e.step_candidates(**kw)
    e.close()


# ---- the worker's sampled requests

def _req(ids, max_new, temp, top_p, seed, top_k="", pen=("", "", "", "", ""), logprobs="", rid=""):
    p = base64.b64encode(" ".join(str(int(i)) for i in ids).encode()).decode()
    cols = [p, str(max_new), str(temp), str(top_p), str(seed)] + list(pen) + ["", str(top_k), rid, str(logprobs)]
    return "\t".join(cols)


def _replay(blob, prompt, n, temp, top_p, seed, top_k=0, cand=False, pen=None, logprobs=False):
    """The worker loop (engine/src/worker.cpp:300-409) through the library's
    calls: the prompt but its last token prefilled, then per step the logits
    (penalised, sampled) or the candidates."""
    e, s = Engine(blob), Sampler(seed)
    P = len(prompt)
    if P > 1:
        e.prefill(prompt[:-1], 0, logits=False)
    mode = {"cand": cand and top_k > 0 and temp > 0 and not pen and not logprobs}

    def step(tok, pos):
        if mode["cand"]:
            r = e.step_candidates(tok, pos, top_k, temp, top_p)
            if r["complete"]:
                return r
            mode["cand"] = False
            return r["full"]
        q, _ = e.step(tok, pos)
        return q.astype(np.float32) / 256

    cur = step(int(prompt[-1]), P - 1)
    out, lps, recent, pos = [], [], [], P
    for i in range(n):
        lp = None
        if isinstance(cur, dict):
            t = s.sample_candidates(cur["values"], cur["tokens"], True, cur["logsumexp"], temp, top_p, top_k)
        else:
            x = apply_penalties(cur, recent, **(pen or {}))
            if logprobs:
                t, lp = argmax_report(x) if temp <= 0 else s.sample_logits(x, temp, top_p, top_k)
            elif temp <= 0:
                t, _ = argmax_report(x)
            else:
                t, _ = s.sample_logits(x, temp, top_p, top_k)
        if t in (1, 2):
            break
        out.append(int(t))
        lps.append(lp)
        recent.append(int(t))
        if i + 1 < n:
            cur = step(int(t), pos)
            pos += 1
    e.close()
    s.close()
    return out, lps


def _events(out):
    return [json.loads(line) for line in out.splitlines() if line.startswith("{")]


def _tokens(evs):
    return [int(t) for e in evs if e["event"] == "token" for t in e["text"].split()]


def test_worker_sampled_requests(gpu, tmp_path):
    spec = _spec(3000)
    blob = synth.container(spec, "q8", seed=31, head_dedup=False)
    path = str(tmp_path / "m.mmcf")
    open(path, "wb").write(blob)
    p = synth.prompt(7, spec.vocab, seed=5)
    cases = [
        ("full", dict(temp=0.9, top_p=0.9, seed=123), {}),
        ("topk", dict(temp=1.2, top_p=0.8, seed=7, top_k=20), {}),
        ("cand", dict(temp=0.8, top_p=0.9, seed=99, top_k=30), dict(cand=True)),
        ("cand_fallback", dict(temp=1.0, top_p=1.0, seed=5, top_k=4), dict(cand=True)),
        ("pen", dict(temp=0.7, top_p=0.95, seed=3), dict(pen=dict(repetition=1.3, frequency=0.2, presence=0.1,
                                                                  no_repeat_ngram=2, min_p=0.01))),
        ("greedy_pen", dict(temp=0.0, top_p=0.9, seed=0), dict(pen=dict(repetition=1.5))),
        ("lp", dict(temp=1.0, top_p=0.9, seed=11), dict(logprobs=True)),
    ]
    for name, kw, extra in cases:
        print("worker case", name, flush=True)
        pen = extra.get("pen")
        pen_cols = (("%g" % pen.get("repetition", 1.0), "%g" % pen.get("frequency", 0.0),
                     "%g" % pen.get("presence", 0.0), "%d" % pen.get("no_repeat_ngram", 0),
                     "%g" % pen.get("min_p", 0.0)) if pen else ("", "", "", "", ""))
        line = _req(p, 12, kw["temp"], kw["top_p"], kw["seed"], top_k=kw.get("top_k", ""), pen=pen_cols,
                    logprobs=1 if extra.get("logprobs") else "", rid=name)
        args = [BIN, "--model", path, "--worker"] + (["--top-k-candidates"] if extra.get("cand") else [])
        r = subprocess.run(args, input=line + "\n", capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        evs = _events(r.stdout)
        assert not [e for e in evs if e["event"] == "error"], evs
        want, lps = _replay(blob, p, 12, kw["temp"], kw["top_p"], kw["seed"], top_k=kw.get("top_k", 0) or 0,
                            cand=bool(extra.get("cand")), pen=pen, logprobs=bool(extra.get("logprobs")))
        assert _tokens(evs) == want, name
        done = [e for e in evs if e["event"] == "done"][0]
        if extra.get("logprobs"):
            rows = done["logprobs"]
            assert [row["id"] for row in rows] == want
            assert all(abs(row["lp"] - lp) < 1e-6 for row, lp in zip(rows, lps))
            assert all(row["lp"] <= 0 for row in rows)
        else:
            assert "logprobs" not in done
    # the same seed draws the same tokens; another seed (almost surely) others
    a = _replay(blob, p, 12, 1.0, 1.0, 1)[0]
    assert a == _replay(blob, p, 12, 1.0, 1.0, 1)[0]
    assert a != _replay(blob, p, 12, 1.0, 1.0, 2)[0]
