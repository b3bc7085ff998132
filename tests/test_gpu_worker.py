"""The engine_mm3 command line and its --worker line protocol
(engine/src/worker.cpp:81-435, server/README.md "Worker protocol") over
the engine: the tokens it streams are those of the library's greedy decode,
the rolling prefix reuse and the MMKV1 prefix cache give the same tokens as
a cold run, and the control lines answer as the reference's do."""
import base64
import json
import os
import subprocess

import numpy as np
import pytest

from vgx import synth
from vgx.engine import Engine

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(__file__), "..", "vc4-gles2-inference_amd", "bin", "engine_mm3")


def _req(ids, max_new, temp=0.0, rid=""):
    p = base64.b64encode(" ".join(str(int(i)) for i in ids).encode()).decode()
    cols = [p, str(max_new), str(temp), "0.9", "0"] + [""] * 7 + [rid]
    return "\t".join(cols)


def _events(out):
    return [json.loads(line) for line in out.splitlines() if line.startswith("{")]


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    spec = synth.tiny_spec(seq=64)
    blob = synth.container(spec, "q8", seed=12)
    path = tmp_path_factory.mktemp("w") / "tiny.mmcf"
    path.write_bytes(blob)
    return str(path), blob, spec


def _tokens(evs):
    return [int(t) for e in evs if e["event"] == "token" for t in e["text"].split()]


def _greedy(blob, prompt, n):
    """The library's greedy run, cut at the first end id (1 or 2) as the worker
    cuts it when the container states no special ids."""
    out, _, _ = Engine(blob).generate(prompt, n)
    res = []
    for t in out:
        if t in (1, 2):
            break
        res.append(int(t))
    return res


def test_worker_protocol(gpu, model_file):
    path, blob, spec = model_file
    p1 = synth.prompt(9, spec.vocab, seed=3)
    p2 = np.concatenate([p1, synth.prompt(4, spec.vocab, seed=4)])
    lines = ['{"op":"stats"}', _req(p1, 12, rid="r1"), _req(p2, 10, rid="r2"), _req(p1, 5, temp=0.7),
             "not base64 ids\t4\t0\t0.9\t0", '{"op":"cancel","id":"x"}', '{"op":"nope"}',
             '{"op":"load","model":"%s"}' % path, _req(p2, 10, rid="r3")]
    r = subprocess.run([BIN, "--model", path, "--worker"], input="\n".join(lines) + "\n", capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    evs = _events(r.stdout)
    assert evs[0]["event"] == "ready" and evs[0]["prefix_cache_tokens"] == 0
    assert evs[1]["event"] == "stats" and evs[1]["seq"] == 64 and evs[1]["kv_pack"] == 16
    by = {}
    for e in evs:
        by.setdefault(e.get("id"), []).append(e)
    r1, r2, r3 = by["r1"], by["r2"], by["r3"]
    assert r1[0]["event"] == "start" and r1[0]["cached_tokens"] == 0 and r1[0]["prefill_tokens"] == 9
    assert _tokens(r1) == _greedy(blob, p1, 12)
    assert r1[-1]["event"] == "done" and r1[-1]["completion_tokens"] == len(_tokens(r1))
    # the second request extends the first: its prompt prefix is not prefilled again
    assert r2[0]["cached_tokens"] == 9 and r2[0]["prefill_tokens"] == 4
    assert _tokens(r2) == _greedy(blob, p2, 10)
    # after a load the rolling cache is gone, and the answer is a cold run's
    assert r3[0]["cached_tokens"] == 0
    assert _tokens(r3) == _tokens(r2)
    errs = [e["message"] for e in evs if e["event"] == "error"]
    assert any("token ids" in m for m in errs)
    # a sampled request (temperature 0.7, seed 0) is answered, not refused
    assert not any("temperature" in m for m in errs)
    assert sum(1 for e in evs if e["event"] == "done") == 4
    assert any("unknown op" in m for m in errs)
    assert any(e["event"] == "cancelled" and e.get("idle") for e in evs)
    assert any(e["event"] == "loaded" and e["seq"] == 64 for e in evs)


def test_cli_prefix_cache(gpu, model_file, tmp_path):
    path, blob, spec = model_file
    prompt = synth.prompt(12, spec.vocab, seed=9)
    ids = ",".join(str(int(t)) for t in prompt)
    cold = subprocess.run([BIN, "--model", path, "--prompt-ids", ids, "--gen", "8"], capture_output=True,
                          text=True, timeout=120)
    assert cold.returncode == 0, cold.stderr
    want, _, _ = Engine(blob).generate(prompt, 8)
    assert [int(t) for t in cold.stdout.split()] == list(want)
    cache = str(tmp_path / "c.mmkv")
    saved = subprocess.run([BIN, "--model", path, "--prompt-ids", ids, "--gen", "8", "--save-prefix", cache],
                           capture_output=True, text=True, timeout=120)
    assert saved.returncode == 0, saved.stderr and os.path.exists(cache) and os.path.exists(cache + ".json")
    assert saved.stdout == cold.stdout
    # the saved prefix is the prompt but its last token
    assert json.load(open(cache + ".json"))["n_tokens"] == 11
    warm = subprocess.run([BIN, "--model", path, "--prompt-ids", ids, "--gen", "8", "--prefix-cache", cache],
                          capture_output=True, text=True, timeout=120)
    assert warm.returncode == 0, warm.stderr
    assert warm.stdout == cold.stdout and "11 cached" in warm.stderr
    # a worker started on the cache reuses it for a prompt that extends it
    r = subprocess.run([BIN, "--model", path, "--worker", "--prefix-cache", cache], input=_req(prompt, 8) + "\n",
                       capture_output=True, text=True, timeout=120)
    evs = _events(r.stdout)
    assert evs[0]["prefix_cache_tokens"] == 11
    start = [e for e in evs if e["event"] == "start"][0]
    assert start["cached_tokens"] == 11 and start["prefill_tokens"] == 1
    assert _tokens(evs) == _greedy(blob, prompt, 8)
