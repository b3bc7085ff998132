#!/usr/bin/env python3
"""Benchmark: q8 dequant-GEMV over the MiniMind3 shapes with cold weights.

One step = one pass of the q8 dequant-GEMV (fp32 activations in, fp32 out, the
per-row q8 container format of MiniMind3-64M) over the five MiniMind3 shapes
768x768, 384x768 (KV projection), 2432x768, 768x2432 and 6400x768 (LM head),
each streamed over enough distinct weight copies (>= --cold-mb MiB per shape)
that no weight is cache-resident when it is read: one launch per shape, all
copies of a shape sharing the activation vector.  `value` is the step's
algorithmic bytes (weight body + f32 row plane + f32 x + f32 y per GEMV, the
byte model of the hot-path survey) over its wall time.  Warm (cache-resident,
1000 reps of one matrix) single-launch figures are reported beside it, and the
CPU restatement (oracle/) of the same GEMV is timed on a bounded sample of the
same shapes on this host's cores.
"""
import argparse
import json
import re
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "vc4-gles2-inference_amd")
sys.path.insert(0, PKG)

SHAPES = [(768, 768), (384, 768), (2432, 768), (768, 2432), (6400, 768)]
HBM_PEAK_GBS = 8000.0
METRIC = "dequant-GEMV GB/s (% HBM peak) + decode tokens/s, MiniMind3-64M q8, 1 GPU"


def algo_bytes(rows, cols, kind="q8"):
    """Weight body + scale planes + f32 x + f32 y for one GEMV: q8 per-row
    (body + f32 row plane), q4 g32 (nibbles + int16 scale and min per group)."""
    if kind == "q4":
        return rows * cols // 2 + rows * (cols // 32) * 4 + cols * 4 + rows * 4
    return rows * cols + rows * 4 + cols * 4 + rows * 4


def weight_bytes(rows, cols, kind):
    return rows * cols // 2 + rows * (cols // 32) * 4 if kind == "q4" else rows * cols + rows * 4


def make_matrix(rng, rows, cols, kind):
    """N(0, 0.02) fp32 weights packed by the container packer (vgx.mmcf); for
    t3, the synthetic per-row ternary weights of the t3 models (vgx.synth)."""
    import numpy as np
    from vgx import mmcf
    if kind == "t3":
        from vgx import synth
        packed, unit, plane = mmcf.t3mat(synth.ternary_matrix(rng, rows, cols))
        return mmcf.Matrix("t3", rows, cols, np.frombuffer(packed, np.uint8), unit, plane=plane)
    if kind != "q4" and kind != "q8":
        raise ValueError("make_matrix: kind must be q8, q4 or t3")
    w = rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(0.02)
    if kind == "q4":
        packed, s16, m16, ps, _ = mmcf.q4mat(w)
        return mmcf.Matrix("q4", rows, cols, packed.ravel(), ps, s16=s16.ravel(), m16=m16.ravel())
    q, unit, plane = mmcf.q8_per_row(w)
    return mmcf.Matrix("q8", rows, cols, (q.view(np.uint8) ^ 0x80).ravel(), unit, True, plane)


def pmc_summary(fetch_csv, write_csv, bench_log):
    """HBM traffic of the cold sweep's launches from two rocprofv3 --pmc runs
    of `bench.py --only gemv --steps 3 --warmup 1 --copy-mb 1024` (counter
    FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by what the
    same counter reads for the 1 GiB elementwise copy of that run.  The first
    four steps (warm-up + 3 timed) are averaged per shape.  `bench_log` is the
    JSON line of a full bench run (for the algorithmic bytes)."""
    import csv

    def load(p):
        with open(p) as f:
            rows = list(csv.DictReader(f))
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        return rows

    def scale(rows, known):
        # the copy calibration's dispatches: the last three elementwise
        # kernels of the run (--copy-mb runs after the library references,
        # whose cache-resident copy must not enter the scale)
        v = [float(r["Counter_Value"]) for r in rows if "AUnaryFunctor" in r["Kernel_Name"]][-3:]
        return known / (sum(v) / len(v) * 1024.0), v

    fe, wr = load(fetch_csv), load(write_csv)
    with open(bench_log) as f:
        bench = [json.loads(line) for line in f if line.startswith("{")][-1]
    kf, cf = scale(fe, 1 << 30)
    kw, cw = scale(wr, 1 << 30)
    names = ["%dx%d" % s for s in SHAPES]
    algo = {"q8": {x["shape"]: x["bytes_per_launch"] for x in bench["gemv"]},
            "q4": {x["shape"]: x["bytes_per_launch"] for x in bench["q4"]["gemv"]}}
    per = {}
    for kind, kid in (("q8", 1), ("q4", 2)):
        def cold(rows):
            # the f32-epilogue launches with 4 rows per lane: gemv_kernel<kind, lpr, 4, 1, 1[, single]>
            pat = re.compile(r"gemv_kernel<%d, \d+, 4, 1, 1(, (true|false))?>" % kid)
            return [r for r in rows if pat.search(r["Kernel_Name"])]
        cfk, cwk = cold(fe), cold(wr)
        per[kind] = {}
        for i, s in enumerate(names):
            fb = sum(float(cfk[k * 5 + i]["Counter_Value"]) for k in range(4)) / 4 * 1024.0 * kf
            wb = sum(float(cwk[k * 5 + i]["Counter_Value"]) for k in range(4)) / 4 * 1024.0 * kw
            per[kind][s] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "algorithmic_bytes": algo[kind][s],
                            "traffic_over_algorithmic": round((fb + wb) / algo[kind][s], 4)}
    return {"source": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE: bench.py --only gemv --steps 3 --warmup 1 "
                      "--warm-reps 5 --copy-mb 1024",
            "calibration": {"kernel": "at::native elementwise mul, float32, 1 GiB read + 1 GiB written",
                            "fetch_KiB": cf, "write_KiB": cw, "fetch_bytes_per_counted_byte": kf,
                            "write_bytes_per_counted_byte": kw},
            "per_launch": per,
            "bytes_per_step": sum(v["fetch_bytes"] + v["write_bytes"] for v in per["q8"].values()),
            "algorithmic_bytes_per_step": sum(algo["q8"].values())}


def traffic_summary():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE runs of this script, scaled by the
    same counters on a copy of known size), or None before one exists."""
    p = os.path.join(ROOT, "profiles", "gemv_q8_cold_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)


def cpu_baseline(seconds):
    """The oracle's q8 GEMV (exact int accumulation, OpenMP over rows) on the
    same five shapes, one matrix each, repeated for about `seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as o
    from vgx import mmcf

    rng = np.random.default_rng(1)
    mats = []
    for rows, cols in SHAPES:
        w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
        q, unit, plane = mmcf.q8_per_row(w)
        body = (q.view(np.uint8) ^ 0x80).ravel()
        mats.append((rows, cols, body, o.row_scales(rows, unit, plane)))
    xs = {c: rng.standard_normal(c).astype(np.float32) for _, c in SHAPES}

    def run(secs):
        nbytes, passes = 0, 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < secs:
            for rows, cols, body, wsr in mats:
                xq = o.quantize_act(xs[cols])
                o.store_f32(o.rowval_q8(body, 1, rows, cols, wsr, xq))
                nbytes += algo_bytes(rows, cols)
            passes += 1
        dt = time.perf_counter() - t0
        return nbytes / dt / 1e9, passes, dt

    cores = o.threads()
    gbps, passes, dt = run(seconds)
    # the same on one core (the survey asks for both)
    o.set_threads(1)
    gbps1, passes1, dt1 = run(max(1.0, seconds / 3))
    o.set_threads(cores)
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "one_core_value": round(gbps1, 3),
            "sample": "%d passes over the 5 MiniMind3 q8 GEMV shapes (one matrix each, warm host caches), "
                      "%.1f s, oracle exact-integer q8 GEMV with OpenMP on %d threads; one_core_value: %d passes, "
                      "%.1f s on 1 thread" % (passes, dt, cores, passes1, dt1)}


GRAPHS = True  # decode steps replayed as one HIP graph (--no-graphs: individual launches)


def decode_step_bytes(blob, kv_bits, n_prompt, n_gen, nseq=1):
    """Algorithmic HBM bytes of one timed decode step: every tensor a step
    reads once whatever the batch (each layer's matrices, their scale planes
    and norm weights, the LM head -- rendered from the embedding when the
    container has no head tiles), plus per sequence its embedding row and, in
    every attention layer, the K and V rows it reads and the row it writes.
    The timed steps attend over n_prompt + 1 .. n_prompt + n_gen - 1 rows, so
    the KV term is taken at their mean, n_prompt + n_gen / 2."""
    from vgx import mmcf
    c = mmcf.Container(blob)
    s = c.spec
    weights = sum(len(r.body) for r in c.records if r.kind not in (mmcf.T_EMB, mmcf.T_EMB_SCALE))
    if not any(r.kind == mmcf.T_LOGITS for r in c.records):
        weights += s.vocab * s.dim + s.vocab * 4
    attn_layers = sum(1 for t in (s.layer_types or ["attn"] * s.layers) if t == "attn")
    kv_row = 2 * s.kv_heads * s.head_dim * kv_bits // 8
    per_seq = s.dim + 4 + attn_layers * kv_row * (n_prompt + n_gen / 2.0 + 1)
    return int(weights + nseq * per_seq)


def decode_roofline(step_bytes, ms_step):
    gbps = step_bytes / (ms_step * 1e-3) / 1e9
    return {"bytes_per_step": step_bytes, "achieved_GBps": round(gbps, 1), "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBS, 4)}


def model_decode(name, spec, scheme, kv_bits, n_prompt, n_gen, runs):
    """A seeded synthetic model through the engine: n_prompt prompt tokens
    (batched prefill) then n_gen greedy tokens; decode tokens/s over the
    n_gen - 1 steps after the prompt, median of `runs` after a warm-up run."""
    import numpy as np
    from vgx import synth
    from vgx.engine import Engine

    blob = synth.container(spec, scheme, seed=0, q8_row=True)
    prompt = synth.prompt(n_prompt, spec.vocab, seed=0)
    eng = Engine(blob, kv_bits=kv_bits)
    eng.set_graphs(GRAPHS)
    eng.generate(prompt, n_gen)
    pf, dc, toks = [], [], None
    for _ in range(runs):
        toks, p, d = eng.generate(prompt, n_gen)
        pf.append(p)
        dc.append(d)
    eng.close()
    ms_tok = float(np.median(dc)) / (n_gen - 1)
    return blob, prompt, toks, {
        "model": name, "prompt": n_prompt, "gen": n_gen, "seq": spec.seq, "kv": "q%d" % kv_bits,
        "tokens_per_s": round(1000.0 / ms_tok, 1), "ms_per_token": round(ms_tok, 4),
        "prefill_ms": round(float(np.median(pf)), 3), "runs": runs, "graphs": GRAPHS,
        "hbm": decode_roofline(decode_step_bytes(blob, kv_bits, n_prompt, n_gen), ms_tok)}


def decode_bench(runs):
    """C1: MiniMind3-64M q8 (per-row scales), KV q16, SEQ 256, 32 prompt
    tokens then 64 greedy tokens."""
    from vgx import synth
    return model_decode("MiniMind3-64M-shaped, q8 per-row, seed 0", synth.minimind3_spec(seq=256), "q8", 16,
                        32, 64, runs)


def hybrid_decode_bench(runs):
    """C4: LFM2.5-230M-shaped hybrid q8 (8 conv + 6 attention layers), KV q16,
    SEQ 256, 64 prompt tokens then 128 greedy tokens."""
    from vgx import synth
    return model_decode("LFM2.5-230M-shaped hybrid, q8 per-row, seed 0", synth.lfm2_spec(seq=256), "q8", 16,
                        64, 128, runs)


def ternary_decode_bench(runs):
    """C5 at batch 1: the 0.5B Llama-shaped ternary (t3) body, KV q16, SEQ 512,
    128 prompt tokens then 256 greedy tokens."""
    from vgx import synth
    return model_decode("0.5B Llama-shaped t3 (per-row ternary P(0)=0.4), seed 0", synth.bitcpm_spec(seq=512),
                        "t3", 16, 128, 256, runs)


def ternary_batch_bench(runs, nseq=32):
    """C5 at batch 32: the same ternary model, 32 sequences of 128 prompt
    tokens (each prefilled on its own KV cache), then 256 greedy steps in
    lockstep; decode tokens/s = 32 x 255 steps over the decode time."""
    import numpy as np
    from vgx import synth
    from vgx.engine import Engine

    spec = synth.bitcpm_spec(seq=512)
    blob = synth.container(spec, "t3", seed=0, q8_row=True)
    prompts = np.stack([synth.prompt(128, spec.vocab, seed=s) for s in range(nseq)])
    eng = Engine(blob, kv_bits=16)
    eng.generate_batch(prompts, 256)
    pf, dc = [], []
    for _ in range(runs):
        _toks, p, d = eng.generate_batch(prompts, 256)
        pf.append(p)
        dc.append(d)
    eng.close()
    ms_step = float(np.median(dc)) / 255
    return {"model": "0.5B Llama-shaped t3 (per-row ternary P(0)=0.4), seed 0", "sequences": nseq, "prompt": 128,
            "gen": 256, "seq": 512, "kv": "q16", "tokens_per_s": round(nseq * 1000.0 / ms_step, 1),
            "ms_per_step": round(ms_step, 4), "prefill_ms_all_sequences": round(float(np.median(pf)), 2),
            "runs": runs, "hbm": decode_roofline(decode_step_bytes(blob, 16, 128, 256, nseq), ms_step),
            "gemm_int8_peak_TOPS": INT8_PEAK_TOPS, "gemms": decode_batch_gemms()}


def decode_batch_gemms(reps=200):
    """The C5 batch-32 step's GEMMs alone, at its shapes (32 tokens, the 0.5B
    t3 layer): qkv, wo + residual then the FFN RMSNorm (rows of 32 k-steps
    are not split), the gate, w2 + residual split over workgroups with the
    next RMSNorm in its epilogue launch -- the calls the batched decode loop
    makes -- timed with HIP events on the launch stream; algorithmic int8 ops
    2*M*N*K (the gate: both matrices) against the matrix-core peak."""
    import numpy as np
    import torch
    from vgx import gpu as vg

    g = vg.GPU(0)
    rng = np.random.default_rng(0)
    M, dim, hidden = 32, 1024, 4096
    x = torch.from_numpy(rng.integers(-3000, 3000, (M, dim)).astype(np.int16)).cuda()
    xh = torch.from_numpy(rng.integers(-3000, 3000, (M, hidden)).astype(np.int16)).cuda()
    res = torch.from_numpy(rng.integers(-3000, 3000, (M, dim)).astype(np.int16)).cuda()
    nw = torch.from_numpy(rng.integers(100, 400, dim).astype(np.int16)).cuda()
    mats = {k: g.upload(make_matrix(rng, r, c, "t3"))
            for k, (r, c) in {"qkv": (1280, dim), "wo": (dim, dim), "w1": (hidden, dim), "w3": (hidden, dim),
                              "w2": (dim, hidden)}.items()}
    calls = [
        ("qkv", 1280, dim, lambda: g.gemm(mats["qkv"], x)),
        ("wo + norm", dim, dim, lambda: g.gemm_norm(mats["wo"], x, res, nw)),
        ("gate (w1, w3)", 2 * hidden, dim, lambda: g.ffn_gate_batch(mats["w1"], mats["w3"], x)),
        ("w2 + split + norm", dim, hidden, lambda: g.gemm_norm(mats["w2"], xh, res, nw, split=hidden // 2)),
    ]
    out = []
    for name, rows, cols, f in calls:
        for _ in range(5):
            f()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            f()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        tops = 2.0 * M * rows * cols / (us * 1e-6) / 1e12
        out.append({"gemm": name, "M_tokens": M, "N": rows, "K": cols, "kind": "t3", "us": round(us, 2),
                    "int8_TOPS": round(tops, 2), "frac_of_peak": round(tops / INT8_PEAK_TOPS, 5)})
    for m in mats.values():
        m.free()
    g.close()
    return out


def attention_bench(reps=200):
    """The C3 attention microbench: MiniMind3's attention (8 query / 4 KV heads
    of 96, q/k norm), KV q8, SEQ 768; K and V ~ N(0,1) written through the
    pack kernel; one decode attention launch (all heads of one layer, no KV
    write) at context 1, 64, 256, 512, 768: microseconds and the KV bytes read
    per microsecond."""
    import numpy as np
    import torch
    from vgx import gpu as vg

    g = vg.GPU(0)
    hd, seq, dim, kvh = 96, 768, 768, 4
    half = hd // 2
    inv = 1.0 / (1e6 ** (np.arange(half) * 2.0 / hd))
    ang = np.outer(np.arange(seq), inv)
    A = g.attention(dim=dim, heads=8, kv_heads=kvh, head_dim=hd, seq=seq, layers=1, kv_bits=8, rope_half=1,
                    qk_norm=1, rope_cos=np.cos(ang).astype(np.float32), rope_sin=np.sin(ang).astype(np.float32),
                    q_norm=np.ones((1, hd), np.float32), k_norm=np.ones((1, hd), np.float32))
    rng = np.random.default_rng(0)
    width = dim + 2 * kvh * hd
    qkv = np.clip(np.rint(rng.standard_normal((seq, width)) * 256.0), -32768, 32767).astype(np.int16)
    rows = torch.from_numpy(qkv).cuda()
    A.block_batch(0, 0, rows)  # every row packed, every position attended once
    out = torch.empty(dim, dtype=torch.int16, device="cuda")
    res = []
    for ctx in (1, 64, 256, 512, 768):
        q = rows[ctx - 1]
        for _ in range(20):
            A.decode(0, ctx - 1, q, out)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            A.decode(0, ctx - 1, q, out)
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        kv_bytes = ctx * A.row_bytes
        res.append({"context": ctx, "us": round(us, 2), "kv_bytes": kv_bytes, "GBps": round(kv_bytes / us / 1e3, 2)})
    A.free()
    g.close()
    return {"shape": "MiniMind3 attention: 8 query / 4 KV heads of 96, q/k norm, KV q8, SEQ 768",
            "launch": "vgx_attn_decode (all heads of one layer)", "reps": reps, "contexts": res}


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix-core peak, TOPS


def prefill_bench(runs):
    """The C3 workload: MiniMind3-64M-shaped q4, KV q8, SEQ 768.  A 256-token
    prompt prefilled in one batch (int8 matrix cores) against the serial loop,
    then 512 greedy tokens; and the prefill GEMMs alone (256 tokens x the
    layer shapes), their algorithmic int8 ops (2*M*N*K) over kernel time
    against the matrix-core peak."""
    import numpy as np
    import torch
    from vgx import gpu as vg
    from vgx import synth
    from vgx.engine import Engine

    spec = synth.minimind3_spec(seq=768)
    blob = synth.container(spec, "q4", seed=0)
    prompt = synth.prompt(256, spec.vocab, seed=0)
    eng = Engine(blob, kv_bits=8)
    eng.set_graphs(GRAPHS)
    eng.prefill(prompt, logits=False)
    batched = []
    for _ in range(runs):
        t0 = time.perf_counter()
        eng.prefill(prompt, logits=False)
        batched.append((time.perf_counter() - t0) * 1e3)
    eng.set_prefill_batch(0)
    t0 = time.perf_counter()
    eng.prefill(prompt, logits=False)
    serial_ms = (time.perf_counter() - t0) * 1e3
    eng.set_prefill_batch(256)
    toks, pf_ms, dc_ms = eng.generate(prompt, 512)
    eng.close()

    # the GEMMs alone, on the stream the wrapper launches on
    g = vg.GPU(0)
    rng = np.random.default_rng(0)
    gemms = []
    for name, rows, cols in (("qkv", 1536, 768), ("wo", 768, 768), ("w1/w3 chunk", 1216, 768), ("w2", 768, 2432)):
        W = g.upload(make_matrix(rng, rows, cols, "q4"))
        x = torch.from_numpy(rng.integers(-3000, 3000, (256, cols)).astype(np.int16)).cuda()
        y = torch.empty((256, rows), dtype=torch.int16, device="cuda")
        for _ in range(3):
            g.gemm(W, x, out=y)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(100):
            g.gemm(W, x, out=y)
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / 100
        tops = 2.0 * 256 * rows * cols / (us * 1e-6) / 1e12
        gemms.append({"gemm": name, "M_tokens": 256, "N": rows, "K": cols, "kind": "q4", "us": round(us, 2),
                      "int8_TOPS": round(tops, 2), "frac_of_peak": round(tops / INT8_PEAK_TOPS, 5)})
        W.free()
    g.close()
    med = float(np.median(batched))
    return {"model": "MiniMind3-64M-shaped, q4 g32, seed 0", "kv": "q8", "seq": 768, "prompt": 256,
            "batched_prefill_ms": round(med, 3), "batched_prefill_tokens_per_s": round(256 / med * 1e3, 1),
            "serial_prefill_ms": round(serial_ms, 3), "serial_prefill_tokens_per_s": round(256 / serial_ms * 1e3, 1),
            "speedup": round(serial_ms / med, 2), "runs": runs,
            "generate_512": {"prefill_ms": round(pf_ms, 3), "decode_ms": round(dc_ms, 3),
                             "decode_tokens_per_s": round(511 / dc_ms * 1e3, 1)},
            "gemm_int8_peak_TOPS": INT8_PEAK_TOPS, "gemms": gemms}


def decode_cpu_baseline(blob, prompt, n_gen):
    """The float CPU path over the GPU leg's own positions: the prompt, then
    greedy steps on its own argmax, timed over the n_gen - 1 steps after the
    first generated token, as the GPU leg is -- the
    reference's float forward on the dequantised container weights
    (oracle/model.py FModel semantics) run by the C/OpenMP float path
    (oracle/vgx_float.c), on every host core this process may use and on one."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    from model import CFModel, float_lib

    f = CFModel(blob)
    lib = float_lib()
    cores = lib.vgxf_threads()
    n_prompt = len(prompt)

    def rate():
        logits = None
        for pos in range(n_prompt):
            logits = f.step(int(prompt[pos]), pos)
        # the first generated token comes from the prompt's last logits; the
        # GPU leg times the n_gen - 1 steps after it, and so does this
        tok = int(np.argmax(logits))
        t0 = time.perf_counter()
        for pos in range(n_prompt, n_prompt + n_gen - 1):
            tok = int(np.argmax(f.step(tok, pos)))
        return (n_gen - 1) / (time.perf_counter() - t0)

    rate()  # first touch of the weights
    all_cores = rate()
    lib.vgxf_set_threads(1)
    one = rate()
    lib.vgxf_set_threads(cores)
    return {"tokens_per_s": round(all_cores, 2), "cores": cores, "one_core_tokens_per_s": round(one, 2),
            "sample": "the GPU leg's positions: a %d-token prompt, then the %d greedy steps after the first "
                      "token timed (C, fp32 FMA dot products, OpenMP over rows, dequantised container weights)"
                      % (n_prompt, n_gen - 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cold-mb", type=int, default=512, help="distinct weight MiB per shape")
    ap.add_argument("--warm-reps", type=int, default=1000)
    ap.add_argument("--warm-mb", type=int, default=64,
                    help="distinct weight MiB per shape of the warm (Infinity-Cache-resident) sweep")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-runs", type=int, default=5)
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--copy-mb", type=int, default=0, help="also time a device copy of this many MiB")
    ap.add_argument("--skip-stream-ref", action="store_true", help="skip the library read/copy bandwidth reference")
    ap.add_argument("--only", choices=["gemv", "decode", "prefill", "hybrid", "ternary", "ternary32", "attention",
                                       "gemm32"],
                    default=None,
                    help="run one leg (for profiling); the JSON line then carries that leg only")
    ap.add_argument("--prefill-runs", type=int, default=5)
    ap.add_argument("--no-graphs", action="store_true",
                    help="decode legs issue each step's launches instead of replaying a HIP graph")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-models", action="store_true", help="skip the C4 hybrid and C5 ternary decode legs")
    ap.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "BENCH_LOG"),
                    help="print the HBM traffic summary of two rocprofv3 --pmc runs and exit (no GPU)")
    args = ap.parse_args()
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary), indent=1))
        return
    global GRAPHS
    GRAPHS = not args.no_graphs
    if args.gpus != 1:
        print("bench.py measures one GPU: the decode path runs on a single device; --gpus %d is not measured"
              % args.gpus, file=sys.stderr)
        sys.exit(2)
    if args.only == "decode":
        blob, prompt, toks, dec = decode_bench(args.decode_runs)
        print(json.dumps({"decode": dec}))
        return
    if args.only == "prefill":
        print(json.dumps({"prefill": prefill_bench(args.prefill_runs)}))
        return
    if args.only == "attention":
        print(json.dumps({"attention_c3": attention_bench()}))
        return
    if args.only == "ternary32":
        print(json.dumps({"decode_c5_batch32": ternary_batch_bench(args.decode_runs)}))
        return
    if args.only == "gemm32":
        print(json.dumps({"decode_c5_batch32_gemms": decode_batch_gemms()}))
        return
    if args.only in ("hybrid", "ternary"):
        fn = hybrid_decode_bench if args.only == "hybrid" else ternary_decode_bench
        print(json.dumps({args.only: fn(args.decode_runs)[3]}))
        return
    if args.only == "gemv":
        args.skip_decode, args.no_cpu, args.skip_prefill, args.skip_models = True, True, True, True

    import numpy as np
    import torch

    from vgx import gpu as vg

    torch.cuda.set_device(0)
    g = vg.GPU(0)

    def cold_sweep(kind, timed):
        """One launch per shape over >= --cold-mb MiB of distinct copies (a
        group sharing x); `timed` steps of the five launches between two
        events, then per shape: the cold launch time, the warm sweep (one
        launch over --warm-mb MiB of the same copies, resident in the
        Infinity Cache after a warm-up launch: the kernel streaming from the
        cache), and the back-to-back launch interval of one matrix (1000 reps,
        the reference's warm measurement; at these sizes a launch-latency
        figure, not a kernel duration)."""
        rng = np.random.default_rng(0 if kind == "q8" else 1)
        xs, per_shape = {}, []
        for rows, cols in SHAPES:
            base = g.upload(make_matrix(rng, rows, cols, kind))
            copies = max(1, (args.cold_mb << 20) // weight_bytes(rows, cols, kind))
            mats = [base] + [g.clone(base) for _ in range(copies - 1)]
            grp = g.group(mats)
            wcopies = max(1, min(copies, (args.warm_mb << 20) // weight_bytes(rows, cols, kind)))
            wgrp = g.group(mats[:wcopies])
            if cols not in xs:
                xs[cols] = torch.from_numpy(rng.standard_normal(cols).astype(np.float32)).cuda()
            y = torch.empty(grp.rows, dtype=torch.float32, device="cuda")
            per_shape.append(dict(rows=rows, cols=cols, copies=copies, mats=mats, grp=grp, y=y, wcopies=wcopies,
                                  wgrp=wgrp, y1=torch.empty(rows, dtype=torch.float32, device="cuda")))
        torch.cuda.synchronize()

        def step():
            for s in per_shape:
                s["grp"].gemv_f32(xs[s["cols"]], s["y"])

        step_bytes = sum(s["copies"] * algo_bytes(s["rows"], s["cols"], kind) for s in per_shape)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(timed):
            step()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_step = e0.elapsed_time(e1) / timed
        shapes_out = []
        for s in per_shape:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(timed):
                s["grp"].gemv_f32(xs[s["cols"]], s["y"])
            b.record()
            torch.cuda.synchronize()
            cold_us = a.elapsed_time(b) * 1e3 / timed
            for _ in range(3):  # bring the warm copies into the Infinity Cache
                s["wgrp"].gemv_f32(xs[s["cols"]], s["y"])
            a.record()
            for _ in range(timed):
                s["wgrp"].gemv_f32(xs[s["cols"]], s["y"])
            b.record()
            torch.cuda.synchronize()
            wsweep_us = a.elapsed_time(b) * 1e3 / timed
            a.record()
            for _ in range(args.warm_reps):
                g.matvec_f32(s["mats"][0], xs[s["cols"]], s["y1"])
            b.record()
            torch.cuda.synchronize()
            warm_us = a.elapsed_time(b) * 1e3 / args.warm_reps
            ab = algo_bytes(s["rows"], s["cols"], kind)
            shapes_out.append({"shape": "%dx%d" % (s["rows"], s["cols"]), "copies": s["copies"],
                               "bytes_per_launch": s["copies"] * ab,
                               "cold_us_per_launch": round(cold_us, 2),
                               "cold_GBps": round(s["copies"] * ab / (cold_us * 1e-6) / 1e9, 1),
                               "warm_sweep_copies": s["wcopies"], "warm_sweep_bytes": s["wcopies"] * ab,
                               "warm_sweep_us_per_launch": round(wsweep_us, 2),
                               "warm_sweep_GBps": round(s["wcopies"] * ab / (wsweep_us * 1e-6) / 1e9, 1),
                               "launch_interval_us_one_matrix": round(warm_us, 3)})
        for s in per_shape:
            s["grp"].free()
            s["wgrp"].free()
            for mm in s["mats"]:
                mm.free()
        torch.cuda.synchronize()
        kern_us = sum(x["cold_us_per_launch"] for x in shapes_out)
        return {"value": step_bytes / (ms_step * 1e-3) / 1e9, "ms_step": ms_step, "wall": wall,
                "step_bytes": step_bytes, "achieved": step_bytes / (kern_us * 1e-6) / 1e9, "shapes": shapes_out}

    q8 = cold_sweep("q8", args.steps)
    q4 = cold_sweep("q4", args.steps)
    traffic = traffic_summary()
    out = {
        "metric": METRIC, "value": round(q8["value"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(q8["ms_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8 weights x q16 activations (exact int32 dot), fp32 scale",
        "data": "synthetic: N(0,0.02) fp32 weights, seed 0, packed q8 per-row; x ~ N(0,1) fp32",
        "config": {"workload": "q8 dequant-GEMV sweep at MiniMind3 shapes, cold weights",
                   "shapes": [x["shape"] for x in q8["shapes"]], "batch": 1,
                   "cold_bytes_per_step": q8["step_bytes"], "wall_s": round(q8["wall"], 3)},
        "roofline": {"bound": "hbm", "achieved": round(q8["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(q8["achieved"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes_per_step"] if traffic else None,
                     "algorithmic_bytes": q8["step_bytes"],
                     "per": "step: one launch per shape, 5 launches; achieved = algorithmic bytes / sum of the "
                            "5 launches' HIP-event durations",
                     "kernel": "gemv_kernel<q8, EPI_STORE_F32> (one launch per shape per step)"},
        "gemv": q8["shapes"],
        "q4": {"value": round(q4["value"], 1), "unit": "GB/s", "achieved": round(q4["achieved"], 1),
               "frac": round(q4["achieved"] / HBM_PEAK_GBS, 4), "ms_per_step": round(q4["ms_step"], 4),
               "cold_bytes_per_step": q4["step_bytes"], "gemv": q4["shapes"]},
    }
    if traffic:
        out["roofline"]["traffic_source"] = traffic.get("source")
    g.close()
    torch.cuda.synchronize()
    if not args.skip_stream_ref:
        # what plain library kernels reach on this part, beside the GEMV: a
        # read-only reduction and an elementwise copy, 1 GiB each way
        big = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(big)
        ref = {}
        for name, fn, nbytes in (("torch.sum, float32, 1 GiB read", lambda: big.sum(), big.numel() * 4),
                                 ("torch.mul, float32, 1 GiB read + 1 GiB written",
                                  lambda: torch.mul(big, 1.0, out=dst), big.numel() * 8)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                fn()
            e1.record()
            torch.cuda.synchronize()
            gbps = nbytes * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
            ref[name] = {"GBps": round(gbps, 1), "frac_of_peak": round(gbps / 8000.0, 4)}
        # the same two kernels on a working set the Infinity Cache holds (the
        # warm sweep's size), after a warm-up pass
        small = torch.ones(args.warm_mb << 17, dtype=torch.float32, device="cuda")  # warm_mb / 2 MiB
        sdst = torch.empty_like(small)
        for name, fn, nbytes in (("torch.sum, float32, %d MiB read, cache-resident" % (args.warm_mb // 2),
                                  lambda: small.sum(), small.numel() * 4),
                                 ("torch.mul, float32, %d MiB read + %d MiB written, cache-resident"
                                  % (args.warm_mb // 2, args.warm_mb // 2),
                                  lambda: torch.mul(small, 1.0, out=sdst), small.numel() * 8)):
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(50):
                fn()
            e1.record()
            torch.cuda.synchronize()
            ref[name] = {"GBps": round(nbytes * 50 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)}
        out["stream_reference"] = ref
        del big, dst, small, sdst
    if args.copy_mb:
        # a plain device copy of known size: the scale for the FETCH_SIZE /
        # WRITE_SIZE counters of a profiling run of this command
        # (an elementwise kernel, not copy_, which a DMA engine may serve)
        a = torch.empty(args.copy_mb << 18, dtype=torch.float32, device="cuda").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(args.steps):
            torch.mul(a, 1.0, out=b)
        torch.cuda.synchronize()
        out["copy_calibration"] = {"kernel": "at::native elementwise mul, float32",
                                   "bytes_read": a.numel() * 4, "bytes_written": b.numel() * 4,
                                   "dispatches": args.steps}
        del a, b
    if not args.skip_decode:
        blob, prompt, toks, dec = decode_bench(args.decode_runs)
        out["decode"] = dec
        out["decode_tokens_per_s"] = dec["tokens_per_s"]
    if not args.skip_prefill:
        out["prefill"] = prefill_bench(args.prefill_runs)
        out["attention_c3"] = attention_bench()
    others = []
    if not args.skip_models:
        others = [("decode_c4", hybrid_decode_bench(args.decode_runs)),
                  ("decode_c5_batch1", ternary_decode_bench(args.decode_runs))]
        for key, (_b, _p, _t, res) in others:
            out[key] = res
        out["decode_c5_batch32"] = ternary_batch_bench(max(1, args.decode_runs // 2))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if not args.skip_decode:
            out["decode"]["cpu_float_path"] = decode_cpu_baseline(blob, prompt, out["decode"]["gen"])
        for key, (b, p, _t, r) in others:
            out[key]["cpu_float_path"] = decode_cpu_baseline(b, p, r["gen"])
    print(json.dumps(out))


if __name__ == "__main__":
    main()
