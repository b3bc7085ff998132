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
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "vc4-gles2-inference_amd")
sys.path.insert(0, PKG)

SHAPES = [(768, 768), (384, 768), (2432, 768), (768, 2432), (6400, 768)]
HBM_PEAK_GBS = 8000.0
METRIC = "dequant-GEMV GB/s (% HBM peak) + decode tokens/s, MiniMind3-64M q8, 1 GPU"


def algo_bytes(rows, cols):
    """body + f32 row plane + f32 x + f32 y for one q8 per-row GEMV."""
    return rows * cols + rows * 4 + cols * 4 + rows * 4


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
    nbytes, passes = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for rows, cols, body, wsr in mats:
            xq = o.quantize_act(xs[cols])
            o.store_f32(o.rowval_q8(body, 1, rows, cols, wsr, xq))
            nbytes += algo_bytes(rows, cols)
        passes += 1
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": o.threads(), "kind": "port",
            "sample": "%d passes over the 5 MiniMind3 q8 GEMV shapes (one matrix each, warm host caches), "
                      "%.1f s, oracle exact-integer q8 GEMV with OpenMP" % (passes, dt)}


def decode_bench(runs):
    """MiniMind3-64M q8 (per-row scales), KV q16, SEQ 256: 32 prompt tokens
    then 64 greedy tokens through the engine; decode tokens/s over the 63
    steps after the prompt, median of `runs` after one warm-up run."""
    import numpy as np
    from vgx import synth
    from vgx.engine import Engine

    spec = synth.minimind3_spec(seq=256)
    blob = synth.container(spec, "q8", seed=0, q8_row=True)
    prompt = synth.prompt(32, spec.vocab, seed=0)
    eng = Engine(blob, kv_bits=16)
    eng.generate(prompt, 64)
    pf, dc, toks = [], [], None
    for _ in range(runs):
        toks, p, d = eng.generate(prompt, 64)
        pf.append(p)
        dc.append(d)
    eng.close()
    ms_tok = float(np.median(dc)) / 63
    return blob, prompt, toks, {
        "model": "MiniMind3-64M-shaped, q8 per-row, seed 0", "prompt": 32, "gen": 64, "seq": 256, "kv": "q16",
        "tokens_per_s": round(1000.0 / ms_tok, 1), "ms_per_token": round(ms_tok, 4),
        "prefill_ms": round(float(np.median(pf)), 3), "runs": runs}


def decode_cpu_baseline(blob, prompt, steps):
    """The float CPU path (oracle/model.py FModel: the reference's numpy
    forward semantics on the dequantised container) for `steps` positions."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as o
    from model import FModel

    f = FModel(blob)
    t0 = time.perf_counter()
    for pos in range(steps):
        f.step(int(prompt[pos % len(prompt)]), pos)
    dt = time.perf_counter() - t0
    return {"tokens_per_s": round(steps / dt, 2), "cores": o.threads(),
            "sample": "%d positions of the float path (numpy fp32 BLAS, dequantised q8 weights)" % steps}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cold-mb", type=int, default=512, help="distinct weight MiB per shape")
    ap.add_argument("--warm-reps", type=int, default=1000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-runs", type=int, default=5)
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--copy-mb", type=int, default=0, help="also time a device copy of this many MiB")
    ap.add_argument("--cpu-decode-steps", type=int, default=16)
    ap.add_argument("--only", choices=["gemv", "decode"], default=None,
                    help="run one leg (for profiling); the JSON line then carries that leg only")
    args = ap.parse_args()
    if args.only == "decode":
        blob, prompt, toks, dec = decode_bench(args.decode_runs)
        print(json.dumps({"decode": dec}))
        return
    if args.only == "gemv":
        args.skip_decode, args.no_cpu = True, True
    if args.gpus != 1:
        print("bench.py runs on one GPU: the decode path is single-device (see DESIGN.md); --gpus %d "
              "is not measured" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from vgx import gpu as vg
    from vgx import mmcf

    torch.cuda.set_device(0)
    g = vg.GPU(0)
    rng = np.random.default_rng(0)
    xs, per_shape = {}, []
    for rows, cols in SHAPES:
        w = rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(0.02)
        q, unit, plane = mmcf.q8_per_row(w)
        m = mmcf.Matrix("q8", rows, cols, (q.view(np.uint8) ^ 0x80).ravel(), unit, True, plane)
        base = g.upload(m)
        copies = max(1, (args.cold_mb << 20) // (rows * cols))
        mats = [base] + [g.clone(base) for _ in range(copies - 1)]
        grp = g.group(mats)
        if cols not in xs:
            xs[cols] = torch.from_numpy(rng.standard_normal(cols).astype(np.float32)).cuda()
        y = torch.empty(grp.rows, dtype=torch.float32, device="cuda")
        per_shape.append(dict(rows=rows, cols=cols, copies=copies, mats=mats, grp=grp, y=y,
                              y1=torch.empty(rows, dtype=torch.float32, device="cuda")))
    torch.cuda.synchronize()

    def step():
        for s in per_shape:
            s["grp"].gemv_f32(xs[s["cols"]], s["y"])

    step_bytes = sum(s["copies"] * algo_bytes(s["rows"], s["cols"]) for s in per_shape)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # per-shape launch durations (cold) and warm single-matrix launches
    shapes_out = []
    for s in per_shape:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            s["grp"].gemv_f32(xs[s["cols"]], s["y"])
        b.record()
        torch.cuda.synchronize()
        cold_us = a.elapsed_time(b) * 1e3 / args.steps
        a.record()
        for _ in range(args.warm_reps):
            g.matvec_f32(s["mats"][0], xs[s["cols"]], s["y1"])
        b.record()
        torch.cuda.synchronize()
        warm_us = a.elapsed_time(b) * 1e3 / args.warm_reps
        ab = algo_bytes(s["rows"], s["cols"])
        shapes_out.append({"shape": "%dx%d" % (s["rows"], s["cols"]), "copies": s["copies"],
                           "cold_us_per_launch": round(cold_us, 2),
                           "cold_GBps": round(s["copies"] * ab / (cold_us * 1e-6) / 1e9, 1),
                           "warm_us_per_gemv": round(warm_us, 3),
                           "warm_GBps": round(ab / (warm_us * 1e-6) / 1e9, 1)})
    kern_us = sum(x["cold_us_per_launch"] for x in shapes_out)
    achieved = step_bytes / (kern_us * 1e-6) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 weights x q16 activations (exact int32 dot), fp32 scale",
        "data": "synthetic: N(0,0.02) fp32 weights, seed 0, packed q8 per-row; x ~ N(0,1) fp32",
        "config": {"workload": "q8 dequant-GEMV sweep at MiniMind3 shapes, cold weights",
                   "shapes": [x["shape"] for x in shapes_out], "batch": 1,
                   "cold_bytes_per_step": step_bytes, "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_kernel<q8, EPI_STORE_F32> (one launch per shape per step)"},
        "gemv": shapes_out,
    }
    for s in per_shape:
        s["grp"].free()
        for mm in s["mats"]:
            mm.free()
    g.close()
    torch.cuda.synchronize()
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
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if not args.skip_decode:
            out["decode"]["cpu_float_path"] = decode_cpu_baseline(blob, prompt, args.cpu_decode_steps)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
