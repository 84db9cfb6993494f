"""Benchmark of the NanoLLM greedy token loop on one MI355X.

Headline (BASELINE.json metric, config c2): decode tokens/s of the 384d x 6L char GPT
(vocab 65, block 256) at batch 1 -- a "step" is one decode step (one new token per sequence)
after a 64-token prefill, inputs resident in HBM.  The same JSON line carries:

* roofline: the dominant decode-step op (by time per step), algorithmic HBM bytes per launch
  over its mean launch time measured with HIP events on the library stream;
* step_roofline: algorithmic bytes per decode step (SURVEY formula) over the step time;
* bs64: c3 decode tokens/s (64 sequences) and its step roofline;
* prefill: MFMA utilisation of the c3 and c4 prefills (executed FLOPs / time / fp32 peak);
* cpu_baseline: the CPU oracle ("port" of the reference algorithm: full-window recompute per
  token, ThreadPool-style row split) on a bounded sample of c2 steps.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import freeml_amd as fh  # noqa: E402
from freeml_amd import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
FP32_MFMA_PEAK_TF = 157.3   # MI355X dense fp32 matrix
METRIC = "decode tok/s bs1/bs64 (384d·6L GPT); % HBM roofline; prefill MFMA util"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def step_bytes(shape, batch, pos):
    """Algorithmic HBM bytes of one decode step at position pos (attends pos + 1 keys)."""
    V, C, L = shape.vocab, shape.n_embed, shape.n_layer
    t = pos + 1
    weights = 4 * (L * 12 * C * C + V * C + 2 * L * C + 2 * C)
    return (weights + batch * 4 * 2 * C + batch * L * 2 * t * C * 4 + batch * L * 2 * C * 4
            + batch * V * 4)


def prefill_flops(shape, batch, P):
    """FLOPs the prefill executes: all prompt rows through every block (causal attention
    counted as its lower triangle) and lm_head on the last row of each sequence."""
    V, C, L = shape.vocab, shape.n_embed, shape.n_layer
    return batch * (2 * P * L * 12 * C * C + L * 2 * C * P * (P + 1) + 2 * V * C)


def timed_decode(m, prompts, n_steps, per_chunk):
    """Decode n_steps steps (re-prefilling outside the timed region when the window fills);
    returns (seconds of decode, list of (first_pos, steps) chunks)."""
    timer = fh.Timer()
    total_ms, chunks, left = 0.0, [], n_steps
    P = prompts.shape[1]
    while left > 0:
        k = min(left, per_chunk)
        m.prefill(prompts)
        fh.synchronize()
        timer.start()
        m.decode(k)
        total_ms += timer.stop()
        fh.synchronize()
        chunks.append((P, k))
        left -= k
    return total_ms / 1e3, chunks


def decode_bench(name, steps, warmup):
    cfg = synth.CONFIGS[name]
    shape, B, P = cfg["shape"], cfg["batch"], cfg["prompt"]
    per_chunk = shape.block_size - P  # decode steps one window allows after the prefill
    w = synth.make_weights(shape, 0)
    prompts = synth.prompts_for(name)
    m = fh.NanoLLM(w, max_batch=B)
    if warmup:
        timed_decode(m, prompts, warmup, per_chunk)
    secs, chunks = timed_decode(m, prompts, steps, per_chunk)
    nbytes = sum(step_bytes(shape, B, p0 + i) for p0, k in chunks for i in range(k))
    tok_s = B * steps / secs
    step_ms = secs * 1e3 / steps
    gbs = nbytes / secs / 1e9
    res = dict(tok_s=tok_s, ms_per_step=step_ms, bytes_per_step=nbytes / steps,
               step_roofline=dict(bound="hbm", achieved=gbs, peak=HBM_PEAK_GBS, unit="GB/s",
                                  frac=gbs / HBM_PEAK_GBS))
    return m, prompts, res


def dominant_op(m, prompts, shape):
    names = ["qkv", "attention", "attn_proj", "mlp_fc", "mlp_proj", "lm_head"]
    per_step = [shape.n_layer] * 5 + [1]
    rows = []
    for op in range(6):
        m.prefill(prompts)
        m.decode(16)  # a realistic attended length for the attention op
        ms, nbytes = m.profile_op(op, 200)
        rows.append(dict(op=names[op], ms=ms, bytes=nbytes, per_step=per_step[op],
                         share_ms=ms * per_step[op], gbs=nbytes / (ms * 1e-3) / 1e9))
    dom = max(rows, key=lambda r: r["share_ms"])
    return dom, rows


def prefill_bench(name, reps=3):
    cfg = synth.CONFIGS[name]
    shape, B, P = cfg["shape"], cfg["batch"], cfg["prompt"]
    w = synth.make_weights(shape, 0)
    m = fh.NanoLLM(w, max_batch=B)
    prompts = synth.prompts_for(name)
    m.prefill(prompts)  # warm-up
    timer = fh.Timer()
    best = None
    for _ in range(reps):
        fh.synchronize()
        timer.start()
        m.prefill(prompts)
        ms = timer.stop()
        best = ms if best is None else min(best, ms)
    flops = prefill_flops(shape, B, P)
    tf = flops / (best * 1e-3) / 1e12
    m.close()
    return dict(config=name, ms=best, gflop=flops / 1e9, tflops=tf, mfma_util=tf / FP32_MFMA_PEAK_TF)


def cpu_baseline(budget_s=12.0):
    """The reference algorithm on the host: full-window recompute per generated token (c2)."""
    import oracle

    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 0)
    threads = max(1, min(16, os.cpu_count() or 1))
    om = oracle.OracleModel(w, nthreads=threads)
    prompt = synth.prompts_for("c2")[0]
    t0 = time.perf_counter()
    om.greedy(prompt, 1, cached=False)
    one = time.perf_counter() - t0
    k = int(max(2, min(40, budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    om.greedy(prompt, k, cached=False)
    secs = time.perf_counter() - t0
    om.close()
    return dict(value=k / secs, unit="tok/s", cores=threads, kind="port",
                sample=f"c2 batch 1: first {k} greedy steps, each a full 256-token window "
                       f"recompute (reference algorithm), {secs:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=191)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-extra", action="store_true", help="skip bs64 / prefill / cpu legs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the token loop shards over independent sequences; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    fh.init(0)
    arch, cus = fh.device_info()
    log(f"device {arch}, {cus} CUs")
    shape = synth.CONFIGS["c2"]["shape"]
    log("c2 decode (batch 1)")
    m, prompts, res = decode_bench("c2", args.steps, args.warmup)
    log(f"c2: {res['tok_s']:.0f} tok/s, {res['ms_per_step'] * 1e3:.1f} us/step")
    dom, ops = dominant_op(m, prompts, shape)
    for r in ops:
        log(f"  op {r['op']:10s} {r['ms'] * 1e3:8.2f} us  {r['gbs']:8.1f} GB/s  x{r['per_step']}")
    m.close()
    out = {
        "metric": METRIC,
        "value": res["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompts; freeml_amd/synth.py)",
        "config": {"workload": "c2: char GPT vocab 65, block 256, 384d, 6 heads, 6 layers; "
                               "batch 1, 64-token prompt, greedy decode steps",
                   "batch": 1, "prompt": 64, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "op": dom["op"], "achieved": dom["gbs"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dom["gbs"] / HBM_PEAK_GBS,
                     "traffic": None, "bytes_per_launch": dom["bytes"],
                     "us_per_launch": dom["ms"] * 1e3},
        "step_roofline": res["step_roofline"],
    }
    if not args.no_extra:
        log("c3 decode (batch 64)")
        m64, _, r64 = decode_bench("c3", 191, 10)
        m64.close()
        log(f"c3: {r64['tok_s']:.0f} tok/s")
        out["bs64"] = {"tok_s": r64["tok_s"], "ms_per_step": r64["ms_per_step"],
                       "step_roofline": r64["step_roofline"]}
        pf = []
        for name in ("c3", "c4"):
            log(f"{name} prefill")
            pf.append(prefill_bench(name))
            log(f"  {pf[-1]['ms']:.2f} ms, {pf[-1]['tflops']:.1f} TFLOP/s")
        out["prefill"] = pf
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
