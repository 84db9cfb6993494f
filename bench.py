"""Benchmark of the NanoLLM greedy token loop on one MI355X.

Headline (the benchmark's metric, config c2): decode tokens/s of the 384d x 6L char GPT
(vocab 65, block 256) at batch 1 -- a "step" is one decode step (one new token per sequence)
after a 64-token prefill, inputs resident in HBM.  The same JSON line carries:

* roofline: the dominant kernel.  At batch 1 that is the relay decode kernel (one launch per
  decode call, all steps of the call inside it; FMLH_RELAY=0 measures the persistent kernel
  instead): algorithmic HBM bytes per launch (the
  per-step bytes summed over the launch's steps) over its mean launch time, measured with HIP
  events on the library stream the kernel is launched on.  traffic: the counter bytes of a
  committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary per algorithmic byte, times this
  launch's algorithmic bytes.  When a shape decodes through the multi-kernel graph path
  instead, the dominant op of the step (profile_op) is reported;
* step_roofline: algorithmic bytes per decode step over the step time;
* bs64: c3 decode tokens/s (64 sequences: the grouped persistent kernel, one launch per decode
  call) with its kernel roofline (or, on the graph path, the dominant op);
* large: c4 (batch 8, 512-token prompts) and c5 (batch 4, 3584-token prompts) decode tokens/s
  over their configs' 511 decode steps, with the step roofline;
* prefill: MFMA utilisation of the c3, c4 and c5 prefills (executed FLOPs / time / fp32 peak),
  best and median of ten calls;
* cpu_baseline: the reference algorithm on the host (full-window recompute per token) on a
  bounded sample of c2 steps: the compiled reference's own MatrixCPU decode (kind "reference",
  FreeML's ThreadPool) with the oracle's restatement ("port") beside it and their ratio, nproc,
  and c3-c5 extrapolated by window FLOPs;
* train: the next row after decoding -- NanoLLM's training iteration (window + shifted target,
  forward, CCE gradient, backward, AdamW) of FreeML's own Model::Run on MatrixHIP<float>
  (oracle/_ref/nanollm_dropin --train), c2 shape, against the same driver on the reference
  MatrixCPU<float> backend for a few iterations.
Not default: exchange (hand-off latency probe), timeline (the grouped kernel's per-hop
timeline), wide_timeline (the wide kernel's per-phase timeline at c4 / c5), relay_timeline (the
relay kernel's per-role timeline at c2 and c3's batch of 64), gemm (the NT GEMM at the prefill
projection shapes and longer ones).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--no-extra | --extra bs64,large,prefill,cpu,train,exchange,timeline,wide_timeline,
                                             relay_timeline,gemm]
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


PMC_TRAFFIC = {("c2", "persistent"): os.path.join(ROOT, "profiles", "decode_persistent_c2_pmc_traffic.md"),
               ("c2", "relay"): os.path.join(ROOT, "profiles", "decode_relay_c2_pmc_traffic.md"),
               ("c3", "grouped"): os.path.join(ROOT, "profiles", "decode_grouped_c3_pmc_traffic.md"),
               ("c3", "relay"): os.path.join(ROOT, "profiles", "decode_relay_c3_pmc_traffic.md"),
               ("c4", "wide"): os.path.join(ROOT, "profiles", "decode_wide_c4_pmc_traffic.md"),
               ("c5", "wide"): os.path.join(ROOT, "profiles", "decode_wide_c5_pmc_traffic.md")}
KERNELS = {"persistent": "decode_persistent_kernel", "grouped": "decode_grouped_kernel",
           "relay": "decode_relay_kernel", "wide": "decode_wide_kernel"}


def measured_traffic(path, algorithmic_bytes):
    """HBM bytes of a launch of algorithmic_bytes, from a committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (counters cannot be read from inside the profiled process): the
    summary's counter bytes per algorithmic byte, times this launch's algorithmic bytes.  A
    launch of another length then scales with its own weight and KV-cache bytes.  Returns
    (bytes, counter/algorithmic ratio) or (None, None) when the summary is absent."""
    try:
        vals = {}
        with open(path) as f:
            for line in f:
                if "=" in line and not line.startswith(("cd ", "`", "|")):
                    k, v = line.split("=", 1)
                    vals[k.strip()] = v.strip()
        ratio = float(vals["traffic_bytes_per_launch"]) / float(vals["algorithmic_bytes_per_launch"])
        return ratio * algorithmic_bytes, ratio
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None, None


def timed_decode(m, prompts, n_steps, per_chunk):
    """Decode n_steps steps (re-prefilling outside the timed region when the window fills);
    returns (seconds of decode, list of (first_pos, steps, ms) chunks -- one decode call, and on
    the persistent path one kernel launch, per chunk)."""
    timer = fh.Timer()
    total_ms, chunks, left = 0.0, [], n_steps
    P = prompts.shape[1]
    while left > 0:
        k = min(left, per_chunk)
        m.prefill(prompts)
        fh.synchronize()
        timer.start()
        m.decode(k)
        ms = timer.stop()
        total_ms += ms
        fh.synchronize()
        chunks.append((P, k, ms))
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
    launch_bytes = [sum(step_bytes(shape, B, p0 + i) for i in range(k)) for p0, k, _ in chunks]
    nbytes = sum(launch_bytes)
    tok_s = B * steps / secs
    step_ms = secs * 1e3 / steps
    gbs = nbytes / secs / 1e9
    path, wgs = m.decode_path(B)
    res = dict(tok_s=tok_s, ms_per_step=step_ms, bytes_per_step=nbytes / steps, path=path,
               workgroups=wgs,
               step_roofline=dict(bound="hbm", achieved=gbs, peak=HBM_PEAK_GBS, unit="GB/s",
                                  frac=gbs / HBM_PEAK_GBS))
    if path in KERNELS:  # one launch per decode call: the launch is the dominant kernel
        us = float(np.mean([ms for _, _, ms in chunks])) * 1e3
        by = float(np.mean(launch_bytes))
        ach = by / (us * 1e-6) / 1e9
        pmc = PMC_TRAFFIC.get((name, path))
        if pmc and not os.path.exists(pmc):
            pmc = None
        traffic, ratio = measured_traffic(pmc, by) if pmc else (None, None)
        res["kernel_roofline"] = dict(
            bound="hbm", kernel=f"{KERNELS[path]} (head_dim {shape.n_embed // shape.n_head}, "
                                f"{wgs} workgroups)",
            achieved=ach, peak=HBM_PEAK_GBS, unit="GB/s", frac=ach / HBM_PEAK_GBS, traffic=traffic,
            traffic_per_algorithmic_byte=ratio,
            traffic_source=os.path.relpath(pmc, ROOT) if pmc else None,
            bytes_per_launch=by, us_per_launch=us, steps_per_launch=float(np.mean([k for _, k, _ in chunks])),
            launches=len(chunks))
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


def prefill_bench(name, reps=20, warmup=30):
    """Best and median of `reps` timed prefills after `warmup` untimed ones (HIP events on the
    library stream around each call, prompt upload included); mfma_util is the best one's.  A
    c3 prefill keeps getting faster over its first ~20 back-to-back calls on a fresh box (1.22 ->
    1.07 ms, the device ramping up), so the warm-up is 30 calls and the timed ones are steady."""
    cfg = synth.CONFIGS[name]
    shape, B, P = cfg["shape"], cfg["batch"], cfg["prompt"]
    w = synth.make_weights(shape, 0)
    m = fh.NanoLLM(w, max_batch=B)
    prompts = synth.prompts_for(name)
    for _ in range(warmup):
        m.prefill(prompts)
    timer = fh.Timer()
    times = []
    for _ in range(reps):
        fh.synchronize()
        timer.start()
        m.prefill(prompts)
        times.append(timer.stop())
    best, med = min(times), float(np.median(times))
    flops = prefill_flops(shape, B, P)
    tf = flops / (best * 1e-3) / 1e12
    m.close()
    return dict(config=name, ms=best, ms_median=med, reps=reps, warmup=warmup, gflop=flops / 1e9, tflops=tf,
                mfma_util=tf / FP32_MFMA_PEAK_TF,
                mfma_util_median=flops / (med * 1e-3) / 1e12 / FP32_MFMA_PEAK_TF)


def window_flops(shape):
    """FLOPs of one full-window forward as the reference's greedy loop runs it for every
    generated token (NanoLLM.cpp:189-205 through Model::Run): all block_size rows through every
    block with full T x T attention per head, and lm_head on every row."""
    T, C, L, V = shape.block_size, shape.n_embed, shape.n_layer, shape.vocab
    return 2 * T * (L * 12 * C * C + V * C) + L * 2 * 2 * T * T * C


def reference_cpu_steps(w, prompt, steps):
    """Seconds per greedy step of the compiled reference's own MatrixCPU<float> path (FreeML's
    Model::Run through oracle/_ref/nanollm_dropin, the reference's ThreadPool of
    hardware_concurrency threads): two runs of 1 and 1 + steps steps, differenced so that
    process start, weight load and graph build cancel.  None when the driver is not built."""
    import subprocess
    import tempfile

    from freeml_amd import dropin

    if not os.path.exists(dropin.DROPIN):
        return None
    secs = []
    with tempfile.TemporaryDirectory() as d:
        for n in (1, 1 + steps):
            inp, out = os.path.join(d, f"in{n}.bin"), os.path.join(d, f"out{n}.bin")
            dropin.write_params(inp, w, prompt, n)
            t0 = time.perf_counter()
            subprocess.run([dropin.DROPIN, "cpu", inp, out], check=True, capture_output=True, timeout=600)
            secs.append(time.perf_counter() - t0)
    return (secs[1] - secs[0]) / steps


def cpu_baseline(budget_s=12.0, ref_steps=4):
    """The reference algorithm on the host cores, c2 batch 1: full-window recompute per
    generated token.  Timed twice on the same box: the compiled reference's MatrixCPU decode
    (the reported value when the driver is built) and the oracle's clean-room restatement
    ("port"), whose ratio calibrates the port; c3-c5 are extrapolated from the measured rate by
    their window FLOPs (hours of CPU time each if run)."""
    import oracle

    cfg = synth.CONFIGS["c2"]
    shape = cfg["shape"]
    w = synth.make_weights(shape, 0)
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    # The port's pool is sized to the box's CPU share, not to every core the host reports.
    threads = max(1, min(16, affinity))
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
    port = dict(value=k / secs, unit="tok/s", cores=threads, kind="port",
                sample=f"c2 batch 1: first {k} greedy steps, each a full 256-token window "
                       f"recompute (reference algorithm, clean-room C restatement), {secs:.1f} s")
    ref_s = reference_cpu_steps(w, prompt, ref_steps)
    if ref_s is not None and ref_s > 0:
        out = dict(value=1.0 / ref_s, unit="tok/s", cores=nproc, kind="reference",
                   sample=f"c2 batch 1: {ref_steps} greedy steps of FreeML's Model::Run on MatrixCPU<float> "
                          f"(oracle/_ref/nanollm_dropin cpu; ThreadPool of hardware_concurrency = {nproc} "
                          f"threads), {ref_s:.3f} s per full-window step",
                   port=port, port_over_reference=port["value"] * ref_s)
    else:
        out = dict(port)
    out["nproc"] = nproc
    out["affinity_cpus"] = affinity
    gflops = window_flops(shape) * out["value"] / 1e9
    out["gflop_per_s"] = gflops
    out["extrapolated"] = {
        n: {"tok_s": gflops * 1e9 / window_flops(synth.CONFIGS[n]["shape"]), "unit": "tok/s",
            "note": f"batch {synth.CONFIGS[n]['batch']}: each generated token costs one full window "
                    f"({window_flops(synth.CONFIGS[n]['shape']) / 1e9:.1f} GFLOP) at the measured "
                    f"{gflops:.1f} GFLOP/s; extrapolated, not run"}
        for n in ("c3", "c4", "c5")}
    return out


def train_flops(shape):
    """FLOPs of one training iteration as the reference computes it (full T x T attention per
    head, no causal skipping): forward products, then two products per forward product in the
    backward (input gradient and weight gradient; for attention, the four per-head products)."""
    T, C, L, V = shape.block_size, shape.n_embed, shape.n_layer, shape.vocab
    dense = 2 * T * C * (3 * C + C + 4 * C + 4 * C)
    attn = 2 * 2 * T * T * C
    fwd = L * (dense + attn) + 2 * T * C * V
    return 3 * fwd


def train_bench(iters=21, cpu_iters=3):
    import subprocess
    import tempfile

    from freeml_amd import dropin

    if not os.path.exists(dropin.DROPIN):
        return {"skipped": "oracle/_ref/nanollm_dropin not built (make -C freeml_amd/host)"}
    shape = synth.CONFIGS["c2"]["shape"]
    w = synth.make_weights(shape, 0)
    corpus = synth.prompt_tokens(shape.vocab, 4 * shape.block_size, 5)
    res = {}
    with tempfile.TemporaryDirectory() as d:
        inp = os.path.join(d, "in.bin")
        dropin.write_params(inp, w, corpus, 0)
        for backend, k in (("hip", iters), ("cpu", cpu_iters)):
            out = os.path.join(d, f"out_{backend}.bin")
            subprocess.run([dropin.DROPIN, backend, inp, out, "--train", str(k)], check=True,
                           capture_output=True, timeout=600)
            losses, secs, copies = dropin.read_train(out, k)
            res[backend] = (losses, float(np.mean(secs[1:])), copies)
    losses, s_hip, copies = res["hip"]
    s_cpu = res["cpu"][1]
    flops = train_flops(shape)
    return {"config": "c2 shape, batch 1, 256-token window; random corpus of 1024 ids; AdamW lr 1e-4",
            "ms_per_iteration": s_hip * 1e3, "tokens_per_s": shape.block_size / s_hip,
            "gflop_per_iteration": flops / 1e9, "tflops": flops / s_hip / 1e12,
            "mfma_frac": flops / s_hip / 1e12 / FP32_MFMA_PEAK_TF,
            "copies_per_iteration": {"d2h": int(copies[0]) / (iters - 1), "h2d": int(copies[1]) / (iters - 1)},
            "loss_first_last": [float(losses[0]), float(losses[-1])],
            "cpu_reference": {"ms_per_iteration": s_cpu * 1e3, "kind": "reference",
                              "sample": f"{cpu_iters} iterations of the same driver on MatrixCPU<float> "
                                        "(the reference's ThreadPool)"},
            "speedup_vs_cpu_reference": s_cpu / s_hip}


def timeline_bench(name="c3", steps=100):
    """Where a grouped decode step goes: the kernel's own per-workgroup timeline
    (FMLH_GROUPED_TRACE, freeml_amd/timeline.py) of one launch of `steps` steps, step 1, mean
    over workgroups and summed over layers (us)."""
    import tempfile

    from freeml_amd import timeline

    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], 0)
    prompts = synth.prompts_for(name)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "trace.bin")
        os.environ["FMLH_GROUPED_TRACE"] = path
        try:
            m = fh.NanoLLM(w, max_batch=cfg["batch"])
        finally:
            del os.environ["FMLH_GROUPED_TRACE"]
        if m.decode_path(cfg["batch"])[0] != "grouped":
            m.close()
            return {"skipped": f"{name} does not decode on the grouped kernel"}
        m.prefill(prompts)
        m.decode(steps)
        m.tokens()
        m.close()
        trace, n_layer = timeline.read(path)[-1]
    res = timeline.summarize(trace, n_layer)
    res["config"] = f"{name}, one launch of {steps} steps from position {cfg['prompt']}; step 1"
    res["points"] = {k: v for k, v in timeline.POINTS}
    return res


def wide_timeline_bench(names=("c4", "c5")):
    """Where a wide decode step goes: the kernel's own per-workgroup timeline (FMLH_WIDE_TRACE,
    freeml_amd/timeline.py) of decode step 1 of a 4-step launch at the prompt's end; per layer
    the median over workgroups of each interval (us), averaged over layers 1 .. L-1."""
    import tempfile

    from freeml_amd import timeline

    out = []
    for name in names:
        cfg = synth.CONFIGS[name]
        w = synth.make_weights(cfg["shape"], 0)
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "trace.bin")
            os.environ["FMLH_WIDE_TRACE"] = path
            try:
                m = fh.NanoLLM(w, max_batch=cfg["batch"])
            finally:
                del os.environ["FMLH_WIDE_TRACE"]
            if m.decode_path(cfg["batch"])[0] != "wide":
                m.close()
                out.append({"config": name, "skipped": "not on the wide kernel"})
                continue
            m.prefill(synth.prompts_for(name))
            m.decode(4)
            m.tokens()
            m.close()
            trace, n_layer, batch = timeline.read_wide(path)[-1]
        res = timeline.summarize_wide(trace, n_layer)
        res["config"] = f"{name}, batch {batch}, one launch of 4 steps from position {cfg['prompt']}; step 1"
        out.append(res)
    return {"runs": out, "points": {k: v for k, v in timeline.WIDE_POINTS + timeline.WIDE_LM}}


def relay_timeline_bench(cases=(("c2", 1), ("c3", 64))):
    """Where a relay decode step goes: the kernel's own per-role timeline (FMLH_RELAY_TRACE,
    freeml_amd/timeline.py) of steps 1-3 of an 8-step launch at the prompt's end: sequence 0's
    path through a layer (the last member of each team) and each team's waiting / working time
    per step."""
    import tempfile

    from freeml_amd import timeline

    out = []
    for name, batch in cases:
        cfg = synth.CONFIGS[name]
        w = synth.make_weights(cfg["shape"], 0)
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "trace.bin")
            os.environ["FMLH_RELAY_TRACE"] = path
            try:
                m = fh.NanoLLM(w, max_batch=batch)
            finally:
                del os.environ["FMLH_RELAY_TRACE"]
            if m.decode_path(batch)[0] != "relay":
                m.close()
                out.append({"config": name, "skipped": "not on the relay kernel"})
                continue
            m.prefill(synth.prompts_for(name)[:batch])
            m.decode(8)
            m.tokens()
            m.close()
            trace, meta = timeline.read_relay(path)[-1]
        res = timeline.summarize_relay(trace, meta)
        res["config"] = f"{name}, batch {batch}, one launch of 8 steps from position {cfg['prompt']}; steps 1-3"
        out.append(res)
    return {"runs": out, "chain": dict(timeline.RELAY_CHAIN)}


# Prefill projection shapes (M, N, K) and longer ones, B stored N x K as the projections keep it.
GEMM_SHAPES = [(4096, 1536, 384), (4096, 1152, 384), (4096, 384, 1536), (16384, 1536, 384),
               (65536, 1536, 384), (4096, 1536, 1536), (16384, 1536, 1536), (8192, 3072, 768)]


def gemm_bench(reps=20):
    """fp32 NT products through fmlh_gemm_ex (no epilogue) at GEMM_SHAPES: mean time of `reps`
    back-to-back calls after three warm-up calls, HIP events on the library stream."""
    r = np.random.default_rng(0)
    rows = []
    for M, N, K in GEMM_SHAPES:
        A = fh.DeviceArray.from_host(r.standard_normal((M, K), dtype=np.float32))
        B = fh.DeviceArray.from_host(r.standard_normal((N, K), dtype=np.float32))
        C = fh.DeviceArray((M, N))
        for _ in range(3):
            fh.gemm_ex(A.ptr, K, B.ptr, K, 1, C.ptr, N, M, N, K)
        fh.synchronize()
        timer = fh.Timer()
        timer.start()
        for _ in range(reps):
            fh.gemm_ex(A.ptr, K, B.ptr, K, 1, C.ptr, N, M, N, K)
        us = timer.stop() * 1e3 / reps
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        rows.append(dict(M=M, N=N, K=K, us=us, tflops=tf, mfma_util=tf / FP32_MFMA_PEAK_TF))
        log(f"  {M:6d} x {N:5d} x {K:5d}: {us:8.1f} us {tf:6.1f} TFLOP/s ({tf / FP32_MFMA_PEAK_TF * 100:.1f} %)")
        for d in (A, B, C):
            d.free()
    return rows


SCOPES = ["device", "xcd", "xcd/global sc0", "xcd/plain store", "xcd/sc1 store", "xcd/inv+load",
          "device/4 polls gap", "device/4 polls", "device/8 polls gap", "plain st/sc1 ld",
          "sc1 st/inv sc1+ld", "plain st/scalar ld", "sc1 st/scalar ld"]


def exchange_bench(rounds=2000):
    """Hand-off latency through exchange words (fmlh_probe_exchange): the per-hop cost that
    bounds the persistent decode kernels.  Groups are picked from the observed placement."""
    _, xcc = fh.probe_exchange(0, [0], rounds=1)
    by_xcd = {}
    for wg, x in enumerate(xcc.tolist()):
        by_xcd.setdefault(x, []).append(wg)
    xs = sorted(by_xcd)
    rows = []

    def run(label, scope, a, b=(), words=0):
        try:
            ns, _ = fh.probe_exchange(scope, a, b, words=words, rounds=rounds)
            rows.append(dict(case=label, scope=SCOPES[scope], na=len(a), nb=len(b),
                             words=words or max(len(a), len(b)), ns_per_hop=ns))
            log(f"  {label:58s} {SCOPES[scope]:16s} {ns:8.1f} ns/hop")
        except fh.FreeMLHipError as e:
            rows.append(dict(case=label, scope=SCOPES[scope], error=str(e)))
            log(f"  {label:58s} {SCOPES[scope]:16s} failed: {e}")

    x0 = by_xcd[xs[0]]
    x1 = by_xcd[xs[1]] if len(xs) > 1 else []
    # One word between two WGs of one XCD, every scope: device scope, the XCD-scope forms (words
    # meeting in the XCD's L2; a failure means the consumer never saw the word), and device
    # scope with pipelined polls.
    if len(x0) >= 2:
        for sc in range(len(SCOPES)):
            run("ping-pong, 1 word, same XCD", sc, x0[:1], x0[1:2])
    if x1:
        for sc in (0, 9, 10, 11, 12):
            run("ping-pong, 1 word, two XCDs", sc, x0[:1], x1[:1])
    for n in (8, 32, 64, 128, 256):
        if n <= len(xcc):
            for words in (n, 384, 1536):
                if words >= n:
                    run(f"all-to-all, WGs 0..{n - 1} (all XCDs), {words} words", 0, list(range(n)), words=words)
    if len(x0) >= 32:
        run("all-to-all, 32 WGs on one XCD, 384 words", 0, x0[:32], words=384)
    for sc in (6, 8):
        run("all-to-all, WGs 0..255 (all XCDs), 384 words", sc, list(range(len(xcc))), words=384)
    # Two disjoint groups (producers are not consumers): the hand-off between two roles of a
    # role-specialised pipeline.  Group A = WGs 0..na-1, B = the next nb (both spread over XCDs).
    for na, nb, words in ((1, 1, 384), (6, 6, 384), (8, 8, 384), (16, 16, 384), (32, 32, 384),
                          (64, 64, 384), (128, 128, 384), (32, 32, 1536), (6, 32, 2304),
                          (32, 6, 1152), (32, 32, 3072), (32, 32, 6144), (32, 32, 12288)):
        if na + nb <= len(xcc):
            run(f"{na} WGs -> {nb} WGs and back, {words} words", 0, list(range(na)),
                list(range(na, na + nb)), words=words)
    if x1 and len(x0) >= 32 and len(x1) >= 32:
        run("32 WGs of one XCD -> 32 of another and back, 384 words", 0, x0[:32], x1[:32], words=384)
        run("32 WGs of one XCD -> 32 of another and back, 3072 words", 0, x0[:32], x1[:32], words=3072)
        run("32 WGs of one XCD -> 32 of another and back, 384 words", 6, x0[:32], x1[:32], words=384)
    return {"placement": {str(k): len(v) for k, v in by_xcd.items()},
            "round_robin": all(x == xcc[i % len(xs)] for i, x in enumerate(xcc.tolist())) if xs else None,
            "rounds": rounds, "cases": rows}


def headline(args):
    """The c2 batch-1 decode leg: the line's metric, value and roofline."""
    shape = synth.CONFIGS["c2"]["shape"]
    log("c2 decode (batch 1)")
    m, prompts, res = decode_bench("c2", args.steps, args.warmup)
    log(f"c2: {res['tok_s']:.0f} tok/s, {res['ms_per_step'] * 1e3:.1f} us/step ({res['path']} path)")
    if "kernel_roofline" in res:
        roofline = res["kernel_roofline"]
        log(f"  {roofline['kernel']}: {roofline['us_per_launch']:.1f} us/launch, "
            f"{roofline['achieved']:.1f} GB/s algorithmic")
    else:
        dom, ops = dominant_op(m, prompts, shape)
        for r in ops:
            log(f"  op {r['op']:10s} {r['ms'] * 1e3:8.2f} us  {r['gbs']:8.1f} GB/s  x{r['per_step']}")
        roofline = {"bound": "hbm", "op": dom["op"], "achieved": dom["gbs"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": dom["gbs"] / HBM_PEAK_GBS, "traffic": None,
                    "bytes_per_launch": dom["bytes"], "us_per_launch": dom["ms"] * 1e3}
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
        "roofline": roofline,
        "step_roofline": res["step_roofline"],
    }
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=191)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-headline", action="store_true",
                    help="skip the c2 headline leg (profiling runs of the other legs: their processes "
                         "then make no cooperative launch); the line then carries no value")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the bs64 / large / prefill / cpu / train legs")
    ap.add_argument("--extra", default="bs64,large,prefill,cpu,train",
                    help="comma-separated legs after the c2 headline: bs64, large, prefill, cpu, "
                         "train; not default: exchange (the hand-off latency probe), timeline "
                         "(the grouped kernel's own per-hop timeline), wide_timeline (the wide "
                         "kernel's per-phase timeline), relay_timeline (the relay kernel's "
                         "per-role timeline) and gemm (the NT GEMM at the prefill "
                         "shapes); profiling runs select one")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run one plain copy of MIB MiB (fmlh_copy), the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the token loop shards over independent sequences, one process per GPU; this run "
              "measures one GPU's share)", file=sys.stderr)
        sys.exit(2)

    fh.init(0)
    arch, cus = fh.device_info()
    log(f"device {arch}, {cus} CUs")
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src, dst = fh.DeviceArray(n), fh.DeviceArray(n)
        fh.fill(src.ptr, 1.0, n)
        fh.copy(dst.ptr, src.ptr, n)
        fh.synchronize()
        src.free()
        dst.free()
        log(f"copy calibration: {args.copy_calibration} MiB read + {args.copy_calibration} MiB written")
    out = {"metric": METRIC, "value": None, "unit": "tok/s", "n_gpus": 1, "note": "--no-headline"}
    if not args.no_headline:
        out = headline(args)
    legs = set() if args.no_extra else {x.strip() for x in args.extra.split(",") if x.strip()}
    if "bs64" in legs:
        log("c3 decode (batch 64)")
        m64, p64, r64 = decode_bench("c3", 191, 10)
        out["bs64"] = {"tok_s": r64["tok_s"], "ms_per_step": r64["ms_per_step"], "path": r64["path"],
                       "workgroups": r64["workgroups"], "step_roofline": r64["step_roofline"]}
        if "kernel_roofline" in r64:
            kr = r64["kernel_roofline"]
            out["bs64"]["kernel_roofline"] = kr
            log(f"c3: {r64['tok_s']:.0f} tok/s, {r64['ms_per_step'] * 1e3:.1f} us/step ({kr['kernel']}, "
                f"{kr['us_per_launch']:.1f} us/launch)")
        else:
            dom64, _ = dominant_op(m64, p64, synth.CONFIGS["c3"]["shape"])
            log(f"c3: {r64['tok_s']:.0f} tok/s ({r64['path']} path), dominant op {dom64['op']}")
            out["bs64"]["dominant_op"] = {"op": dom64["op"], "us_per_launch": dom64["ms"] * 1e3,
                                          "bytes_per_launch": dom64["bytes"], "achieved": dom64["gbs"],
                                          "frac": dom64["gbs"] / HBM_PEAK_GBS}
        m64.close()
    if "large" in legs:
        out["decode_large"] = []
        for name in ("c4", "c5"):
            cfg = synth.CONFIGS[name]
            log(f"{name} decode (batch {cfg['batch']})")
            ml, _, rl = decode_bench(name, cfg["n_gen"] - 1, 8)
            ml.close()
            log(f"{name}: {rl['tok_s']:.0f} tok/s, {rl['ms_per_step'] * 1e3:.1f} us/step ({rl['path']} path)")
            out["decode_large"].append({"config": name, "batch": cfg["batch"], "prompt": cfg["prompt"],
                                        "steps": cfg["n_gen"] - 1, "tok_s": rl["tok_s"],
                                        "ms_per_step": rl["ms_per_step"], "path": rl["path"],
                                        "step_roofline": rl["step_roofline"]})
            if "kernel_roofline" in rl:
                out["decode_large"][-1]["kernel_roofline"] = rl["kernel_roofline"]
    if "prefill" in legs:
        pf = []
        for name in ("c3", "c4", "c5"):
            log(f"{name} prefill")
            pf.append(prefill_bench(name))
            log(f"  {pf[-1]['ms']:.3f} ms best, {pf[-1]['ms_median']:.3f} ms median of {pf[-1]['reps']}: "
                f"{pf[-1]['tflops']:.1f} TFLOP/s ({pf[-1]['mfma_util'] * 100:.1f} % of fp32 MFMA peak)")
        out["prefill"] = pf
    if "cpu" in legs:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline()
    if "train" in legs:
        log("c2 training iterations (Model::Run on MatrixHIP vs MatrixCPU)")
        out["train"] = train_bench()
        if "ms_per_iteration" in out["train"]:
            log(f"  {out['train']['ms_per_iteration']:.2f} ms/iteration, "
                f"{out['train']['speedup_vs_cpu_reference']:.0f}x the CPU reference")
    if "timeline" in legs:
        log("c3 grouped decode timeline (FMLH_GROUPED_TRACE)")
        out["timeline"] = timeline_bench()
    if "wide_timeline" in legs:
        log("c4 / c5 wide decode timeline (FMLH_WIDE_TRACE)")
        out["wide_timeline"] = wide_timeline_bench()
        for r in out["wide_timeline"]["runs"]:
            if "layer" in r:
                log(f"  {r['config']}: layer {r.get('layer_us', 0):.1f} us, step {r['step_us']:.1f} us; per layer "
                    + ", ".join(f"{k} {v:.2f}" for k, v in r["layer"].items()))
    if "relay_timeline" in legs:
        log("c2 / c3 relay decode timeline (FMLH_RELAY_TRACE)")
        out["relay_timeline"] = relay_timeline_bench()
        for r in out["relay_timeline"]["runs"]:
            if "chain" in r:
                log(f"  {r['config']}: step {r['step_us']:.1f} us; sequence 0 per layer "
                    + ", ".join(f"{k} {v:.2f}" for k, v in r["chain"].items()) + "; per step (wait / busy) "
                    + ", ".join(f"{k} {v['wait']:.1f} / {v['busy']:.1f}" for k, v in r["teams"].items()))
    if "exchange" in legs:
        log("exchange-word hand-off latency (fmlh_probe_exchange)")
        out["exchange"] = exchange_bench()
    if "gemm" in legs:
        log("NT GEMM shape sweep (fmlh_gemm_ex)")
        out["gemm"] = gemm_bench()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
