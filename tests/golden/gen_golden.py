"""Writes tests/golden/<config>.npz from the compiled FreeML reference (oracle/_ref).

Run in the development container, where /root/reference exists:

    make -C oracle ref && python tests/golden/gen_golden.py c1 c2 c3 c4 c5

Each fixture holds inputs (seed, prompt rows) and the reference's outputs for them:

* c1, c2 -- every greedy step of sequence 0: tokens and the full logits row of each step,
  from ``ref_greedy`` (full-window Model::Run per step, NanoLLM.cpp semantics).
* c3     -- sequences 0 and 63 of the batch-64 config, every step (the reference has batch 1
  only, so batched configs are B independent loops).
* c4, c5 -- sequence 0: the token history comes from the bit-exact cached oracle (the
  reference needs minutes per full window at these sizes), then the reference's own
  ``Model::Run`` is evaluated on the windows of the first and last step; the fixture keeps
  those logits rows and the reference-checked history.

Fixture arrays are plain numeric/unicode (``np.load(..., allow_pickle=False)``).
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from freeml_amd import synth  # noqa: E402
import oracle  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def _save(name: str, **arrays) -> None:
    path = os.path.join(OUT, f"{name}.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)", flush=True)


def full_loop(name: str, rows) -> None:
    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], seed=0)
    prompts = synth.prompts_for(name)
    ref = oracle.RefModel(w)
    toks, logits = [], []
    for b in rows:
        t0 = time.time()
        t, l = ref.greedy(prompts[b], cfg["n_gen"])
        print(f"{name} row {b}: {time.time() - t0:.1f}s", flush=True)
        toks.append(t)
        logits.append(l)
    _save(name, rows=np.array(rows, dtype=np.int32), prompts=prompts[list(rows)],
          tokens=np.stack(toks), logits=np.stack(logits),
          weights_seed=np.array(0), weights_checksum=np.array(w.checksum()),
          ref_threads=np.array(oracle.RefModel.threads()))


def sampled(name: str) -> None:
    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], seed=0)
    prompt = synth.prompts_for(name)[0]
    T, V, P, n_gen = cfg["shape"].block_size, cfg["shape"].vocab, cfg["prompt"], cfg["n_gen"]
    t0 = time.time()
    orc = oracle.OracleModel(w, nthreads=os.cpu_count() or 1)
    toks, orc_logits = orc.greedy(prompt, n_gen, cached=True)
    print(f"{name} oracle cached loop: {time.time() - t0:.1f}s", flush=True)
    ref = oracle.RefModel(w)
    steps = [0, n_gen - 1]
    rows = []
    for s in steps:
        hist = np.concatenate([prompt, toks[:s]]).astype(np.int32)
        window = np.zeros(T, dtype=np.int32)
        window[: hist.size] = hist
        t0 = time.time()
        full = ref.forward_window(window)
        row = full[hist.size - 1].copy()
        print(f"{name} step {s}: ref window {time.time() - t0:.1f}s, "
              f"oracle==ref {np.array_equal(row, orc_logits[s])}", flush=True)
        if int(np.argmax(row == row.max())) != int(toks[s]):
            raise SystemExit(f"{name} step {s}: reference argmax differs from oracle history")
        rows.append(row)
    _save(name, rows=np.array([0], dtype=np.int32), prompts=prompt[None, :],
          tokens=toks[None, :], steps=np.array(steps, dtype=np.int32),
          logits=np.stack(rows)[None, :, :],
          weights_seed=np.array(0), weights_checksum=np.array(w.checksum()),
          ref_threads=np.array(oracle.RefModel.threads()))


def main(argv) -> None:
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libfreeml_ref.so missing: run `make -C oracle ref`")
    for name in argv or ["c1", "c2"]:
        if name in ("c1", "c2"):
            full_loop(name, [0])
        elif name == "c3":
            full_loop(name, [0, 63])
        else:
            sampled(name)


if __name__ == "__main__":
    main(sys.argv[1:])
