"""Files of the drop-in driver (freeml_amd/host/nanollm_dropin.cpp): FreeML's own Model /
Layer / loss / optimiser code compiled against the reference headers with MatrixHIP<float>
plugged in, built by freeml_amd/host/Makefile into oracle/_ref/nanollm_dropin (it contains
reference code, so it is not committed).

``write_params`` writes its in.bin; ``read_generate`` and ``read_train`` parse its out.bin
(formats in the driver's header comment).
"""
from __future__ import annotations

import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "oracle", "_ref", "nanollm_dropin")


def write_params(path, w, prompt, n_gen):
    """in.bin: int32[9] header, the parameters in FreeML's storage layout, the prompt ids."""
    s = w.shape
    with open(path, "wb") as f:
        np.array([s.vocab, s.block_size, s.n_embed, s.n_head, s.n_layer, int(s.tied),
                  prompt.size, n_gen, 0], np.int32).tofile(f)
        w.tok_emb.tofile(f)
        w.pos_emb.tofile(f)
        for lw in w.layers:
            for a in (lw.w_qkv, lw.w_proj, lw.w_fc, lw.w_proj2, lw.ln0_g, lw.ln1_g):
                a.tofile(f)
        w.lnf_g.tofile(f)
        if not s.tied:
            w.lm_head.tofile(f)
        np.asarray(prompt, np.int32).tofile(f)


def read_generate(path, n_gen, vocab):
    """(tokens, logits, {d2h, h2d} copies) of a generation run."""
    raw = open(path, "rb").read()
    toks = np.frombuffer(raw, np.int32, count=n_gen)
    logits = np.frombuffer(raw, np.float32, count=n_gen * vocab, offset=4 * n_gen).reshape(n_gen, vocab)
    copies = np.frombuffer(raw, np.uint64, count=2, offset=4 * n_gen + 4 * n_gen * vocab)
    return toks, logits, copies


def read_train(path, iters):
    """(losses, seconds per iteration, {d2h, h2d} copies of iterations 1..K-1) of --train K."""
    raw = open(path, "rb").read()
    losses = np.frombuffer(raw, np.float64, count=iters)
    secs = np.frombuffer(raw, np.float64, count=iters, offset=8 * iters)
    copies = np.frombuffer(raw, np.uint64, count=2, offset=16 * iters)
    return losses, secs, copies
