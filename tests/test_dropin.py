"""The drop-in boundary: FreeML's own Model / Datablob / MatrixManager / Layer code running
NanoLLM on MatrixHIP<float> (freeml_amd/host/MatrixLibrary/GPU/HIP) via Model::Run.

oracle/_ref/nanollm_dropin is built in the development container from the reference headers
plus this backend's headers (freeml_amd/host/Makefile) and travels with the tree.  Its `cpu`
mode runs the same graph on the reference MatrixCPU<float> backend, which pins the driver's
graph construction bit-for-bit against the reference's NanoLLM.cpp fixtures.
"""
import os
import subprocess
import tempfile

import numpy as np
import pytest

from freeml_amd import synth
from freeml_amd.dropin import DROPIN, read_generate, write_params

pytestmark = pytest.mark.skipif(not os.path.exists(DROPIN), reason="drop-in driver not built")


def run_dropin(backend, w, prompt, n_gen):
    with tempfile.TemporaryDirectory() as d:
        inp, out = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        write_params(inp, w, prompt, n_gen)
        print(f"nanollm_dropin {backend}: V={w.shape.vocab} T={w.shape.block_size} n_gen={n_gen}", flush=True)
        subprocess.run([DROPIN, backend, inp, out], check=True, timeout=600)
        toks, logits, copies = read_generate(out, n_gen, w.shape.vocab)
    return toks, logits, copies


def test_dropin_cpu_graph_equals_reference_fixture(golden):
    """The driver's graph on MatrixCPU<float> reproduces NanoLLM.cpp's graph bit-for-bit."""
    g = golden("c1")
    w = synth.make_weights(synth.CONFIGS["c1"]["shape"], 0)
    toks, logits, _ = run_dropin("cpu", w, g["prompts"][0], 48)
    np.testing.assert_array_equal(toks, g["tokens"][0])
    np.testing.assert_array_equal(logits, g["logits"][0])


@pytest.mark.gpu
@pytest.mark.parametrize("name,n_gen", [("c1", 48), ("c2", 24)])
def test_dropin_model_run_on_matrixhip(name, n_gen, golden):
    """Model::Run on MatrixHIP<float>: per-step logits within 1e-4 (normwise) of the reference,
    identical greedy tokens, and no host round trip inside the forward beyond the input window
    and the logits read."""
    g = golden(name)
    w = synth.make_weights(synth.CONFIGS[name]["shape"], 0)
    toks, logits, copies = run_dropin("hip", w, g["prompts"][0], n_gen)
    ref = g["logits"][0][:n_gen].astype(np.float64)
    err = np.max(np.abs(logits - ref), axis=1) / np.max(np.abs(ref), axis=1)
    assert err.max() <= 1e-4, err.max()
    np.testing.assert_array_equal(toks, g["tokens"][0][:n_gen])
    assert copies.tolist() == [n_gen - 1, n_gen - 1], copies


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c1", "c2"])
def test_token_loop_on_model_blobs(name, golden):
    """NanoLLMTokenLoop over a Model<float, MatrixHIP<float>> built with the reference API:
    the KV-cache loop reads the blobs' device matrices and reproduces the reference steps."""
    g = golden(name)
    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], 0)
    toks, logits, _ = run_dropin("hiploop", w, g["prompts"][0], cfg["n_gen"])
    ref = g["logits"][0].astype(np.float64)
    err = np.max(np.abs(logits - ref), axis=1) / np.max(np.abs(ref), axis=1)
    assert err.max() <= 1e-4, err.max()
    np.testing.assert_array_equal(toks, g["tokens"][0])


@pytest.mark.gpu
def test_token_loop_in_a_second_process(golden):
    """A process that decodes while another one holds a NanoLLM whose persistent (cooperative)
    decode kernel has run: the device's cooperative-launch resource belongs to one process at
    a time, so the second process's decode must fall back to the graph path, not fail."""
    import freeml_amd as fh

    fh.init(0)
    g = golden("c2")
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 0)
    m = fh.NanoLLM(w, max_batch=1)
    try:
        assert m.decode_path(1)[0] in ("relay", "persistent")  # both cooperative launches
        m.generate(g["prompts"][:1], 4)
        toks, logits, _ = run_dropin("hiploop", w, g["prompts"][0], cfg["n_gen"])
    finally:
        m.close()
    ref = g["logits"][0].astype(np.float64)
    err = np.max(np.abs(logits - ref), axis=1) / np.max(np.abs(ref), axis=1)
    assert err.max() <= 1e-4, err.max()
    np.testing.assert_array_equal(toks, g["tokens"][0])
