"""FreeML checkpoints (Model::Save / Model::Load through Loading/SaveLoader.h) with this backend.

Checkpoints are written by the drop-in driver (oracle/_ref/nanollm_dropin --save), i.e. by the
reference's own Model::Save on MatrixCPU<float> or MatrixHIP<float>, so the files are the
reference's format by construction.  The CPU tests pin ``freeml_amd.checkpoint`` against them:
every parameter read back equals the synthetic weights written, bit for bit, and the saved
lm_head output holds the reference's logits.  The GPU tests decode loaded checkpoints (the
reference's Model::Load into MatrixHIP, then NanoLLMTokenLoop; and the Python reader into
fmlh_nanollm) against the golden fixtures, and save from MatrixHIP after Model::Run, which
reads every device-written matrix back through GetRawData.
"""
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import freeml_amd as fh
from freeml_amd import checkpoint, synth
from freeml_amd.dropin import DROPIN, write_params

needs_driver = pytest.mark.skipif(not os.path.exists(DROPIN), reason="drop-in driver not built")
MODEL = "NanoLLM_dropin"


def zero_weights(shape):
    """Weights of the right shape, all zero: with --load the driver must not use them."""
    w = synth.make_weights(shape, 0)
    for a in w.tensors():
        a[...] = 0
    return w


def driver(backend, w, prompt, n_gen, tmp, *extra, check=True):
    inp, out = os.path.join(tmp, "in.bin"), os.path.join(tmp, "out.bin")
    write_params(inp, w, prompt, n_gen)
    print(f"nanollm_dropin {backend} {' '.join(extra)}: V={w.shape.vocab} n_gen={n_gen}", flush=True)
    r = subprocess.run([DROPIN, backend, inp, out, *extra], capture_output=True, text=True, timeout=600)
    if check:
        assert r.returncode == 0, r.stderr
        raw = open(out, "rb").read()
        V = w.shape.vocab
        toks = np.frombuffer(raw, np.int32, count=n_gen)
        logits = np.frombuffer(raw, np.float32, count=n_gen * V, offset=4 * n_gen).reshape(n_gen, V)
        return toks, logits
    return r


def save_cpu(name, golden, tmp, n_gen=1):
    """Checkpoint of config `name` written by Model::Save on MatrixCPU after n_gen steps."""
    g = golden(name)
    w = synth.make_weights(synth.CONFIGS[name]["shape"], 0)
    d = os.path.join(tmp, "ck")
    driver("cpu", w, g["prompts"][0], n_gen, tmp, "--save", d)
    return os.path.join(d, MODEL), w, g


def rel_err_rows(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.max(np.abs(got - ref), axis=1) / np.max(np.abs(ref), axis=1)


@needs_driver
@pytest.mark.parametrize("name", ["c1", "c2"])
def test_reader_recovers_saved_parameters(name, golden, tmp_path):
    """load_nanollm reads back exactly the parameters Model::Save wrote (tied and untied
    lm_head), and the saved lm_head output holds the reference's logits for the step run."""
    path, w, g = save_cpu(name, golden, str(tmp_path))
    got = checkpoint.load_nanollm(path)
    assert got.shape == w.shape
    assert got.checksum() == w.checksum()
    for a, b in zip(got.tensors(), w.tensors()):
        np.testing.assert_array_equal(a, b)
    assert (got.lm_head is got.tok_emb) == w.shape.tied
    ck = checkpoint.read_checkpoint(path)
    assert ck.input_dims == (1, w.shape.block_size, 1)
    assert ck.optimiser is not None and ck.loss is not None
    # Output_0 of lm_head: {V, T} logits of the padded window; row P-1 is step 0's.
    out = ck.layer("lm_head").matrix("Output_0").array()[0]
    P = g["prompts"][0].size
    np.testing.assert_array_equal(out[P - 1], g["logits"][0][0])


@needs_driver
def test_reference_reload_cannot_run_graph(golden, tmp_path):
    """The reference's Model::Load rebuilds lm_head without TransposedWeights, so Model::Run
    on a reloaded NanoLLM stops; the driver reports it rather than running a wrong product."""
    path, w, g = save_cpu("c1", golden, str(tmp_path))
    r = driver("cpu", zero_weights(w.shape), g["prompts"][0], 1, str(tmp_path), "--load",
               os.path.dirname(path), check=False)
    assert r.returncode == 10, (r.returncode, r.stderr)
    assert "TransposedWeights=false" in r.stderr


def test_reader_rejects_damaged_checkpoints(tmp_path):
    with pytest.raises(checkpoint.CheckpointError, match="model.guide"):
        checkpoint.load_nanollm(str(tmp_path))


@needs_driver
def test_reader_rejects_truncated_and_biased(golden, tmp_path):
    path, w, _ = save_cpu("c1", golden, str(tmp_path))
    ck = checkpoint.read_checkpoint(path)
    # A data file shorter than DIMX*DIMY*DIMZ floats.
    qkv = ck.layer("block_0").sub("AttentionLayerData").sub("CSA_AttentionLayer")
    data = qkv.matrix("Dense_Weights").data_file
    keep = open(data, "rb").read()
    open(data, "wb").write(keep[:-4])
    with pytest.raises(checkpoint.CheckpointError, match="floats"):
        checkpoint.load_nanollm(path)
    open(data, "wb").write(keep)
    # A Dense_Bias (NanoLLM use_bias=true) is refused: the device graph has no dense bias.
    fc = ck.layer("block_1").sub("DenseFCData")
    w_file = os.path.basename(fc.matrix("Dense_Weights").path)
    with open(fc.path, "a") as f:
        f.write(f"NAME Dense_Bias\nDATA {w_file}\nTYPE MATRIX\n;\n")
    with pytest.raises(checkpoint.CheckpointError, match="Dense_Bias"):
        checkpoint.load_nanollm(path)


@pytest.mark.gpu
@needs_driver
@pytest.mark.parametrize("name", ["c1", "c2"])
def test_token_loop_decodes_reference_loaded_checkpoint(name, golden, tmp_path):
    """Model::Load into MatrixHIP (SaveLoader writes each matrix through DataWrite), then the
    KV-cache token loop over the loaded blobs: the golden steps, with in.bin's weights zero."""
    path, w, g = save_cpu(name, golden, str(tmp_path))
    n_gen = synth.CONFIGS[name]["n_gen"]
    toks, logits = driver("hiploop", zero_weights(w.shape), g["prompts"][0], n_gen, str(tmp_path),
                          "--load", os.path.dirname(path))
    assert rel_err_rows(logits, g["logits"][0]).max() <= 1e-4
    np.testing.assert_array_equal(toks, g["tokens"][0])


@pytest.mark.gpu
@needs_driver
def test_python_nanollm_from_checkpoint(golden, tmp_path):
    fh.init(0)
    path, w, g = save_cpu("c2", golden, str(tmp_path))
    m = fh.NanoLLM.from_checkpoint(path)
    try:
        toks, logits = m.generate(g["prompts"][:1], synth.CONFIGS["c2"]["n_gen"], with_logits=True)
    finally:
        m.close()
    assert rel_err_rows(logits[0], g["logits"][0]).max() <= 1e-4
    np.testing.assert_array_equal(toks[0], g["tokens"][0])


# Matrices the forward writes: layer inputs/outputs, LayerNorm's XHat and the attention
# layer's per-step scratch.  Error and gradient buffers are never written by inference and
# hold whatever the allocator returned (MatrixCPU does not clear new memory), so they are
# not compared.  Neither are the per-head attention dropout sublayers' buffers: at dropout 0
# they are an identity copy of Scratch_AttHead_h, which the MatrixHIP attention layer skips.
FORWARD = re.compile(r"/(Output_\d+|Input_\d+|XHat|Scratch_[QKVY]|Scratch_AttHead_\d+)$")
SKIPPED = re.compile(r"CSA_AttentionDropout_\d+:/")


def _walk(rec, prefix=""):
    for k, m in rec.matrices.items():
        yield f"{prefix}{rec.name}/{k}", m
    for k, sub in rec.sublayers.items():
        yield from _walk(sub, f"{prefix}{rec.name}/{k}:")


@pytest.mark.gpu
@needs_driver
def test_save_from_matrixhip_after_model_run(golden, tmp_path):
    """Model::Save of a MatrixHIP model after Model::Run: every matrix goes through GetRawData,
    so the device-written activations are read back.  Against Model::Save of the MatrixCPU
    model after the same steps: parameters bit-identical, every matrix the forward writes
    within its 1e-4 tolerance (normwise per matrix)."""
    g = golden("c1")
    w = synth.make_weights(synth.CONFIGS["c1"]["shape"], 0)
    n_gen = 8
    cpu_dir, hip_dir = str(tmp_path / "cpu"), str(tmp_path / "hip")
    os.makedirs(cpu_dir)
    os.makedirs(hip_dir)
    driver("cpu", w, g["prompts"][0], n_gen, cpu_dir, "--save", os.path.join(cpu_dir, "ck"))
    toks, _ = driver("hip", w, g["prompts"][0], n_gen, hip_dir, "--save", os.path.join(hip_dir, "ck"))
    np.testing.assert_array_equal(toks, g["tokens"][0][:n_gen])
    a = checkpoint.read_checkpoint(os.path.join(cpu_dir, "ck", MODEL))
    b = checkpoint.read_checkpoint(os.path.join(hip_dir, "ck", MODEL))
    assert checkpoint.load_nanollm(b.path).checksum() == w.checksum()
    ma = {k: m for rec in a.layers for k, m in _walk(rec) if not SKIPPED.search(k)}
    mb = {k: m for rec in b.layers for k, m in _walk(rec) if not SKIPPED.search(k)}
    assert ma.keys() == mb.keys()
    checked = 0
    for key, m in ma.items():
        if not FORWARD.search(key):
            continue
        x, y = m.array(), mb[key].array()
        assert x.shape == y.shape, key
        scale = np.max(np.abs(x))
        if scale == 0:
            assert np.max(np.abs(y)) == 0, key
            continue
        err = np.max(np.abs(x.astype(np.float64) - y)) / scale
        assert err <= 1e-4, (key, err)
        checked += 1
    assert checked >= 70, checked
    out = b.layer("lm_head").matrix("Output_0").array()[0]
    P = g["prompts"][0].size
    ref = g["logits"][0][n_gen - 1]
    assert np.max(np.abs(out[P + n_gen - 2] - ref)) / np.max(np.abs(ref)) <= 1e-4
    shutil.rmtree(str(tmp_path), ignore_errors=True)
