"""GPU parity of the NanoLLM token loop (fmlh_nanollm_*) against the reference.

Bar (north_star): at every decode step the logits match the reference MatrixCPU path within
a relative error of 1e-4 -- measured normwise per step, max|gpu - ref| / max|ref| -- and the
greedy tokens match exactly.  References: the compiled-reference fixtures in tests/golden/
(every step for c1/c2, rows 0 and 63 of c3, first/last step of c4/c5) and the bit-exact CPU
oracle for what the fixtures do not hold.
"""
import contextlib
import os

import numpy as np
import pytest

import freeml_amd as fh
import oracle
from freeml_amd import synth

pytestmark = pytest.mark.gpu

REL_TOL = 1e-4


@contextlib.contextmanager
def env(**kv):
    """Environment switches the library reads at engine creation or at each decode call."""
    old = {k: os.environ.get(k) for k in kv}
    os.environ.update(kv)
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.fixture(scope="module", autouse=True)
def device():
    fh.init(0)


def rel_err_rows(got, ref):
    got = np.asarray(got, np.float64).reshape(-1, ref.shape[-1])
    ref = np.asarray(ref, np.float64).reshape(-1, ref.shape[-1])
    return np.max(np.abs(got - ref), axis=1) / np.max(np.abs(ref), axis=1)


def margins(logits):
    s = np.sort(logits.reshape(-1, logits.shape[-1]), axis=1)
    return s[:, -1] - s[:, -2]


_models = {}


def model_for(name, max_batch=None):
    cfg = synth.CONFIGS[name]
    key = (name, max_batch or cfg["batch"])
    if key not in _models:
        w = synth.make_weights(cfg["shape"], 0)
        _models[key] = (fh.NanoLLM(w, max_batch=key[1]), w)
    return _models[key]


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_every_step_matches_reference_fixture(name, golden):
    g = golden(name)
    cfg = synth.CONFIGS[name]
    print(f"{name}: generate {cfg['n_gen']} tokens", flush=True)
    m, w = model_for(name)
    assert w.checksum() == str(g["weights_checksum"])
    toks, logits = m.generate(g["prompts"], cfg["n_gen"], with_logits=True)
    err = rel_err_rows(logits[0], g["logits"][0])
    print(f"{name}: max rel err {err.max():.2e}, min ref top-2 margin {margins(g['logits'][0]).min():.2e}")
    assert err.max() <= REL_TOL
    np.testing.assert_array_equal(toks[0], g["tokens"][0])


def test_batch64_rows_match_fixture_and_oracle(golden):
    g = golden("c3")
    cfg = synth.CONFIGS["c3"]
    m, w = model_for("c3")
    prompts = synth.prompts_for("c3")
    print("c3: batch 64 generate", flush=True)
    toks, logits = m.generate(prompts, cfg["n_gen"], with_logits=True)
    for i, b in enumerate(g["rows"]):
        assert rel_err_rows(logits[b], g["logits"][i]).max() <= REL_TOL
        np.testing.assert_array_equal(toks[b], g["tokens"][i])
    om = oracle.OracleModel(w, nthreads=8)
    for b in (9, 31, 50):
        t_ref, l_ref = om.greedy(prompts[b], cfg["n_gen"], cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"row {b}"
        np.testing.assert_array_equal(toks[b], t_ref)


def test_batch_rows_are_independent():
    """A sequence decoded alone gives the tokens it gets inside a batch of 64."""
    cfg = synth.CONFIGS["c3"]
    m64, w = model_for("c3")
    prompts = synth.prompts_for("c3")
    toks64, _ = m64.generate(prompts, 40)
    m1, _ = model_for("c3", max_batch=1)
    for b in (0, 17, 63):
        t1, _ = m1.generate(prompts[b:b + 1], 40)
        np.testing.assert_array_equal(t1[0], toks64[b])


def test_fused_prefill_parts_and_unfused_path(golden):
    """c3's prefill (fused: residual projections as two K halves whose reduction applies the
    next LayerNorm) in 1, 2 and 3 stream parts: every row's arithmetic is the same whatever the
    part, so the logits are bit-identical; the unfused path (separate LayerNorms, other split
    orders) agrees within tolerance, and both match the fixture rows."""
    g = golden("c3")
    m, _ = model_for("c3")
    prompts = synth.prompts_for("c3")
    got = {}
    for parts in ("1", "2", "3"):
        with env(FMLH_PREFILL_STREAMS=parts):
            m.prefill(prompts)
            got[parts] = m.logits()
    np.testing.assert_array_equal(got["1"], got["2"])
    np.testing.assert_array_equal(got["1"], got["3"])
    with env(FMLH_PREFILL_FUSED="0"):
        m.prefill(prompts)
        unfused = m.logits()
    assert rel_err_rows(got["2"], unfused).max() <= REL_TOL
    for i, b in enumerate(g["rows"]):
        assert rel_err_rows(got["2"][b], g["logits"][i][0]).max() <= REL_TOL


@pytest.mark.parametrize("C,H,B", [(256, 8, 16), (64, 4, 48)])
def test_prefill_kv_cache_epilogue_head_dims_below_64(C, H, B):
    """A prefill large enough for the NT GEMM (B x 64 rows; QKV grids of 384 and 288 64 x 64
    tiles) writes the keys and values straight into the caches through LDS-staged 16-byte
    stores, a 64-wide tile then spanning 64 / head_dim heads (head_dim 32 and 16 here).  The
    first four tokens and logits of every tenth sequence against the oracle: the decode steps
    read the cache rows the prefill wrote."""
    shape = synth.NanoLLMShape(65, 128, C, H, 2)
    w = synth.make_weights(shape, 5)
    prompts = np.stack([synth.prompt_tokens(65, 64, 100 + b) for b in range(B)])
    m = fh.NanoLLM(w, max_batch=B)
    try:
        toks, logits = m.generate(prompts, 4, with_logits=True)
    finally:
        m.close()
    om = oracle.OracleModel(w, nthreads=8)
    for b in range(0, B, 10):
        t_ref, l_ref = om.greedy(prompts[b], 4, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"sequence {b}"
        np.testing.assert_array_equal(toks[b], t_ref)


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_large_configs_first_and_last_step(name, golden):
    g = golden(name)
    cfg = synth.CONFIGS[name]
    m, w = model_for(name)
    assert w.checksum() == str(g["weights_checksum"])
    prompts = synth.prompts_for(name)
    np.testing.assert_array_equal(prompts[0], g["prompts"][0])
    print(f"{name}: prefill batch {prompts.shape}", flush=True)
    m.prefill(prompts)
    first = m.logits()
    assert rel_err_rows(first[0], g["logits"][0][0]).max() <= REL_TOL
    m.decode(cfg["n_gen"] - 2)
    m.decode(1)
    last = m.logits()
    assert rel_err_rows(last[0], g["logits"][0][1]).max() <= REL_TOL
    toks = m.tokens()
    assert toks.shape == (cfg["batch"], cfg["n_gen"])
    np.testing.assert_array_equal(toks[0], g["tokens"][0])
    print(f"{name}: tokens of row 0 match over {cfg['n_gen']} steps", flush=True)


def test_full_window_matches_oracle():
    for name in ("c1", "c2"):
        m, w = model_for(name)
        om = oracle.OracleModel(w, nthreads=8)
        ids = synth.prompt_tokens(w.shape.vocab, w.shape.block_size, 1234)
        got = m.forward_window(ids)[0]
        ref = om.forward_window(ids)
        assert rel_err_rows(got, ref).max() <= REL_TOL


def test_cached_decode_equals_window_recompute():
    """KV-cache step s logits == the full-window forward of the same history at row len-1."""
    m, w = model_for("c2")
    p = synth.prompt_tokens(65, 64, 77)
    toks, logits = m.generate(p, 30, with_logits=True)
    hist = np.concatenate([p, toks[0]])
    for s in (0, 7, 29):
        window = np.zeros(256, np.int32)
        L = 64 + s
        window[:L] = hist[:L]
        full = m.forward_window(window)[0]
        assert rel_err_rows(logits[0, s], full[L - 1]).max() <= REL_TOL


def test_deterministic_and_graph_equals_eager():
    cfg = synth.CONFIGS["c2"]
    m, w = model_for("c2")
    p = synth.prompts_for("c2")
    t1, l1 = m.generate(p, 50, with_logits=True)
    t2, l2 = m.generate(p, 50, with_logits=True)
    np.testing.assert_array_equal(t1, t2)
    np.testing.assert_array_equal(l1, l2)
    os.environ["FMLH_NO_GRAPH"] = "1"
    try:
        eager = fh.NanoLLM(w, max_batch=1)
    finally:
        del os.environ["FMLH_NO_GRAPH"]
    t3, l3 = eager.generate(p, 50, with_logits=True)
    eager.close()
    np.testing.assert_array_equal(t1, t3)
    np.testing.assert_array_equal(l1, l3)


def test_incremental_api_equals_generate():
    m, w = model_for("c2")
    p = synth.prompts_for("c2")
    t_all, _ = m.generate(p, 20)
    m.prefill(p)
    m.decode(5)
    m.decode(14)
    assert m.status() == (20, 1)
    np.testing.assert_array_equal(m.tokens(), t_all)
    np.testing.assert_array_equal(m.tokens(3, 4), t_all[:, 3:7])


def test_error_paths():
    m, w = model_for("c1")
    with pytest.raises(fh.FreeMLHipError):
        m.prefill(np.array([[1, 2, 65]], np.int32))  # id outside the vocabulary
    m.prefill(np.arange(16, dtype=np.int32)[None, :] % 65)
    with pytest.raises(fh.FreeMLHipError):
        m.decode(64)  # would pass block_size
    with pytest.raises(fh.FreeMLHipError):
        m.tokens(0, 5)  # only 1 generated
    with pytest.raises(fh.FreeMLHipError):
        m.generate(np.zeros((2, 4), np.int32), 3)  # batch above max_batch


@pytest.mark.parametrize("name,batch", [("c1", 1), ("c2", 1), ("c2", 3), ("c2", 8), ("c1", 5),
                                        ("c1", 12), ("c2", 12), ("c2", 16)])
def test_persistent_decode_matches_multikernel_path(name, batch):
    """The persistent decode kernel (default for 2-8 sequences, and for one where the relay kernel
    does not apply -- FMLH_RELAY=0 keeps it for c2; above 8 the grouped kernel is the default and
    FMLH_GROUPED=0 keeps the persistent kernel's two groups of up to 8) and the
    multi-kernel graph path (FMLH_DECODE=graph) give the same tokens and logits to fp32
    reassociation."""
    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], 0)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, cfg["prompt"], 1 + b) for b in range(batch)])
    n = min(cfg["n_gen"], 40)
    os.environ["FMLH_DECODE"] = "graph"
    try:
        ref = fh.NanoLLM(w, max_batch=batch)
    finally:
        del os.environ["FMLH_DECODE"]
    assert ref.decode_path(batch) == ("graph", 0)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    os.environ["FMLH_GROUPED"] = "0"
    os.environ["FMLH_RELAY"] = "0"
    try:
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "persistent"
        print(f"{name} batch {batch}: persistent decode of {n} steps", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    finally:
        del os.environ["FMLH_GROUPED"]
        del os.environ["FMLH_RELAY"]
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5


@pytest.mark.parametrize("kernel", ["default", "mfma16", "mfma32"])
@pytest.mark.parametrize("name,length,batch", [("c2", 256, 1), ("c2", 100, 1), ("c2", 1, 1),
                                               ("c2", 129, 2), ("c2", 64, 3), ("c5", 700, 1),
                                               ("c5", 1920, 2)])
def test_prefill_attention_on_matrix_cores_matches_per_lane_kernel(kernel, name, length, batch):
    """The MFMA prefill attention kernels for head_dim 64 (default: 32x32x2 MFMA with 128
    queries per work-group from 256 rows on, else 16x16x4 with 64; FMLH_ATTN_PREFILL=mfma16 /
    mfma32: one of them at every length) and the per-lane kernel
    (FMLH_ATTN_PREFILL=simt) give the same prefill logits (every sequence's last row) to fp32
    reassociation, for full and partial query blocks, one key tile, and several sequences."""
    print(f"prefill attention {kernel} {name} length {length} batch {batch}", flush=True)
    m, w = model_for(name, max_batch=4)
    ids = np.stack([synth.prompt_tokens(w.shape.vocab, length, 4242 + k) for k in range(batch)])

    def run(mode):
        if mode == "default":
            os.environ.pop("FMLH_ATTN_PREFILL", None)
        else:
            os.environ["FMLH_ATTN_PREFILL"] = mode
        try:
            m.prefill(ids)
            return m.logits()
        finally:
            os.environ.pop("FMLH_ATTN_PREFILL", None)

    fast = run(kernel)
    ref = run("simt")
    assert fast.shape == (batch, w.shape.vocab)
    assert rel_err_rows(fast, ref).max() <= 1e-5


@pytest.mark.parametrize("name,rows", [("c4", range(1, 8)), ("c5", range(1, 4))])
def test_large_configs_every_row_matches_oracle(name, rows):
    """Rows the fixtures do not hold (c4 rows 1-7, c5 rows 1-3): each row's prefill logits and
    its first cached-decode steps against the CPU oracle run on that row alone, so a per-sequence
    indexing error in the KV cache at T = 1024 / 4096 shows up."""
    cfg = synth.CONFIGS[name]
    m, w = model_for(name)
    prompts = synth.prompts_for(name)
    n = 4
    print(f"{name}: batch {cfg['batch']} generate {n} tokens", flush=True)
    toks, logits = m.generate(prompts, n, with_logits=True)
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in rows:
        print(f"{name}: oracle row {b}", flush=True)
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        err = rel_err_rows(logits[b], l_ref)
        assert err.max() <= REL_TOL, f"{name} row {b}: rel err {err}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"{name} row {b}")
    om.close()


@pytest.mark.parametrize("name,rows", [("c4", (1, 4, 7)), ("c5", (1, 3))])
def test_large_configs_late_step_every_row_matches_oracle(name, rows):
    """Late positions on rows the fixtures do not hold: the whole decode (c4 511 steps to
    position 1022, c5 511 steps to 4094), then the oracle recomputes each listed row's last
    step from that row's own token history (teacher forcing): logits within 1e-4, same token."""
    cfg = synth.CONFIGS[name]
    m, w = model_for(name)
    prompts = synth.prompts_for(name)
    n = cfg["n_gen"]
    print(f"{name}: batch {cfg['batch']} generate {n} tokens ({m.decode_path(cfg['batch'])[0]} path)", flush=True)
    m.prefill(prompts)
    m.decode(n - 1)
    toks, last = m.tokens(), m.logits()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    try:
        for b in rows:
            print(f"{name}: oracle row {b}, position {prompts.shape[1] + n - 2}", flush=True)
            hist = np.concatenate([prompts[b], toks[b][:n - 1]]).astype(np.int32)
            t_ref, l_ref = om.greedy(hist, 1, cached=True)
            err = rel_err_rows(last[b], l_ref[0]).max()
            assert err <= REL_TOL, f"{name} row {b}: rel err {err}"
            assert toks[b][n - 1] == t_ref[0], f"{name} row {b}"
    finally:
        om.close()


@pytest.mark.parametrize("batch", [3, 8])
def test_persistent_batches_match_oracle(batch):
    """The persistent kernel at batch > 1 (FMLH_RELAY=0: c2's shape takes the relay kernel by
    default) against the oracle (not only against the graph path): every row's tokens and
    per-step logits over 24 steps."""
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 0)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, cfg["prompt"], 1 + b) for b in range(batch)])
    with env(FMLH_RELAY="0"):
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "persistent"
        n = 24
        print(f"c2 batch {batch}: persistent decode of {n} steps", flush=True)
        toks, logits = m.generate(prompts, n, with_logits=True)
        m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(batch):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"row {b}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"row {b}")
    om.close()


HD32_SHAPES = [synth.NanoLLMShape(65, 64, 64, 2, 2), synth.NanoLLMShape(65, 256, 256, 8, 2)]


@pytest.mark.parametrize("path", ["persistent", "graph"])
@pytest.mark.parametrize("batch", [1, 5])
@pytest.mark.parametrize("shape", HD32_SHAPES, ids=["C64H2", "C256H8"])
def test_head_dim_32_matches_oracle(shape, batch, path):
    """head_dim 32 (the hd32 persistent kernels and the hd32 decode / prefill attention) on both
    decode paths against the oracle: tokens equal, per-step logits within 1e-4."""
    w = synth.make_weights(shape, 3)
    assert shape.head_dim == 32
    P = 24
    prompts = np.stack([synth.prompt_tokens(shape.vocab, P, 100 + b) for b in range(batch)])
    if path == "graph":
        os.environ["FMLH_DECODE"] = "graph"
    try:
        m = fh.NanoLLM(w, max_batch=batch)
    finally:
        os.environ.pop("FMLH_DECODE", None)
    assert m.decode_path(batch)[0] == path
    n = 20
    print(f"hd32 C={shape.n_embed} H={shape.n_head} batch {batch} {path}", flush=True)
    toks, logits = m.generate(prompts, n, with_logits=True)
    m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(batch):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"row {b}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"row {b}")
    om.close()


def test_token_range_checks_do_not_wrap():
    """first + count and prompt_len + n_gen - 1 are checked without 32-bit wrap-around: a first
    of 2^32 - 1 (what -1 becomes at the C ABI) or a huge n_gen is rejected before any copy."""
    m, w = model_for("c1")
    m.generate(synth.prompts_for("c1"), 3)
    with pytest.raises(fh.FreeMLHipError):
        m.tokens(-1, 2)
    with pytest.raises(fh.FreeMLHipError):
        m.tokens(2, 2**32 - 1)
    with pytest.raises(fh.FreeMLHipError):
        m.generate(synth.prompts_for("c1"), 2**32 - 1)
    np.testing.assert_array_equal(m.tokens(0, 1).shape, (1, 1))


def test_refresh_weights_follows_in_place_updates():
    """An engine built on device parameters (weights_on_device = 1) that are then changed in
    place gives the new model's tokens and logits after fmlh_nanollm_refresh_weights, on both
    decode paths; an engine built on host weights owns its copies and refuses the refresh."""
    shape = synth.NanoLLMShape(65, 64, 64, 4, 2)
    w0 = synth.make_weights(shape, 0)
    w1 = synth.make_weights(shape, 1)
    prompts = synth.prompt_tokens(65, 16, 9)[None, :]
    for path in ("persistent", "graph"):
        if path == "graph":
            os.environ["FMLH_DECODE"] = "graph"
        try:
            m = fh.NanoLLM(w0, max_batch=1, on_device=True)
            fresh = fh.NanoLLM(w1, max_batch=1)
        finally:
            os.environ.pop("FMLH_DECODE", None)
        t_new, l_new = fresh.generate(prompts, 30, with_logits=True)
        fresh.close()
        m.generate(prompts, 30)
        for l0, l1 in zip(w0.layers, w1.layers):  # every parameter of w0 becomes w1's
            for a0, a1 in ((l0.w_qkv, l1.w_qkv), (l0.w_proj, l1.w_proj), (l0.w_fc, l1.w_fc),
                           (l0.w_proj2, l1.w_proj2)):
                m.device_weights[id(a0)].upload(a1)
        m.device_weights[id(w0.tok_emb)].upload(w1.tok_emb)
        m.device_weights[id(w0.pos_emb)].upload(w1.pos_emb)
        m.refresh_weights()
        t, l = m.generate(prompts, 30, with_logits=True)
        m.close()
        np.testing.assert_array_equal(t, t_new, err_msg=path)
        assert rel_err_rows(l, l_new).max() <= 1e-5, path
    host = fh.NanoLLM(w0, max_batch=1)
    with pytest.raises(fh.FreeMLHipError):
        host.refresh_weights()
    host.close()


@pytest.mark.parametrize("name,batch", [("c2", 9), ("c2", 16), ("c2", 64), ("c1", 16), ("c1", 12)])
def test_grouped_decode_matches_graph_path_and_oracle(name, batch):
    """The grouped persistent kernel (batches beyond one group of 8: groups of up to 8 sequences,
    matrix-core products) against the multi-kernel graph path (FMLH_DECODE=graph) on every
    row and step, and against the oracle on a few rows: tokens equal, logits within 1e-4
    (graph path: 1e-5, fp32 reassociation)."""
    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], 0)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, cfg["prompt"], 1 + b) for b in range(batch)])
    n = min(cfg["n_gen"], 40)
    os.environ["FMLH_DECODE"] = "graph"
    try:
        ref = fh.NanoLLM(w, max_batch=batch)
    finally:
        del os.environ["FMLH_DECODE"]
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    with env(FMLH_RELAY="0"):  # c2's shape takes the relay kernel by default
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "grouped"
        print(f"{name} batch {batch}: grouped decode of {n} steps", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, batch // 2, batch - 1}):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("prompt_len", [1, 17])
def test_grouped_decode_from_one_key_to_the_last_position(prompt_len):
    """Grouped decode from position prompt_len to block_size - 1: a prompt of one token leaves
    three of the four waves without a key in the first steps (their softmax max stays -inf),
    and the last step fills the cache's final 16-row group."""
    cfg = synth.CONFIGS["c1"]
    w = synth.make_weights(cfg["shape"], 3)
    batch, T = 10, w.shape.block_size
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, prompt_len, 40 + b) for b in range(batch)])
    n = T - prompt_len + 1  # the last decode step feeds position T - 1
    m = fh.NanoLLM(w, max_batch=batch)
    assert m.decode_path(batch)[0] == "grouped"
    print(f"c1 batch {batch}: grouped decode from position {prompt_len} to {T - 1}", flush=True)
    t, l = m.generate(prompts, n, with_logits=True)
    m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in (0, 7, batch - 1):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("shape,batch", [(synth.NanoLLMShape(65, 128, 256, 8, 2), 20),
                                         (synth.NanoLLMShape(65, 64, 64, 2, 2), 10)],
                         ids=["C256H8-20", "C64H2-10"])
def test_grouped_decode_head_dim_32_matches_oracle(shape, batch):
    w = synth.make_weights(shape, 5)
    P = 24
    prompts = np.stack([synth.prompt_tokens(shape.vocab, P, 300 + b) for b in range(batch)])
    m = fh.NanoLLM(w, max_batch=batch)
    assert m.decode_path(batch)[0] == "grouped"
    n = 20
    print(f"grouped hd32 C={shape.n_embed} batch {batch}", flush=True)
    t, l = m.generate(prompts, n, with_logits=True)
    m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(batch):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.fixture
def relay_on():
    """The relay decode kernel (the default for up to 64 sequences at n_embed 256 / 384 / 512);
    FMLH_RELAY=1, read at each decode call, keeps it wherever it plans."""
    with env(FMLH_RELAY="1"):
        yield


def test_relay_decode_matches_reference_fixture(golden, relay_on):
    """c2 at batch 1 on the relay kernel (one cooperative launch per decode call, a team of
    workgroups per product: 229 roles, one per workgroup; each attention role forms its head's
    q): every step against the compiled-reference fixture, tokens equal and logits within
    1e-4."""
    g = golden("c2")
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 0)
    assert w.checksum() == str(g["weights_checksum"])
    m = fh.NanoLLM(w, max_batch=1)
    assert m.decode_path(1)[0] == "relay"
    print(f"c2: relay decode of {cfg['n_gen']} tokens", flush=True)
    toks, logits = m.generate(g["prompts"], cfg["n_gen"], with_logits=True)
    m.close()
    err = rel_err_rows(logits[0], g["logits"][0])
    print(f"c2 relay: max rel err {err.max():.2e}")
    assert err.max() <= REL_TOL
    np.testing.assert_array_equal(toks[0], g["tokens"][0])


@pytest.mark.parametrize("n_layer", [4, 8], ids=["one-role", "two-roles"])
def test_relay_decode_one_and_two_roles_per_workgroup(n_layer, relay_on):
    """4 layers: 169 roles, one per workgroup, weights kept on the chip for the whole launch; 8
    layers: 337 roles on 256 workgroups, so 81 take two and load each role's weights in turn.
    Against the oracle, several runs (a race between workgroups would show as a run that
    differs)."""
    shape = synth.NanoLLMShape(65, 256, 384, 6, n_layer)
    w = synth.make_weights(shape, 5)
    p = synth.prompts_for("c2")
    n = 24
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    tr, lr = om.greedy(p[0], n, cached=True)
    om.close()
    m = fh.NanoLLM(w, max_batch=1)
    assert m.decode_path(1)[0] == "relay"
    for run in range(3):
        print(f"{n_layer} layers: relay run {run}", flush=True)
        t, l = m.generate(p, n, with_logits=True)
        np.testing.assert_array_equal(t[0], tr, err_msg=f"run {run}")
        assert rel_err_rows(l[0], lr).max() <= REL_TOL, f"run {run}"
    m.close()


@pytest.mark.parametrize("prompt_len", [1, 17])
def test_relay_decode_from_one_key_to_the_last_position(prompt_len, relay_on):
    """Relay decode from position prompt_len to block_size - 1: with a one-token prompt three of
    the four waves of each attention workgroup have no key in the first steps; the last step
    fills the cache's final 16-key group."""
    w = synth.make_weights(synth.CONFIGS["c2"]["shape"], 2)
    T = w.shape.block_size
    prompt = synth.prompt_tokens(w.shape.vocab, prompt_len, 11)[None, :]
    n = T - prompt_len + 1  # the last decode step feeds position T - 1
    m = fh.NanoLLM(w, max_batch=1)
    assert m.decode_path(1)[0] == "relay"
    print(f"c2: relay decode from position {prompt_len} to {T - 1}", flush=True)
    t, l = m.generate(prompt, n, with_logits=True)
    m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    tr, lr = om.greedy(prompt[0], n, cached=True)
    om.close()
    np.testing.assert_array_equal(t[0], tr)
    assert rel_err_rows(l[0], lr).max() <= REL_TOL


def test_relay_decode_calls_continue_one_another(relay_on):
    """Several decode calls (each one launch with its own epochs) continue the sequence exactly
    as one call does: the tokens, and the last step's logits, against the oracle."""
    w = synth.make_weights(synth.CONFIGS["c2"]["shape"], 0)
    p = synth.prompts_for("c2")
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    tr, lr = om.greedy(p[0], 30, cached=True)
    om.close()
    m = fh.NanoLLM(w, max_batch=1)
    m.prefill(p)
    for k in (3, 1, 20, 5):
        print(f"c2: relay decode call of {k} steps", flush=True)
        m.decode(k)
    toks = m.tokens()
    last = m.logits()
    m.close()
    np.testing.assert_array_equal(toks[0][:30], tr)
    assert rel_err_rows(last[0], lr[29][None, :]).max() <= REL_TOL


@pytest.mark.parametrize("batch", [2, 8, 31, 32, 64])
def test_relay_batches_match_graph_path_and_oracle(batch, relay_on):
    """Batches on the relay kernel (the sequences flow through the teams as a pipeline, each
    with its own exchange words; from 32 sequences the FC team adds up an item's rows two items
    later) against the multi-kernel graph path on every row and step (tokens equal, logits
    within 1e-5) and against the oracle on the first, a middle and the last row (logits within
    1e-4)."""
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 0)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, cfg["prompt"], 1 + b) for b in range(batch)])
    n = 40
    with env(FMLH_DECODE="graph"):
        ref = fh.NanoLLM(w, max_batch=batch)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    m = fh.NanoLLM(w, max_batch=batch)
    assert m.decode_path(batch)[0] == "relay"
    print(f"c2 batch {batch}: relay decode of {n} steps", flush=True)
    t, l = m.generate(prompts, n, with_logits=True)
    m.close()
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, batch // 2, batch - 1}):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("batch,qa", [(1, "0"), (8, "1"), (40, "1")])
def test_relay_q_in_attention_role_either_way(batch, qa, relay_on):
    """At batch 1 each attention role forms its head's q (the Q team holds only the k / v
    rows); above, the Q team forms q as well.  FMLH_RELAY_QA forces the other cut: batch 1 with
    q from the Q team, batches 8 and 40 (the FC team's lagged row sums) with q in the attention
    roles, against the graph path on every row (tokens equal, logits within 1e-5)
    and the oracle on the first and last rows."""
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 3)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, 20, 90 + b) for b in range(batch)])
    n = 24
    with env(FMLH_DECODE="graph"):
        ref = fh.NanoLLM(w, max_batch=batch)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    with env(FMLH_RELAY_QA=qa):
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "relay"
        print(f"c2 batch {batch}: relay decode, FMLH_RELAY_QA={qa}", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, batch - 1}):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("batch,big", [(8, "1"), (40, "0")])
def test_relay_row_sum_team_either_way(batch, big, relay_on):
    """From 16 sequences the relay kernel's Q team has 192-row slices and the rows of x_{l+1}
    are added up by a team of their own (F2) from the FC team's partials and its published x'
    rows; below, by the FC team itself.  FMLH_RELAY_BIG forces the other cut: batch 8 with the
    F2 team, batch 40 without it, against the graph path on every row (tokens equal, logits
    within 1e-5) and the oracle on the first and last rows."""
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 4)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, 24, 150 + b) for b in range(batch)])
    n = 24
    with env(FMLH_DECODE="graph"):
        ref = fh.NanoLLM(w, max_batch=batch)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    with env(FMLH_RELAY_BIG=big):
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "relay"
        print(f"c2 batch {batch}: relay decode, FMLH_RELAY_BIG={big}", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, batch - 1}):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("batch,switches", [(17, {"FMLH_RELAY_SPLIT": "1"}), (17, {"FMLH_RELAY_HCUT": "1"}),
                                             (40, {}), (40, {"FMLH_RELAY_HCUT": "0"}),
                                             (40, {"FMLH_RELAY_SPLIT": "0"})])
def test_relay_split_cut_either_way(batch, switches, relay_on):
    """The split cut (from 16 sequences at n_embed 384: two attention workgroups per head and
    two lm_head workgroups, each taking every other sequence, FC slices of 96 rows, the row-sum
    team) and, from 33 sequences, its h cut (FC slices of 128 rows that publish h, the MLP
    projection's rows in the F2 team), each forced on at an odd batch and either way at 40,
    against the graph path on every row (tokens equal, logits within 1e-5) and the oracle on
    the first and last rows."""
    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 9)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, 24, 400 + b) for b in range(batch)])
    n = 24
    with env(FMLH_DECODE="graph"):
        ref = fh.NanoLLM(w, max_batch=batch)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    with env(**switches):
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "relay"
        print(f"c2 batch {batch}: relay decode, {switches}", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, batch - 1}):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("hcut", ["1", "0"])
def test_relay_split_cut_with_two_roles_per_workgroup(hcut, relay_on):
    """41 sequences with 8 layers on the h cut (6 Q, 12 attention, 12 FC and 12 F2 workgroups
    per layer and 2 lm_head workgroups: 338 roles on 256 workgroups, so 82 take two) and on the
    split cut without it (16 FC and 6 F2: 322 roles, 66 take two), from a one-token prompt over
    40 steps, against the oracle on three rows."""
    shape = synth.NanoLLMShape(65, 256, 384, 6, 8)
    w = synth.make_weights(shape, 10)
    batch, n = 41, 40
    prompts = np.stack([synth.prompt_tokens(shape.vocab, 1, 450 + b) for b in range(batch)])
    with env(FMLH_RELAY_HCUT=hcut):
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "relay"
        print(f"8 layers, batch {batch}: relay decode (split cut, FMLH_RELAY_HCUT={hcut}) of {n} steps", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in (0, 21, 40):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


def test_relay_row_sum_team_with_two_roles_per_workgroup(relay_on):
    """33 sequences with 8 layers on the relay kernel's big cut (6 Q, 6 attention, 24 FC and
    6 F2 workgroups per layer: 337 roles on 256 workgroups, so 81 take two, F2 roles among
    them), from a one-token prompt over 40 steps, against the oracle on three rows."""
    shape = synth.NanoLLMShape(65, 256, 384, 6, 8)
    w = synth.make_weights(shape, 8)
    batch, n = 33, 40
    prompts = np.stack([synth.prompt_tokens(shape.vocab, 1, 200 + b) for b in range(batch)])
    m = fh.NanoLLM(w, max_batch=batch)
    assert m.decode_path(batch)[0] == "relay"
    print(f"8 layers, batch {batch}: relay decode (big cut) of {n} steps", flush=True)
    t, l = m.generate(prompts, n, with_logits=True)
    m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in (0, 16, 32):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


@pytest.mark.parametrize("batch", [1, 20, 40])
def test_relay_timeline_reads_back(tmp_path, batch, relay_on):
    """FMLH_RELAY_TRACE: a relay launch's per-role timeline reads back (freeml_amd/timeline.py)
    with the plan's team sizes (batch 1: q in the attention roles, 8 Q / 6 attention / 24 FC
    workgroups per layer; batch 20: the split cut, 6 Q / 12 attention / 16 FC / 6 row-sum
    workgroups and two lm_head roles; batch 40: the h cut, 12 FC / 12 F2); sequence 0's path
    through a layer adds up to the layer
    and every interval is non-negative; the traced launch's tokens and logits equal an untraced
    one's bit for bit (the stamps change no arithmetic)."""
    from freeml_amd import timeline

    cfg = synth.CONFIGS["c2"]
    w = synth.make_weights(cfg["shape"], 5)
    prompts = np.stack([synth.prompt_tokens(w.shape.vocab, 40, 300 + b) for b in range(batch)])
    n = 8
    ref = fh.NanoLLM(w, max_batch=batch)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    path = tmp_path / "relay_trace.bin"
    with env(FMLH_RELAY_TRACE=str(path)):
        m = fh.NanoLLM(w, max_batch=batch)
    assert m.decode_path(batch)[0] == "relay"
    print(f"c2 batch {batch}: relay decode with FMLH_RELAY_TRACE", flush=True)
    t, l = m.generate(prompts, n, with_logits=True)
    m.close()
    np.testing.assert_array_equal(t, t_ref)
    np.testing.assert_array_equal(l, l_ref)
    launches = timeline.read_relay(str(path))
    assert launches
    trace, meta = launches[-1]
    expect = {1: dict(nq=8, nf=24, nf2=0, nA=1, nlm=1), 20: dict(nq=6, nf=16, nf2=6, nA=2, nlm=2),
              40: dict(nq=6, nf=12, nf2=12, nA=2, nlm=2)}[batch]
    assert {k: meta[k] for k in expect} == expect
    assert meta["n_layer"] == 6 and meta["n_head"] == 6
    per = meta["nq"] + meta["nA"] * 6 + meta["nf"] + meta["nf2"]
    assert trace.shape[1] == 6 * per + meta["nlm"]
    r = timeline.summarize_relay(trace, meta)
    c = r["chain"]
    parts = [c[k] for k, _ in timeline.RELAY_CHAIN]
    assert min(parts) >= 0.0 and c["layer"] > 0.0
    assert abs(sum(parts) - c["layer"]) < 1e-6
    assert r["step_us"] > 0.0
    assert set(r["teams"]) == ({"Q", "A", "F", "lm"} | ({"F2"} if batch > 1 else set()))


@pytest.mark.parametrize("C,H,L,batch,switches", [(256, 4, 4, 1, {}), (256, 4, 4, 20, {}), (512, 8, 4, 1, {}),
                                                   (512, 8, 3, 6, {}), (256, 4, 2, 60, {}),
                                                   (256, 4, 4, 20, {"FMLH_RELAY_SPLIT": "0"})])
def test_relay_other_widths(C, H, L, batch, switches):
    """The relay kernel at n_embed 256 and 512 (head_dim 64; batches 20 and 60 at 256 take the
    split cut, and 20 once with the row-sum team alone) against the graph path on every row
    (tokens equal, logits within 1e-5) and the oracle on the first and last rows."""
    shape = synth.NanoLLMShape(65, 256, C, H, L)
    w = synth.make_weights(shape, 6)
    prompts = np.stack([synth.prompt_tokens(shape.vocab, 20, 250 + b) for b in range(batch)])
    n = 24
    with env(FMLH_DECODE="graph"):
        ref = fh.NanoLLM(w, max_batch=batch)
    t_ref, l_ref = ref.generate(prompts, n, with_logits=True)
    ref.close()
    with env(**switches):
        m = fh.NanoLLM(w, max_batch=batch)
        assert m.decode_path(batch)[0] == "relay"
        print(f"C {C}, {L} layers, batch {batch}: relay decode of {n} steps {switches}", flush=True)
        t, l = m.generate(prompts, n, with_logits=True)
        m.close()
    np.testing.assert_array_equal(t, t_ref)
    assert rel_err_rows(l, l_ref).max() <= 1e-5
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, batch - 1}):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


def test_relay_batch_from_one_key_to_the_last_position_with_two_roles(relay_on):
    """A batch of 5 on the relay kernel with 8 layers (337 roles on 256 workgroups: 81 take two
    roles and reload each role's weights every step), from a one-token prompt to the last
    position, against the oracle on every row."""
    shape = synth.NanoLLMShape(65, 256, 384, 6, 8)
    w = synth.make_weights(shape, 7)
    batch, T = 5, shape.block_size
    prompts = np.stack([synth.prompt_tokens(shape.vocab, 1, 60 + b) for b in range(batch)])
    n = T
    m = fh.NanoLLM(w, max_batch=batch)
    assert m.decode_path(batch)[0] == "relay"
    print(f"8 layers, batch {batch}: relay decode from position 1 to {T - 1}", flush=True)
    t, l = m.generate(prompts, n, with_logits=True)
    m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(batch):
        tr, lr = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(t[b], tr, err_msg=f"row {b}")
        assert rel_err_rows(l[b], lr).max() <= REL_TOL, f"row {b}"
    om.close()


def test_decode_attention_counts_survive_a_smaller_batch():
    """Decode attention over several 256-key chunks (graph path, block_size 600) merges the
    chunk partials in the work-group that arrives last, counted per (sequence, head).  The
    counts sit at offsets that do not depend on the batch: one engine decoding batch 8 and then
    batch 4 gives the oracle's tokens and logits both times (with the counts placed after the
    batch's own partials, batch 4's counts fell on batch 8's leftover partials)."""
    shape = synth.NanoLLMShape(65, 600, 128, 2, 2)
    w = synth.make_weights(shape, 11)
    with env(FMLH_DECODE="graph"):
        m = fh.NanoLLM(w, max_batch=8)
    assert m.decode_path(8) == ("graph", 0)
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    try:
        for batch, seed in ((8, 300), (4, 400), (8, 500)):
            prompts = np.stack([synth.prompt_tokens(65, 300, seed + b) for b in range(batch)])
            print(f"graph decode, block_size 600: batch {batch}", flush=True)
            toks, logits = m.generate(prompts, 6, with_logits=True)
            for b in range(batch):
                t_ref, l_ref = om.greedy(prompts[b], 6, cached=True)
                assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"batch {batch} row {b}"
                np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"batch {batch} row {b}")
    finally:
        m.close()
        om.close()


@pytest.mark.parametrize("name,batch,path_env", [("c2", 1, {}), ("c1", 1, {}), ("c1", 12, {})])
def test_epoch_count_wraps_cleanly(name, batch, path_env, golden):
    """Exchange words carry 32-bit epochs.  An engine whose count starts just below 2^32
    (FMLH_EPOCH_START) decodes two calls, the second of which would pass 2^32: the library
    clears the exchange buffers and restarts the count, and the tokens and last logits equal
    the reference's (relay kernel for c2, persistent for c1, grouped for c1 x 12)."""
    cfg = synth.CONFIGS[name]
    w = synth.make_weights(cfg["shape"], 0)
    if batch == 1:
        prompts = synth.prompts_for(name)
    else:
        prompts = np.stack([synth.prompt_tokens(w.shape.vocab, cfg["prompt"], 1 + b) for b in range(batch)])
    n = 40
    per_step = 1 if name == "c2" else 5 * w.shape.n_layer + 1
    start = 2**32 - 1 - (20 * per_step + 1) - 5  # the first call fits, the second wraps
    with env(FMLH_EPOCH_START=str(start), **path_env):
        m = fh.NanoLLM(w, max_batch=batch)
    try:
        kind = m.decode_path(batch)[0]
        print(f"{name} batch {batch}: {kind} decode across the epoch wrap", flush=True)
        assert kind == {"c2": "relay", "c1": "persistent" if batch == 1 else "grouped"}[name]
        m.prefill(prompts)
        m.decode(20)
        m.decode(n - 21)
        toks, last = m.tokens(), m.logits()
    finally:
        m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(batch):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"row {b}")
        assert rel_err_rows(last[b], l_ref[-1]).max() <= REL_TOL
    om.close()


def test_wide_epoch_count_wraps_cleanly():
    """The wide kernel's epochs (7 per layer and step + 1 per step + 1 per launch) across the
    32-bit wrap: the second decode call would pass 2^32, so the library clears the exchange
    buffers and restarts the count; tokens and last logits equal the oracle's."""
    V, T, C, H, L, B, P = 65, 320, 256, 4, 2, 3, 40
    shape = synth.NanoLLMShape(V, T, C, H, L)
    w = synth.make_weights(shape, 29)
    prompts = np.stack([synth.prompt_tokens(V, P, 700 + b) for b in range(B)])
    n = 40
    start = 2**32 - 1 - (20 * (7 * L + 1) + 1) - 5  # the first call fits, the second wraps
    with env(FMLH_EPOCH_START=str(start), FMLH_WIDE="1"):  # FMLH_WIDE is read at each decode
        m = fh.NanoLLM(w, max_batch=B)
        try:
            assert m.decode_path(B)[0] == "wide"
            print(f"wide batch {B}: decode across the epoch wrap", flush=True)
            m.prefill(prompts)
            m.decode(20)
            m.decode(n - 21)
            toks, last = m.tokens(), m.logits()
        finally:
            m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(B):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"row {b}")
        assert rel_err_rows(last[b], l_ref[-1]).max() <= REL_TOL
    om.close()


@pytest.mark.parametrize("C,H,B,P,parts", [(1024, 16, 16, 64, "2"), (1024, 16, 1, 576, "2"),
                                           (384, 6, 22, 64, "4")])
def test_fused_prefill_part_workspace(C, H, B, P, parts):
    """Each part of the fused prefill gets a workspace slice sized for what its QKV and FC
    products plan at the part's rows (they can split K where a part is small) -- C = 1024 at
    16 x 64 and 1 x 576 rows, and four parts of c3's width at 22 sequences.  Every sequence's
    prefill logits and first decode step against the oracle, on a one-layer model."""
    shape = synth.NanoLLMShape(65, 640, C, H, 1)
    w = synth.make_weights(shape, 21)
    prompts = np.stack([synth.prompt_tokens(65, P, 700 + b) for b in range(B)])
    with env(FMLH_PREFILL_STREAMS=parts, FMLH_PREFILL_FUSED="1", FMLH_DECODE="graph"):
        m = fh.NanoLLM(w, max_batch=B)
        try:
            print(f"fused prefill C={C} batch {B} x {P} rows, {parts} parts", flush=True)
            toks, logits = m.generate(prompts, 2, with_logits=True)
        finally:
            m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in sorted({0, B // 2, B - 1}):
        t_ref, l_ref = om.greedy(prompts[b], 2, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"sequence {b}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"sequence {b}")
    om.close()


WIDE_CASES = [
    # (vocab, block, n_embed, n_head, layers, batch, prompt, steps)
    (65, 320, 256, 4, 2, 1, 40, 24),
    (65, 320, 256, 4, 2, 3, 40, 24),
    (100, 96, 512, 8, 1, 8, 20, 12),
    (300, 64, 768, 12, 2, 5, 10, 20),
    (65, 1200, 256, 4, 1, 2, 1100, 12),   # block_size beyond the persistent kernel: key slices
    (70, 96, 256, 4, 16, 2, 20, 8),       # 16 layers (deeper than the kernel's timeline buffer)
]


@pytest.mark.parametrize("V,T,C,H,L,B,P,n", WIDE_CASES)
def test_wide_decode_matches_oracle(V, T, C, H, L, B, P, n):
    """The wide decode kernel (FMLH_WIDE=1 also takes shapes the persistent kernel plans) against
    the oracle: every sequence's tokens and per-step logits, for n_embed 256 / 512 / 768, batch
    1 to 8, one key slice per few keys up to block_size 1200 (slices of ~75-600 keys)."""
    shape = synth.NanoLLMShape(V, T, C, H, L)
    w = synth.make_weights(shape, 17)
    prompts = np.stack([synth.prompt_tokens(V, P, 500 + b) for b in range(B)])
    with env(FMLH_WIDE="1", FMLH_RELAY="0"):  # (the relay kernel also plans the 16-layer case)
        m = fh.NanoLLM(w, max_batch=B)
        try:
            assert m.decode_path(B)[0] == "wide"
            print(f"wide decode C={C} H={H} L={L} T={T} batch {B}: {n} steps", flush=True)
            toks, logits = m.generate(prompts, n, with_logits=True)
        finally:
            m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(B):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"sequence {b}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"sequence {b}")
    om.close()


@pytest.mark.parametrize("path,C,batch,switches", [
    ("relay", 384, 1, {}), ("relay", 384, 8, {}), ("relay", 384, 20, {}), ("relay", 256, 1, {}),
    ("persistent", 384, 3, {"FMLH_RELAY": "0"}), ("grouped", 384, 12, {"FMLH_RELAY": "0"})])
def test_decode_kernels_with_layernorm_biases(path, C, batch, switches):
    """LayerNorm gains != 1 and biases present in every LayerNorm (the relay kernel applies
    them after its products through the row sums of w g and w b; the persistent and grouped
    kernels normalise first) on the relay kernel's three team cuts (batch 1: q in the attention
    roles; 8; 20: the row-sum team), the persistent and the grouped kernels, against the oracle
    on every row."""
    V, T, L, P, n = 65, 96, 2, 24, 10
    H = C // 64
    shape = synth.NanoLLMShape(V, T, C, H, L)
    w = synth.make_weights(shape, 31)
    rng = np.random.default_rng(7)
    vec = lambda mu: (mu + 0.2 * rng.standard_normal(C)).astype(np.float32)
    for lw in w.layers:
        lw.ln0_g, lw.ln0_b, lw.ln1_g, lw.ln1_b = vec(1.0), vec(0.0), vec(1.0), vec(0.0)
    w.lnf_g, w.lnf_b = vec(1.0), vec(0.0)
    prompts = np.stack([synth.prompt_tokens(V, P, 950 + b) for b in range(batch)])
    with env(**switches):
        m = fh.NanoLLM(w, max_batch=batch)
        try:
            assert m.decode_path(batch)[0] == path
            print(f"{path} decode with LayerNorm biases, C={C}, batch {batch}: {n} steps", flush=True)
            toks, logits = m.generate(prompts, n, with_logits=True)
        finally:
            m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(batch):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"sequence {b}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"sequence {b}")
    om.close()


@pytest.mark.parametrize("C,H", [(256, 4), (1024, 16)])
def test_wide_decode_with_layernorm_biases(C, H):
    """The wide kernel with LayerNorm gains != 1 and biases present (the kernel stages every
    gain and bias in LDS; a model without biases skips them) against the oracle, n_embed 256
    and 1024 (the widest LDS layout)."""
    V, T, L, B, P, n = 120, 96, 2, 3, 24, 10
    shape = synth.NanoLLMShape(V, T, C, H, L)
    w = synth.make_weights(shape, 23)
    rng = np.random.default_rng(5)
    vec = lambda mu: (mu + 0.2 * rng.standard_normal(C)).astype(np.float32)
    for lw in w.layers:
        lw.ln0_g, lw.ln0_b, lw.ln1_g, lw.ln1_b = vec(1.0), vec(0.0), vec(1.0), vec(0.0)
    w.lnf_g, w.lnf_b = vec(1.0), vec(0.0)
    prompts = np.stack([synth.prompt_tokens(V, P, 900 + b) for b in range(B)])
    with env(FMLH_WIDE="1"):
        m = fh.NanoLLM(w, max_batch=B)
        try:
            assert m.decode_path(B)[0] == "wide"
            print(f"wide decode with LayerNorm biases C={C}: {n} steps", flush=True)
            toks, logits = m.generate(prompts, n, with_logits=True)
        finally:
            m.close()
    om = oracle.OracleModel(w, nthreads=min(16, os.cpu_count() or 1))
    for b in range(B):
        t_ref, l_ref = om.greedy(prompts[b], n, cached=True)
        assert rel_err_rows(logits[b], l_ref).max() <= REL_TOL, f"sequence {b}"
        np.testing.assert_array_equal(toks[b], t_ref, err_msg=f"sequence {b}")
    om.close()


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_large_configs_decode_on_the_wide_kernel(name):
    """c4 and c5 decode on the wide kernel by default, and the kernel's steps match the graph
    path's (FMLH_DECODE=graph) to fp32 reassociation over 12 steps at the prompt's end."""
    cfg = synth.CONFIGS[name]
    m, w = model_for(name)
    assert m.decode_path(cfg["batch"])[0] == "wide"
    prompts = synth.prompts_for(name)
    toks, logits = m.generate(prompts, 12, with_logits=True)
    with env(FMLH_DECODE="graph"):
        g = fh.NanoLLM(w, max_batch=cfg["batch"])
    try:
        assert g.decode_path(cfg["batch"])[0] == "graph"
        t_ref, l_ref = g.generate(prompts, 12, with_logits=True)
    finally:
        g.close()
    np.testing.assert_array_equal(toks, t_ref)
    assert rel_err_rows(logits, l_ref).max() <= 1e-5
