"""Sampling beyond greedy (fmlh_nanollm_set_sampling).  The reference decodes greedily only, so
this path has no reference result to match ("parity unpinned" against the reference); it is
pinned against its own stated definition instead:

* the random stream: splitmix64 against its published first outputs, and uniformity of u;
* the selection: the restatement (oracle.sample_token) against brute force on small rows --
  top-k set by (value desc, index asc), inverse CDF in index order -- and its limits (top_k 1
  is the greedy first maximum, a tiny temperature concentrates on the maximum);
* the device: every sampled token of a run equals the restatement applied to that step's
  logits, except within float rounding of a CDF boundary.
"""
import numpy as np
import pytest

import oracle


def test_splitmix64_published_outputs():
    # splitmix64 with state 0: the first two outputs of Vigna's reference generator.
    assert oracle.splitmix64(0) == 0xE220A8397B1DCDAF
    assert oracle.splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4


def test_uniform_stream_is_uniform():
    u = np.array([oracle.sample_uniform(7, b, p) for b in range(20) for p in range(1000)])
    assert u.min() >= 0 and u.max() < 1
    counts, _ = np.histogram(u, bins=20, range=(0, 1))
    chi2 = ((counts - u.size / 20) ** 2 / (u.size / 20)).sum()
    assert chi2 < 45  # 19 dof: p ~ 1e-3
    assert len(set(u.tolist())) > 0.99 * u.size


def brute(z, temperature, top_k, u):
    V = z.size
    ranked = sorted(range(V), key=lambda i: (-float(z[i]), i))
    kept = set(ranked[: top_k if 0 < top_k < V else V])
    m = max(float(v) for v in z)
    inv_t = float(np.float32(1.0) / np.float32(temperature))
    w = [np.exp((float(z[i]) - m) * inv_t) if i in kept else 0.0 for i in range(V)]
    t = u * sum(w)
    acc = 0.0
    for i in range(V):
        acc += w[i]
        if w[i] > 0 and acc > t:
            return i
    return max(kept)


@pytest.mark.parametrize("top_k", [0, 1, 3, 8, 40])
def test_restatement_matches_brute_force(top_k):
    r = np.random.default_rng(top_k)
    for trial in range(50):
        z = (r.standard_normal(40) * 2).astype(np.float32)
        z[5] = z[9] = z[17] = z.max()  # ties at the top
        tok, _ = oracle.sample_token(z, 0.8, top_k, 11, trial, 3)
        assert tok == brute(z, 0.8, top_k, oracle.sample_uniform(11, trial, 3))
        if top_k == 1:
            assert tok == int(np.argmax(z))  # the first maximum, as greedy picks


def test_sampling_frequencies_follow_the_distribution():
    z = np.array([2.0, 1.0, 0.0, -1.0, 0.5], np.float32)
    T, k = 0.9, 3
    toks = np.array([oracle.sample_token(z, T, k, 5, b, 0)[0] for b in range(20000)])
    kept = [0, 1, 4]
    w = np.exp((z[kept] - z.max()) / T)
    p = w / w.sum()
    freq = np.array([(toks == i).mean() for i in kept])
    assert set(np.unique(toks)) <= set(kept)
    np.testing.assert_allclose(freq, p, atol=0.015)


def _model(shape, seed=0):
    import freeml_amd as fh
    from freeml_amd import synth

    return fh.NanoLLM(synth.make_weights(shape, seed), max_batch=4)


@pytest.mark.gpu
@pytest.mark.parametrize("temperature,top_k", [(0.8, 0), (1.3, 5), (0.5, 64)])
def test_device_draws_follow_the_definition(temperature, top_k, golden):
    import freeml_amd as fh
    from freeml_amd import synth

    fh.init(0)
    cfg = synth.CONFIGS["c1"]
    m = _model(cfg["shape"])
    prompts = np.stack([golden("c1")["prompts"][0]] * 3)
    try:
        m.set_sampling(temperature, top_k, seed=1234)
        assert m.decode_path(3)[0] == "graph"
        toks, logits = m.generate(prompts, 24, with_logits=True)
    finally:
        m.close()
    P = prompts.shape[1]
    checked = 0
    for b in range(3):
        for s in range(24):
            tok, margin = oracle.sample_token(logits[b, s], temperature, top_k, 1234, b, P + s)
            if margin < 1e-5:
                continue
            assert toks[b, s] == tok, (b, s)
            checked += 1
    assert checked >= 70
    assert len({tuple(t) for t in toks}) > 1  # the three sequences draw differently


@pytest.mark.gpu
def test_top_k_one_is_greedy_and_zero_temperature_restores_greedy(golden):
    import freeml_amd as fh
    from freeml_amd import synth

    fh.init(0)
    g = golden("c2")
    m = _model(synth.CONFIGS["c2"]["shape"])
    try:
        m.set_sampling(0.7, 1, seed=9)
        toks, _ = m.generate(g["prompts"][:1], 32)
        np.testing.assert_array_equal(toks[0], g["tokens"][0][:32])
        m.set_sampling(0.0)
        assert m.decode_path(1)[0] in ("relay", "persistent")  # a one-launch greedy kernel again
        toks, _ = m.generate(g["prompts"][:1], 32)
        np.testing.assert_array_equal(toks[0], g["tokens"][0][:32])
    finally:
        m.close()


@pytest.mark.gpu
def test_top_k_ties_large_vocabulary():
    """A 50304-token vocabulary where half the embedding rows are zero: their logits are all
    exactly 0, so the top-k boundary falls inside a block of equal logits and only the lowest
    indices of it are kept."""
    import freeml_amd as fh
    from freeml_amd import synth

    fh.init(0)
    shape = synth.NanoLLMShape(50304, 64, 64, 4, 2)
    w = synth.make_weights(shape, 3)
    w.tok_emb[1::2] = 0  # tied lm_head: every odd token's logit is 0
    prompt = (np.arange(16, dtype=np.int32) * 2)[None, :]  # even (non-zero) tokens
    m = fh.NanoLLM(w, max_batch=1)
    try:
        m.set_sampling(1.0, 30000, seed=77)
        toks, logits = m.generate(prompt, 24, with_logits=True)
    finally:
        m.close()
    checked = 0
    for s in range(24):
        z = logits[0, s]
        assert np.sum(z > 0) < 30000 < np.sum(z >= 0)  # the boundary is inside the zeros
        tok, margin = oracle.sample_token(z, 1.0, 30000, 77, 0, 16 + s)
        # ~30000 kept weights of ~3e-5 of the total each: the device's fp32 running sums
        # (50-element chunks, then a scan) are good to ~1e-6 of the total.
        if margin < 2e-6:
            continue
        assert toks[0, s] == tok, s
        checked += 1
    assert checked >= 12
