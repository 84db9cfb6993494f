"""Pins the oracle's training-step restatements (oracle/nanollm_oracle.c) on the CPU.

Each restatement is checked two ways:
* bit for bit against the reference's own routine, compiled from the reference sources into
  oracle/_ref/libfreeml_ref.so (SoftmaxBackwards, LayerNormBackwardsOp, GeluDerivtiveMat,
  ScatterAddRows, MergeQKV, CategoricalCrossEntropyWithLogits, AdamWUpdate);
* against what the mathematics fixes, independently of both: finite differences of the
  forward function for the derivatives (in float64), the closed form of the first AdamW step,
  numpy's index arithmetic for the data movement, and the softmax-gradient identities.
"""
import numpy as np
import pytest

import oracle

needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
IMPLS = ["oracle", pytest.param("ref", marks=needs_ref)]


def rng(seed=0):
    return np.random.default_rng(seed)


def softmax64(x):
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


# ---- bit-exact against the compiled reference ----------------------------------------------

@needs_ref
@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (64, 64), (33, 257)])
def test_softmax_backward_matches_reference(rows, cols):
    r = rng(rows * 100 + cols)
    p = softmax64(r.standard_normal((rows, cols))).astype(np.float32)
    dp = r.standard_normal((rows, cols)).astype(np.float32)
    np.testing.assert_array_equal(oracle.softmax_backward(p, dp),
                                  oracle.softmax_backward(p, dp, impl="ref"))


@needs_ref
@pytest.mark.parametrize("rows,cols", [(1, 8), (7, 64), (64, 384), (3, 1000)])
@pytest.mark.parametrize("with_xhat", [True, False])
@pytest.mark.parametrize("with_beta", [True, False])
def test_layernorm_backward_matches_reference(rows, cols, with_xhat, with_beta):
    r = rng(rows + cols)
    x = (r.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
    dy = r.standard_normal((rows, cols)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    xhat = None
    if with_xhat:
        mu = x.mean(axis=1, keepdims=True, dtype=np.float64)
        xhat = ((x - mu) / np.sqrt(x.var(axis=1, keepdims=True, dtype=np.float64) + 1e-5)).astype(np.float32)
    a = oracle.layernorm_backward(dy, x, g, xhat, with_beta)
    b = oracle.layernorm_backward(dy, x, g, xhat, with_beta, impl="ref")
    for u, v in zip(a, b):
        if u is None:
            assert v is None
        else:
            np.testing.assert_array_equal(u, v)


@needs_ref
def test_gelu_derivative_matches_reference():
    x = np.concatenate([np.linspace(-9, 9, 4001), rng(1).standard_normal(1000) * 3]).astype(np.float32)
    np.testing.assert_array_equal(oracle.gelu_derivative(x), oracle.gelu_derivative(x, impl="ref"))


@needs_ref
@pytest.mark.parametrize("src_batch,out_batch", [(1, 1), (3, 1), (3, 3)])
def test_scatter_add_rows_matches_reference(src_batch, out_batch):
    r = rng(src_batch * 10 + out_batch)
    width, src_rows, out_rows = 37, 50, 9  # many repeated destination rows
    out = r.standard_normal((out_batch, out_rows, width)).astype(np.float32)
    src = r.standard_normal((src_batch, src_rows, width)).astype(np.float32)
    idx = r.integers(0, out_rows, (src_batch, src_rows)).astype(np.float32)
    np.testing.assert_array_equal(oracle.scatter_add_rows(out, src, idx),
                                  oracle.scatter_add_rows(out, src, idx, impl="ref"))


@needs_ref
def test_merge_qkv_matches_reference():
    r = rng(3)
    q, k, v = (r.standard_normal((6, 40, 16)).astype(np.float32) for _ in range(3))
    np.testing.assert_array_equal(oracle.merge_qkv(q, k, v), oracle.merge_qkv(q, k, v, impl="ref"))


@needs_ref
@pytest.mark.parametrize("kind", ["index", "index_ignore", "onehot", "index_batched"])
def test_cce_logits_matches_reference(kind):
    r = rng(4)
    batch = 3 if kind == "index_batched" else 1
    steps, vocab = 31, 65
    z = (r.standard_normal((batch, steps, vocab)) * 3).astype(np.float32)
    if kind.startswith("index"):
        t = r.integers(0, vocab, (batch, steps)).astype(np.float32)
        if kind == "index_ignore":
            t[0, ::4] = -1
    else:
        t = np.zeros((1, steps, vocab), np.float32)
        t[0, np.arange(steps), r.integers(0, vocab, steps)] = 1
    g1, l1 = oracle.cce_logits(t, z)
    g2, l2 = oracle.cce_logits(t, z, impl="ref")
    np.testing.assert_array_equal(g1, g2)
    assert l1 == l2


@needs_ref
@pytest.mark.parametrize("t", [1, 2, 50])
def test_adamw_matches_reference(t):
    r = rng(t)
    n = 4097
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    g[:5] = 0
    m = (r.standard_normal(n) * 1e-4).astype(np.float32)
    v = (r.random(n) * 1e-6).astype(np.float32)
    a = oracle.adamw_update(p, g, m, v, 1e-4, 0.9, 0.999, t, 1e-8, 0.01)
    b = oracle.adamw_update(p, g, m, v, 1e-4, 0.9, 0.999, t, 1e-8, 0.01, impl="ref")
    for u, w in zip(a, b):
        np.testing.assert_array_equal(u, w)


# ---- what the mathematics fixes -------------------------------------------------------------

@pytest.mark.parametrize("impl", IMPLS)
def test_softmax_backward_is_the_softmax_vjp(impl):
    """out = J^T dp for p = softmax(x): compared with central differences of sum(dp * softmax(x))."""
    r = rng(5)
    x = r.standard_normal((4, 9))
    dp = r.standard_normal((4, 9))
    p = softmax64(x)
    got = oracle.softmax_backward(p.astype(np.float32), dp.astype(np.float32), impl=impl)
    h = 1e-6
    num = np.zeros_like(x)
    for i in range(x.shape[1]):
        e = np.zeros_like(x)
        e[:, i] = h
        num[:, i] = ((dp * softmax64(x + e)).sum(1) - (dp * softmax64(x - e)).sum(1)) / (2 * h)
    np.testing.assert_allclose(got, num, atol=2e-6)
    np.testing.assert_allclose(got.sum(axis=1), 0, atol=1e-6)  # rows of J^T dp sum to zero


def ln64(x, g, eps=1e-5):
    mu = x.mean(1, keepdims=True)
    return (x - mu) / np.sqrt(x.var(1, keepdims=True) + eps) * g


@pytest.mark.parametrize("impl", IMPLS)
def test_layernorm_backward_is_the_gradient(impl):
    """dx, dgamma, dbeta are the gradients of sum(dy * (LN(x) gamma + beta))."""
    r = rng(6)
    rows, cols = 3, 12
    x = r.standard_normal((rows, cols)) * 1.5
    g = 1 + 0.2 * r.standard_normal(cols)
    dy = r.standard_normal((rows, cols))
    dx, dg, db = oracle.layernorm_backward(dy.astype(np.float32), x.astype(np.float32),
                                           g.astype(np.float32), None, True, impl=impl)
    f = lambda xx, gg: (dy * ln64(xx, gg)).sum()
    h = 1e-6
    ndx = np.zeros_like(x)
    for i in range(rows):
        for j in range(cols):
            e = np.zeros_like(x)
            e[i, j] = h
            ndx[i, j] = (f(x + e, g) - f(x - e, g)) / (2 * h)
    ndg = np.array([(f(x, g + h * np.eye(cols)[j]) - f(x, g - h * np.eye(cols)[j])) / (2 * h)
                    for j in range(cols)])
    np.testing.assert_allclose(dx, ndx, atol=5e-5)
    np.testing.assert_allclose(dg, ndg, atol=5e-5)
    np.testing.assert_allclose(db, dy.sum(0), atol=1e-5)


@pytest.mark.parametrize("impl", IMPLS)
def test_gelu_derivative_is_the_derivative(impl):
    from scipy.special import erf

    x = np.linspace(-6, 6, 601)
    gelu = lambda v: 0.5 * v * (1 + erf(v / np.sqrt(2)))
    h = 1e-5
    num = (gelu(x + h) - gelu(x - h)) / (2 * h)
    np.testing.assert_allclose(oracle.gelu_derivative(x.astype(np.float32), impl=impl), num, atol=2e-6)


@pytest.mark.parametrize("impl", IMPLS)
def test_scatter_add_rows_is_index_add(impl):
    r = rng(7)
    out = np.zeros((2, 5, 3), np.float32)
    src = r.standard_normal((2, 8, 3)).astype(np.float32)
    idx = r.integers(0, 5, (2, 8)).astype(np.float32)
    expect = np.zeros((2, 5, 3))
    for z in range(2):
        np.add.at(expect[z], idx[z].astype(int), src[z].astype(np.float64))
    np.testing.assert_allclose(oracle.scatter_add_rows(out, src, idx, impl=impl), expect, atol=1e-6)


@pytest.mark.parametrize("impl", IMPLS)
def test_merge_qkv_is_the_split_inverse(impl):
    """MergeQKV undoes the forward's per-head split: packed[t, s*C + h*hd + d] = S[h, t, d]."""
    r = rng(8)
    nh, T, hd = 3, 5, 4
    q, k, v = (r.standard_normal((nh, T, hd)).astype(np.float32) for _ in range(3))
    packed = oracle.merge_qkv(q, k, v, impl=impl)
    for s, src in enumerate((q, k, v)):
        blk = packed[:, s * nh * hd:(s + 1) * nh * hd].reshape(T, nh, hd).transpose(1, 0, 2)
        np.testing.assert_array_equal(blk, src)


@pytest.mark.parametrize("impl", IMPLS)
def test_cce_gradient_is_negative_loss_gradient(impl):
    """Index targets: grad = -(d loss / d z) (the codebase's negative-gradient convention);
    the loss is mean(logsumexp - z[target]) over non-ignored rows."""
    r = rng(9)
    steps, vocab = 5, 7
    z = r.standard_normal((1, steps, vocab))
    t = r.integers(0, vocab, (1, steps)).astype(np.float32)
    t[0, 2] = -1
    grad, loss = oracle.cce_logits(t, z.astype(np.float32), impl=impl)
    valid = [i for i in range(steps) if t[0, i] != -1]

    def L(zz):
        lse = np.log(np.exp(zz[0]).sum(1))
        return np.mean([lse[i] - zz[0, i, int(t[0, i])] for i in valid])

    assert abs(loss - L(z)) < 1e-5
    h = 1e-6
    num = np.zeros_like(z)
    for i in range(steps):
        for j in range(vocab):
            e = np.zeros_like(z)
            e[0, i, j] = h
            num[0, i, j] = (L(z + e) - L(z - e)) / (2 * h)
    np.testing.assert_allclose(grad, -num, atol=1e-6)
    np.testing.assert_array_equal(grad[0, 2], 0)


@pytest.mark.parametrize("impl", IMPLS)
def test_adamw_first_step_closed_form(impl):
    """t = 1 from zero moments: m^ = g, v^ = g^2, so p' = p + lr g / (|g| + eps) - lr wd p."""
    r = rng(10)
    n = 1000
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-2).astype(np.float32)
    z = np.zeros(n, np.float32)
    lr, wd = 1e-3, 0.01
    p1, m1, v1 = oracle.adamw_update(p, g, z, z, lr, 0.9, 0.999, 1, 1e-8, wd, impl=impl)
    g64, p64 = g.astype(np.float64), p.astype(np.float64)
    # 1 - beta is formed in float (MatrixBase_Functions.h:1524-1525).
    ib1 = float(np.float32(1) - np.float32(0.9))
    ib2 = float(np.float32(1) - np.float32(0.999))
    np.testing.assert_allclose(p1, p64 + lr * g64 / (np.abs(g64) + 1e-8) - lr * wd * p64, atol=1e-8)
    np.testing.assert_allclose(m1, ib1 * g64, rtol=1e-6)
    np.testing.assert_allclose(v1, ib2 * g64 * g64, rtol=1e-6)


# ---- SumColumns and the dropout mask ---------------------------------------------------------

@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 3), (256, 384), (1000, 65)])
def test_sum_columns_is_the_row_ordered_column_sum(impl, rows, cols):
    """SumColumns (MatrixBase_Functions.h:1098-1118): float32 sums taken row by row, so equal
    to numpy's sequential accumulation over axis 0 and within float32 rounding of float64."""
    x = (rng(rows + cols).standard_normal((rows, cols)) * 3).astype(np.float32)
    got = oracle.sum_columns(x, impl=impl)
    seq = np.zeros(cols, np.float32)
    for r in range(rows):
        seq = (seq + x[r]).astype(np.float32)
    np.testing.assert_array_equal(got, seq)
    np.testing.assert_allclose(got, x.astype(np.float64).sum(0), rtol=0, atol=1e-4 * max(1, rows) ** 0.5)


@needs_ref
def test_sum_columns_matches_reference():
    x = rng(9).standard_normal((333, 129)).astype(np.float32)
    np.testing.assert_array_equal(oracle.sum_columns(x), oracle.sum_columns(x, impl="ref"))
    # a transposed-index mistake (summing rows instead of columns) fails
    assert not np.array_equal(oracle.sum_columns(x)[:5], x.sum(1)[:5].astype(np.float32))


@needs_ref
def test_dropout_mask_matches_reference_update_mask():
    """DropoutLayer::UpdateMask of the compiled reference against the restatement: the draws
    come from RandomUtils' uniform buffer at the process-wide running index (starting at 0 in
    this process, continuing across calls), 0 where the draw is below the probability; p <= 0
    and p >= 1 fill without drawing."""
    n1, n2 = 1000, 4097
    uni, count = oracle.ref_uniform_buffer(n1 + n2 + 64)
    assert count == 4 * 1024 * 1024 and uni.min() >= 0 and uni.max() < 1
    got1 = oracle.ref_dropout_mask(n1, 0.1)
    exp1, used1 = oracle.dropout_mask(n1, uni, 0, 0.1)
    assert used1 == n1
    np.testing.assert_array_equal(got1, exp1)
    np.testing.assert_array_equal(oracle.ref_dropout_mask(16, 0.0), np.ones(16, np.float32))  # no draws
    np.testing.assert_array_equal(oracle.ref_dropout_mask(16, 1.0), np.zeros(16, np.float32))
    got2 = oracle.ref_dropout_mask(n2, 0.5)
    exp2, _ = oracle.dropout_mask(n2, uni, n1, 0.5)
    np.testing.assert_array_equal(got2, exp2)
    # the index really continued: drawing from 0 again differs
    assert not np.array_equal(exp2, oracle.dropout_mask(n2, uni, 0, 0.5)[0])


def test_dropout_mask_wraps_and_keeps_the_rate():
    u = rng(4).random(1000).astype(np.float32)
    m, used = oracle.dropout_mask(2500, u, 900, 0.25)
    assert used == 2500
    idx = (900 + np.arange(2500)) % 1000
    np.testing.assert_array_equal(m, np.where(u[idx] < 0.25, 0, 1).astype(np.float32))
    big = rng(5).random(1 << 16).astype(np.float32)
    frac = 1 - oracle.dropout_mask(1 << 16, big, 0, 0.3)[0].mean()
    assert abs(frac - 0.3) < 0.01
