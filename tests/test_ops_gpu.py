"""GPU parity of the matrix-op entry points (the MatrixHIP<float> overload set).

Each op runs through the C ABI on device memory and is compared with the oracle's
restatement of the reference routine (same fp32 formula) or float64.  Tolerances (normwise,
written per test) cover fp32 reassociation and libm-vs-device exp/erf ulps; data movement ops
(copy, gather, split, fill, argmax) must be exact.
"""
import numpy as np
import pytest

import freeml_amd as fh
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    fh.init(0)
    arch, cus = fh.device_info()
    print(f"device {arch} with {cus} CUs", flush=True)
    assert arch.startswith("gfx950")


D = fh.DeviceArray.from_host


def _rng(s):
    return np.random.default_rng(s)


def _close(got, ref64, tol, scale=None):
    scale = np.max(np.abs(ref64)) if scale is None else scale
    err = np.max(np.abs(got.astype(np.float64) - ref64)) / max(scale, 1e-30)
    assert err <= tol, f"normwise error {err:.3e} > {tol:.1e}"


# Shapes hit: skinny NN/NT (M <= 8), MFMA 64x64 / 128x128 tiles, split-K, ragged edges,
# K not a multiple of 16 (strided fallback).
MUL_SHAPES = [(1, 1152, 384), (4, 1536, 384), (8, 65, 64), (64, 1152, 384), (64, 384, 1536),
              (257, 130, 64), (1024, 512, 768), (37, 50, 65), (3, 7, 5)]


@pytest.mark.parametrize("mode", [fh.NONE, fh.RIGHT, fh.LEFT, fh.BOTH])
@pytest.mark.parametrize("shape", MUL_SHAPES)
def test_mul(mode, shape):
    M, N, K = shape
    print(f"mul mode={mode} M={M} N={N} K={K}", flush=True)
    r = _rng(M * 7 + N + K)
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    L = np.ascontiguousarray(A.T) if mode in (fh.LEFT, fh.BOTH) else A
    R = np.ascontiguousarray(B.T) if mode in (fh.RIGHT, fh.BOTH) else B
    dL, dR, dO = D(L), D(R), fh.DeviceArray((M, N))
    fh.mul(mode, dO.ptr, dL.ptr, dR.ptr, M, N, K)
    got = dO.numpy()
    ref64 = A.astype(np.float64) @ B.astype(np.float64)
    # fp32 accumulation error bound ~ K * eps * sum|a||b|; normwise against |A||B|.
    absprod = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    _close(got, ref64, 2e-6 * np.sqrt(K) + 1e-6, scale=np.max(absprod))


@pytest.mark.parametrize("epi", [fh.EPI_NONE, fh.EPI_GELU, fh.EPI_RESID])
@pytest.mark.parametrize("shape,bt", [((1, 1536, 384), 0), ((1, 384, 384), 1), ((8, 50304, 768), 1),
                                      ((64, 1152, 384), 0), ((4096, 384, 1536), 0),
                                      ((512, 768, 768), 1), ((64, 65, 384), 1),
                                      # skinny NT on matrix cores: ragged N, the longest K held in
                                      # LDS, and one K past it (per-column kernel)
                                      ((5, 100, 4096), 1), ((8, 768, 3072), 1), ((2, 2304, 768), 1),
                                      ((7, 33, 16), 1), ((3, 40, 4112), 1)])
def test_gemm_ex_epilogues(epi, shape, bt):
    M, N, K = shape
    print(f"gemm_ex epi={epi} M={M} N={N} K={K} bt={bt}", flush=True)
    r = _rng(M + N + K + epi)
    A = (r.standard_normal((M, K)) * 0.5).astype(np.float32)
    W = (r.standard_normal((K, N)) * 0.02).astype(np.float32)
    Rm = r.standard_normal((M, N)).astype(np.float32)
    Wd = np.ascontiguousarray(W.T) if bt else W
    dA, dW, dC, dR = D(A), D(Wd), fh.DeviceArray((M, N)), D(Rm)
    fh.gemm_ex(dA.ptr, K, dW.ptr, K if bt else N, bt, dC.ptr, N, M, N, K, epi,
               dR.ptr if epi == fh.EPI_RESID else 0, N)
    got = dC.numpy()
    acc = A.astype(np.float64) @ W.astype(np.float64)
    if epi == fh.EPI_GELU:
        from scipy.special import erf
        ref = 0.5 * acc * (1 + erf(acc / np.sqrt(2)))
    elif epi == fh.EPI_RESID:
        ref = Rm + acc
    else:
        ref = acc
    _close(got, ref, 1e-5)


_NT_REF = {}


def _nt_case(M, N, K, seed):
    key = (M, N, K, seed)
    if key not in _NT_REF:
        r = _rng(seed)
        A = (r.standard_normal((M, K)) * 0.5).astype(np.float32)
        Wt = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
        Rm = r.standard_normal((M, N)).astype(np.float32)
        _NT_REF[key] = (A, Wt, Rm, A.astype(np.float64) @ Wt.T.astype(np.float64))
    return _NT_REF[key]


# NT kernel (B stored N x K, direct-to-LDS copies, three stages): ragged M and N (clamped edge
# rows), K of 1, 2, 3 and many 16-wide blocks (pipeline prologue and tail), every tile shape
# (forced through FMLH_GEMM_NT_TILE) and the default choice.
@pytest.mark.parametrize("tile", ["", "128x128", "128x64", "64x64"])
@pytest.mark.parametrize("shape", [(1000, 1030, 384), (300, 2000, 48), (520, 2100, 16),
                                   (1100, 700, 32), (4096, 2304, 768)])
def test_gemm_nt_kernel_tiles(tile, shape, monkeypatch):
    M, N, K = shape
    print(f"gemm nt tile={tile or 'default'} M={M} N={N} K={K}", flush=True)
    if tile:
        monkeypatch.setenv("FMLH_GEMM_NT_TILE", tile)
    A, Wt, Rm, acc = _nt_case(M, N, K, 11)
    dA, dW, dC = D(A), D(Wt), fh.DeviceArray((M, N))
    fh.gemm_ex(dA.ptr, K, dW.ptr, K, 1, dC.ptr, N, M, N, K, fh.EPI_NONE, 0, N)
    _close(dC.numpy(), acc, 1e-5)


@pytest.mark.parametrize("epi", [fh.EPI_GELU, fh.EPI_RESID])
@pytest.mark.parametrize("tile", ["128x128", "64x64"])
def test_gemm_nt_kernel_epilogues_in_place(epi, tile, monkeypatch):
    M, N, K = 1000, 1030, 384
    print(f"gemm nt epi={epi} tile={tile}", flush=True)
    monkeypatch.setenv("FMLH_GEMM_NT_TILE", tile)
    A, Wt, Rm, acc = _nt_case(M, N, K, 11)
    dA, dW, dX = D(A), D(Wt), D(Rm)
    if epi == fh.EPI_RESID:  # C aliases R, as the block's residual add does
        fh.gemm_ex(dA.ptr, K, dW.ptr, K, 1, dX.ptr, N, M, N, K, epi, dX.ptr, N)
        ref = Rm + acc
    else:
        fh.gemm_ex(dA.ptr, K, dW.ptr, K, 1, dX.ptr, N, M, N, K, epi, 0, N)
        from scipy.special import erf
        ref = 0.5 * acc * (1 + erf(acc / np.sqrt(2)))
    _close(dX.numpy(), ref, 1e-5)


@pytest.mark.parametrize("epi", [fh.EPI_NONE, fh.EPI_GELU, fh.EPI_RESID])
@pytest.mark.parametrize("shape", [(4096, 384, 1536), (2000, 330, 1056)])
def test_gemm_nt_two_k_halves(epi, shape, monkeypatch):
    """NT products with fewer than two 64 x 64 tiles per CU and K >= 1024 run as two K halves
    (partials) plus the reduction with the epilogue; the residual case writes in place.  The
    same product with the split turned off (FMLH_GEMM_NT_SPLIT_K=0) agrees to fp32 rounding."""
    M, N, K = shape
    print(f"gemm nt two K halves epi={epi} M={M} N={N} K={K}", flush=True)
    A, Wt, Rm, acc = _nt_case(M, N, K, 5)
    dA, dW = D(A), D(Wt)
    outs = []
    for split in ("1", "0"):
        monkeypatch.setenv("FMLH_GEMM_NT_SPLIT_K", split)
        dX = D(Rm)
        fh.gemm_ex(dA.ptr, K, dW.ptr, K, 1, dX.ptr, N, M, N, K, epi, dX.ptr if epi == fh.EPI_RESID else 0, N)
        outs.append(dX.numpy())
    if epi == fh.EPI_RESID:
        ref = Rm + acc
    elif epi == fh.EPI_GELU:
        from scipy.special import erf
        ref = 0.5 * acc * (1 + erf(acc / np.sqrt(2)))
    else:
        ref = acc
    _close(outs[0], ref, 1e-5)
    _close(outs[0], outs[1], 1e-5)


@pytest.mark.parametrize("bt", [0, 1])
def test_split_k_products_back_to_back(bt):
    """Split-K products (batched-decode shapes) reduce in the launch: the last split of each
    tile adds the partials and resets the tile's arrival counter.  Several products in a row,
    of different tile counts and split factors, each with fresh inputs, must all be right (a
    counter left non-zero would skip a tile's reduction in the next product)."""
    r = _rng(17 + bt)
    shapes = [(64, 1152, 384, fh.EPI_NONE), (64, 384, 1536, fh.EPI_RESID), (64, 1152, 384, fh.EPI_NONE),
              (48, 1536, 384, fh.EPI_GELU), (64, 384, 1536, fh.EPI_RESID), (64, 1152, 384, fh.EPI_NONE)]
    for rep, (M, N, K, epi) in enumerate(shapes * 4):
        print(f"split-K product {rep}: M={M} N={N} K={K} epi={epi} bt={bt}", flush=True)
        A = (r.standard_normal((M, K)) * 0.5).astype(np.float32)
        W = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
        X = r.standard_normal((M, N)).astype(np.float32)
        dA, dW, dX = D(A), D(np.ascontiguousarray(W.T) if bt else W), D(X)
        fh.gemm_ex(dA.ptr, K, dW.ptr, K if bt else N, bt, dX.ptr, N, M, N, K, epi,
                   dX.ptr if epi == fh.EPI_RESID else 0, N)
        acc = A.astype(np.float64) @ W.astype(np.float64)
        if epi == fh.EPI_RESID:
            ref = X + acc
        elif epi == fh.EPI_GELU:
            from scipy.special import erf
            ref = 0.5 * acc * (1 + erf(acc / np.sqrt(2)))
        else:
            ref = acc
        _close(dX.numpy(), ref, 1e-5)


def test_gemm_ex_residual_in_place():
    M, N, K = 16, 384, 384
    r = _rng(5)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    X = r.standard_normal((M, N)).astype(np.float32)
    dA, dW, dX = D(A), D(W), D(X)
    fh.gemm_ex(dA.ptr, K, dW.ptr, K, 1, dX.ptr, N, M, N, K, fh.EPI_RESID, dX.ptr, N)
    _close(dX.numpy(), X + A.astype(np.float64) @ W.T.astype(np.float64), 1e-5)


@pytest.mark.parametrize("T,C,H", [(64, 64, 4), (256, 384, 6), (200, 96, 3)])
def test_matmul_strided_attention_views(T, C, H):
    """The per-head views of CausalSelfAttentionLayer.h:430-497: Q_h K_h^T with row stride C,
    then P V_h written into a column slice of Y (K = T: past one 64-wide chunk for T > 64),
    and the backward's transposed-left products P^T dY_h and dS^T Q_h (:612-660)."""
    hd = C // H
    r = _rng(9)
    Q = r.standard_normal((T, C)).astype(np.float32)
    K = r.standard_normal((T, C)).astype(np.float32)
    V = r.standard_normal((T, C)).astype(np.float32)
    dQ, dK, dV = D(Q), D(K), D(V)
    dS, dY = fh.DeviceArray((H, T, T)), fh.DeviceArray((T, C))
    for h in range(H):
        fh.matmul_strided(fh.RIGHT, dS.at(h * T * T), dQ.at(h * hd), dK.at(h * hd), T, T, hd,
                          C, 1, C, 1, T, 1)
    S = dS.numpy()
    for h in range(H):
        ref = Q[:, h * hd:(h + 1) * hd].astype(np.float64) @ K[:, h * hd:(h + 1) * hd].T.astype(np.float64)
        _close(S[h], ref, 1e-6)
    P = np.abs(S[0]) / np.abs(S[0]).sum(1, keepdims=True)
    dP = D(P.astype(np.float32))
    for h in range(H):
        fh.matmul_strided(fh.NONE, dY.at(h * hd), dP.ptr, dV.at(h * hd), T, hd, T, T, 1, C, 1, C, 1)
    Y = dY.numpy()
    for h in range(H):
        _close(Y[:, h * hd:(h + 1) * hd], P.astype(np.float64) @ V[:, h * hd:(h + 1) * hd], 1e-6)
    # dV_h = P^T dY_h: Left mode, L = P (T x T, row stride T), R = a column slice of Y.
    dVh = fh.DeviceArray((H, T, hd))
    for h in range(H):
        fh.matmul_strided(fh.LEFT, dVh.at(h * T * hd), dP.ptr, dY.at(h * hd), T, hd, T, T, 1, C, 1, hd, 1)
    G = dVh.numpy()
    for h in range(H):
        _close(G[h], P.astype(np.float64).T @ Y[:, h * hd:(h + 1) * hd].astype(np.float64), 1e-6)


@pytest.mark.parametrize("M,N,K", [(20, 30, 40), (70, 33, 300)])
def test_matmul_strided_batched_planes(M, N, K):
    r = _rng(10)
    B = 3
    A = r.standard_normal((B, M, K)).astype(np.float32)
    Bm = r.standard_normal((B, N, K)).astype(np.float32)
    dA, dB, dO = D(A), D(Bm), fh.DeviceArray((B, M, N))
    fh.matmul_strided(fh.RIGHT, dO.ptr, dA.ptr, dB.ptr, M, N, K, K, 1, K, 1, N, 1, B, M * K, N * K, M * N)
    ref = np.einsum("bmk,bnk->bmn", A.astype(np.float64), Bm.astype(np.float64))
    _close(dO.numpy(), ref, 1e-6)


@pytest.mark.parametrize("mode", [fh.NONE, fh.LEFT, fh.RIGHT, fh.BOTH])
@pytest.mark.parametrize("M,N,K", [(6, 5, 7), (40, 33, 70), (64, 64, 64)])
def test_matmul_strided_against_oracle_all_modes(mode, M, N, K):
    """fmlh_matmul_strided on operands read through element strides (row strides wider than
    the row, column strides > 1, a column-strided output) against the oracle's MulStrided
    restatement (bit-exact to the compiled reference); elements of the output buffer the product
    does not address keep their contents."""
    r = _rng(100 + mode)
    tl, tr = mode in (fh.LEFT, fh.BOTH), mode in (fh.RIGHT, fh.BOTH)
    a_rows, a_cols = (K, M) if tl else (M, K)
    b_rows, b_cols = (N, K) if tr else (K, N)
    a_cs, b_cs, c_cs = 2, 3, 2
    a_rs, b_rs, c_rs = a_cols * a_cs + 5, b_cols * b_cs + 1, N * c_cs + 3
    A = r.standard_normal(a_rows * a_rs).astype(np.float32)
    B = r.standard_normal(b_rows * b_rs).astype(np.float32)
    ref = oracle.mul_strided(mode, A, B, M, N, K, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, M * c_rs)
    dA, dB = D(A), D(B)
    dO = D(np.zeros(M * c_rs, np.float32))
    fh.matmul_strided(mode, dO.ptr, dA.ptr, dB.ptr, M, N, K, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs)
    got = dO.numpy()
    assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))
    written = np.zeros(M * c_rs, bool)
    for i in range(M):
        written[i * c_rs + np.arange(N) * c_cs] = True
    assert not got[~written].any()


@pytest.mark.parametrize("rows,cols", [(1, 64), (256, 256), (5, 4096), (3, 65)])
def test_softmax(rows, cols):
    r = _rng(rows + cols)
    x = (r.standard_normal((rows, cols)) * 3).astype(np.float32)
    if cols >= 64:
        x = oracle.scale_add(x, 0.125, oracle.triangle_lower(rows, cols, 0.0, -np.inf))
    dX, dO = D(x), fh.DeviceArray((rows, cols))
    fh.softmax(dO.ptr, dX.ptr, rows, cols)
    got = dO.numpy()
    ref = oracle.softmax(x)
    np.testing.assert_allclose(got, ref, rtol=5e-6, atol=1e-9)
    assert np.all(got[np.isinf(x)] == 0.0)


@pytest.mark.parametrize("rows,cols,beta", [(1, 384, False), (300, 768, True), (7, 64, False), (2, 100, True)])
def test_layernorm(rows, cols, beta):
    r = _rng(rows * cols)
    x = (r.standard_normal((rows, cols)) * 2 + 0.3).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    b = r.standard_normal(cols).astype(np.float32) if beta else None
    dX, dG, dO, dH = D(x), D(g), fh.DeviceArray((rows, cols)), fh.DeviceArray((rows, cols))
    dB = D(b) if beta else None
    fh.layernorm(dO.ptr, dX.ptr, dG.ptr, dB.ptr if beta else 0, dH.ptr, rows, cols)
    ref = oracle.layernorm(x, g, b)
    np.testing.assert_allclose(dO.numpy(), ref, rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(dH.numpy(), oracle.layernorm(x, np.ones(cols, np.float32)), rtol=1e-5, atol=2e-6)


def test_gelu_and_elementwise():
    r = _rng(12)
    n = 100_003
    x = (r.standard_normal(n) * 3).astype(np.float32)
    y = r.standard_normal(n).astype(np.float32)
    dx, dy, do = D(x), D(y), fh.DeviceArray(n)
    fh.gelu(do.ptr, dx.ptr, n)
    np.testing.assert_allclose(do.numpy(), oracle.gelu(x), rtol=2e-6, atol=5e-7)
    fh.add(do.ptr, dx.ptr, dy.ptr, n)
    np.testing.assert_array_equal(do.numpy(), x + y)
    fh.per_element_mul(do.ptr, dx.ptr, dy.ptr, n)
    np.testing.assert_array_equal(do.numpy(), x * y)
    fh.scale_scalar(do.ptr, dx.ptr, 0.25, n)
    np.testing.assert_array_equal(do.numpy(), x * np.float32(0.25))
    s = D(np.array([1.5], np.float32))
    fh.scale(do.ptr, dx.ptr, s.ptr, n)
    np.testing.assert_array_equal(do.numpy(), x * np.float32(1.5))
    fh.fill(do.ptr, 2.5, n)
    np.testing.assert_array_equal(do.numpy(), np.full(n, 2.5, np.float32))
    fh.fill_from(do.ptr, s.ptr, n)
    np.testing.assert_array_equal(do.numpy(), np.full(n, 1.5, np.float32))
    fh.copy(do.ptr, dy.ptr, n)
    np.testing.assert_array_equal(do.numpy(), y)
    m = D(oracle.triangle_lower(1, n, 0.0, -np.inf)[0])
    fh.scale_add(do.ptr, dx.ptr, s.ptr, m.ptr, n)
    np.testing.assert_array_equal(do.numpy(), oracle.scale_add(x, 1.5, oracle.triangle_lower(1, n, 0.0, -np.inf)[0]))
    bias = r.standard_normal(7).astype(np.float32)
    db = D(bias)
    fh.broadcast_add(do.ptr, dx.ptr, db.ptr, 7 * 1000, 7)
    np.testing.assert_array_equal(do.numpy()[:7000], x[:7000] + np.tile(bias, 1000))


def test_gather_split_argmax():
    r = _rng(13)
    V, C, T = 65, 64, 33
    W = r.standard_normal((V, C)).astype(np.float32)
    ids = r.integers(0, V, size=(2, T)).astype(np.float32)
    ids[1, 3] = V + 5  # out of range -> zero row
    dW, dI, dO = D(W), D(ids), fh.DeviceArray((2, T, C))
    fh.gather_rows(dO.ptr, dW.ptr, dI.ptr, C, T, 2, V, 1)
    got = dO.numpy()
    exp = W[np.minimum(ids.astype(np.int64), V - 1)]
    exp[1, 3] = 0.0
    np.testing.assert_array_equal(got, exp)
    # In-range rows against the oracle's GatherRows restatement (bit-exact to the reference).
    np.testing.assert_array_equal(got[0], oracle.gather_rows(W, ids[0]))
    keep = np.arange(T) != 3
    np.testing.assert_array_equal(got[1][keep], oracle.gather_rows(W, ids[1][keep]))
    packed = r.standard_normal((T, 3 * C)).astype(np.float32)
    dp = D(packed)
    q, k, v = (fh.DeviceArray((T, C)) for _ in range(3))
    fh.split_qkv(q.ptr, k.ptr, v.ptr, dp.ptr, T, C)
    np.testing.assert_array_equal(q.numpy(), packed[:, :C])
    np.testing.assert_array_equal(k.numpy(), packed[:, C:2 * C])
    np.testing.assert_array_equal(v.numpy(), packed[:, 2 * C:])
    logits = r.standard_normal((9, 50304)).astype(np.float32)
    logits[2, 10] = logits[2, 40000] = 99.0  # tie: first index wins
    logits[5, :] = 1.0
    dl, di = D(logits), fh.DeviceArray(9, np.int32)
    fh.row_argmax(di.ptr, dl.ptr, 9, 50304)
    got = di.numpy()
    exp = [oracle.argmax(row) for row in logits]
    assert got.tolist() == exp
    assert got[2] == 10 and got[5] == 0


def test_bad_arguments_raise():
    with pytest.raises(fh.FreeMLHipError):
        fh.mul(7, 0, 0, 0, 1, 1, 1)
    a = fh.DeviceArray(4)
    with pytest.raises(fh.FreeMLHipError):
        fh.gemm_ex(a.ptr, 2, a.ptr, 2, 0, a.ptr, 2, 2, 2, 2, fh.EPI_RESID, 0, 2)
