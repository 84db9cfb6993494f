"""CPU oracle for the NanoLLM token loop — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the timed CPU baseline: the product path
(``freeml_amd``) never does.

* ``OracleModel`` wraps ``libnanollm_oracle.so``, the plain-C restatement of the reference's
  MatrixCPU arithmetic (``nanollm_oracle.c``; per-function reference citations there).
* ``RefModel`` wraps ``_ref/libfreeml_ref.so``, the reference itself compiled from
  ``/root/reference`` by ``make -C oracle ref`` (built in the development container; the file
  travels with the tree, the sources do not).

Parity pins for each oracle function are listed in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "libnanollm_oracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libfreeml_ref.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32 = ctypes.c_uint32

NONE, LEFT, RIGHT, BOTH = 0, 1, 2, 3


def build(reference: bool = False) -> None:
    """Compile the oracle (and with ``reference=True`` the reference harness) via make."""
    cmd = ["make", "-s", "-C", _HERE, "ref" if reference else "all"]
    subprocess.run(cmd, check=True)


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def _ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_i32p)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        L.orc_mul.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _u32, _u32, _u32, ctypes.c_int]
        L.orc_mul_strided.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p] + [_u32] * 9
        L.orc_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _u32, _u32, ctypes.c_float]
        L.orc_softmax.argtypes = [_f32p, _f32p, _u32, _u32]
        L.orc_scale_add.argtypes = [_f32p, _f32p, ctypes.c_float, _f32p, _u32]
        L.orc_gelu.argtypes = [_f32p, _f32p, _u32]
        L.orc_add.argtypes = [_f32p, _f32p, _f32p, _u32]
        L.orc_gather_rows.argtypes = [_f32p, _f32p, _f32p, _u32, _u32]
        L.orc_split_qkv.argtypes = [_f32p, _f32p, _f32p, _f32p, _u32, _u32]
        L.orc_triangle_lower.argtypes = [_f32p, _u32, _u32, ctypes.c_float, ctypes.c_float]
        L.orc_argmax.argtypes = [_f32p, _u32]
        L.orc_argmax.restype = _u32
        L.orc_model_create.argtypes = [_u32] * 5 + [_f32p, _f32p, ctypes.POINTER(_f32p), _f32p,
                                                    _f32p, _f32p, ctypes.c_int]
        L.orc_model_create.restype = ctypes.c_void_p
        L.orc_model_destroy.argtypes = [ctypes.c_void_p]
        L.orc_forward_window.argtypes = [ctypes.c_void_p, _i32p, _f32p]
        for fn in (L.orc_greedy_window, L.orc_greedy_cached):
            fn.argtypes = [ctypes.c_void_p, _i32p, _u32, _u32, _i32p, _f32p]
        _lib = L
    return _lib


# ---- per-op wrappers (numpy in, numpy out) ----------------------------------------------

def mul(mode: int, L: np.ndarray, R: np.ndarray, nthreads: int = 1) -> np.ndarray:
    tl = mode in (LEFT, BOTH)
    tr = mode in (RIGHT, BOTH)
    M, K = (L.shape[1], L.shape[0]) if tl else L.shape
    N = R.shape[0] if tr else R.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    lib().orc_mul(mode, _fp(out), _fp(L), _fp(R), M, N, K, nthreads)
    return out


def layernorm(x: np.ndarray, gamma: np.ndarray, beta=None, eps: float = 1e-5) -> np.ndarray:
    out = np.empty_like(x)
    rows, cols = x.shape
    lib().orc_layernorm(_fp(out), _fp(x), _fp(gamma), _fp(beta) if beta is not None else None,
                        None, rows, cols, eps)
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    lib().orc_softmax(_fp(out), _fp(x), x.shape[0], x.shape[1])
    return out


def gelu(x: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    lib().orc_gelu(_fp(out), _fp(x), x.size)
    return out


def scale_add(x: np.ndarray, scale: float, add: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    lib().orc_scale_add(_fp(out), _fp(x), scale, _fp(add), x.size)
    return out


def triangle_lower(rows: int, cols: int, true_val: float, false_val: float) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    lib().orc_triangle_lower(_fp(out), rows, cols, true_val, false_val)
    return out


def argmax(row: np.ndarray) -> int:
    return int(lib().orc_argmax(_fp(row), row.size))


# ---- training-step ops: the oracle's restatements (impl="oracle") and the compiled
# reference's own routines (impl="ref", oracle/_ref/libfreeml_ref.so), same signatures -------

_TRAIN_SIGS = {
    "softmax_backward": ([_f32p] * 3 + [_u32] * 2, None),
    "layernorm_backward": ([_f32p] * 7 + [_u32, _u32, ctypes.c_float], None),
    "gelu_derivative": ([_f32p, _f32p, _u32], None),
    "scatter_add_rows": ([_f32p] * 3 + [_u32] * 5, None),
    "merge_qkv": ([_f32p] * 4 + [_u32] * 3, None),
    "cce_logits": ([_f32p] * 3 + [_u32] * 5, ctypes.c_float),
    "adamw_update": ([_f32p] * 4 + [_u32] + [ctypes.c_float] * 7, None),
    "sum_columns": ([_f32p] * 2 + [_u32] * 2, None),
}


def _train_fn(impl: str, name: str):
    L = lib() if impl == "oracle" else ref_lib()
    f = getattr(L, ("orc_" if impl == "oracle" else "ref_") + name)
    f.argtypes, f.restype = _TRAIN_SIGS[name]
    return f


def _opt(a):
    return _fp(a) if a is not None else ctypes.cast(None, _f32p)


def softmax_backward(p: np.ndarray, dp: np.ndarray, impl: str = "oracle") -> np.ndarray:
    """p, dp: (rows, cols)."""
    out = np.empty_like(p)
    _train_fn(impl, "softmax_backward")(_fp(out), _fp(p), _fp(dp), p.shape[0], p.shape[1])
    return out


def layernorm_backward(dy, x, gamma, xhat=None, with_beta=True, eps=1e-5, impl="oracle"):
    """dy, x, xhat: (rows, cols).  Returns (dx, dgamma, dbeta or None)."""
    rows, cols = x.shape
    dx = np.empty_like(x)
    dg = np.empty(cols, np.float32)
    db = np.empty(cols, np.float32) if with_beta else None
    _train_fn(impl, "layernorm_backward")(_fp(dx), _fp(dy), _fp(x), _fp(gamma), _fp(dg), _opt(db),
                                          _opt(xhat), rows, cols, eps)
    return dx, dg, db


def gelu_derivative(x: np.ndarray, impl: str = "oracle") -> np.ndarray:
    out = np.empty_like(x)
    _train_fn(impl, "gelu_derivative")(_fp(out), _fp(x), x.size)
    return out


def scatter_add_rows(out: np.ndarray, src: np.ndarray, idx: np.ndarray, impl: str = "oracle"):
    """out: (out_batch, out_rows, width), accumulated into a copy; src: (src_batch, src_rows,
    width); idx: (src_batch, src_rows) float ids."""
    res = out.copy()
    _train_fn(impl, "scatter_add_rows")(_fp(res), _fp(src), _fp(idx), src.shape[2], src.shape[1],
                                        src.shape[0], out.shape[1], out.shape[0])
    return res


def merge_qkv(q: np.ndarray, k: np.ndarray, v: np.ndarray, impl: str = "oracle") -> np.ndarray:
    """q, k, v: (n_head, tokens, head_dim) -> (tokens, 3 * n_head * head_dim)."""
    nh, tokens, hd = q.shape
    out = np.empty((tokens, 3 * nh * hd), np.float32)
    _train_fn(impl, "merge_qkv")(_fp(out), _fp(q), _fp(k), _fp(v), hd, tokens, nh)
    return out


def sum_columns(x: np.ndarray, impl: str = "oracle") -> np.ndarray:
    """SumColumns (MatrixBase_Functions.h:1098-1118) of a (rows, cols) matrix."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape[1], np.float32)
    _train_fn(impl, "sum_columns")(_fp(out), _fp(x), x.shape[0], x.shape[1])
    return out


def dropout_mask(n: int, uniforms: np.ndarray, start: int, prob: float):
    """UpdateMask's mask of n elements with draws from `uniforms` starting at `start`: (mask,
    draws made)."""
    uniforms = np.ascontiguousarray(uniforms, np.float32)
    out = np.empty(n, np.float32)
    f = lib().orc_dropout_mask
    f.argtypes = [_f32p, ctypes.c_uint64, _f32p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]
    f.restype = ctypes.c_uint64
    used = f(_fp(out), n, _fp(uniforms), uniforms.size, start, prob)
    return out, int(used)


def ref_uniform_buffer(n: int):
    """(first n floats of the compiled reference's RandomUtils uniform buffer, its size)."""
    out = np.empty(n, np.float32)
    f = ref_lib().ref_uniform_buffer
    f.argtypes, f.restype = [_f32p, ctypes.c_uint64], ctypes.c_uint64
    count = f(_fp(out), n)
    return out, int(count)


def ref_dropout_mask(n: int, prob: float) -> np.ndarray:
    """The compiled reference's DropoutLayer::UpdateMask on n elements (advances its index)."""
    out = np.empty(n, np.float32)
    f = ref_lib().ref_dropout_mask
    f.argtypes = [_f32p, _u32, ctypes.c_float]
    f(_fp(out), n, prob)
    return out


def cce_logits(target: np.ndarray, logits: np.ndarray, impl: str = "oracle"):
    """logits: (batch, steps, vocab); target: (target_batch, steps) ids or (target_batch,
    steps, vocab) one-hot.  Returns (gradient, loss)."""
    batch, steps, vocab = logits.shape
    tcols = 1 if target.ndim == 2 else target.shape[2]
    grad = np.empty_like(logits)
    loss = _train_fn(impl, "cce_logits")(_fp(grad), _fp(target), _fp(logits), vocab, steps, batch,
                                         tcols, target.shape[0])
    return grad, float(loss)


def adam_powers(beta1: float, beta2: float, t: int):
    """beta^t as AdamWOptimiser::Step forms them: std::pow(float, uint64_t) evaluates in
    double and is stored as float (OptimiserLibrary/AdamWOptimiser.h:163-165)."""
    return (float(np.float32(float(np.float32(beta1)) ** t)), float(np.float32(float(np.float32(beta2)) ** t)))


def adamw_update(param, grad, mt, vt, lr, beta1, beta2, t, eps, weight_decay, impl="oracle"):
    """Returns updated copies (param, mt, vt)."""
    p, m, v = param.copy(), mt.copy(), vt.copy()
    b1t, b2t = adam_powers(beta1, beta2, t)
    _train_fn(impl, "adamw_update")(_fp(p), _fp(grad), _fp(m), _fp(v), p.size, lr, beta1, beta2, b1t,
                                    b2t, eps, weight_decay)
    return p, m, v


# ---- models ------------------------------------------------------------------------------

def _layer_ptr_array(weights):
    ptrs = []
    for lw in weights.layers:
        for a in (lw.w_qkv, lw.w_proj, lw.w_fc, lw.w_proj2, lw.ln0_g, lw.ln0_b, lw.ln1_g, lw.ln1_b):
            ptrs.append(_fp(a) if a is not None else ctypes.cast(None, _f32p))
    return (_f32p * len(ptrs))(*ptrs)


class OracleModel:
    """The C restatement over one set of ``freeml_amd.synth.NanoLLMWeights``."""

    def __init__(self, weights, nthreads: int = 1):
        s = weights.shape
        self.w = weights  # keeps the arrays alive
        self.V = s.vocab
        self.T = s.block_size
        self._ptrs = _layer_ptr_array(weights)
        lnf_b = _fp(weights.lnf_b) if weights.lnf_b is not None else None
        self.h = lib().orc_model_create(s.vocab, s.block_size, s.n_embed, s.n_head, s.n_layer,
                                        _fp(weights.tok_emb), _fp(weights.pos_emb), self._ptrs,
                                        _fp(weights.lnf_g), lnf_b, _fp(weights.lm_head), nthreads)
        if not self.h:
            raise ValueError("orc_model_create rejected the shape")

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward_window(self, ids: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((self.T, self.V), dtype=np.float32)
        rc = lib().orc_forward_window(self.h, _ip(ids), _fp(out))
        if rc:
            raise ValueError(f"orc_forward_window failed ({rc})")
        return out

    def greedy(self, prompt: np.ndarray, n_gen: int, cached: bool = True):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.empty(n_gen, dtype=np.int32)
        logits = np.empty((n_gen, self.V), dtype=np.float32)
        fn = lib().orc_greedy_cached if cached else lib().orc_greedy_window
        rc = fn(self.h, _ip(prompt), prompt.size, n_gen, _ip(toks), _fp(logits))
        if rc:
            raise ValueError(f"oracle greedy failed ({rc})")
        return toks, logits


_ref = None


def gather_rows(src: np.ndarray, ids: np.ndarray, impl: str = "oracle") -> np.ndarray:
    """GatherRows (MatrixBase_Functions.h:202-242) of one plane: out[r] = src[int(ids[r])]."""
    src = np.ascontiguousarray(src, np.float32)
    ids = np.ascontiguousarray(ids, np.float32)
    out = np.empty((ids.shape[0], src.shape[1]), np.float32)
    if impl == "oracle":
        lib().orc_gather_rows(_fp(out), _fp(src), _fp(ids), src.shape[1], ids.shape[0])
    else:
        f = ref_lib().ref_gather_rows
        f.argtypes = [_f32p, _f32p, _f32p, _u32, _u32, _u32]
        f(_fp(out), _fp(src), _fp(ids), src.shape[1], ids.shape[0], src.shape[0])
    return out


def mul_strided(mode: int, A: np.ndarray, B: np.ndarray, M: int, N: int, K: int, a_rs: int, a_cs: int,
                b_rs: int, b_cs: int, c_rs: int, c_cs: int, c_size: int, impl: str = "oracle") -> np.ndarray:
    """MulStrided<Mode> (MatrixBase_Mul.h:88-144) over flat buffers A, B; returns the flat C
    buffer of c_size elements (elements the product does not write stay 0)."""
    A = np.ascontiguousarray(A, np.float32).reshape(-1)
    B = np.ascontiguousarray(B, np.float32).reshape(-1)
    C = np.zeros(c_size, np.float32)
    if impl == "oracle":
        lib().orc_mul_strided(mode, _fp(C), _fp(A), _fp(B), M, N, K, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs)
    else:
        f = ref_lib().ref_mul_strided
        f.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p] + [_u32] * 9
        f(mode, _fp(C), _fp(A), _fp(B), M, N, K, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs)
    return C


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        L = ctypes.CDLL(REF_SO)
        L.ref_create.argtypes = [_u32] * 5 + [_f32p, _f32p, ctypes.POINTER(_f32p), _f32p, _f32p]
        L.ref_create.restype = ctypes.c_void_p
        L.ref_forward_window.argtypes = [ctypes.c_void_p, _i32p, _f32p]
        L.ref_greedy.argtypes = [ctypes.c_void_p, _i32p, _u32, _u32, _i32p, _f32p]
        L.ref_thread_count.restype = _u32
        _ref = L
    return _ref


class RefModel:
    """The compiled reference (MatrixCPU<float>, its global ThreadPool) over the same weights."""

    def __init__(self, weights):
        s = weights.shape
        if weights.lnf_b is not None or any(l.ln0_b is not None for l in weights.layers):
            raise ValueError("the reference NanoLLM graph has use_bias=false")
        self.w = weights
        self.V = s.vocab
        self.T = s.block_size
        self._ptrs = _layer_ptr_array(weights)
        self.h = ref_lib().ref_create(s.vocab, s.block_size, s.n_embed, s.n_head, s.n_layer,
                                      _fp(weights.tok_emb), _fp(weights.pos_emb), self._ptrs,
                                      _fp(weights.lnf_g), _fp(weights.lm_head))
        if not self.h:
            raise ValueError("ref_create rejected the config")

    @staticmethod
    def threads() -> int:
        return int(ref_lib().ref_thread_count())

    def forward_window(self, ids: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((self.T, self.V), dtype=np.float32)
        if ref_lib().ref_forward_window(self.h, _ip(ids), _fp(out)):
            raise RuntimeError("ref_forward_window failed")
        return out

    def greedy(self, prompt: np.ndarray, n_gen: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.empty(n_gen, dtype=np.int32)
        logits = np.empty((n_gen, self.V), dtype=np.float32)
        if ref_lib().ref_greedy(self.h, _ip(prompt), prompt.size, n_gen, _ip(toks), _fp(logits)):
            raise RuntimeError("ref_greedy failed")
        return toks, logits


# ---- the NanoLLM example's text front end, compiled from the reference (oracle/_ref) -------

def _ref_text_lib():
    L = ref_lib()
    c_p = ctypes.c_char_p
    u32p = ctypes.POINTER(_u32)
    L.ref_build_vocab.argtypes = [c_p, ctypes.c_size_t, ctypes.c_void_p, u32p]
    L.ref_build_vocab.restype = _u32
    L.ref_encode.argtypes = [c_p, _u32, c_p, ctypes.c_size_t, u32p]
    L.ref_decode.argtypes = [c_p, _u32, u32p, ctypes.c_size_t, ctypes.c_void_p]
    L.ref_decode_matrix_tokens.argtypes = [_f32p, _u32, _u32, c_p, _u32, ctypes.c_void_p]
    L.ref_count_correct.argtypes = [_f32p, _f32p, _u32, _u32]
    L.ref_count_correct.restype = _u32
    return L


def ref_build_vocab(data: bytes):
    """(unique chars, ids) from the reference's BuildVocab (NanoLLM.cpp:121-144)."""
    L = _ref_text_lib()
    uniq = ctypes.create_string_buffer(256)
    ids = np.empty(len(data), np.uint32)
    n = L.ref_build_vocab(data, len(data), uniq, ids.ctypes.data_as(ctypes.POINTER(_u32)))
    return uniq.raw[:n], ids


def ref_encode(unique: bytes, s: bytes) -> np.ndarray:
    L = _ref_text_lib()
    ids = np.empty(len(s), np.uint32)
    L.ref_encode(unique, len(unique), s, len(s), ids.ctypes.data_as(ctypes.POINTER(_u32)))
    return ids


def ref_decode(unique: bytes, ids) -> bytes:
    L = _ref_text_lib()
    ids = np.ascontiguousarray(ids, np.uint32)
    out = ctypes.create_string_buffer(max(1, ids.size))
    L.ref_decode(unique, len(unique), ids.ctypes.data_as(ctypes.POINTER(_u32)), ids.size, out)
    return out.raw[:ids.size]


def ref_decode_matrix_tokens(mat: np.ndarray, unique: bytes) -> bytes:
    L = _ref_text_lib()
    mat = np.ascontiguousarray(mat, np.float32)
    steps, cols = mat.shape
    out = ctypes.create_string_buffer(max(1, steps))
    L.ref_decode_matrix_tokens(_fp(mat), cols, steps, unique, len(unique), out)
    return out.raw[:steps]


def ref_count_correct(logits: np.ndarray, target) -> int:
    L = _ref_text_lib()
    logits = np.ascontiguousarray(logits, np.float32)
    t = np.ascontiguousarray(target, np.float32)
    return int(L.ref_count_correct(_fp(logits), _fp(t), logits.shape[0], logits.shape[1]))


# ---- sampling restatement (fmlh_nanollm_set_sampling; no counterpart in the reference) -----

_M64 = (1 << 64) - 1


def splitmix64(x: int) -> int:
    """Vigna's splitmix64 output function applied to x + golden gamma."""
    x = (x + 0x9E3779B97F4A7C15) & _M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _M64
    return x ^ (x >> 31)


def sample_uniform(seed: int, b: int, p: int) -> float:
    """u in [0, 1) on a 2^-24 grid for sequence b filling position p."""
    key = ((b & 0xFFFFFFFF) << 32) | (p & 0xFFFFFFFF)
    return (splitmix64((seed ^ splitmix64(key)) & _M64) >> 40) / float(1 << 24)


def sample_token(z: np.ndarray, temperature: float, top_k: int, seed: int, b: int, p: int):
    """(token, margin): the draw fmlh_nanollm_set_sampling defines, evaluated in float64 from
    the float32 logits row; margin = distance of u * total to the nearest CDF boundary over
    total (a device draw can differ only when it is within float rounding of a boundary)."""
    z = np.asarray(z, np.float32)
    V = z.size
    keep = np.ones(V, bool)
    if 0 < top_k < V:
        order = np.lexsort((np.arange(V), -z.astype(np.float64)))  # value desc, index asc
        keep[:] = False
        keep[order[:top_k]] = True
    inv_t = float(np.float32(1.0) / np.float32(temperature))
    m = float(z.max())
    w = np.where(keep, np.exp((z.astype(np.float64) - m) * inv_t), 0.0)
    cdf = np.cumsum(w)
    total = cdf[-1]
    target = sample_uniform(seed, b, p) * total
    idx = np.nonzero((cdf > target) & (w > 0))[0]
    tok = int(idx[0]) if idx.size else int(np.nonzero(w > 0)[0][-1])
    margin = float(np.min(np.abs(cdf[w > 0] - target)) / total)
    return tok, margin
