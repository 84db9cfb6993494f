"""MI355X (gfx950) backend for FreeML's NanoLLM token loop — Python host binding.

This package binds ``lib/libfreeml_hip.so`` (the C ABI declared in ``include/freeml_hip.h``)
with ctypes.  It mirrors the reference's operator API for the hot path — ``mul``,
``matmul_strided``, ``softmax``, ``layernorm``, ``gelu``, ``gather_rows``, ... with the
argument meaning of FreeML's free functions (MatrixLibrary/MatrixBase_Functions.h,
MatrixBase_Mul.h) — and the NanoLLM graph (Examples/NanoLLM/NanoLLM.cpp:255-376) as
``NanoLLM``.  There is no CPU fallback: if the native library is missing or no gfx950 device
is present every call raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import synth  # noqa: F401  (re-exported: seeded benchmark inputs)

_HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(_HERE, "lib", "libfreeml_hip.so")
PROBE_LIB_PATH = os.path.join(_HERE, "lib", "libfreeml_probe.so")
HEADER = os.path.join(ROOT, "include", "freeml_hip.h")
PROBE_HEADER = os.path.join(ROOT, "include", "freeml_probe.h")

NONE, LEFT, RIGHT, BOTH = 0, 1, 2, 3  # TransposeMode (MatrixBase_Mul.h:27)
EPI_NONE, EPI_GELU, EPI_RESID = 0, 1, 2


class FreeMLHipError(RuntimeError):
    """A C-ABI call returned a non-zero status; the message is fmlh_last_error()."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def build(force: bool = False) -> None:
    """Compile libfreeml_hip.so for gfx950 in-tree (make -C freeml_amd/csrc)."""
    cmd = ["make", "-s", "-C", os.path.join(_HERE, "csrc"), f"-j{min(8, os.cpu_count() or 1)}"]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)


_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32 = ctypes.c_uint32
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t


class NanoLLMConfig(ctypes.Structure):
    _fields_ = [("vocab", _u32), ("block_size", _u32), ("n_embed", _u32), ("n_head", _u32),
                ("n_layer", _u32), ("max_batch", _u32)]


class NanoLLMWeightsC(ctypes.Structure):
    _fields_ = [("tok_emb", _f32p), ("pos_emb", _f32p), ("layers", ctypes.POINTER(_f32p)),
                ("lnf_gamma", _f32p), ("lnf_beta", _f32p), ("lm_head", _f32p)]


_SIGS = {
    "fmlh_init": [ctypes.c_int],
    "fmlh_shutdown": [],
    "fmlh_device_info": [ctypes.c_char_p, _sz, ctypes.POINTER(ctypes.c_int)],
    "fmlh_malloc": [ctypes.POINTER(_vp), _sz],
    "fmlh_free": [_vp],
    "fmlh_memcpy_h2d": [_vp, _vp, _sz],
    "fmlh_memcpy_d2h": [_vp, _vp, _sz],
    "fmlh_memcpy_d2d": [_vp, _vp, _sz],
    "fmlh_synchronize": [],
    "fmlh_event_create": [ctypes.POINTER(_vp)],
    "fmlh_event_destroy": [_vp],
    "fmlh_event_record": [_vp],
    "fmlh_event_elapsed_ms": [_vp, _vp, ctypes.POINTER(ctypes.c_float)],
    "fmlh_mul": [ctypes.c_int, _vp, _vp, _vp, _u32, _u32, _u32],
    "fmlh_gemm_ex": [_vp, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int,
                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int],
    "fmlh_gemm_ex_noalloc": [_vp, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int,
                             ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int],
    "fmlh_matmul_strided": [ctypes.c_int, _vp, _vp, _vp] + [_u32] * 10 + [_sz] * 3,
    "fmlh_softmax": [_vp, _vp, _u32, _u32],
    "fmlh_layernorm": [_vp, _vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float],
    "fmlh_gelu": [_vp, _vp, _sz],
    "fmlh_add": [_vp, _vp, _vp, _sz],
    "fmlh_copy": [_vp, _vp, _sz],
    "fmlh_gather_rows": [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32],
    "fmlh_split_qkv": [_vp, _vp, _vp, _vp, _u32, _u32],
    "fmlh_scale_add": [_vp, _vp, _vp, _vp, _sz],
    "fmlh_broadcast_add": [_vp, _vp, _vp, _sz, _u32],
    "fmlh_fill": [_vp, ctypes.c_float, _sz],
    "fmlh_fill_from": [_vp, _vp, _sz],
    "fmlh_per_element_mul": [_vp, _vp, _vp, _sz],
    "fmlh_scale": [_vp, _vp, _vp, _sz],
    "fmlh_scale_scalar": [_vp, _vp, ctypes.c_float, _sz],
    "fmlh_row_argmax": [_vp, _vp, _u32, _u32],
    "fmlh_softmax_backward": [_vp, _vp, _vp, _u32, _u32],
    "fmlh_layernorm_backward": [_vp] * 8 + [_u32, _u32, ctypes.c_float],
    "fmlh_gelu_derivative": [_vp, _vp, _sz],
    "fmlh_scatter_add_rows": [_vp, _vp, _vp] + [_u32] * 5,
    "fmlh_cce_logits": [_vp] * 5 + [_u32] * 5,
    "fmlh_adamw_update": [_vp, _vp, _vp, _vp, _sz] + [ctypes.c_float] * 7,
    "fmlh_sum_columns": [_vp, _vp, _u32, _u32],
    "fmlh_dropout_mask": [_vp, ctypes.c_uint64, _vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float],
    "fmlh_merge_qkv": [_vp] * 4 + [_u32] * 3,
    "fmlh_attention_softmax_heads": [ctypes.POINTER(_vp), _sz, _vp, _vp, _vp, _u32, _u32],
    "fmlh_attention_softmax_backward_heads": [_vp, ctypes.POINTER(_vp), _vp, _vp, _u32, _u32],
    "fmlh_nanollm_create": [ctypes.POINTER(NanoLLMConfig), ctypes.POINTER(NanoLLMWeightsC),
                            ctypes.c_int, ctypes.POINTER(_vp)],
    "fmlh_nanollm_destroy": [_vp],
    "fmlh_nanollm_refresh_weights": [_vp],
    "fmlh_nanollm_prefill": [_vp, _i32p, _u32, _u32],
    "fmlh_nanollm_decode": [_vp, _u32],
    "fmlh_nanollm_read_tokens": [_vp, _i32p, _u32, _u32],
    "fmlh_nanollm_read_logits": [_vp, _f32p],
    "fmlh_nanollm_status": [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u32)],
    "fmlh_nanollm_decode_path": [_vp, _u32, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)],
    "fmlh_nanollm_generate": [_vp, _i32p, _u32, _u32, _u32, _i32p, _f32p],
    "fmlh_nanollm_set_sampling": [_vp, ctypes.c_float, _u32, ctypes.c_ulonglong],
    "fmlh_nanollm_forward_window": [_vp, _i32p, _u32, _f32p],
    "fmlh_nanollm_profile_op": [_vp, ctypes.c_int, _u32, ctypes.POINTER(ctypes.c_float),
                                ctypes.POINTER(ctypes.c_double)],
}
# The measurement library (include/freeml_probe.h), loaded on first use.
_PROBE_SIGS = {
    "fmlh_probe_exchange": [ctypes.c_int, _i32p, _u32, _i32p, _u32, _u32, _u32, _i32p,
                            ctypes.POINTER(ctypes.c_double)],
}

_lib = None
_shut = False  # fmlh_shutdown ran at interpreter exit: objects freed later skip the library


def _shutdown_at_exit() -> None:
    """Releases the library's device objects while the HIP runtime is still alive; objects
    collected after this (during interpreter teardown) leave their memory to the process exit."""
    global _shut
    _shut = True
    if _lib is not None:
        _lib.fmlh_shutdown()


def lib() -> ctypes.CDLL:
    """The loaded native library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FreeMLHipError("load", -1, f"{LIB_PATH} is missing: run freeml_amd.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.fmlh_last_error.argtypes = []
        L.fmlh_last_error.restype = ctypes.c_char_p
        L.fmlh_get_stream.argtypes = []
        L.fmlh_get_stream.restype = _vp
        _lib = L
        import atexit

        atexit.register(_shutdown_at_exit)
    return _lib


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        msg = lib().fmlh_last_error().decode(errors="replace")
        raise FreeMLHipError(fn, rc, msg)


def call(fn: str, *args) -> None:
    _check(fn, getattr(lib(), fn)(*args))


def init(device: int = 0) -> None:
    call("fmlh_init", device)


def device_info():
    buf = ctypes.create_string_buffer(64)
    cus = ctypes.c_int(0)
    call("fmlh_device_info", buf, 64, ctypes.byref(cus))
    return buf.value.decode(), cus.value


def synchronize() -> None:
    call("fmlh_synchronize")


class DeviceArray:
    """A device fp32/int32 buffer owned by Python (fmlh_malloc / fmlh_free)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = _vp()
        call("fmlh_malloc", ctypes.byref(p), max(self.nbytes, 4))
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        call("fmlh_memcpy_h2d", self.ptr, a.ctypes.data, self.nbytes)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        call("fmlh_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def at(self, elem_offset: int) -> int:
        """Device address of element ``elem_offset`` (a view, as SetData(ptr, offset))."""
        return self.ptr + int(elem_offset) * self.dtype.itemsize

    def free(self) -> None:
        if getattr(self, "ptr", None):
            if not _shut:
                call("fmlh_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Timer:
    """HIP events on the library stream bracketing enqueued work."""

    def __init__(self):
        self.a, self.b = _vp(), _vp()
        call("fmlh_event_create", ctypes.byref(self.a))
        call("fmlh_event_create", ctypes.byref(self.b))

    def start(self):
        call("fmlh_event_record", self.a)

    def stop(self) -> float:
        call("fmlh_event_record", self.b)
        ms = ctypes.c_float()
        call("fmlh_event_elapsed_ms", self.a, self.b, ctypes.byref(ms))
        return ms.value


# ---- operator API (device pointers in, results in device memory) -------------------------

def mul(mode: int, out: int, L: int, R: int, M: int, N: int, K: int) -> None:
    """Mul<Mode>(out, L, R) (MatrixBase_Mul.h:591-615)."""
    call("fmlh_mul", mode, out, L, R, M, N, K)


def gemm_ex(A: int, lda: int, B: int, ldb: int, b_trans: int, C: int, ldc: int, M: int, N: int,
            K: int, epi: int = EPI_NONE, R: int = 0, ldr: int = 0) -> None:
    """Dense projection with fused epilogue (Dense.h:201-222 + the residual Add)."""
    call("fmlh_gemm_ex", A, lda, B, ldb, b_trans, C, ldc, M, N, K, epi, R or None, ldr)


def matmul_strided(mode, out, L, R, M, N, K, l_rs, l_cs, r_rs, r_cs, o_rs, o_cs, batch=1,
                   l_plane=0, r_plane=0, o_plane=0) -> None:
    """MatMul_Strided<Mode> (MatrixBase_Mul.h:617-722)."""
    call("fmlh_matmul_strided", mode, out, L, R, M, N, K, l_rs, l_cs, r_rs, r_cs, o_rs, o_cs,
         batch, l_plane, r_plane, o_plane)


def softmax(out, inp, rows, cols):
    call("fmlh_softmax", out, inp, rows, cols)


def layernorm(out, inp, gamma, beta, xhat, rows, cols, eps=1e-5):
    call("fmlh_layernorm", out, inp, gamma, beta or None, xhat or None, rows, cols, eps)


def gelu(out, inp, n):
    call("fmlh_gelu", out, inp, n)


def add(out, a, b, n):
    call("fmlh_add", out, a, b, n)


def copy(out, inp, n):
    call("fmlh_copy", out, inp, n)


def gather_rows(out, src, idx, width, out_rows, out_batch, src_rows, src_batch):
    call("fmlh_gather_rows", out, src, idx, width, out_rows, out_batch, src_rows, src_batch)


def split_qkv(q, k, v, packed, rows, dC):
    call("fmlh_split_qkv", q, k, v, packed, rows, dC)


def scale_add(out, inp, scale, addm, n):
    call("fmlh_scale_add", out, inp, scale, addm, n)


def broadcast_add(out, L, R, n, dims_x):
    call("fmlh_broadcast_add", out, L, R, n, dims_x)


def fill(out, value, n):
    call("fmlh_fill", out, value, n)


def fill_from(out, value_ptr, n):
    call("fmlh_fill_from", out, value_ptr, n)


def per_element_mul(out, a, b, n):
    call("fmlh_per_element_mul", out, a, b, n)


def scale(out, inp, value_ptr, n):
    call("fmlh_scale", out, inp, value_ptr, n)


def scale_scalar(out, inp, value, n):
    call("fmlh_scale_scalar", out, inp, value, n)


def row_argmax(out_idx, inp, rows, cols):
    call("fmlh_row_argmax", out_idx, inp, rows, cols)


# ---- training step (Model::Run with a target, ModelLibrary/Model.h:790-878) ---------------

def softmax_backward(out, softmax_out, grad_in, rows, cols):
    """SoftmaxBackwards (MatrixBase_Functions.h:83-111)."""
    call("fmlh_softmax_backward", out, softmax_out, grad_in, rows, cols)


def layernorm_backward(dx, dy, inp, gamma, dgamma, dbeta, xhat, ws, rows, cols, eps=1e-5):
    """LayerNormBackwardsOp (MatrixBase_Functions.h:552-705); dbeta, xhat may be 0 (None)."""
    call("fmlh_layernorm_backward", dx, dy, inp, gamma, dgamma, dbeta or None, xhat or None,
         ws or None, rows, cols, eps)


def gelu_derivative(out, inp, n):
    """GeluDerivtiveMat (MatrixBase_Functions.h:1002-1017)."""
    call("fmlh_gelu_derivative", out, inp, n)


def scatter_add_rows(out, src, idx, width, src_rows, src_batch, out_rows, out_batch):
    """ScatterAddRows (MatrixBase_Functions.h:285-327)."""
    call("fmlh_scatter_add_rows", out, src, idx, width, src_rows, src_batch, out_rows, out_batch)


def cce_logits(grad, loss, ws, target, logits, vocab, steps, batch, target_cols, target_batch):
    """CategoricalCrossEntropyWithLogits Gradient/Loss (CategoricalCrossEntropyWithLogits.h)."""
    call("fmlh_cce_logits", grad or None, loss or None, ws or None, target, logits, vocab, steps,
         batch, target_cols, target_batch)


def adamw_update(param, grad, mt, vt, n, lr, beta1, beta2, beta1_pow_t, beta2_pow_t, eps, wd):
    """AdamWUpdate (MatrixBase_Functions.h:1497-1545)."""
    call("fmlh_adamw_update", param, grad, mt, vt, n, lr, beta1, beta2, beta1_pow_t, beta2_pow_t,
         eps, wd)


def attention_softmax_heads(p_heads, p_offset, p_all, scores, scale_ptr, n_head, T):
    """Scale + causal mask + Softmax for all heads (CausalSelfAttentionLayer.h:453-458);
    p_heads: device pointers, one per head."""
    arr = (_vp * len(p_heads))(*p_heads)
    call("fmlh_attention_softmax_heads", arr, p_offset, p_all, scores, scale_ptr, n_head, T)


def attention_softmax_backward_heads(ds_all, p_heads, datt_all, scale_ptr, n_head, T):
    """SoftmaxBackwards + mask + scale for all heads (CausalSelfAttentionLayer.h:640-642)."""
    arr = (_vp * len(p_heads))(*p_heads)
    call("fmlh_attention_softmax_backward_heads", ds_all, arr, datt_all, scale_ptr, n_head, T)


def merge_qkv(packed, q, k, v, head_dim, tokens, n_head):
    """MergeQKV (MatrixBase_Functions.h:369-431)."""
    call("fmlh_merge_qkv", packed, q, k, v, head_dim, tokens, n_head)


def sum_columns(out, inp, rows, cols):
    """SumColumns (MatrixBase_Functions.h:1098-1118): column sums of a rows x cols matrix, in
    row order."""
    call("fmlh_sum_columns", out, inp, rows, cols)


def dropout_mask(mask, n, uniforms, count, start, prob):
    """DropoutLayer::UpdateMask's draws for 0 < prob < 1 (DropoutLayer.h:97-123) from a device
    copy of RandomUtils' uniform buffer, starting at draw `start`."""
    call("fmlh_dropout_mask", mask, n, uniforms, count, start, prob)


_probe_lib = None


def probe_lib() -> ctypes.CDLL:
    """The measurement library (lib/libfreeml_probe.so; raises if it is not built)."""
    global _probe_lib
    if _probe_lib is None:
        lib()  # the product library first: the probe links against it
        if not os.path.exists(PROBE_LIB_PATH):
            raise FreeMLHipError("load", -1, f"{PROBE_LIB_PATH} is missing: run freeml_amd.build()")
        P = ctypes.CDLL(PROBE_LIB_PATH)
        for name, args in _PROBE_SIGS.items():
            fn = getattr(P, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _probe_lib = P
    return _probe_lib


def probe_exchange(scope: int, group_a, group_b=(), words: int = 0, rounds: int = 2000):
    """Latency of one exchange-word hand-off (fmlh_probe_exchange, the measurement library):
    (ns per hop, XCD of every workgroup).  scope 0: device scope; the others are the store /
    load forms probe.hip lists."""
    _, cus = device_info()
    a = np.ascontiguousarray(group_a, dtype=np.int32)
    b = np.ascontiguousarray(group_b, dtype=np.int32)
    words = words or max(len(a), len(b))
    xcc = np.full(cus, -1, dtype=np.int32)
    ns = ctypes.c_double()
    rc = probe_lib().fmlh_probe_exchange(scope, a.ctypes.data_as(_i32p), len(a),
                                         b.ctypes.data_as(_i32p) if len(b) else ctypes.cast(None, _i32p),
                                         len(b), words, rounds, xcc.ctypes.data_as(_i32p), ctypes.byref(ns))
    if rc != 0:
        raise FreeMLHipError("fmlh_probe_exchange", rc, lib().fmlh_last_error().decode(errors="replace"))
    return ns.value, xcc


# ---- NanoLLM token loop ------------------------------------------------------------------

def _fp(a):
    return a.ctypes.data_as(_f32p) if a is not None else ctypes.cast(None, _f32p)


class NanoLLM:
    """The NanoLLM graph on the device with a greedy token loop (fmlh_nanollm_*)."""

    # fmlh_nanollm_profile_op ids
    OP_QKV, OP_ATTN, OP_PROJ, OP_FC, OP_PROJ2, OP_LM_HEAD = range(6)

    def __init__(self, weights, max_batch: int = 1, on_device: bool = False):
        """on_device: the parameters are first uploaded to device buffers the engine references
        (weights_on_device = 1, as NanoLLMTokenLoop passes a model's blobs); ``device_weights``
        then maps each parameter's id() to its DeviceArray, and after changing one in place
        ``refresh_weights()`` re-takes the engine's transposed copies."""
        s = weights.shape
        self.shape = s
        self.V = s.vocab
        self.T = s.block_size
        self.max_batch = max_batch
        cfg = NanoLLMConfig(s.vocab, s.block_size, s.n_embed, s.n_head, s.n_layer, max_batch)
        self.device_weights = {}

        def ptr(a):
            if a is None:
                return ctypes.cast(None, _f32p)
            if not on_device:
                return _fp(a)
            if id(a) not in self.device_weights:
                self.device_weights[id(a)] = DeviceArray.from_host(np.ascontiguousarray(a, np.float32))
            return ctypes.cast(self.device_weights[id(a)].ptr, _f32p)

        ptrs = []
        for lw in weights.layers:
            for a in (lw.w_qkv, lw.w_proj, lw.w_fc, lw.w_proj2, lw.ln0_g, lw.ln0_b, lw.ln1_g, lw.ln1_b):
                ptrs.append(ptr(a))
        self._ptrs = (_f32p * len(ptrs))(*ptrs)
        tok = ptr(weights.tok_emb)
        lm = tok if s.tied else ptr(weights.lm_head)
        w = NanoLLMWeightsC(tok, ptr(weights.pos_emb), self._ptrs, ptr(weights.lnf_g), ptr(weights.lnf_b), lm)
        h = _vp()
        call("fmlh_nanollm_create", ctypes.byref(cfg), ctypes.byref(w), 1 if on_device else 0, ctypes.byref(h))
        self.h = h.value

    def refresh_weights(self) -> None:
        """fmlh_nanollm_refresh_weights: re-take the transposed copies of W_qkv, W_fc, W_proj2."""
        call("fmlh_nanollm_refresh_weights", self.h)

    @classmethod
    def from_checkpoint(cls, path: str, max_batch: int = 1) -> "NanoLLM":
        """The NanoLLM of a FreeML checkpoint folder (what Model::Save writes, the folder
        holding ``model.guide``), read by ``freeml_amd.checkpoint.load_nanollm``."""
        from .checkpoint import load_nanollm

        return cls(load_nanollm(path), max_batch=max_batch)

    def close(self):
        if getattr(self, "h", None):
            if not _shut:
                call("fmlh_nanollm_destroy", self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill(self, prompts: np.ndarray) -> None:
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), dtype=np.int32)
        call("fmlh_nanollm_prefill", self.h, prompts.ctypes.data_as(_i32p), prompts.shape[0],
             prompts.shape[1])

    def decode(self, n_steps: int) -> None:
        call("fmlh_nanollm_decode", self.h, n_steps)

    def status(self):
        g, b = _u32(), _u32()
        call("fmlh_nanollm_status", self.h, ctypes.byref(g), ctypes.byref(b))
        return g.value, b.value

    def decode_path(self, batch: int):
        """("relay" | "persistent" | "grouped" | "wide" | "graph", workgroups) for decoding `batch` sequences."""
        path, wgs = ctypes.c_int(), ctypes.c_int()
        call("fmlh_nanollm_decode_path", self.h, batch, ctypes.byref(path), ctypes.byref(wgs))
        return {0: "graph", 1: "persistent", 2: "grouped", 3: "relay", 4: "wide"}[path.value], wgs.value

    def tokens(self, first: int = 0, count: int | None = None) -> np.ndarray:
        gen, batch = self.status()
        count = gen - first if count is None else count
        out = np.empty((batch, count), dtype=np.int32)
        call("fmlh_nanollm_read_tokens", self.h, out.ctypes.data_as(_i32p), first, count)
        return out

    def logits(self) -> np.ndarray:
        _, batch = self.status()
        out = np.empty((batch, self.V), dtype=np.float32)
        call("fmlh_nanollm_read_logits", self.h, out.ctypes.data_as(_f32p))
        return out

    def generate(self, prompts: np.ndarray, n_gen: int, with_logits: bool = False):
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), dtype=np.int32)
        B, P = prompts.shape
        toks = np.empty((B, n_gen), dtype=np.int32)
        logits = np.empty((B, n_gen, self.V), dtype=np.float32) if with_logits else None
        call("fmlh_nanollm_generate", self.h, prompts.ctypes.data_as(_i32p), B, P, n_gen,
             toks.ctypes.data_as(_i32p), _fp(logits))
        return toks, logits

    def set_sampling(self, temperature: float = 0.0, top_k: int = 0, seed: int = 0) -> None:
        """Sampled instead of greedy picks (fmlh_nanollm_set_sampling); temperature 0 = greedy."""
        call("fmlh_nanollm_set_sampling", self.h, temperature, top_k, seed)

    def generate_text(self, prompt, n_gen: int, vocab) -> bytes:
        """Greedy completion of a text prompt: chars to ids and back with the example's
        character vocabulary (freeml_amd.text; Examples/NanoLLM/NanoLLM.cpp:146-166)."""
        from . import text

        ids = text.encode(prompt, vocab).astype(np.int32)
        toks, _ = self.generate(ids[None, :], n_gen)
        return text.decode(toks[0], vocab)

    def forward_window(self, ids: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(np.atleast_2d(ids), dtype=np.int32)
        B, T = ids.shape
        assert T == self.T
        out = np.empty((B, T, self.V), dtype=np.float32)
        call("fmlh_nanollm_forward_window", self.h, ids.ctypes.data_as(_i32p), B,
             out.ctypes.data_as(_f32p))
        return out

    def profile_op(self, op: int, iters: int):
        """Average device time (ms) of one launch of a decode-step op and its algorithmic bytes."""
        ms = ctypes.c_float()
        by = ctypes.c_double()
        call("fmlh_nanollm_profile_op", self.h, op, iters, ctypes.byref(ms), ctypes.byref(by))
        return ms.value, by.value
