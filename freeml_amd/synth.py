"""Seeded synthetic weights and prompts for the NanoLLM token loop.

FreeML initialises weights with a ``std::random_device``-seeded ``mt19937`` feeding
``std::normal_distribution`` (ToolsLibrary/Tools.h:15-27, Dense.h:75-85, Embedding.h:51-56),
which is neither reproducible nor portable across standard libraries.  Benchmarks and parity
tests therefore build their inputs here, from a counter-based generator whose every value is
a pure function of ``(seed, stream, index)``:

* ``splitmix64`` finalisers give 64-bit words (integer arithmetic only, so identical on every
  IEEE/two's-complement machine);
* Box-Muller in float64 turns word pairs into normals, rounded once to float32;
* prompts use the high 32 bits of a word, multiplied by the vocabulary size and shifted
  (Lemire's multiply-shift range reduction), so no modulo bias is introduced.

The canonical fill order assigns each tensor a fixed stream id (``STREAM_*`` below), so a
tensor's values do not depend on which other tensors were generated first.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_STREAM_MUL = 0xD1B54A32D192ED03
_MASK64 = (1 << 64) - 1

STREAM_TOK_EMB = 0
STREAM_POS_EMB = 1
STREAM_LM_HEAD = 2
STREAM_PROMPT = 7
STREAM_LAYER_BASE = 16  # layer l uses streams 16 + 16*l + {0: qkv, 1: attn proj, 2: fc, 3: mlp proj}


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _key(seed: int, stream: int) -> np.uint64:
    k = (seed * 0x9E3779B97F4A7C15 + stream * _STREAM_MUL + 1) & _MASK64
    return _mix(np.array([k], dtype=np.uint64))[0]


def words(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """64-bit words ``start .. start+count-1`` of stream ``(seed, stream)``."""
    idx = np.arange(start + 1, start + 1 + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(_key(seed, stream) + idx * _GOLDEN)


def normal_f32(count: int, seed: int, stream: int, std: float = 0.02, mean: float = 0.0,
               chunk_pairs: int = 1 << 22) -> np.ndarray:
    """``count`` float32 samples of N(mean, std^2): Box-Muller over consecutive word pairs."""
    out = np.empty(count, dtype=np.float32)
    pairs = (count + 1) // 2
    two_pi = 2.0 * math.pi
    for p0 in range(0, pairs, chunk_pairs):
        n = min(chunk_pairs, pairs - p0)
        w = words(seed, stream, 2 * p0, 2 * n).reshape(n, 2)
        u1 = ((w[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
        u2 = (w[:, 1] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.empty((n, 2), dtype=np.float64)
        z[:, 0] = r * np.cos(two_pi * u2)
        z[:, 1] = r * np.sin(two_pi * u2)
        vals = (mean + std * z).astype(np.float32).reshape(-1)
        lo = 2 * p0
        hi = min(count, lo + 2 * n)
        out[lo:hi] = vals[: hi - lo]
    return out


def prompt_tokens(vocab: int, length: int, seed: int) -> np.ndarray:
    """``length`` token ids uniform over ``[0, vocab)`` (multiply-shift range reduction)."""
    w = words(seed, STREAM_PROMPT, 0, length)
    hi = (w >> np.uint64(32)).astype(np.uint64)
    with np.errstate(over="ignore"):
        ids = (hi * np.uint64(vocab)) >> np.uint64(32)
    return ids.astype(np.int32)


@dataclasses.dataclass(frozen=True)
class NanoLLMShape:
    """Shape of a NanoLLM graph (Examples/NanoLLM/NanoLLM.cpp:47-66, :255-376)."""

    vocab: int
    block_size: int
    n_embed: int
    n_head: int
    n_layer: int
    tied: bool = True  # lm_head shares Embedding_Weights (NanoLLM.cpp:333-345)

    @property
    def head_dim(self) -> int:
        return self.n_embed // self.n_head


@dataclasses.dataclass
class LayerWeights:
    """One TransformerBlock's parameters, in FreeML's storage layout (row-major).

    * ``w_qkv``  (C, 3C): CSA_AttentionLayer ``Dense_Weights``, dims {3C, C}, read by
      ``Mul<None>`` (CausalSelfAttentionLayer.h:47, Dense.h:207).
    * ``w_proj`` (C, C):  CSA_ProjLayer ``Dense_Weights`` stored out-rows x in-cols, dims {C, C},
      read by ``Mul<Right>`` (CausalSelfAttentionLayer.h:51, Dense.h:203).
    * ``w_fc``   (C, 4C): DenseFCData ``Dense_Weights`` (TransformerBlock.h:288).
    * ``w_proj2``(4C, C): DenseProjData ``Dense_Weights`` (TransformerBlock.h:316).
    * ``ln0_g``/``ln1_g`` (C,): ``GammaScale`` = 1 (LayerNorm.h:115); ``*_b`` = ``BetaShift`` or None.
    """

    w_qkv: np.ndarray
    w_proj: np.ndarray
    w_fc: np.ndarray
    w_proj2: np.ndarray
    ln0_g: np.ndarray
    ln1_g: np.ndarray
    ln0_b: np.ndarray | None = None
    ln1_b: np.ndarray | None = None


@dataclasses.dataclass
class NanoLLMWeights:
    shape: NanoLLMShape
    tok_emb: np.ndarray  # (V, C)  embedding_token Embedding_Weights, dims {C, V}
    pos_emb: np.ndarray  # (T, C)  embedding_pos Embedding_Weights, dims {C, T}
    layers: list
    lnf_g: np.ndarray
    lnf_b: np.ndarray | None
    lm_head: np.ndarray  # (V, C) lm_head Dense_Weights (transposed dense); aliases tok_emb if tied

    def checksum(self) -> str:
        """Order-sensitive digest of every parameter, recorded in golden fixtures."""
        import hashlib

        h = hashlib.sha256()
        for a in self.tensors():
            h.update(np.ascontiguousarray(a).tobytes())
        return h.hexdigest()[:16]

    def tensors(self):
        yield self.tok_emb
        yield self.pos_emb
        for lw in self.layers:
            yield from (lw.w_qkv, lw.w_proj, lw.w_fc, lw.w_proj2, lw.ln0_g, lw.ln1_g)
        yield self.lnf_g
        if not self.shape.tied:
            yield self.lm_head


def make_weights(shape: NanoLLMShape, seed: int = 0, std: float = 0.02) -> NanoLLMWeights:
    """fp32 ~N(0, std^2) weights, LayerNorm gain 1 / no bias (NanoLLM use_bias=false)."""
    V, T, C, L = shape.vocab, shape.block_size, shape.n_embed, shape.n_layer
    tok = normal_f32(V * C, seed, STREAM_TOK_EMB, std).reshape(V, C)
    pos = normal_f32(T * C, seed, STREAM_POS_EMB, std).reshape(T, C)
    layers = []
    for l in range(L):
        b = STREAM_LAYER_BASE + 16 * l
        layers.append(LayerWeights(
            w_qkv=normal_f32(C * 3 * C, seed, b + 0, std).reshape(C, 3 * C),
            w_proj=normal_f32(C * C, seed, b + 1, std).reshape(C, C),
            w_fc=normal_f32(C * 4 * C, seed, b + 2, std).reshape(C, 4 * C),
            w_proj2=normal_f32(4 * C * C, seed, b + 3, std).reshape(4 * C, C),
            ln0_g=np.ones(C, dtype=np.float32),
            ln1_g=np.ones(C, dtype=np.float32),
        ))
    lm = tok if shape.tied else normal_f32(V * C, seed, STREAM_LM_HEAD, std).reshape(V, C)
    return NanoLLMWeights(shape, tok, pos, layers, np.ones(C, dtype=np.float32), None, lm)


# The benchmark workloads c1..c5 (shapes, batch, prompt length, tokens generated).
CONFIGS = {
    "c1": dict(shape=NanoLLMShape(65, 64, 64, 4, 2, tied=False), batch=1, prompt=16, n_gen=48),
    "c2": dict(shape=NanoLLMShape(65, 256, 384, 6, 6), batch=1, prompt=64, n_gen=192),
    "c3": dict(shape=NanoLLMShape(65, 256, 384, 6, 6), batch=64, prompt=64, n_gen=192),
    "c4": dict(shape=NanoLLMShape(50304, 1024, 768, 12, 12), batch=8, prompt=512, n_gen=512),
    "c5": dict(shape=NanoLLMShape(256, 4096, 512, 8, 4), batch=4, prompt=3584, n_gen=512),
}


def prompts_for(config: str) -> np.ndarray:
    """(B, P) int32 prompts: row b uses seed 1 + b (c1: seed 1, batch 1)."""
    c = CONFIGS[config]
    return np.stack([prompt_tokens(c["shape"].vocab, c["prompt"], 1 + b) for b in range(c["batch"])])
