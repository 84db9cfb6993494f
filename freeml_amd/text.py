"""Character-level text front end of the NanoLLM example (Examples/NanoLLM/NanoLLM.cpp:95-252).

The example trains on the bytes of a text file: the vocabulary is the sorted set of distinct
chars, a char's id is its index in that set, and generated ids map back to chars.  This module
keeps those definitions so that text prompts and completions read the same as the reference's:

* ``build_vocab`` = BuildVocab (:121-144).  The chars are C++ ``char`` -- signed on x86 -- and
  ``std::sort`` orders them by that signed value, so bytes >= 0x80 sort before ASCII.
* ``encode`` = encode (:146-155): ``std::map::operator[]`` gives 0 for a char outside the
  vocabulary.  ``decode`` = decode (:157-166): an id outside it gives the char 0.
* ``decode_matrix_tokens`` = DecodeMatrixTokens (:168-206): a one-column matrix holds ids
  (truncated floats); a wider one holds logits and each row decodes to its first maximum
  (strict ``>`` from element 0).  An id outside the vocabulary prints ``?``.
* ``count_correct`` = CountCorrectTokensBatch (:226-252).
* ``windows`` = the TrainLoop's CopyRange pair (:440-442): input window at ``start``, target
  window one token later.

Host-side only (parsing and bookkeeping); generation itself runs through ``freeml_amd.NanoLLM``.
"""
from __future__ import annotations

import dataclasses

import numpy as np


def _signed(b: int) -> int:
    return b - 256 if b >= 128 else b


@dataclasses.dataclass
class Vocab:
    unique: bytes         # distinct chars in signed-char order; id = index
    ids: np.ndarray       # uint32 id of every char of the corpus it was built from

    @property
    def size(self) -> int:
        return len(self.unique)

    def lookup(self) -> np.ndarray:
        """256-entry byte -> id table (0 for bytes outside the vocabulary)."""
        t = np.zeros(256, np.uint32)
        for i, b in enumerate(self.unique):
            t[b] = i
        return t


def load_text_file(path: str) -> bytes:
    """LoadTextFile (NanoLLM.cpp:103-119): the file's bytes."""
    with open(path, "rb") as f:
        return f.read()


def build_vocab(data: bytes) -> Vocab:
    unique = bytes(sorted(set(data), key=_signed))
    v = Vocab(unique, np.empty(0, np.uint32))
    v.ids = v.lookup()[np.frombuffer(data, np.uint8)] if data else np.empty(0, np.uint32)
    return v


def encode(s, vocab: Vocab) -> np.ndarray:
    b = s.encode("latin-1") if isinstance(s, str) else bytes(s)
    return vocab.lookup()[np.frombuffer(b, np.uint8)] if b else np.empty(0, np.uint32)


def decode(ids, vocab: Vocab) -> bytes:
    ids = np.asarray(ids, np.int64).reshape(-1)
    table = np.frombuffer(vocab.unique, np.uint8)
    ok = (ids >= 0) & (ids < vocab.size)
    out = np.zeros(ids.size, np.uint8)
    out[ok] = table[ids[ok]]
    return out.tobytes()


def _first_max(rows: np.ndarray) -> np.ndarray:
    """Index of each row's first maximum by the reference's strict '>' scan from element 0: a
    NaN is never taken after element 0, and a NaN at element 0 is never replaced."""
    rows = np.asarray(rows, np.float32)
    masked = np.where(np.isnan(rows), -np.inf, rows)
    idx = np.argmax(masked, axis=1)
    # A row whose maximum is not above element 0 keeps index 0 (all -inf, or NaN first).
    first = rows[:, 0]
    keep0 = np.isnan(first) | ~(masked[np.arange(rows.shape[0]), idx] > first)
    return np.where(keep0, 0, idx)


def decode_matrix_tokens(mat: np.ndarray, vocab: Vocab) -> bytes:
    """mat: (steps, cols) float32 -- ids when cols == 1, logits otherwise."""
    mat = np.asarray(mat, np.float32)
    if mat.ndim == 1:
        mat = mat[:, None]
    ids = mat[:, 0].astype(np.int64) if mat.shape[1] == 1 else _first_max(mat)
    # The reference converts the float id to uint32; an id beyond the vocabulary prints '?'.
    table = np.frombuffer(vocab.unique, np.uint8)
    out = np.full(ids.size, ord("?"), np.uint8)
    ok = (ids >= 0) & (ids < vocab.size)
    out[ok] = table[ids[ok]]
    return out.tobytes()


def count_correct(logits: np.ndarray, target) -> int:
    """logits: (block, vocab); target: (block,) ids."""
    pred = _first_max(np.asarray(logits, np.float32))
    return int(np.sum(pred == np.asarray(target).astype(np.int64).reshape(-1)))


def windows(corpus_ids, block: int, start: int):
    """(input, target) windows of the TrainLoop at ``start``: corpus[start:start+block] and
    corpus[start+1:start+1+block]."""
    c = np.asarray(corpus_ids)
    if start < 0 or start + block + 1 > c.size:
        raise ValueError(f"window at {start} of {block} + 1 ids exceeds the corpus ({c.size} ids)")
    return c[start:start + block], c[start + 1:start + 1 + block]
