"""The character-level text front end (freeml_amd/text.py) against the reference's own
BuildVocab / encode / decode / DecodeMatrixTokens / CountCorrectTokensBatch
(Examples/NanoLLM/NanoLLM.cpp:95-252, compiled into oracle/_ref/libfreeml_ref.so), on the
example's own corpus (Examples/NanoLLM/Data/input.txt, read where the reference tree is
present) and on byte strings that reach the corner cases: bytes >= 0x80 (signed-char order),
chars and ids outside the vocabulary, ties and NaNs in logits rows."""
import os

import numpy as np
import pytest

import oracle
from freeml_amd import text

needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
CORPUS = "/root/reference/Examples/NanoLLM/Data/input.txt"


@needs_ref
@pytest.mark.skipif(not os.path.exists(CORPUS), reason="reference corpus not present")
def test_vocab_of_the_example_corpus():
    data = text.load_text_file(CORPUS)
    v = text.build_vocab(data)
    uniq, ids = oracle.ref_build_vocab(data)
    assert v.unique == uniq and v.size == 65  # the vocabulary size of configs c1-c3
    np.testing.assert_array_equal(v.ids, ids)
    assert text.decode(v.ids, v) == data


@needs_ref
def test_vocab_with_high_bytes_sorts_as_signed_char():
    rng = np.random.default_rng(0)
    data = bytes(rng.integers(0, 256, 5000, dtype=np.uint8)) + b"hello \x80\xff"
    v = text.build_vocab(data)
    uniq, ids = oracle.ref_build_vocab(data)
    assert v.unique == uniq
    assert v.unique[0] == 0x80  # -128 first
    np.testing.assert_array_equal(v.ids, ids)


@needs_ref
def test_encode_decode_match_reference_outside_the_vocabulary():
    v = text.build_vocab(b"the quick brown fox")
    s = b"the lazy dog!"  # l, a, z, y, d, g, ! are not in the vocabulary
    np.testing.assert_array_equal(text.encode(s, v), oracle.ref_encode(v.unique, s))
    ids = np.array([0, 3, v.size - 1, v.size, 1000], np.uint32)
    assert text.decode(ids, v) == oracle.ref_decode(v.unique, ids)
    assert text.decode(text.encode(b"fox", v), v) == b"fox"


@needs_ref
def test_decode_matrix_tokens_matches_reference():
    v = text.build_vocab(bytes(range(32, 97)))  # 65 chars
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((40, v.size)).astype(np.float32)
    logits[3, 7] = logits[3, 20] = 9.0         # a tie: the first maximum wins
    logits[5, 0] = np.nan                      # NaN first: index 0 kept
    logits[6, 11] = np.nan                     # NaN later: skipped
    logits[8, :] = -np.inf
    assert text.decode_matrix_tokens(logits, v) == oracle.ref_decode_matrix_tokens(logits, v.unique)
    ids = np.array([[0], [5], [64], [65], [3.7], [200]], np.float32)
    assert text.decode_matrix_tokens(ids, v) == oracle.ref_decode_matrix_tokens(ids, v.unique)


@needs_ref
def test_count_correct_matches_reference():
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((64, 65)).astype(np.float32)
    target = np.argmax(logits, 1).astype(np.float32)
    target[::3] = (target[::3] + 1) % 65
    assert text.count_correct(logits, target) == oracle.ref_count_correct(logits, target)


def test_windows_are_shifted_by_one():
    corpus = np.arange(100)
    x, y = text.windows(corpus, 16, 10)
    np.testing.assert_array_equal(x, np.arange(10, 26))
    np.testing.assert_array_equal(y, np.arange(11, 27))
    with pytest.raises(ValueError):
        text.windows(corpus, 16, 84)


@pytest.mark.gpu
def test_generate_text_on_the_device(golden):
    """Text in, text out through the token loop: the completion of the decoded golden prompt is
    the decoded golden token sequence (c2 weights; a 65-char vocabulary)."""
    import freeml_amd as fh
    from freeml_amd import synth

    fh.init(0)
    g = golden("c2")
    v = text.build_vocab(bytes(range(32, 97)))
    prompt = text.decode(g["prompts"][0], v)
    m = fh.NanoLLM(synth.make_weights(synth.CONFIGS["c2"]["shape"], 0))
    try:
        out = m.generate_text(prompt, 48, v)
    finally:
        m.close()
    assert out == text.decode(g["tokens"][0][:48], v)
