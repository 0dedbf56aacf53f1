"""The WordPiece tokenizer and the embed command's chunk plan and pooling
(io/tokenizer.zig; main.zig:786-923): the oracle pinned against the
reference's own tokenizer tests and known answers read off the algorithm,
then the library's host tokenizer against the oracle, id for id.  CPU only:
the tokenizer entry points make no GPU calls."""
import json
import os

import numpy as np
import pytest

from oracle import wordpiece as wp
from tenzor_amd import TzhError, synth
from tenzor_amd.tokenizer import Tokenizer, chunk_count
from tests.conftest import GOLDEN

CASES = json.load(open(os.path.join(GOLDEN, "tokenizer_cases.json")))["cases"]


def lib_tokenizer(vocab: dict) -> Tokenizer:
    t = Tokenizer.init()
    for k, v in vocab.items():
        t.put(k, v)
    return t


def case_vocab(case):
    return {k.encode(): v for k, v in case["vocab"]}


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_reference_known_answers(case):
    vocab = case_vocab(case)
    text = case["text"].encode()
    assert wp.encode(vocab, text, 32) == case["expected"]
    assert lib_tokenizer(vocab).encode(text, 32).tolist() == case["expected"]


# Special cases read off tokenizer.zig (line numbers there); each would fail
# for a plausible slip: shortest instead of longest match, pieces kept
# before an [UNK], "##" on the first piece, capacity off by one, the 200-byte
# limit off by one, non-ASCII lowercased, vertical tab taken as whitespace.
V = {b"[UNK]": 100, b"[CLS]": 101, b"[SEP]": 102, b"a": 5, b"ab": 6, b"abc": 7, b"##d": 8, b"##cd": 9,
     b"test": 10, b"##ing": 11, b"##s": 12, b"hello": 13, b"!": 14, b"world": 15, b"##test": 16,
     b"x" * 200: 17, b"caf\xc3\xa9": 18}
KNOWN = [
    (b"abcd", 32, [101, 7, 8, 102]),                    # longest prefix first (177-190)
    (b"abd", 32, [101, 6, 8, 102]),
    (b"testx", 32, [101, 100, 102]),                    # whole word [UNK] (200-204)
    (b"testtest", 32, [101, 10, 16, 102]),              # "##" only after the first piece
    (b"tests testing", 32, [101, 10, 12, 10, 11, 102]),
    (b"hello!world", 32, [101, 13, 14, 15, 102]),       # punctuation splits words (96-110)
    (b"hello?", 32, [101, 13, 100, 102]),               # punctuation outside the vocab
    (b"HeLLo\tWORLD\r\nhello", 32, [101, 13, 15, 13, 102]),
    (b"hello\x0bworld", 32, [101, 100, 102]),           # only space, tab, LF, CR are whitespace
    (b"CAF\xc3\x89", 32, [101, 100, 102]),              # ASCII lowercasing only (E-acute stays upper)
    (b"CAF\xc3\xa9", 32, [101, 18, 102]),
    (b"x" * 200, 32, [101, 17, 102]),                   # 200 bytes is still a word
    (b"x" * 201, 32, [101, 100, 102]),                  # over 200: [UNK] (215-218)
    (b"", 32, [101, 102]),
    (b"   \n ", 32, [101, 102]),
    (b"hello world hello", 4, [101, 13, 15, 102]),      # capacity: pieces stop at cap - 1
    (b"testing", 3, [101, 10, 102]),                    # ... inside a word too (229)
    (b"hello", 2, [101, 102]),
    (b"hello, world", 3, [101, 13, 102]),               # punctuation needs room too (104-108)
]


@pytest.mark.parametrize("text,cap,expected", KNOWN)
def test_algorithm_known_answers(text, cap, expected):
    assert wp.encode(V, text, cap) == expected
    assert lib_tokenizer(V).encode(text, cap).tolist() == expected
    if cap == 32:
        assert wp.encode_raw(V, text) == expected[1:-1]
        assert lib_tokenizer(V).encodeRaw(text).tolist() == expected[1:-1]


def test_vocab_lines():
    """loadVocabFromBytes (tokenizer.zig:54-74): ids are line indices, empty
    lines count, a trailing CR is stripped, a repeated token takes its later
    line (StringHashMap.put replaces)."""
    data = b"[PAD]\n\nfoo\r\nbar\nfoo\n\r\nbaz"
    assert wp.load_vocab_bytes(data) == {b"[PAD]": 0, b"foo": 4, b"bar": 3, b"baz": 6}
    t = Tokenizer.init()
    t.loadVocabFromBytes(data)
    # "[PAD]" in text is "[", "pad", "]": none of them in this vocabulary
    assert t.encodeRaw(b"foo bar baz [PAD] qux").tolist() == [4, 3, 6, 100, 100, 100, 100]


def test_vocab_file(tmp_path):
    data, _ = synth.make_vocab(3, 2000)
    p = tmp_path / "vocab.txt"
    p.write_bytes(data)
    t = Tokenizer.init()
    t.loadVocab(str(p))
    text = synth.make_text(4, synth.make_vocab(3, 2000)[1], 300)
    assert t.encodeRaw(text).tolist() == wp.encode_raw(wp.load_vocab_bytes(data), text)
    with pytest.raises(TzhError):
        t.loadVocab(str(tmp_path / "missing.txt"))


def test_capacity_below_two_is_rejected():
    with pytest.raises(TzhError):
        lib_tokenizer(V).encode(b"hello", 1)


@pytest.mark.parametrize("seed", range(6))
def test_library_matches_oracle_on_random_text(seed):
    data, words = synth.make_vocab(seed, 3000)
    vocab = wp.load_vocab_bytes(data)
    t = Tokenizer.init()
    t.loadVocabFromBytes(data)
    text = synth.make_text(100 + seed, words, 400)
    raw = wp.encode_raw(vocab, text)
    assert t.encodeRaw(text).tolist() == raw
    assert len(raw) > 400
    for cap in (2, 3, 17, 64, 511, 512, 4096):
        assert t.encode(text, cap).tolist() == wp.encode(vocab, text, cap), cap


def test_chunk_count_known_answers():
    """main.zig:803-806: chunks start every 460 pieces; a new chunk only once
    the pieces reach 461 past its start, so a tail of up to 410 pieces after
    the last chunk's 510 is dropped."""
    known = {0: 1, 1: 1, 510: 1, 511: 1, 920: 1, 921: 2, 970: 2, 971: 2, 1380: 2, 1381: 3, 1840: 3, 1841: 4}
    for total, n in known.items():
        assert wp.chunk_count(total) == n and chunk_count(total) == n, total


def test_chunk_count_brute_force():
    """Closed form against a count of the chunk starts 460k with
    460k + 461 <= total (above one chunk's 510 pieces)."""
    for total in range(0, 6000, 7):
        brute = 1 if total <= 510 else sum(1 for k in range(total) if 460 * k + 461 <= total)
        assert wp.chunk_count(total) == brute == chunk_count(total), total


def test_chunks_layout():
    pieces = list(range(1000, 1000 + 1400))
    ch = wp.chunks(pieces)
    assert len(ch) == 3
    assert ch[0] == [101] + pieces[0:510] + [102]
    assert ch[1] == [101] + pieces[460:970] + [102]
    assert ch[2] == [101] + pieces[920:1400] + [102]
    assert wp.chunks([]) == [[101, 102]]


def test_chunk_pooling_closed_forms():
    e = np.eye(384, dtype=np.float32)
    # one chunk: its own direction
    u = np.random.default_rng(0).standard_normal(384).astype(np.float32)
    u /= np.linalg.norm(u)
    assert np.allclose(wp.chunk_mean_l2(u[None]), u, atol=1e-6)
    # orthogonal unit chunks: the normalised sum
    got = wp.chunk_mean_l2(np.stack([e[0], e[5], e[7]]))
    ref = np.zeros(384, np.float32)
    ref[[0, 5, 7]] = 1 / np.sqrt(3)
    assert np.allclose(got, ref, atol=1e-7)
    # weights follow the counts: two chunks along e0, one along e1
    got = wp.chunk_mean_l2(np.stack([e[0], e[0], e[1]]))
    assert np.allclose(got[:2], np.array([2, 1]) / np.sqrt(5), atol=1e-7)
    # cancelling chunks: zero mean, no division
    z = wp.chunk_mean_l2(np.stack([u, -u]))
    assert not z.any()
