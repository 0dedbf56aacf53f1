"""TEST INFRASTRUCTURE ONLY — pure-Python restatement of the reference's
WordPiece tokenizer (io/tokenizer.zig) and of the embed command's chunking
and chunk pooling (main.zig:786-923).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; it is the checker, never the thing measured or shipped.

Pinning (tests/test_tokenizer.py): the five known-answer tests of
tokenizer.zig:291-437 (fixture tests/golden/tokenizer_cases.json), special
cases read off the algorithm (longest match, whole-word [UNK], capacity cuts,
the 200-byte word limit, vocabulary line numbering), a brute-force count of
the chunk starts against the closed form below, and closed forms of the
pooling (one chunk, orthogonal chunks, cancelling chunks).
"""
from __future__ import annotations

import numpy as np

UNK, CLS, SEP = 100, 101, 102          # tokenizer.zig:12-14
MAX_WORD = 200                         # tokenizer.zig:15
WHITESPACE = b" \t\n\r"                # tokenizer.zig:267-269
PUNCT = b"!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~"  # tokenizer.zig:271-276
CHUNK, OVERLAP = 510, 50               # main.zig:783-784


def load_vocab_bytes(data: bytes) -> dict:
    """loadVocabFromBytes (tokenizer.zig:54-74): id = line index, empty lines
    count, one trailing CR stripped, a repeated token keeps the later id."""
    vocab = {}
    for idx, line in enumerate(data.split(b"\n")):
        if line.endswith(b"\r"):
            line = line[:-1]
        if line:
            vocab[line] = idx
    return vocab


def _lower(word: bytes) -> bytes:
    return bytes(c + 32 if 65 <= c <= 90 else c for c in word)  # tokenizer.zig:278-284


def _word(vocab: dict, word: bytes, room) -> tuple[list, bool]:
    """Pieces of one word (tokenizer.zig:154-206, 209-259): longest prefix
    first, "##" on pieces after the first.  Returns (pieces, whole_unk)."""
    if len(word) > MAX_WORD:
        return [UNK], True
    low = _lower(word)
    out, start, first = [], 0, True
    while start < len(low) and room(len(out)):
        for end in range(len(low), start, -1):
            piece = low[start:end] if first else b"##" + low[start:end]
            if piece in vocab:
                out.append(vocab[piece])
                start, first = end, False
                break
        else:
            return [UNK], True
    return out, False


def encode(vocab: dict, text: bytes, capacity: int) -> list:
    """encode (tokenizer.zig:78-118): [CLS] pieces [SEP] within capacity."""
    assert capacity >= 2
    out = [CLS]
    i, n = 0, len(text)
    while i < n and len(out) < capacity - 1:
        while i < n and text[i] in WHITESPACE:
            i += 1
        if i >= n:
            break
        ws = i
        while i < n and text[i] not in WHITESPACE and text[i] not in PUNCT:
            i += 1
        if i > ws:
            base = len(out)
            pieces, _ = _word(vocab, text[ws:i], lambda k: base + k < capacity - 1)
            out.extend(pieces)
        if i < n and text[i] in PUNCT:
            if len(out) < capacity - 1:
                out.append(vocab.get(text[i:i + 1], UNK))
            i += 1
    out.append(SEP)
    return out


def encode_raw(vocab: dict, text: bytes) -> list:
    """encodeRaw (tokenizer.zig:122-151): all pieces, no markers."""
    out = []
    i, n = 0, len(text)
    while i < n:
        while i < n and text[i] in WHITESPACE:
            i += 1
        if i >= n:
            break
        ws = i
        while i < n and text[i] not in WHITESPACE and text[i] not in PUNCT:
            i += 1
        if i > ws:
            out.extend(_word(vocab, text[ws:i], lambda k: True)[0])
        if i < n and text[i] in PUNCT:
            out.append(vocab.get(text[i:i + 1], UNK))
            i += 1
    return out


def chunk_count(total: int) -> int:
    """main.zig:803-806."""
    if total <= CHUNK:
        return 1
    return 1 + (total - CHUNK + OVERLAP - 1) // (CHUNK - OVERLAP)


def chunks(pieces: list) -> list:
    """The chunk id lists of main.zig:854-864 (and 894-898 for one chunk)."""
    stride = CHUNK - OVERLAP
    out = []
    for k in range(chunk_count(len(pieces))):
        s = k * stride
        out.append([CLS] + list(pieces[s:min(s + CHUNK, len(pieces))]) + [SEP])
    return out


def chunk_mean_l2(emb: np.ndarray) -> np.ndarray:
    """main.zig:908-923 in f32 and in its order: chunk rows added in order
    onto zeros, times the f32 reciprocal of the count, the squares summed
    from column 0 up, then divided by sqrt of that sum when it is positive."""
    emb = np.asarray(emb, np.float32)
    acc = np.zeros(emb.shape[1], np.float32)
    for row in emb:
        acc = acc + row
    scale = np.float32(1.0) / np.float32(emb.shape[0])
    acc = acc * scale
    sq = acc * acc
    norm = np.float32(0.0)
    for v in sq:
        norm = np.float32(norm + v)
    norm = np.sqrt(norm)
    return acc / norm if norm > 0 else acc
