"""WordPiece tokenizer: the mirror of io/tokenizer.zig's Tokenizer over the
C ABI (tokenizer.cpp in the library).

    tok = Tokenizer.init()                   # tokenizer.zig:17-22
    tok.loadVocab("vocab.txt")               # tokenizer.zig:34-51
    ids = tok.encode(b"hello world", 512)    # tokenizer.zig:78-118
    pieces = tok.encodeRaw(b"long text")     # tokenizer.zig:122-151

Texts are bytes (str is encoded as UTF-8); ids are numpy uint32 arrays.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import TzhError, check, lib

TZH_ERR_TOO_LARGE = -11


def _bytes(text) -> bytes:
    return text.encode("utf-8") if isinstance(text, str) else bytes(text)


class Tokenizer:
    unk_id, cls_id, sep_id = 100, 101, 102  # tokenizer.zig:12-14

    def __init__(self, handle: C.c_void_p):
        self.handle = handle

    @staticmethod
    def init() -> "Tokenizer":
        h = C.c_void_p()
        check(lib().tzh_tokenizer_create(C.byref(h)))
        return Tokenizer(h)

    def deinit(self) -> None:
        if self.handle:
            lib().tzh_tokenizer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.deinit()
        except Exception:
            pass

    def loadVocab(self, path: str) -> None:
        check(lib().tzh_tokenizer_load_vocab(self.handle, str(path).encode()))

    def loadVocabFromBytes(self, data: bytes) -> None:
        data = bytes(data)
        check(lib().tzh_tokenizer_load_vocab_bytes(self.handle, data, len(data)))

    def put(self, token, token_id: int) -> None:
        """vocab.put(token, id), as the reference's tests fill the vocabulary."""
        t = _bytes(token)
        check(lib().tzh_tokenizer_put(self.handle, t, len(t), int(token_id)))

    def encode(self, text, capacity: int = 512) -> np.ndarray:
        t = _bytes(text)
        out = np.empty(max(int(capacity), 0), np.uint32)
        n = C.c_int64()
        check(lib().tzh_tokenizer_encode(self.handle, t, len(t), out.ctypes.data, int(capacity), C.byref(n)))
        return out[:n.value].copy()

    def encodeRaw(self, text) -> np.ndarray:
        t = _bytes(text)
        n = C.c_int64()
        rc = lib().tzh_tokenizer_encode_raw(self.handle, t, len(t), None, 0, C.byref(n))
        if rc not in (0, TZH_ERR_TOO_LARGE):
            check(rc)
        out = np.empty(n.value, np.uint32)
        check(lib().tzh_tokenizer_encode_raw(self.handle, t, len(t), out.ctypes.data if n.value else None, n.value,
                                             C.byref(n)))
        return out


def chunk_count(total_tokens: int) -> int:
    """Chunks runEmbed cuts a document of that many pieces into (main.zig:803-806)."""
    n = C.c_int64()
    check(lib().tzh_embed_chunk_count(int(total_tokens), C.byref(n)))
    return n.value


def _text_array(texts):
    data = [_bytes(t) for t in texts]
    arr = (C.c_char_p * max(len(data), 1))(*data)
    lens = np.array([len(d) for d in data], np.int64)
    return data, arr, lens


__all__ = ["Tokenizer", "TzhError", "chunk_count"]
