"""Seeded synthetic inputs for the Arctic-embed-xs configurations.

Weights follow the configurations' recipe: every matrix N(0, 0.02) in f32
(biases N(0, 0.02) as well; LayerNorm gamma = 1, beta = 0 unless
`ln_random`), then the 36 encoder linears quantized per row to int8 with f16
scales (quantize_arctic_xs.zig:94-115).  Token batches put the [CLS] id
101 first and draw the rest uniformly from [1000, 30521]; padded positions
hold id 0.  Everything is numpy (PCG64) from one seed, so the GPU path and
the CPU checker read identical bytes.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _abi, quantize_rows_host


@dataclass
class Config:
    """arctic.Config (arctic.zig:29-42)."""

    hidden_size: int = 384
    num_hidden_layers: int = 6
    num_attention_heads: int = 12
    intermediate_size: int = 1536
    vocab_size: int = 30522
    max_position_embeddings: int = 512
    type_vocab_size: int = 2
    layer_norm_eps: float = 1e-12

    def to_c(self) -> _abi.ArcticConfig:
        return _abi.ArcticConfig(self.hidden_size, self.num_hidden_layers, self.num_attention_heads,
                                 self.intermediate_size, self.vocab_size, self.max_position_embeddings,
                                 self.type_vocab_size, self.layer_norm_eps)


LINEARS = ("attention.self.query", "attention.self.key", "attention.self.value", "attention.output.dense",
           "intermediate.dense", "output.dense")


def make_arctic_f32(seed: int, cfg: Config = Config(), ln_random: bool = False) -> dict:
    """f32 weights keyed by HF parameter names (no "bert." prefix)."""
    rng = np.random.default_rng(seed)
    h, inter = cfg.hidden_size, cfg.intermediate_size

    def normal(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    def ln(prefix):
        if ln_random:
            w[prefix + ".weight"] = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
            w[prefix + ".bias"] = (0.1 * rng.standard_normal(h)).astype(np.float32)
        else:
            w[prefix + ".weight"] = np.ones(h, np.float32)
            w[prefix + ".bias"] = np.zeros(h, np.float32)

    w = {}
    w["embeddings.word_embeddings.weight"] = normal(cfg.vocab_size, h)
    w["embeddings.position_embeddings.weight"] = normal(cfg.max_position_embeddings, h)
    w["embeddings.token_type_embeddings.weight"] = normal(cfg.type_vocab_size, h)
    ln("embeddings.LayerNorm")
    shapes = {"attention.self.query": (h, h), "attention.self.key": (h, h), "attention.self.value": (h, h),
              "attention.output.dense": (h, h), "intermediate.dense": (inter, h), "output.dense": (h, inter)}
    for l in range(cfg.num_hidden_layers):
        p = f"encoder.layer.{l}."
        for name in LINEARS:
            w[p + name + ".weight"] = normal(*shapes[name])
            w[p + name + ".bias"] = normal(shapes[name][0])
        ln(p + "attention.output.LayerNorm")
        ln(p + "output.LayerNorm")
    return w


def should_quantize(name: str, arr: np.ndarray) -> bool:
    """quantize_arctic_xs.zig:22-34."""
    return (arr.dtype == np.float32 and arr.ndim == 2 and name.endswith(".weight") and "LayerNorm" not in name
            and arr.shape[0] > 0 and arr.shape[1] > 0 and arr.size >= 4096)


def quantize(w: dict, embeddings: bool = False) -> dict:
    """Quantize the encoder linears (and, with `embeddings`, every tensor the
    quantize_arctic_xs rule selects, i.e. also word/position embeddings).
    Returns a new dict with I8 `<name>` and uint16 (f16 bits) `<name>.scale`."""
    out = {}
    for name, arr in w.items():
        sel = should_quantize(name, arr) and (embeddings or not name.startswith("embeddings."))
        if sel:
            q, s = quantize_rows_host(arr)
            out[name] = q
            out[name + ".scale"] = s
        else:
            out[name] = arr
    return out


def dequantize(w: dict) -> dict:
    """f32 view of a quantized dict: W = f32(q) * f32(scale[row])."""
    out = {}
    for name, arr in w.items():
        if name.endswith(".scale"):
            continue
        if arr.dtype == np.int8:
            s = w[name + ".scale"].view(np.float16).astype(np.float32)
            out[name] = arr.astype(np.float32) * s[:, None]
        else:
            out[name] = arr
    return out


class HostWeights:
    """ctypes tzh_arctic_weights over a weight dict (keeps the arrays alive)."""

    def __init__(self, w: dict, cfg: Config = Config()):
        self.cfg = cfg
        self._keep = {k: np.ascontiguousarray(v) for k, v in w.items()}
        self._layers = (_abi.LayerWeights * cfg.num_hidden_layers)()
        s = _abi.ArcticWeights()
        s.config = cfg.to_c()
        s.word_embeddings = self._mat("embeddings.word_embeddings.weight")
        s.position_embeddings = self._mat("embeddings.position_embeddings.weight")
        s.token_type_embeddings = self._mat("embeddings.token_type_embeddings.weight")
        s.layer_norm_gamma = self._ptr("embeddings.LayerNorm.weight")
        s.layer_norm_beta = self._ptr("embeddings.LayerNorm.bias")
        for l in range(cfg.num_hidden_layers):
            p = f"encoder.layer.{l}."
            a, f = self._layers[l].attention, self._layers[l].ffn
            a.query_weight, a.query_bias = self._mat(p + "attention.self.query.weight"), self._ptr(p + "attention.self.query.bias")
            a.key_weight, a.key_bias = self._mat(p + "attention.self.key.weight"), self._ptr(p + "attention.self.key.bias")
            a.value_weight, a.value_bias = self._mat(p + "attention.self.value.weight"), self._ptr(p + "attention.self.value.bias")
            a.output_weight, a.output_bias = self._mat(p + "attention.output.dense.weight"), self._ptr(p + "attention.output.dense.bias")
            a.output_ln_gamma = self._ptr(p + "attention.output.LayerNorm.weight")
            a.output_ln_beta = self._ptr(p + "attention.output.LayerNorm.bias")
            f.intermediate_weight, f.intermediate_bias = self._mat(p + "intermediate.dense.weight"), self._ptr(p + "intermediate.dense.bias")
            f.output_weight, f.output_bias = self._mat(p + "output.dense.weight"), self._ptr(p + "output.dense.bias")
            f.output_ln_gamma = self._ptr(p + "output.LayerNorm.weight")
            f.output_ln_beta = self._ptr(p + "output.LayerNorm.bias")
        s.layers = C.cast(self._layers, C.POINTER(_abi.LayerWeights))
        self.struct = s

    def _ptr(self, name):
        a = self._keep.get(name)
        return None if a is None else a.ctypes.data

    def _mat(self, name) -> _abi.MatView:
        v = _abi.MatView()
        a = self._keep.get(name)
        if a is None:
            return v
        v.data = a.ctypes.data
        v.rows, v.cols = a.shape
        if a.dtype == np.int8:
            v.dtype = _abi.I8
            sc = self._keep.get(name + ".scale")
            v.scale = None if sc is None else sc.ctypes.data
        elif a.dtype == np.float32:
            v.dtype = _abi.F32
        else:
            v.dtype = -1
        return v


def make_batch(seed: int, batch: int, seq_len: int = 512, min_len: int = 16, fixed: bool = False):
    """(ids u32 [batch, seq_len] padded with 0, lengths int32 [batch])."""
    rng = np.random.default_rng(seed)
    if fixed:
        lengths = np.full(batch, seq_len, dtype=np.int32)
    else:
        lengths = rng.integers(min_len, seq_len + 1, size=batch, dtype=np.int64).astype(np.int32)
    ids = np.zeros((batch, seq_len), dtype=np.uint32)
    for b in range(batch):
        L = int(lengths[b])
        ids[b, 0] = 101
        ids[b, 1:L] = rng.integers(1000, 30522, size=L - 1, dtype=np.int64).astype(np.uint32)
    return ids, lengths


def packed(ids: np.ndarray, lengths: np.ndarray):
    """(packed ids [sum L], offsets int64 [batch]) of a padded batch."""
    offs = np.zeros(len(lengths), dtype=np.int64)
    offs[1:] = np.cumsum(lengths[:-1])
    flat = np.concatenate([ids[b, : int(lengths[b])] for b in range(len(lengths))]).astype(np.uint32)
    return flat, offs


def make_vocab(seed: int, size: int = 30522) -> tuple[bytes, list]:
    """A BERT-shaped vocab.txt of `size` lines (no real vocabulary is
    available offline): [PAD], [unused*] up to id 99, [UNK] 100, [CLS] 101,
    [SEP] 102, [MASK] 103, the ASCII punctuation, single letters and digits
    with their "##" forms, then random lowercase words and "##" suffixes.
    Returns (file bytes, the whole words of the vocabulary)."""
    rng = np.random.default_rng(seed)
    lines = ["[PAD]"] + [f"[unused{i}]" for i in range(99)] + ["[UNK]", "[CLS]", "[SEP]", "[MASK]"]
    lines += list("!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~")
    chars = "abcdefghijklmnopqrstuvwxyz0123456789"
    lines += list(chars) + ["##" + c for c in chars]
    seen, words = set(lines), []
    letters = np.array(list("abcdefghijklmnopqrstuvwxyz"))
    while len(lines) < size:
        w = "".join(rng.choice(letters, size=int(rng.integers(2, 9))))
        tok = ("##" + w) if rng.random() < 0.3 else w
        if tok in seen:
            continue
        seen.add(tok)
        lines.append(tok)
        if not tok.startswith("##"):
            words.append(tok)
    return ("\n".join(lines[:size]) + "\n").encode(), words


def make_text(seed: int, words: list, n_words: int, plain: bool = False) -> bytes:
    """Synthetic text of n_words words drawn from `words`.  plain: single
    spaces only, so every word is exactly one piece; otherwise mixed case,
    punctuation, tabs/newlines, out-of-vocabulary and run-together words."""
    rng = np.random.default_rng(seed)
    picks = [words[int(i)] for i in rng.integers(0, len(words), size=n_words)]
    if plain:
        return " ".join(picks).encode()
    out = []
    for w in picks:
        r = rng.random()
        if r < 0.1:
            w = w.upper()
        elif r < 0.15:
            w = w + words[int(rng.integers(0, len(words)))]
        elif r < 0.2:
            w = w + "qzx"
        out.append(w)
        r = rng.random()
        out.append(", " if r < 0.1 else ". " if r < 0.15 else "\t" if r < 0.17 else "\n" if r < 0.19 else " ")
    return "".join(out).encode()
