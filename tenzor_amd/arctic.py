"""Arctic-embed-xs on the GPU: the mirror of model/arctic.zig's entry points.

    ctx = InferenceContext(device=0)                       # arctic.zig:436-465
    weights = ModelWeights.fromSafeTensors(ctx, path)      # arctic.zig:113-166
    forward(out, token_ids, weights, ctx)                  # arctic.zig:874-898
    forwardBatch(outs, ids, lengths, weights, ctx)         # arctic.zig:902-918 / 959-1013

Outputs are L2-normalised CLS embeddings [hidden] per sequence.  Device
tensors are torch tensors on the context's device; ids are uint32 values
stored in an int32 tensor.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import Context, _abi, check, lib
from .synth import Config, HostWeights

InferenceContext = Context
arctic_embed_xs_config = Config()


class ModelWeights:
    """Device-resident weights (tzh_model)."""

    def __init__(self, handle: C.c_void_p, ctx: Context, config: Config):
        self.handle, self.ctx, self.config = handle, ctx, config

    @staticmethod
    def fromSafeTensors(ctx: Context, path: str, config: Config = Config()) -> "ModelWeights":
        h = C.c_void_p()
        cfg = config.to_c()
        check(lib().tzh_arctic_load_safetensors(ctx.handle, str(path).encode(), C.byref(cfg), C.byref(h)))
        return ModelWeights(h, ctx, config)

    @staticmethod
    def fromTenzor(ctx: Context, path: str, config: Config = Config()) -> "ModelWeights":
        """The same weights from a .tenzor file (tenzor_format.zig), read
        from the mapped file."""
        h = C.c_void_p()
        cfg = config.to_c()
        check(lib().tzh_arctic_load_tenzor(ctx.handle, str(path).encode(), C.byref(cfg), C.byref(h)))
        return ModelWeights(h, ctx, config)

    @staticmethod
    def fromHost(ctx: Context, weights: dict, config: Config = Config()) -> "ModelWeights":
        hw = HostWeights(weights, config)
        h = C.c_void_p()
        check(lib().tzh_arctic_upload(ctx.handle, C.byref(hw.struct), C.byref(h)))
        return ModelWeights(h, ctx, config)

    def bad_id_count(self) -> int:
        n = C.c_int32()
        check(lib().tzh_arctic_bad_id_count(self.handle, C.byref(n)))
        return n.value

    def last_launch_count(self) -> int:
        return lib().tzh_arctic_last_launch_count(self.handle)

    def set_precision(self, dtype: str) -> None:
        """Activation precision of later forwards: "float32" (the default,
        the reference's arithmetic) or "float16" (opt-in, f16 activations)."""
        codes = {"float32": _abi.F32, "float16": _abi.F16}
        if dtype not in codes:
            raise ValueError(f"precision must be float32 or float16, not {dtype!r}")
        check(lib().tzh_arctic_set_precision(self.handle, codes[dtype]))

    def set_ffn_fusion(self, enable: bool) -> None:
        """Run each feed-forward block as one kernel where it applies (the
        default) or, with False, as the GEMM pair (no reference counterpart)."""
        check(lib().tzh_arctic_set_ffn_fusion(self.handle, 1 if enable else 0))

    @property
    def precision(self) -> str:
        d = C.c_int32()
        check(lib().tzh_arctic_precision(self.handle, C.byref(d)))
        return "float32" if d.value == _abi.F32 else "float16"

    def set_timing(self, enable: bool, reps: int = 1) -> None:
        """Record a HIP event around every stage of later forwards, each stage
        after the id packing issued `reps` times between its events."""
        check(lib().tzh_arctic_set_timing(self.handle, max(1, int(reps)) if enable else 0))

    def launch_times(self) -> list:
        """[(stage name, microseconds)] of the most recent timed forward, in
        launch order (waits for it to finish)."""
        n = C.c_int32()
        check(lib().tzh_arctic_launch_times(self.handle, None, None, 0, C.byref(n)))
        us = (C.c_float * max(1, n.value))()
        names = (C.c_char_p * max(1, n.value))()
        check(lib().tzh_arctic_launch_times(self.handle, us, names, n.value, C.byref(n)))
        return [(names[i].decode(), float(us[i])) for i in range(n.value)]

    def deinit(self) -> None:
        if self.handle:
            lib().tzh_arctic_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.deinit()
        except Exception:
            pass


def forward(output, token_ids, weights: ModelWeights, ctx: Context | None = None) -> None:
    """Embed one sequence: output f32 [hidden] (device), token_ids [L] (device)."""
    if output.numel() != weights.config.hidden_size:
        raise ValueError("output must hold hidden_size floats")
    check(lib().tzh_arctic_forward(weights.handle, C.c_void_p(output.data_ptr()),
                                   C.c_void_p(token_ids.data_ptr()), int(token_ids.numel())))


def feedForward(output, input, weights: ModelWeights, layer: int, seq_len: int) -> None:
    """arctic.feedForward (arctic.zig:760-811) of encoder layer `layer`:
    output = LayerNorm(input + GELU(input W1^T + b1) W2^T + b2) for device
    f32 tensors input and output of seq_len * hidden_size floats (distinct
    buffers), in f32."""
    n = int(seq_len) * weights.config.hidden_size
    if input.numel() < n or output.numel() < n:
        raise ValueError("input and output must hold seq_len * hidden_size floats")
    check(lib().tzh_arctic_feed_forward(weights.handle, int(layer), C.c_void_p(input.data_ptr()),
                                        C.c_void_p(output.data_ptr()), int(seq_len)))


def forwardBatch(outputs, ids, lengths, weights: ModelWeights, ctx: Context | None = None) -> None:
    """Embed a batch.  ids: device [batch, S] padded (S = row stride) or a
    packed 1-D device tensor of sum(lengths) ids; lengths: host ints."""
    lengths = np.ascontiguousarray(np.asarray(lengths, dtype=np.int32))
    batch = int(lengths.shape[0])
    if outputs.numel() != batch * weights.config.hidden_size:
        raise ValueError("outputs must hold batch * hidden_size floats")
    stride = int(ids.shape[1]) if ids.dim() == 2 else 0
    check(lib().tzh_arctic_forward_batch(weights.handle, C.c_void_p(outputs.data_ptr()), C.c_void_p(ids.data_ptr()),
                                         lengths.ctypes.data, batch, stride))


def forwardBatchHost(outputs: np.ndarray, token_ids_batch, weights: ModelWeights) -> None:
    """arctic.forwardBatch with the reference's host arguments: outputs a host
    f32 array of batch * hidden_size, token_ids_batch a list of host u32
    sequences of any lengths (one upload, one batched forward)."""
    seqs = [np.ascontiguousarray(np.asarray(t, dtype=np.uint32)) for t in token_ids_batch]
    h = weights.config.hidden_size
    if outputs.dtype != np.float32 or not outputs.flags.c_contiguous or outputs.size != len(seqs) * h:
        raise ValueError("outputs must be a contiguous f32 array of batch * hidden_size")
    arr = (_abi.IdsSlice * max(1, len(seqs)))()
    for i, t in enumerate(seqs):
        arr[i].ids = t.ctypes.data
        arr[i].len = t.size
    check(lib().tzh_arctic_forward_batch_host(weights.handle, outputs.ctypes.data, arr, len(seqs)))


def embedDocuments(outputs, texts, tokenizer, weights: ModelWeights) -> np.ndarray:
    """runEmbed's document path (main.zig:786-933) for several documents at
    once: chunks of 510 pieces every 460, one batched forward over all
    chunks, mean of each document's chunk embeddings, L2.  outputs: device
    f32 [len(texts), hidden].  Returns each document's chunk count."""
    from .tokenizer import _text_array

    keep, arr, lens = _text_array(texts)
    n = len(keep)
    if outputs.numel() != n * weights.config.hidden_size:
        raise ValueError("outputs must hold len(texts) * hidden_size floats")
    counts = np.zeros(max(n, 1), np.int32)
    check(lib().tzh_arctic_embed_documents(weights.handle, tokenizer.handle, arr, lens.ctypes.data_as(C.POINTER(C.c_int64)),
                                           n, C.c_void_p(outputs.data_ptr()),
                                           counts.ctypes.data_as(C.POINTER(C.c_int32))))
    return counts[:n]


def embedTexts(outputs, texts, tokenizer, weights: ModelWeights) -> np.ndarray:
    """runEmbed's positional-text path (main.zig:935-1019): each text
    encoded into at most 512 ids, one batched forward.  outputs: device f32
    [len(texts), hidden].  Returns each text's id count."""
    from .tokenizer import _text_array

    keep, arr, lens = _text_array(texts)
    n = len(keep)
    if outputs.numel() != n * weights.config.hidden_size:
        raise ValueError("outputs must hold len(texts) * hidden_size floats")
    counts = np.zeros(max(n, 1), np.int32)
    check(lib().tzh_arctic_embed_texts(weights.handle, tokenizer.handle, arr, lens.ctypes.data_as(C.POINTER(C.c_int64)),
                                       n, C.c_void_p(outputs.data_ptr()), counts.ctypes.data_as(C.POINTER(C.c_int32))))
    return counts[:n]
