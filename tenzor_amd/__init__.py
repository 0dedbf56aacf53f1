"""tenzor_amd — MI355X (gfx950) backend for tenzor's hot path.

Python binding of libtenzor_hip.so (include/tenzor_hip.h).  The library is
the product; this module only loads it, raises on its error codes and
mirrors the reference's entry points (`tenzor_amd.expr`: Tensor / *Expr /
eval / evalInto; `tenzor_amd.arctic`: Config / ModelWeights /
InferenceContext / forward / forwardBatch).

There is no CPU fallback: if the shared library is missing, or no gfx950
device is present, the calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

from . import _abi

LIB_PATH = Path(__file__).resolve().parent / "libtenzor_hip.so"
_lib = None


class TzhError(RuntimeError):
    """A non-zero status from the C-ABI; `.code` is the TZH_ERR_* value."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.name = _abi.ERROR_NAMES.get(code, f"Error{code}")
        super().__init__(f"{self.name} ({code}): {message}")


def lib() -> C.CDLL:
    """The loaded libtenzor_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m tenzor_amd.build`")
        _lib = _abi.bind(C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL))
    return _lib


def check(rc: int) -> None:
    if rc != _abi.OK:
        msg = lib().tzh_last_error()
        raise TzhError(rc, msg.decode() if msg else "")


class Context:
    """A device context (tzh_ctx): one GPU, one HIP stream.

    By default it enqueues on torch's current stream of `device` (handle 0 is
    the default stream), so work issued through torch and through this
    library is ordered.
    """

    def __init__(self, device: int = 0, stream: int | None = None, use_torch_stream: bool = True):
        self.device = device
        if stream is None and use_torch_stream:
            import torch

            stream = torch.cuda.current_stream(device).cuda_stream
        h = C.c_void_p()
        check(lib().tzh_init(device, C.c_void_p(stream or 0), C.byref(h)))
        self.handle = h

    @property
    def stream(self) -> int:
        return lib().tzh_stream(self.handle)

    def sync(self) -> None:
        check(lib().tzh_sync(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().tzh_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def quantize_rows_host(w):
    """Host quantizer (quantize_arctic_xs.zig:94-115): f32 [rows, cols] ->
    (int8 codes [rows, cols], f16 scale bits as uint16 [rows])."""
    import numpy as np

    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.int8)
    s = np.empty((rows,), dtype=np.uint16)
    check(lib().tzh_quantize_rows_host(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data))
    return q, s


def quantize_safetensors(in_path: str, out_path: str) -> int:
    """The quantize_arctic_xs tool; returns the number of tensors quantized."""
    n = C.c_int32()
    check(lib().tzh_quantize_safetensors(str(in_path).encode(), str(out_path).encode(), C.byref(n)))
    return n.value
