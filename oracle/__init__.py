"""TEST INFRASTRUCTURE ONLY — ctypes loader of the CPU oracle (oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.  It restates the reference's CPU algorithms; it is the
checker, never the thing measured or shipped.

Pinning (see tests/test_oracle_pins.py): every function here is checked
against the reference's own known-answer tests and against independent
implementations (numpy, torch, HuggingFace BertModel built from a config)
or closed forms chosen so that a dropped term, wrong sign, transposed
operand or wrong index fails.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

from tenzor_amd import _abi

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None

vp, i32, i64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float


def build() -> Path:
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [f32]),
            "orc_f16_to_f32": (f32, [C.c_uint16]),
            "orc_quantize_rows": (None, [vp, i64, i64, vp, vp]),
            "orc_matmul_w8a32": (None, [vp, vp, vp, vp, vp, i64, i64, i64]),
            "orc_linear_f32": (None, [vp, vp, vp, vp, i64, i64, i64]),
            "orc_layernorm": (None, [vp, vp, vp, vp, i64, i64, f32]),
            "orc_gelu": (f32, [f32]),
            "orc_gelu_vec": (None, [vp, vp, i64]),
            "orc_l2_normalize": (None, [vp, i64]),
            "orc_attention_head": (None, [vp, vp, vp, vp, i64, i64, i64, vp]),
            "orc_embeddings": (None, [vp, vp, i64, C.POINTER(_abi.ArcticWeights)]),
            "orc_arctic_forward": (C.c_int, [C.POINTER(_abi.ArcticWeights), vp, i64, vp]),
            "orc_arctic_hidden": (C.c_int, [C.POINTER(_abi.ArcticWeights), vp, i64, i32, vp]),
            "orc_arctic_forward_batch": (C.c_int, [C.POINTER(_abi.ArcticWeights), vp, vp, vp, i32, vp, i32]),
            "orc_eval": (C.c_int, [C.POINTER(_abi.Node), i32, C.POINTER(_abi.Leaf), i32, i32, vp]),
            "orc_unary_f32": (f32, [i32, f32]),
            "orc_binary_f32": (f32, [i32, f32, f32]),
            "orc_unary_vec_f32": (None, [i32, vp, vp, i64]),
            "orc_binary_vec_f32": (None, [i32, vp, vp, vp, i64]),
            "orc_chain_add_mul_exp": (None, [vp, vp, vp, vp, i64, i64, vp, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def quantize_rows(w):
    w = _f32(w)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.uint16)
    lib().orc_quantize_rows(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data)
    return q, s


def matmul_w8a32(a, wq, scale, bias=None):
    a = _f32(a)
    wq = np.ascontiguousarray(wq, np.int8)
    scale = np.ascontiguousarray(scale, np.uint16)
    m, k = a.shape
    n = wq.shape[0]
    c = np.empty((m, n), np.float32)
    b = None if bias is None else _f32(bias)
    lib().orc_matmul_w8a32(a.ctypes.data, wq.ctypes.data, scale.ctypes.data, None if b is None else b.ctypes.data,
                           c.ctypes.data, m, k, n)
    return c


def linear_f32(a, w, bias=None):
    """The f32 model's linear (arctic.zig:609-621): C = A W^T, then += bias."""
    a, w = _f32(a), _f32(w)
    m, k = a.shape
    n = w.shape[0]
    c = np.empty((m, n), np.float32)
    b = None if bias is None else _f32(bias)
    lib().orc_linear_f32(a.ctypes.data, w.ctypes.data, None if b is None else b.ctypes.data, c.ctypes.data, m, k, n)
    return c


def layernorm(x, gamma, beta, eps):
    x = _f32(x)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    g, b = _f32(gamma), _f32(beta)
    lib().orc_layernorm(x.ctypes.data, g.ctypes.data, b.ctypes.data, y.ctypes.data, rows, n, eps)
    return y


def gelu(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_gelu_vec(x.ctypes.data, y.ctypes.data, x.size)
    return y


def l2_normalize(v):
    v = _f32(v).copy()
    lib().orc_l2_normalize(v.ctypes.data, v.size)
    return v


def attention_head(q, k, v):
    """q, k, v: [L, d] -> [L, d] (one head, arctic.zig:660-713)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    L, d = q.shape
    out = np.empty_like(q)
    scores = np.empty(L * L, np.float32)
    lib().orc_attention_head(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data, L, d, d,
                             scores.ctypes.data)
    return out


def unary(op: str, x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_unary_vec_f32(_abi.OP[op], x.ctypes.data, y.ctypes.data, x.size)
    return y


def binary(op: str, a, b):
    a, b = _f32(a), _f32(b)
    y = np.empty_like(a)
    lib().orc_binary_vec_f32(_abi.OP[op], a.ctypes.data, b.ctypes.data, y.ctypes.data, a.size)
    return y


def arctic_forward(host_weights, ids):
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty(host_weights.cfg.hidden_size, np.float32)
    rc = lib().orc_arctic_forward(C.byref(host_weights.struct), ids.ctypes.data, ids.size, out.ctypes.data)
    if rc:
        raise ValueError("oracle forward rejected its arguments")
    return out


def arctic_hidden(host_weights, ids, n_layers):
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty((ids.size, host_weights.cfg.hidden_size), np.float32)
    rc = lib().orc_arctic_hidden(C.byref(host_weights.struct), ids.ctypes.data, ids.size, n_layers, out.ctypes.data)
    if rc:
        raise ValueError("oracle forward rejected its arguments")
    return out


def arctic_forward_batch(host_weights, flat_ids, offsets, lengths, nthreads=1):
    flat_ids = np.ascontiguousarray(flat_ids, np.uint32)
    offsets = np.ascontiguousarray(offsets, np.int64)
    lengths = np.ascontiguousarray(lengths, np.int32)
    out = np.empty((len(lengths), host_weights.cfg.hidden_size), np.float32)
    rc = lib().orc_arctic_forward_batch(C.byref(host_weights.struct), flat_ids.ctypes.data, offsets.ctypes.data,
                                        lengths.ctypes.data, len(lengths), out.ctypes.data, nthreads)
    if rc:
        raise ValueError("oracle batch forward rejected its arguments")
    return out


def eval_tape(nodes, leaf_arrays, dtype=np.float32):
    """Evaluate a tenzor_amd.expr tape with host numpy leaves."""
    leaves = (_abi.Leaf * max(1, len(leaf_arrays)))()
    keep = []
    for i, a in enumerate(leaf_arrays):
        a = np.ascontiguousarray(a, dtype)
        keep.append(a)
        leaves[i].data = a.ctypes.data
        leaves[i].ndim = a.ndim
        for j, d in enumerate(a.shape):
            leaves[i].shape[j] = d
    root = nodes[-1]
    shape = tuple(root.shape[i] for i in range(root.ndim))
    out = np.empty(shape, dtype)
    tape = (_abi.Node * len(nodes))(*nodes)
    rc = lib().orc_eval(tape, len(nodes), leaves, len(leaf_arrays), _abi.F64 if dtype == np.float64 else _abi.F32,
                        out.ctypes.data)
    return rc, out


def chain_add_mul_exp(a, b_row, c):
    a, b_row, c = _f32(a), _f32(b_row), _f32(c)
    rows, cols = a.shape
    out = np.empty_like(a)
    t1 = np.empty_like(a)
    t2 = np.empty_like(a)
    lib().orc_chain_add_mul_exp(a.ctypes.data, b_row.ctypes.data, c.ctypes.data, out.ctypes.data, rows, cols,
                                t1.ctypes.data, t2.ctypes.data)
    return out
