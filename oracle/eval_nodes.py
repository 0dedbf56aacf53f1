"""TEST INFRASTRUCTURE ONLY — numpy restatement of the executor's softmax,
layernorm, transpose and reshape nodes (executor.zig:363-535) and of an
expression tree that mixes them with exact elementwise ops.

Only tests/ may import this module; it is the checker, never shipped.
Gather is numpy's take on the table; rows outside it are NaN here.  Matmul
is numpy's matmul in float64, rounded to the element type (the reference's
BLAS summation order is unobservable; tests bound the difference).

Pinning (tests/test_eval_nodes_oracle.py): the reference's own tests
(executor.zig:854-1072, softmax.zig:357-490, transpose.zig:146-240),
torch float64 softmax and layer_norm, and numpy's transpose on the
reference's permutations.
"""
from __future__ import annotations

import numpy as np

EPS = np.float32(1e-5)  # layernorm.zig:15, an f32 constant (widened for f64)


def softmax(x: np.ndarray, axis: int) -> np.ndarray:
    """softmaxRow / softmaxAxis (softmax.zig:38-213): max, exp(x - max),
    sum, 1 / sum, product; in x's element type."""
    t = x.dtype.type
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m).astype(x.dtype)
    inv = t(1) / np.sum(e, axis=axis, keepdims=True, dtype=x.dtype)
    return (e * inv).astype(x.dtype)


def layernorm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, norm_dims: int) -> np.ndarray:
    """layerNorm (layernorm.zig:123-185) over the last norm_dims dims."""
    t = x.dtype.type
    n = int(np.prod(x.shape[x.ndim - norm_dims:]))
    rows = x.reshape(-1, n)
    inv_n = t(1) / t(n)
    mean = (rows.sum(axis=1, dtype=x.dtype) * inv_n)[:, None]
    d = rows - mean
    var = (d * d).sum(axis=1, dtype=x.dtype) * inv_n
    inv_std = (t(1) / np.sqrt(var + t(EPS)))[:, None]
    y = (d * inv_std) * gamma.reshape(1, n) + beta.reshape(1, n)
    return y.astype(x.dtype).reshape(x.shape)


def evaluate(expr, host: dict):
    """Evaluate a tenzor_amd.expr tree on the host; `host` maps id(Tensor)
    to its numpy value.  Elementwise ops are restricted to add/sub/mul
    (bit-exact in numpy's element type)."""
    from tenzor_amd import expr as E

    if isinstance(expr, E.Tensor):
        return host[id(expr)]
    if isinstance(expr, E.ScalarExpr):
        return np.array(expr.value, dtype=expr.dtype)
    if isinstance(expr, E.BinaryExpr):
        a, b = evaluate(expr.lhs, host), evaluate(expr.rhs, host)
        return {"add": np.add, "sub": np.subtract, "mul": np.multiply}[expr.op](a, b).astype(expr.dtype)
    if isinstance(expr, E.MatmulExpr):
        a, b = evaluate(expr.lhs, host), evaluate(expr.rhs, host)
        return np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(a.dtype)
    if isinstance(expr, E.GatherExpr):
        table, idx = evaluate(expr.table, host), host[id(expr.indices)]
        ok = (idx >= 0) & (idx < table.shape[0])
        out = table[np.where(ok, idx, 0)].astype(table.dtype)
        out[~ok] = np.nan  # a row outside the table is NaN (the reference panics)
        return out
    if isinstance(expr, E.SoftmaxExpr):
        return softmax(evaluate(expr.input, host), expr.softmax_axis)
    if isinstance(expr, E.LayerNormExpr):
        return layernorm(evaluate(expr.input, host), evaluate(expr.gamma, host), evaluate(expr.beta, host),
                         expr.norm_dims)
    if isinstance(expr, E.TransposeExpr):
        return np.ascontiguousarray(np.transpose(evaluate(expr.input, host), expr.permutation))
    if isinstance(expr, E.ReshapeExpr):
        return evaluate(expr.input, host).reshape(expr.shape)
    if isinstance(expr, E.ReduceExpr) and expr.op == "sum":
        x = evaluate(expr.input, host)
        axis = tuple(a % x.ndim for a in expr.axes) or None
        return np.sum(x, axis=axis, keepdims=expr.keepdims, dtype=x.dtype)
    raise TypeError(f"no restatement for {type(expr).__name__}")
