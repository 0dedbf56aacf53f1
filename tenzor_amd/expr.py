"""Lazy expressions evaluated on the GPU: the mirror of ops/expr.zig and
backend/cpu/executor.zig's eval/evalInto.

    a = Tensor(torch_tensor)               # device-resident leaf (tensor.zig:28)
    e = BinaryExpr("add", a, b).mul(c).exp()  # builds a DAG, computes nothing
    out = eval(e)                          # executor.eval  (executor.zig:29-45)
    evalInto(e, out_tensor)                # executor.evalInto (executor.zig:49-54)

Construction checks what Zig checks at comptime (expr.zig:212-217,
352-376): element types match, shapes broadcast (NumPy rules,
shape.zig:168-204); violations raise TypeError / ValueError.  eval walks
the DAG once into a post-order node tape (`to_tape`) and hands it to
tzh_eval_into, which runs each elementwise chain as one kernel.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import _abi, check, lib

UNARY_OPS = ("neg", "abs", "exp", "log", "sqrt", "rsqrt", "sin", "cos", "tanh", "sigmoid", "relu", "gelu",
             "silu", "softplus", "floor", "ceil", "round", "exp2", "log2", "log10", "tan", "sinh", "cosh",
             "asin", "acos", "atan", "leaky_relu", "sign")
BINARY_OPS = ("add", "sub", "mul", "div", "pow", "max", "min", "mod", "atan2", "eq", "ne", "lt", "le", "gt", "ge")
REDUCE_OPS = ("sum", "prod", "reduce_max", "reduce_min", "mean", "variance")

_DTYPES = {"float32": _abi.F32, "float64": _abi.F64}
# integer leaves, allowed only as gather indices (TZH_I32, TZH_I64)
_INDEX_DTYPES = {"int32": 6, "int64": 7}


def broadcast_shape(a: Sequence[int], b: Sequence[int]) -> tuple:
    """shape.zig:168-204 (raises ValueError when incompatible)."""
    n = max(len(a), len(b))
    out = []
    for i in range(n):
        da = a[len(a) - n + i] if i >= n - len(a) else 1
        db = b[len(b) - n + i] if i >= n - len(b) else 1
        if da != db and da != 1 and db != 1:
            raise ValueError(f"Shapes not broadcast compatible: {tuple(a)} vs {tuple(b)}")
        out.append(max(da, db))
    return tuple(out)


def reduce_shape(shape: Sequence[int], axes: Sequence[int], keepdims: bool) -> tuple:
    """shape.zig:279-320 ReduceShape (one axis or all)."""
    if len(axes) == 0:
        return tuple(1 for _ in shape) if keepdims else ()
    if len(axes) != 1:
        raise ValueError("only a single reduction axis is supported (executor.zig:347-348)")
    ax = axes[0] + len(shape) if axes[0] < 0 else axes[0]
    if not 0 <= ax < len(shape):
        raise ValueError(f"axis {axes[0]} out of range for rank {len(shape)}")
    if keepdims:
        return tuple(1 if i == ax else d for i, d in enumerate(shape))
    return tuple(d for i, d in enumerate(shape) if i != ax)


class Expr:
    kind: int
    shape: tuple
    dtype: str

    # unary methods (expr.zig:236-287)
    def neg(self): return UnaryExpr("neg", self)
    def abs(self): return UnaryExpr("abs", self)
    def exp(self): return UnaryExpr("exp", self)
    def log(self): return UnaryExpr("log", self)
    def sqrt(self): return UnaryExpr("sqrt", self)
    def rsqrt(self): return UnaryExpr("rsqrt", self)
    def sin(self): return UnaryExpr("sin", self)
    def cos(self): return UnaryExpr("cos", self)
    def tanh(self): return UnaryExpr("tanh", self)
    def sigmoid(self): return UnaryExpr("sigmoid", self)
    def relu(self): return UnaryExpr("relu", self)
    def gelu(self): return UnaryExpr("gelu", self)
    def silu(self): return UnaryExpr("silu", self)

    # binary methods (expr.zig:289-316)
    def add(self, o): return BinaryExpr("add", self, as_expr(o, self.dtype))
    def sub(self, o): return BinaryExpr("sub", self, as_expr(o, self.dtype))
    def mul(self, o): return BinaryExpr("mul", self, as_expr(o, self.dtype))
    def div(self, o): return BinaryExpr("div", self, as_expr(o, self.dtype))
    def pow(self, o): return BinaryExpr("pow", self, as_expr(o, self.dtype))
    def maximum(self, o): return BinaryExpr("max", self, as_expr(o, self.dtype))
    def minimum(self, o): return BinaryExpr("min", self, as_expr(o, self.dtype))

    # reductions over all axes (expr.zig:323-342)
    def matmul(self, o): return MatmulExpr(self, o)
    def softmax(self, axis: int): return SoftmaxExpr(self, axis)
    def transpose(self, perm): return TransposeExpr(self, perm)
    def reshape(self, shape): return ReshapeExpr(self, shape)

    def sum(self): return ReduceExpr("sum", self)
    def mean(self): return ReduceExpr("mean", self)
    def prod(self): return ReduceExpr("prod", self)
    def reduceMax(self): return ReduceExpr("reduce_max", self)
    def reduceMin(self): return ReduceExpr("reduce_min", self)

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class Tensor(Expr):
    """Leaf: a contiguous device tensor (torch, float32 or float64)."""

    kind = _abi.NODE_TENSOR

    def __init__(self, data):
        name = str(data.dtype).replace("torch.", "")
        if name not in _DTYPES and name not in _INDEX_DTYPES:
            raise TypeError(f"element type {data.dtype} is not supported (float32, float64; int32/int64 indices)")
        if not data.is_contiguous():
            raise ValueError("leaf tensors must be contiguous row-major")
        if len(data.shape) > _abi.MAX_RANK:
            raise ValueError("rank above MAX_RANK (shape.zig:10)")
        self.data = data
        self.shape = tuple(data.shape)
        self.dtype = str(data.dtype).replace("torch.", "")


class ScalarExpr(Expr):
    """Rank-0 constant (expr.zig:1010-1035)."""

    kind = _abi.NODE_CONSTANT

    def __init__(self, value: float, dtype: str = "float32"):
        self.value = float(value)
        self.shape = ()
        self.dtype = dtype


def as_expr(x, dtype: str) -> Expr:
    """AsExpr/asExpr (expr.zig:1041-1063): expressions pass through, Python
    numbers become ScalarExpr of the other operand's element type."""
    if isinstance(x, Expr):
        return x
    if isinstance(x, (int, float)):
        return ScalarExpr(x, dtype)
    raise TypeError(f"Cannot convert {type(x).__name__} to expression")


class UnaryExpr(Expr):
    kind = _abi.NODE_UNARY

    def __init__(self, op: str, input: Expr):
        if op not in UNARY_OPS:
            raise TypeError(f"Expected unary operation, got {op}")
        self.op, self.input = op, input
        self.shape, self.dtype = input.shape, input.dtype


class BinaryExpr(Expr):
    kind = _abi.NODE_BINARY

    def __init__(self, op: str, lhs: Expr, rhs: Expr):
        if op not in BINARY_OPS:
            raise TypeError(f"Expected binary operation, got {op}")
        if lhs.dtype != rhs.dtype:
            raise TypeError(f"Type mismatch in binary operation: {lhs.dtype} vs {rhs.dtype}")
        self.op, self.lhs, self.rhs = op, lhs, rhs
        self.shape = broadcast_shape(lhs.shape, rhs.shape)
        self.dtype = lhs.dtype


class ReduceExpr(Expr):
    kind = _abi.NODE_REDUCE

    def __init__(self, op: str, input: Expr, axes: Sequence[int] = (), keepdims: bool = False):
        if op not in REDUCE_OPS:
            raise TypeError(f"Expected reduction operation, got {op}")
        self.op, self.input = op, input
        self.axes, self.keepdims = tuple(axes), keepdims
        self.shape = reduce_shape(input.shape, self.axes, keepdims)
        self.dtype = input.dtype


class MatmulExpr(Expr):
    """MatmulExpr (executor.zig:199-326): 1-D operands are a row / a column
    whose unit dimension the result drops; batch dimensions broadcast."""

    kind = _abi.NODE_MATMUL

    def __init__(self, lhs: Expr, rhs: Expr):
        if lhs.dtype != rhs.dtype:
            raise TypeError(f"Type mismatch in matmul: {lhs.dtype} vs {rhs.dtype}")
        ls, rs = tuple(lhs.shape), tuple(rhs.shape)
        if not ls or not rs:
            raise TypeError("matmul needs operands of rank >= 1")
        k = ls[-1]
        k2 = rs[0] if len(rs) == 1 else rs[-2]
        if k != k2:
            raise TypeError(f"Matmul inner dimensions differ: {k} vs {k2}")
        batch = broadcast_shape(ls[:-2], rs[:-2]) if (len(ls) > 2 or len(rs) > 2) else ()
        self.lhs, self.rhs = lhs, rhs
        self.shape = tuple(batch) + ((ls[-2],) if len(ls) > 1 else ()) + ((rs[-1],) if len(rs) > 1 else ())
        self.dtype = lhs.dtype


class GatherExpr(Expr):
    """GatherExpr (expr.zig:775-830): rows of a 2-D table [vocab, embed]
    picked by an integer index tensor; shape = indices.shape ++ [embed]."""

    kind = _abi.NODE_GATHER

    def __init__(self, table: Expr, indices: "Tensor"):
        if len(table.shape) != 2:
            raise TypeError(f"Gather table must be 2D [vocab, embed], got {len(table.shape)}D")
        if not isinstance(indices, Tensor) or indices.dtype not in _INDEX_DTYPES:
            raise TypeError("Gather indices must be an integer tensor")
        self.table, self.indices = table, indices
        self.shape = tuple(indices.shape) + (table.shape[1],)
        self.dtype = table.dtype


class SoftmaxExpr(Expr):
    """SoftmaxExpr (expr.zig:665-696): softmax along one axis (negative
    axes count from the end, shape.normalizeAxis)."""

    kind = _abi.NODE_SOFTMAX

    def __init__(self, input: Expr, axis: int):
        nd = len(input.shape)
        ax = axis + nd if axis < 0 else axis
        if not 0 <= ax < nd:
            raise ValueError(f"axis {axis} out of range for rank {nd}")
        self.input, self.softmax_axis = input, ax
        self.shape, self.dtype = input.shape, input.dtype


class LayerNormExpr(Expr):
    """LayerNormExpr (expr.zig:705-760): normalise over the last norm_dims
    dimensions; gamma and beta have exactly those dimensions."""

    kind = _abi.NODE_LAYERNORM

    def __init__(self, input: Expr, gamma: Expr, beta: Expr, norm_dims: int = 1):
        nd = len(input.shape)
        if not 1 <= norm_dims <= nd:
            raise ValueError(f"norm_dims {norm_dims} out of range for rank {nd}")
        if len(gamma.shape) != norm_dims or len(beta.shape) != norm_dims:
            raise TypeError("Gamma/beta rank must equal normalized_dims")
        if tuple(gamma.shape) != tuple(input.shape[nd - norm_dims:]) or tuple(beta.shape) != tuple(gamma.shape):
            raise TypeError("Gamma/beta shape must match last dimensions of input")
        if not (input.dtype == gamma.dtype == beta.dtype):
            raise TypeError("LayerNorm operands must share one element type")
        self.input, self.gamma, self.beta, self.norm_dims = input, gamma, beta, norm_dims
        self.shape, self.dtype = input.shape, input.dtype


class TransposeExpr(Expr):
    """TransposeExpr (expr.zig:925-990): output axis i is input axis perm[i]."""

    kind = _abi.NODE_TRANSPOSE

    def __init__(self, input: Expr, perm):
        perm = tuple(int(p) for p in perm)
        nd = len(input.shape)
        if len(perm) != nd:
            raise TypeError(f"Permutation length {len(perm)} must match rank {nd}")
        if sorted(perm) != list(range(nd)):
            raise TypeError("Invalid transpose permutation")
        self.input, self.permutation = input, perm
        self.shape = tuple(input.shape[p] for p in perm)
        self.dtype = input.dtype


class ReshapeExpr(Expr):
    """ReshapeExpr: the same elements under another shape."""

    kind = _abi.NODE_RESHAPE

    def __init__(self, input: Expr, shape):
        shape = tuple(int(d) for d in shape)
        if int(np.prod(shape, dtype=np.int64)) != input.numel():
            raise TypeError("Reshape must preserve the element count")
        self.input = input
        self.shape, self.dtype = shape, input.dtype


def to_tape(expr: Expr):
    """Post-order node tape + leaf list (what a comptime walk emits)."""
    nodes, leaves, leaf_ids = [], [], {}

    def visit(e: Expr) -> int:
        n = _abi.Node()
        n.kind = e.kind
        n.lhs = n.rhs = n.leaf = -1
        n.axis = -1
        n.ndim = len(e.shape)
        for i, d in enumerate(e.shape):
            n.shape[i] = d
        if isinstance(e, Tensor):
            key = id(e)
            if key not in leaf_ids:
                leaf_ids[key] = len(leaves)
                leaves.append(e)
            n.leaf = leaf_ids[key]
        elif isinstance(e, ScalarExpr):
            n.value = e.value
        elif isinstance(e, UnaryExpr):
            n.op = _abi.OP[e.op]
            n.lhs = visit(e.input)
        elif isinstance(e, BinaryExpr):
            n.op = _abi.OP[e.op]
            n.lhs = visit(e.lhs)
            n.rhs = visit(e.rhs)
        elif isinstance(e, ReduceExpr):
            n.op = _abi.OP[e.op]
            n.lhs = visit(e.input)
            n.keepdims = int(e.keepdims)
            if e.axes:
                ax = e.axes[0]
                n.axis = ax + len(e.input.shape) if ax < 0 else ax
        elif isinstance(e, MatmulExpr):
            n.lhs = visit(e.lhs)
            n.rhs = visit(e.rhs)
        elif isinstance(e, GatherExpr):
            n.lhs = visit(e.table)
            n.rhs = visit(e.indices)
        elif isinstance(e, SoftmaxExpr):
            n.lhs = visit(e.input)
            n.axis = e.softmax_axis
        elif isinstance(e, LayerNormExpr):
            n.lhs = visit(e.input)
            n.rhs = visit(e.gamma)
            n.aux = visit(e.beta)
            n.axis = e.norm_dims
        elif isinstance(e, TransposeExpr):
            n.lhs = visit(e.input)
            for i, p in enumerate(e.permutation):
                n.perm[i] = p
        elif isinstance(e, ReshapeExpr):
            n.lhs = visit(e.input)
        else:
            raise TypeError(f"unsupported expression node {type(e).__name__}")
        nodes.append(n)
        return len(nodes) - 1

    visit(expr)
    return nodes, leaves


def _leaf_structs(leaves) -> "C.Array":
    arr = (_abi.Leaf * max(1, len(leaves)))()
    for i, t in enumerate(leaves):
        arr[i].data = t.data.data_ptr()
        arr[i].ndim = len(t.shape)
        arr[i].dtype = _INDEX_DTYPES.get(t.dtype, 0)
        for j, d in enumerate(t.shape):
            arr[i].shape[j] = d
    return arr


_default_ctx = {}


def _ctx_for(device: int):
    from . import Context

    if device not in _default_ctx:
        _default_ctx[device] = Context(device)
    return _default_ctx[device]


def evalInto(expr: Expr, output, ctx=None) -> None:
    """executor.evalInto: evaluate `expr` into the contiguous device tensor
    `output` (same element type, numel of expr.shape)."""
    import torch

    if str(output.dtype).replace("torch.", "") != expr.dtype:
        raise TypeError(f"output dtype {output.dtype} != expression dtype {expr.dtype}")
    if output.numel() != expr.numel() or not output.is_contiguous():
        raise ValueError("output must be contiguous with numel of the expression shape")
    nodes, leaves = to_tape(expr)
    device = output.device.index if output.device.index is not None else torch.cuda.current_device()
    for t in leaves:
        if t.data.device != output.device:
            raise ValueError("all leaves must live on the output's device")
    ctx = ctx or _ctx_for(device)
    tape = (_abi.Node * len(nodes))(*nodes)
    check(lib().tzh_eval_into(ctx.handle, tape, len(nodes), _leaf_structs(leaves), len(leaves),
                              _DTYPES[expr.dtype], C.c_void_p(output.data_ptr())))


def eval(expr: Expr, ctx=None, device=None):
    """executor.eval: allocate the result tensor and evaluate into it."""
    import torch

    dev = device
    if dev is None:
        _, leaves = to_tape(expr)
        dev = leaves[0].data.device if leaves else torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(expr.shape, dtype=getattr(torch, expr.dtype), device=dev)
    evalInto(expr, out, ctx)
    return out
