"""TEST INFRASTRUCTURE ONLY — numpy restatement of the ONNX executor's
MatMul and Gemm (onnx/executor.zig:1489-1990, 4561-4634) and of the fused
matmul epilogue (fusion/codegen.zig:78-147).

Only tests/ may import this module; it is the checker, never shipped.
Sums are formed in float64 from the element-type operands and rounded to
the element type once (the reference's summation order, `matmulTiled` /
`batchedMatmul` / its Gemm triple loop, is not observable; the tests bound
the difference).

Pinning (tests/test_onnx_ops_oracle.py): the reference's own MatMul test
(executor.zig:6246-6291: [2,3] @ [3,2] = [[22,28],[49,64]]) and fused
epilogue test (codegen.zig:330-347: relu(A @ I + [-10, 10])); numpy's
matmul on every shape branch of execMatMul; brute-force triple loops of
execGemm's formula on small shapes for every transpose flag and C shape.
"""
from __future__ import annotations

import numpy as np


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """execMatMul (executor.zig:1489-1990).  A zero dimension gives an empty
    (or, with k == 0, zero) result; B of shape [] or [1] scales A
    elementwise (1545-1577); otherwise NumPy matmul: 2-D, batched 3-D/4-D,
    batch broadcasting (3-D x 2-D, 2-D x 3-D, 4-D x 2-D) and the 1-D
    promotions (1850-1990)."""
    t = a.dtype
    if b.ndim == 0 or (b.ndim == 1 and b.shape[0] == 1):
        s = b.reshape(-1)[0] if b.size else t.type(1)
        return (a.astype(np.float64) * np.float64(s)).astype(t)
    return np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(t)


def gemm(a: np.ndarray, b: np.ndarray, c: np.ndarray | None, alpha: float, beta: float, trans_a: bool,
         trans_b: bool) -> np.ndarray:
    """execGemm (executor.zig:4561-4634): out = beta * C (broadcast to
    [M, N]) + alpha * op(A) @ op(B) in f32.  C of one element broadcasts
    that element, a 1-D C is a row vector [N], an [M, N] C adds elementwise
    (4598-4604).  The restatement broadcasts a [1, N] or [M, 1] C the way
    ONNX defines (the reference's index rule, out_idx % c_size, gives the
    same for [1, N] and [M, N] only)."""
    A = a.T if trans_a else a
    B = b.T if trans_b else b
    m, n = A.shape[0], B.shape[1]
    acc = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    out = np.zeros((m, n), np.float32)
    if c is not None:
        cc = c.reshape(n) if c.ndim == 1 else c
        out = (np.float32(beta) * np.broadcast_to(cc, (m, n))).astype(np.float32)
    return (out + (np.float32(alpha) * acc).astype(np.float32)).astype(np.float32)


def gemm_bruteforce(a, b, c, alpha, beta, trans_a, trans_b):
    """execGemm's own loops (4598-4629), element by element in f32, for
    pinning `gemm` on small shapes."""
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    out = np.zeros((M, N), np.float32)
    if c is not None:
        csize = c.size
        flat = c.reshape(-1)
        for i in range(M):
            for j in range(N):
                idx = 0 if csize == 1 else (j if c.ndim == 1 else i * N + j)
                out[i, j] = np.float32(beta) * flat[idx % csize]
    for i in range(M):
        for j in range(N):
            s = np.float32(0)
            for k in range(K):
                av = a[k, i] if trans_a else a[i, k]
                bv = b[j, k] if trans_b else b[k, j]
                s = np.float32(s + np.float32(av) * np.float32(bv))
            out[i, j] = np.float32(out[i, j] + np.float32(alpha) * s)
    return out


def fused_matmul_epilogue(a, b, bias, ops, unary):
    """FusedMatmulEpilogueKernel.apply (codegen.zig:84-147): the matmul,
    then per output the epilogue ops in order: "add" adds bias[j], any
    other op is unary(op, v) (the elementwise engine's op semantics)."""
    y = matmul(a, b)
    for op in ops:
        y = (y + bias).astype(y.dtype) if op == "add" else unary(op, y)
    return y
