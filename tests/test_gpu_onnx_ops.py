"""GPU parity of the matrix-core f32/f64 GEMM (gemm_fp.hip) behind ONNX
Gemm / MatMul (onnx/executor.zig:1489-1990, 4561-4634) and the eval
planner's fused matmul epilogue (fusion/codegen.zig:78-147), against the
numpy restatement in oracle/onnx_ops.py.

Bounds: products are exact in the element type and summed in it in
another order than the reference's, so |gpu - oracle| <= (k + 2) eps
(|alpha| |A| |B|) + 2 eps |result| per element (eps = 2^-24 f32, 2^-53
f64); a transposed operand, a dropped C or a wrong alpha/beta is far
outside it."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import onnx_ops as oo
from tenzor_amd import TzhError, _abi, check, lib
from tenzor_amd.expr import BinaryExpr, Tensor, UnaryExpr, eval

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def gemm(ctx, A, B, Cm, alpha, beta, ta, tb, lda=None, ldb=None):
    m = A.shape[1] if ta else A.shape[0]
    k = A.shape[0] if ta else A.shape[1]
    n = B.shape[0] if tb else B.shape[1]
    Ad, Bd = dev(A), dev(B)
    Cd = None if Cm is None else dev(Cm)
    cr, cc = (0, 0) if Cm is None else ((1, Cm.shape[0]) if Cm.ndim == 1 else Cm.shape)
    Y = torch.full((m, n), float("nan"), device="cuda")
    check(lib().tzh_gemm_f32(ctx.handle, int(ta), int(tb), m, n, k, alpha, Ad.data_ptr(), lda or A.shape[1],
                             Bd.data_ptr(), ldb or B.shape[1], beta, None if Cd is None else Cd.data_ptr(), cr, cc,
                             Y.data_ptr()))
    return Y.cpu().numpy()


def bound(A, B, alpha, ta, tb, ref, eps=2.0 ** -24):
    Aop = np.abs(A.T if ta else A).astype(np.float64)
    Bop = np.abs(B.T if tb else B).astype(np.float64)
    k = Aop.shape[1]
    return abs(alpha) * (Aop @ Bop) * (k + 2) * eps + 2 * eps * np.abs(ref) + 1e-30


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("m,n,k,cshape", [(1, 1, 1, None), (5, 7, 3, (1, 1)), (130, 20, 17, (20,)),
                                          (33, 129, 300, (1, 129)), (257, 300, 64, (257, 300)),
                                          (64, 64, 16, (64, 1)), (9, 200, 0, (9, 200)), (1024, 768, 384, (768,))])
def test_gemm_vs_oracle(ctx, ta, tb, m, n, k, cshape):
    rng = np.random.default_rng(m * 31 + n * 7 + k + ta * 2 + tb)
    A = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    B = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    Cm = None if cshape is None else rng.standard_normal(cshape).astype(np.float32)
    y = gemm(ctx, A, B, Cm, 0.75, -1.5, ta, tb)
    ref = oo.gemm(A, B, Cm, 0.75, -1.5, bool(ta), bool(tb))
    assert (np.abs(y - ref) <= bound(A, B, 0.75, ta, tb, ref) + 2.0 ** -23 * 1.5 * (0 if Cm is None else np.abs(Cm).max())).all()


def test_gemm_row_pitch_and_unaligned(ctx):
    """Row pitches larger than the row (lda > k) and operands off 16-byte
    boundaries (scalar loads)."""
    rng = np.random.default_rng(4)
    Apad = rng.standard_normal((70, 41)).astype(np.float32)
    B = rng.standard_normal((37, 50)).astype(np.float32)
    Ad = dev(np.concatenate([[0.0], Apad.reshape(-1)]).astype(np.float32))
    Bd = dev(B)
    Y = torch.empty((70, 50), device="cuda")
    check(lib().tzh_gemm_f32(ctx.handle, 0, 0, 70, 50, 37, 1.0, Ad.data_ptr() + 4, 41, Bd.data_ptr(), 50, 0.0, None,
                             0, 0, Y.data_ptr()))
    ref = oo.gemm(np.ascontiguousarray(Apad[:, :37]), B, None, 1.0, 0.0, False, False)
    assert (np.abs(Y.cpu().numpy() - ref) <= bound(Apad[:, :37], B, 1.0, 0, 0, ref)).all()


def test_gemm_rejects(ctx):
    A = dev(np.zeros((4, 4), np.float32))
    Y = torch.empty((4, 4), device="cuda")
    with pytest.raises(TzhError) as ei:  # C [3, 4] does not broadcast to [4, 4]
        check(lib().tzh_gemm_f32(ctx.handle, 0, 0, 4, 4, 4, 1.0, A.data_ptr(), 4, A.data_ptr(), 4, 1.0,
                                 A.data_ptr(), 3, 4, Y.data_ptr()))
    assert ei.value.code == _abi.ERR_SHAPE
    with pytest.raises(TzhError) as ei:  # row pitch below the row
        check(lib().tzh_gemm_f32(ctx.handle, 0, 0, 4, 4, 4, 1.0, A.data_ptr(), 3, A.data_ptr(), 4, 0.0, None, 0, 0,
                                 Y.data_ptr()))
    assert ei.value.code == _abi.ERR_INVALID_ARGS


def matmul_nd(ctx, A, B):
    dt = _abi.F64 if A.dtype == np.float64 else _abi.F32
    ys, yn = (C.c_int64 * 8)(), C.c_int32()
    sa, sb = (C.c_int64 * 8)(*A.shape), (C.c_int64 * 8)(*B.shape)
    Ad, Bd = dev(A), dev(B)
    check(lib().tzh_matmul_nd(ctx.handle, dt, Ad.data_ptr(), sa, A.ndim, Bd.data_ptr(), sb, B.ndim, None, ys, C.byref(yn)))
    shape = tuple(ys[i] for i in range(yn.value))
    Y = torch.full(shape, float("nan"), dtype=torch.float64 if A.dtype == np.float64 else torch.float32, device="cuda")
    check(lib().tzh_matmul_nd(ctx.handle, dt, Ad.data_ptr(), sa, A.ndim, Bd.data_ptr(), sb, B.ndim,
                              Y.data_ptr() if Y.numel() else None, ys, C.byref(yn)))
    return Y.cpu().numpy()


def test_matmul_reference_test(ctx):
    """executor.zig:6246-6291: [[1,2,3],[4,5,6]] @ [[1,2],[3,4],[5,6]]."""
    y = matmul_nd(ctx, np.arange(1, 7, dtype=np.float32).reshape(2, 3), np.arange(1, 7, dtype=np.float32).reshape(3, 2))
    assert y.tolist() == [[22, 28], [49, 64]]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("sa,sb", [((7,), (7,)), ((7,), (7, 5)), ((9, 7), (7,)), ((3, 9, 7), (3, 7, 20)),
                                   ((3, 9, 7), (7, 20)), ((9, 7), (3, 7, 20)), ((2, 3, 65, 33), (2, 3, 33, 40)),
                                   ((2, 3, 65, 33), (33, 40)), ((2, 1, 9, 7), (3, 7, 20)), ((300, 129), (129, 257)),
                                   ((4, 6), ()), ((4, 6), (1,)), ((0, 5), (5, 3)), ((4, 0), (0, 3))])
def test_matmul_shapes_vs_oracle(ctx, dt, sa, sb):
    rng = np.random.default_rng(sum(sa) * 3 + sum(sb))
    A = rng.standard_normal(sa).astype(dt)
    B = rng.standard_normal(sb).astype(dt)
    y = matmul_nd(ctx, A, B)
    ref = oo.matmul(A, B)
    assert y.shape == ref.shape
    eps = 2.0 ** -24 if dt == np.float32 else 2.0 ** -53
    if ref.size:
        k = sa[-1] if len(sb) not in (0,) and sb != (1,) else 1
        mag = np.abs(oo.matmul(np.abs(A), np.abs(B)).astype(np.float64))
        assert (np.abs(y.astype(np.float64) - ref) <= mag * (k + 2) * eps + 2 * eps * np.abs(ref) + 1e-300).all()


def leaf(x):
    return Tensor(torch.from_numpy(np.ascontiguousarray(x)).cuda())


def test_fused_epilogue_reference_test():
    """codegen.zig:330-347: relu(A @ I + [-10, 10]) = [[0, 12], [0, 14]]."""
    a = leaf(np.array([[1, 2], [3, 4]], np.float32))
    e = UnaryExpr("relu", BinaryExpr("add", a.matmul(leaf(np.eye(2, dtype=np.float32))),
                                     leaf(np.array([-10, 10], np.float32))))
    assert eval(e).cpu().numpy().tolist() == [[0, 12], [0, 14]]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_fused_epilogue_equals_unfused(dt):
    """A bias add and activations fused into the matmul kernel give the
    same bits as the same ops over the materialised matmul (one op text,
    the same values)."""
    rng = np.random.default_rng(8)
    A = leaf(rng.standard_normal((3, 100, 64)).astype(dt))
    B = leaf(rng.standard_normal((64, 130)).astype(dt))
    bias = leaf(rng.standard_normal(130).astype(dt))
    mm = A.matmul(B)
    tm = Tensor(eval(mm))
    builds = [lambda x: UnaryExpr("relu", BinaryExpr("add", x, bias)), lambda x: UnaryExpr("gelu", x),
              lambda x: UnaryExpr("silu", UnaryExpr("tanh", BinaryExpr("add", bias, x))),
              lambda x: UnaryExpr("sigmoid", BinaryExpr("add", BinaryExpr("add", x, bias), bias))]
    for build in builds:
        fused = eval(build(mm)).cpu().numpy()
        split = eval(build(tm)).cpu().numpy()
        assert np.array_equal(fused, split)
