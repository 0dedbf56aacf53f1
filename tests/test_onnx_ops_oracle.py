"""Pins of oracle/onnx_ops.py (the restatement of the ONNX executor's
MatMul / Gemm and of the fused matmul epilogue) on the CPU: the
reference's own tests, execGemm's element loops, and the MatMul shape
branches' closed forms."""
import numpy as np

from oracle import onnx_ops as oo


def test_matmul_reference_test():  # onnx/executor.zig:6246-6291
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(1, 7, dtype=np.float32).reshape(3, 2)
    assert oo.matmul(a, b).tolist() == [[22, 28], [49, 64]]


def test_matmul_scalar_operand_scales():  # executor.zig:1545-1577
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    for b in (np.float32(2.5), np.array([2.5], np.float32)):
        y = oo.matmul(a, np.asarray(b))
        assert y.shape == (2, 3) and y.tolist() == (a * 2.5).tolist()


def test_matmul_branches_against_loops():
    """Each shape branch (2-D, 3-D, 3-D x 2-D, 2-D x 3-D, 4-D, 4-D x 2-D,
    1-D x 2-D, 2-D x 1-D) against explicit loops over batches and k."""
    rng = np.random.default_rng(1)

    def loops(a, b):
        a2 = a[None, :] if a.ndim == 1 else a
        b2 = b[:, None] if b.ndim == 1 else b
        batch = np.broadcast_shapes(a2.shape[:-2], b2.shape[:-2])
        A = np.broadcast_to(a2, batch + a2.shape[-2:]).reshape(-1, *a2.shape[-2:])
        B = np.broadcast_to(b2, batch + b2.shape[-2:]).reshape(-1, *b2.shape[-2:])
        out = np.zeros((A.shape[0], A.shape[1], B.shape[2]))
        for z in range(A.shape[0]):
            for i in range(A.shape[1]):
                for j in range(B.shape[2]):
                    out[z, i, j] = sum(float(A[z, i, k]) * float(B[z, k, j]) for k in range(A.shape[2]))
        out = out.reshape(batch + (A.shape[1], B.shape[2]))
        if a.ndim == 1:
            out = out[..., 0, :]
        if b.ndim == 1:
            out = out[..., 0]
        return out

    for sa, sb in [((3, 4), (4, 5)), ((2, 3, 4), (2, 4, 5)), ((2, 3, 4), (4, 5)), ((3, 4), (2, 4, 5)),
                   ((2, 2, 3, 4), (2, 2, 4, 5)), ((2, 2, 3, 4), (4, 5)), ((4,), (4, 5)), ((3, 4), (4,))]:
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32)
        got = oo.matmul(a, b)
        want = loops(a, b)
        assert got.shape == want.shape and np.abs(got - want).max() <= 1e-5, (sa, sb)


def test_gemm_matches_reference_loops():
    """gemm against execGemm's own element loops (4598-4629) for every
    transpose flag and every C shape the reference indexes as ONNX does."""
    rng = np.random.default_rng(3)
    for ta in (False, True):
        for tb in (False, True):
            for cshape in (None, (1, 1), (4,), (1, 4), (3, 4)):
                A = rng.standard_normal((5, 3) if ta else (3, 5)).astype(np.float32)
                B = rng.standard_normal((4, 5) if tb else (5, 4)).astype(np.float32)
                Cm = None if cshape is None else rng.standard_normal(cshape).astype(np.float32)
                got = oo.gemm(A, B, Cm, 0.5, 2.0, ta, tb)
                want = oo.gemm_bruteforce(A, B, Cm, 0.5, 2.0, ta, tb)
                assert np.abs(got - want).max() <= 1e-5, (ta, tb, cshape)


def test_fused_epilogue_reference_test():  # fusion/codegen.zig:330-347
    a = np.array([[1, 2], [3, 4]], np.float32)
    y = oo.fused_matmul_epilogue(a, np.eye(2, dtype=np.float32), np.array([-10, 10], np.float32), ["add", "relu"],
                                 lambda op, v: np.maximum(v, 0))
    assert y.tolist() == [[0, 12], [0, 14]]
