"""GPU parity of the softmax, layernorm, transpose and reshape nodes of
`eval` (executor.zig:363-535) against the numpy restatement
(oracle/eval_nodes.py).  Bars: transpose and reshape bit-exact; softmax and
layernorm within 1e-5 (f32) / 1e-12 (f64) of the restatement, relative to
the largest output magnitude (exp, sqrt and summation order differ from
numpy's by ulps; the reference's own order is unobservable)."""
import numpy as np
import pytest
import torch

from oracle import eval_nodes as en

from tenzor_amd.expr import LayerNormExpr, ReduceExpr, Tensor, eval

pytestmark = pytest.mark.gpu


def leaf(a):
    t = Tensor(torch.from_numpy(np.ascontiguousarray(a)).cuda())
    return t


def check_close(e, host, dt):
    got = eval(e).cpu().numpy()
    ref = en.evaluate(e, host)
    tol = 1e-5 if dt == np.float32 else 1e-12
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= tol * max(1.0, float(np.abs(ref).max()))
    return got, ref


def test_reference_known_answers():
    """executor.zig:854-1030 through the GPU path."""
    y = eval(leaf(np.array([[1, 2, 3], [0, 0, 0]], np.float32)).softmax(-1)).cpu().numpy()
    assert np.allclose(y.sum(1), 1, atol=1e-5) and np.allclose(y[1], 1 / 3, atol=1e-5)
    x = leaf(np.array([[1, 2, 3, 4], [10, 20, 30, 40]], np.float32))
    g, b = leaf(np.ones(4, np.float32)), leaf(np.zeros(4, np.float32))
    y = eval(LayerNormExpr(x, g, b, 1)).cpu().numpy()
    assert np.allclose(y.mean(1), 0, atol=1e-5) and np.allclose(y[0], y[1], atol=1e-5)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_nodes_vs_restatement(dt):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((6, 33, 300)) * 4).astype(dt)
    y = rng.standard_normal((33, 300)).astype(dt)
    g, b = rng.standard_normal(300).astype(dt), rng.standard_normal(300).astype(dt)
    tx, ty, tg, tb = leaf(x), leaf(y), leaf(g), leaf(b)
    host = {id(tx): x, id(ty): y, id(tg): g, id(tb): b}
    for e in [tx.softmax(-1), tx.softmax(1), tx.softmax(0), LayerNormExpr(tx, tg, tb, 1),
              tx.softmax(-1).mul(3.0).add(ty), LayerNormExpr(tx.mul(ty), tg, tb, 1).transpose((2, 0, 1)),
              tx.softmax(-1).sum(), ReduceExpr("sum", tx.transpose((2, 1, 0)), (0,))]:
        check_close(e, host, dt)
    g2 = rng.standard_normal((33, 300)).astype(dt)
    tg2 = leaf(g2)
    host[id(tg2)] = g2
    check_close(LayerNormExpr(tx, tg2, tg2, 2), host, dt)


@pytest.mark.parametrize("perm", [(1, 0, 2, 3), (0, 2, 1, 3), (3, 2, 1, 0), (0, 1, 2, 3), (2, 0, 3, 1)])
def test_transpose_bit_exact(perm):
    """Includes the attention pattern [B,S,H,D] -> [B,H,S,D] (executor.zig:505-520)."""
    x = np.random.default_rng(6).standard_normal((4, 128, 12, 32)).astype(np.float32)
    got = eval(leaf(x).transpose(perm)).cpu().numpy()
    assert np.array_equal(got, np.transpose(x, perm))


def test_reshape_and_large_rows():
    x = np.random.default_rng(7).standard_normal((4096, 1000)).astype(np.float32)
    tx = leaf(x)
    assert np.array_equal(eval(tx.reshape((1000, 4096))).cpu().numpy(), x.reshape(1000, 4096))
    got = eval(tx.softmax(-1)).cpu().numpy()
    assert np.abs(got - en.softmax(x, 1)).max() < 1e-6
    assert np.abs(got.sum(1) - 1).max() < 1e-5


def test_malformed_layernorm_is_rejected():
    x = leaf(np.zeros((2, 4), np.float32))
    g = leaf(np.zeros(3, np.float32))
    with pytest.raises(TypeError):
        LayerNormExpr(x, g, g, 1)  # the mirror's compile-time check
    from tenzor_amd.expr import to_tape
    e = LayerNormExpr(x, leaf(np.zeros(4, np.float32)), leaf(np.zeros(4, np.float32)), 1)
    nodes, leaves = to_tape(e)
    nodes[-1].axis = 3  # norm_dims beyond the rank
    import ctypes as C
    from tenzor_amd import _abi, lib
    from tenzor_amd.expr import _ctx_for, _leaf_structs
    out = torch.empty((2, 4), device="cuda")
    tape = (_abi.Node * len(nodes))(*nodes)
    rc = lib().tzh_eval_into(_ctx_for(0).handle, tape, len(nodes), _leaf_structs(leaves), len(leaves), _abi.F32,
                             C.c_void_p(out.data_ptr()))
    assert rc == -10  # TZH_ERR_SHAPE



def test_gather_reference_known_answers():
    """executor.zig:1074-1168: rows of a [4, 3] table by [0, 2, 1]; a
    [10, 4] table whose row i holds i, by [[0, 5, 9], [1, 2, 3]]."""
    from tenzor_amd.expr import GatherExpr

    table = leaf(np.arange(1, 13, dtype=np.float32).reshape(4, 3))
    idx = Tensor(torch.tensor([0, 2, 1], dtype=torch.int32).cuda())
    got = eval(GatherExpr(table, idx)).cpu().numpy()
    assert got.tolist() == [[1, 2, 3], [7, 8, 9], [4, 5, 6]]
    table = leaf(np.repeat(np.arange(10, dtype=np.float32), 4).reshape(10, 4))
    idx = Tensor(torch.tensor([[0, 5, 9], [1, 2, 3]], dtype=torch.int64).cuda())
    got = eval(GatherExpr(table, idx)).cpu().numpy()
    assert got.shape == (2, 3, 4) and np.array_equal(got[..., 0], [[0, 5, 9], [1, 2, 3]])


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_gather_chains_and_out_of_range(dt):
    from tenzor_amd.expr import GatherExpr

    rng = np.random.default_rng(8)
    tab = rng.standard_normal((30522, 384)).astype(dt)
    idx = rng.integers(0, 30522, size=(16, 128)).astype(np.int32)
    idx[3, 5] = 30522
    idx[7, 0] = -1
    tt, ti = leaf(tab), Tensor(torch.from_numpy(idx).cuda())
    host = {id(tt): tab, id(ti): idx}
    for e in [GatherExpr(tt, ti), GatherExpr(tt, ti).mul(2.0).add(1.0), GatherExpr(tt, ti).softmax(-1)]:
        got = eval(e).cpu().numpy()
        ref = en.evaluate(e, host)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan)
        assert np.abs(got[~nan] - ref[~nan]).max() <= (1e-5 if dt == np.float32 else 1e-12) * max(1.0, np.abs(ref[~nan]).max())


def test_matmul_reference_known_answers():
    """executor.zig:675-693 ([[1,2],[3,4]] @ [[5,6],[7,8]]) and 936-968
    (softmax of Q @ K, rows summing to 1)."""
    a = leaf(np.array([[1, 2], [3, 4]], np.float32))
    b = leaf(np.array([[5, 6], [7, 8]], np.float32))
    assert eval(a.matmul(b)).cpu().numpy().tolist() == [[19, 22], [43, 50]]
    q = leaf(np.array([[1, 0, 0], [0, 1, 0]], np.float32))
    k = leaf(np.array([[1, 0], [0, 1], [0, 0]], np.float32))
    y = eval(q.matmul(k).softmax(-1)).cpu().numpy()
    assert y.shape == (2, 2) and np.allclose(y.sum(1), 1, atol=1e-5)


def test_matmul_many_batches_and_rows():
    """More than 65535 batches ([70000, 2, 2] @ [2, 2]) and more than 2^20
    rows: the GEMM's grid is one-dimensional over batches and tiles."""
    rng = np.random.default_rng(12)
    for sa, sb in [((70000, 2, 2), (2, 2)), (((1 << 20) + 5, 2), (2, 3))]:
        A = rng.standard_normal(sa).astype(np.float32)
        B = rng.standard_normal(sb).astype(np.float32)
        got = eval(leaf(A).matmul(leaf(B))).cpu().numpy()
        ref = np.matmul(A.astype(np.float64), B.astype(np.float64))
        assert got.shape == ref.shape and np.abs(got - ref).max() <= 1e-5 * max(1.0, float(np.abs(ref).max()))


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_matmul_shapes_vs_restatement(dt):
    rng = np.random.default_rng(9)
    for sa, sb in [((64,), (64,)), ((64,), (64, 48)), ((100, 64), (64,)), ((129, 300), (300, 77)),
                   ((12, 65, 32), (12, 32, 65)), ((4, 100, 384), (384, 128)), ((2, 1, 33, 16), (3, 16, 40))]:
        A = rng.standard_normal(sa).astype(dt)
        B = rng.standard_normal(sb).astype(dt)
        ta, tb = leaf(A), leaf(B)
        host = {id(ta): A, id(tb): B}
        for e in [ta.matmul(tb), ta.matmul(tb).mul(0.5).add(1.0)]:
            got = eval(e).cpu().numpy()
            ref = en.evaluate(e, host)
            # |sum error| <= k eps sum |a||b|; with unit normals that is below 1e-5 relative (f32)
            tol = 2e-5 if dt == np.float32 else 1e-12
            assert got.shape == ref.shape
            assert np.abs(got - ref).max() <= tol * max(1.0, float(np.abs(ref).max())) * np.sqrt(sa[-1]), (sa, sb)
