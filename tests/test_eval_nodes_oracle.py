"""Pins of the softmax / layernorm / transpose / reshape node oracle
(oracle/eval_nodes.py) and the Python mirror's shape rules for those
expressions.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import eval_nodes as en
from tenzor_amd import _abi
from tenzor_amd.expr import LayerNormExpr, Tensor, to_tape


def test_reference_softmax_known_answers():
    """executor.zig:854-934: rows sum to 1, order follows the inputs, a
    constant row is uniform."""
    y = en.softmax(np.array([1, 2, 3, 4], np.float32), 0)
    assert abs(y.sum() - 1) < 1e-5 and y[3] > y[2] > y[1] > y[0]
    y = en.softmax(np.array([[1, 2, 3], [0, 0, 0]], np.float32), 1)
    assert np.allclose(y.sum(1), 1, atol=1e-5) and np.allclose(y[1], 1 / 3, atol=1e-5)
    y = en.softmax(np.array([1.0, 2, 3, 4, 0, 0, 1, -1], np.float32).reshape(1, 2, 2, 2), 3)
    assert np.allclose(y.sum(-1), 1, atol=1e-5) and np.allclose(y[0, 1, 0], 0.5, atol=1e-5)
    # numerical stability (softmax.zig:378-396): huge inputs stay finite
    y = en.softmax(np.array([1000, 1001, 1002], np.float32), 0)
    assert np.isfinite(y).all() and abs(y.sum() - 1) < 1e-5


def test_reference_layernorm_known_answers():
    """executor.zig:970-1030: zero mean per instance, scaled rows normalise
    to the same values."""
    y = en.layernorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), np.zeros(4, np.float32), 1)
    assert abs(y.mean()) < 1e-5
    y = en.layernorm(np.array([[1, 2, 3, 4], [10, 20, 30, 40]], np.float32), np.ones(4, np.float32),
                     np.zeros(4, np.float32), 1)
    assert np.allclose(y.mean(1), 0, atol=1e-5) and np.allclose(y[0], y[1], atol=1e-5)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_softmax_vs_torch(dtype):
    x = np.random.default_rng(1).standard_normal((3, 7, 5)).astype(dtype) * 4
    for axis in (0, 1, 2):
        ref = torch.softmax(torch.from_numpy(x.astype(np.float64)), axis).numpy()
        tol = 1e-6 if dtype == np.float32 else 1e-14
        assert np.abs(en.softmax(x, axis) - ref).max() < tol, axis


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_layernorm_vs_torch(dtype):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 6, 8)).astype(dtype) * 3 + 1
    for nd in (1, 2, 3):
        g = rng.standard_normal(x.shape[3 - nd:]).astype(dtype)
        b = rng.standard_normal(x.shape[3 - nd:]).astype(dtype)
        ref = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), x.shape[3 - nd:],
                                             torch.from_numpy(g.astype(np.float64)),
                                             torch.from_numpy(b.astype(np.float64)), eps=float(np.float32(1e-5)))
        tol = 2e-5 if dtype == np.float32 else 1e-12
        assert np.abs(en.layernorm(x, g, b, nd) - ref.numpy()).max() < tol, nd


def test_reference_transpose_cases():
    """transpose.zig:146-240: 2-D, general 3-D, the 4-D attention pattern
    [B,S,H,D] -> [B,H,S,D], and the identity."""
    assert np.transpose(np.arange(6).reshape(2, 3), (1, 0)).ravel().tolist() == [0, 3, 1, 4, 2, 5]
    x = np.arange(24).reshape(2, 3, 4)
    assert np.transpose(x, (2, 0, 1))[1, 1, 2] == x[1, 2, 1]
    x = np.arange(2 * 3 * 4 * 5).reshape(2, 3, 4, 5)
    assert np.transpose(x, (0, 2, 1, 3))[1, 3, 2, 4] == x[1, 2, 3, 4]
    assert np.array_equal(np.transpose(x, (0, 1, 2, 3)), x)


def test_mirror_shapes_and_tape():
    x = Tensor.__new__(Tensor)
    x.shape, x.dtype = (2, 3, 4), "float32"
    g = Tensor.__new__(Tensor)
    g.shape, g.dtype = (3, 4), "float32"
    assert x.transpose((2, 0, 1)).shape == (4, 2, 3)
    assert x.reshape((6, 4)).shape == (6, 4)
    assert x.softmax(-1).softmax_axis == 2
    with pytest.raises(TypeError):
        x.transpose((0, 0, 1))
    with pytest.raises(TypeError):
        x.reshape((5, 5))
    with pytest.raises(TypeError):
        LayerNormExpr(x, g, g, 1)  # gamma rank must equal norm_dims
    nodes, leaves = to_tape(LayerNormExpr(x, g, g, 2).transpose((1, 0, 2)))
    assert [n.kind for n in nodes] == [_abi.NODE_TENSOR, _abi.NODE_TENSOR, _abi.NODE_TENSOR, _abi.NODE_LAYERNORM,
                                       _abi.NODE_TRANSPOSE]
    assert nodes[3].axis == 2 and nodes[3].rhs == 1 and nodes[3].aux == 2
    assert list(nodes[4].perm)[:3] == [1, 0, 2]


def test_gather_oracle_and_mirror():
    """The reference's gather known answer (executor.zig:1074-1115) through
    the restatement; index rules of the mirror (expr.zig:775-830)."""
    from tenzor_amd.expr import GatherExpr

    tab = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    t = Tensor.__new__(Tensor)
    t.shape, t.dtype = (4, 3), "float32"
    i = Tensor.__new__(Tensor)
    i.shape, i.dtype = (3,), "int32"
    e = GatherExpr(t, i)
    assert e.shape == (3, 3)
    got = en.evaluate(e, {id(t): tab, id(i): np.array([0, 2, 1], np.int32)})
    assert got.tolist() == [[1, 2, 3], [7, 8, 9], [4, 5, 6]]
    got = en.evaluate(e, {id(t): tab, id(i): np.array([0, 4, -1], np.int32)})
    assert np.isnan(got[1:]).all() and got[0].tolist() == [1, 2, 3]
    with pytest.raises(TypeError):
        GatherExpr(t, t)  # float indices
    nodes, leaves = to_tape(e)
    assert nodes[-1].kind == _abi.NODE_GATHER and nodes[-1].lhs == 0 and nodes[-1].rhs == 1
