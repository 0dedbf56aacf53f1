"""CPU: pin the oracle before trusting it.

No golden vectors exist in the reference for this path (its fixtures are
produced from a network download and gitignored), so each oracle function is
pinned by (a) the reference's own known-answer tests, restated with the same
inputs and expected values, and (b) independent implementations — numpy,
torch and HuggingFace's BertModel built from a config — on inputs chosen so
that a dropped term, wrong sign, transposed operand or wrong index fails."""
import os

import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import _abi, synth
from tenzor_amd.expr import BinaryExpr, ReduceExpr, ScalarExpr, Tensor, UnaryExpr, to_tape
from tests.conftest import GOLDEN, ulp_diff


# ------------------------------------------------------------------ f16
def test_f16_to_f32_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 100,
        rng.uniform(-7e-5, 7e-5, 20000).astype(np.float32),           # subnormal f16 range
        np.array([65504, 65519.99, 65520, 65536, 1e9, -65520, 0.0, -0.0, np.inf, -np.inf], np.float32),
        # exact ties between neighbouring f16 values
        (np.arange(1024, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
        np.float32(2.0 ** -25) * np.arange(1, 200, dtype=np.float32),
    ])
    got = np.array([oracle.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


# ------------------------------------------------------------------ A1 quantizer
def test_quantizer_golden_cases():
    g = np.load(os.path.join(GOLDEN, "quantize_cases.npz"))
    q, s = oracle.quantize_rows(g["w"])
    assert np.array_equal(q, g["q"]) and np.array_equal(s, g["scale"])


def test_quantizer_known_answers():
    w = np.zeros((3, 8), np.float32)
    w[1, :6] = [127, -63.5, 0.5, -0.5, 1.5, 2.5]
    w[2, :] = 254.0  # scale 2.0 exactly -> codes 127
    q, s = oracle.quantize_rows(w)
    assert s[0] == 0x3C00 and q[0].tolist() == [0] * 8           # zero row: scale 1 (quantize_arctic_xs.zig:103)
    assert q[1, :6].tolist() == [127, -64, 1, -1, 2, 3]          # @round: half away from zero
    assert s[2] == np.float16(2.0).view(np.uint16) and q[2].tolist() == [127] * 8


def test_quantizer_scale_rounding_and_clamp():
    # A normal f16 scale is within 2^-11 of max_abs/127, so the max element
    # lands on +-127; only a subnormal f16 scale (max_abs < ~8e-3) can round
    # down far enough that max_abs * inv > 127.5 and the clamp binds.
    rng = np.random.default_rng(1)
    hit_clamp = False
    for i in range(2000):
        row = (rng.standard_normal(64) * (10.0 ** rng.uniform(-5, 1))).astype(np.float32)
        q, s = oracle.quantize_rows(row[None])
        sf = float(np.float16(s[0].view(np.float16)))
        mx = float(np.abs(row).max())
        assert np.abs(q).max() <= 127
        x = row.astype(np.float64) / sf
        unclamped = np.abs(x) < 127.0
        # reconstruction error of every unclamped element is half a step plus
        # the two f32 roundings of v * (1/s) (|v/s| <= 127, 2 * 2^-24 each)
        assert (np.abs(q[0][unclamped] * sf - row[unclamped]) <= sf * (0.5 + 127 * 2.0 ** -23)).all()
        hit_clamp |= mx / sf > 127.5
    assert hit_clamp, "no row exercised the [-127, 127] clamp"


def test_quantizer_scale_underflow_saturates():
    """max_abs/127 below the smallest f16 subnormal rounds the scale to 0 and
    the reference's @intFromFloat(+-inf) is undefined; this build defines it
    as saturation: sign(w) * 127, and 0 for w == 0."""
    w = np.array([[1e-6, -2e-6, 0.0, 3e-7]], np.float32)
    q, s = oracle.quantize_rows(w)
    assert s[0] == 0 and q[0].tolist() == [127, -127, 0, 127]


# ------------------------------------------------------------------ A5 int8 linear
def test_matmul_w8a32_known_answer():
    a = np.array([[1, 2, 3], [-1, 0, 4]], np.float32)
    wq = np.array([[1, 0, -1], [2, 2, 2]], np.int8)
    scale = np.array([np.float16(0.5).view(np.uint16), np.float16(0.25).view(np.uint16)], np.uint16)
    bias = np.array([1.0, -1.0], np.float32)
    c = oracle.matmul_w8a32(a, wq, scale, bias)
    # row 0: (1-3)*0.5+1 = 0, (2+4+6)*0.25-1 = 2; row 1: (-1-4)*0.5+1 = -1.5, (-2+0+8)*0.25-1 = 0.5
    assert c.tolist() == [[0.0, 2.0], [-1.5, 0.5]]


@pytest.mark.parametrize("m,k,n", [(3, 385, 5), (7, 64, 1), (1, 1536, 9)])
def test_matmul_w8a32_vs_float64(m, k, n):
    rng = np.random.default_rng(m * k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    scale = rng.uniform(0.001, 0.02, n).astype(np.float16).view(np.uint16)
    bias = rng.standard_normal(n).astype(np.float32)
    c = oracle.matmul_w8a32(a, wq, scale, bias)
    sf = scale.view(np.float16).astype(np.float64)
    ref = (a.astype(np.float64) @ wq.astype(np.float64).T) * sf + bias
    bound = (np.abs(a) @ np.abs(wq.astype(np.float64)).T) * sf * (k + 2) * 2.0 ** -24 + np.abs(ref) * 2.0 ** -23
    assert (np.abs(c - ref) <= bound).all()


# ------------------------------------------------------------------ A4 LayerNorm
def test_layernorm_reference_known_answers():  # layernorm.zig:413-528 (eps 1e-5)
    one, zero = np.ones(4, np.float32), np.zeros(4, np.float32)
    out = oracle.layernorm(np.array([[1, 2, 3, 4]], np.float32), one, zero, 1e-5)[0]
    assert abs(out.mean()) < 1e-5 and 0.9 < out.var() < 1.1
    out = oracle.layernorm(np.array([[1, 2, 3, 4]], np.float32), 2 * one, one, 1e-5)[0]
    assert abs(out.mean() - 1.0) < 1e-5
    out = oracle.layernorm(np.array([[1, 2, 3, 4], [10, 20, 30, 40]], np.float32), one, zero, 1e-5)
    assert np.allclose(out[0], out[1], atol=1e-5)
    out = oracle.layernorm(np.array([[1e6, 1e6 + 1, 1e6 + 2, 1e6 + 3]], np.float32), one, zero, 1e-5)[0]
    assert np.isfinite(out).all() and abs(out.mean()) < 1e-4


def test_layernorm_vs_torch_float64():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((33, 384)) * 3 + 2).astype(np.float32)
    g = rng.standard_normal(384).astype(np.float32)
    b = rng.standard_normal(384).astype(np.float32)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (384,), torch.from_numpy(g).double(),
                                         torch.from_numpy(b).double(), eps=1e-12).numpy()
    np.testing.assert_allclose(oracle.layernorm(x, g, b, 1e-12), ref, rtol=2e-5, atol=2e-5)


# ------------------------------------------------------------------ A8 GELU, A10 L2
def test_gelu_reference_known_answers():  # arctic.zig:1032-1045
    g = oracle.gelu(np.array([0.0, -3.0, 3.0, 1.0, 2.0], np.float32))
    assert abs(g[0]) < 1e-6 and -0.01 < g[1] < 0 and abs(g[2] - 3) < 0.01 and g[3] < g[4]


def test_gelu_vs_torch_tanh_gelu():
    x = np.arange(-6, 6.25, 0.25, dtype=np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    np.testing.assert_allclose(oracle.gelu(x), ref, atol=2e-6, rtol=2e-6)


def test_l2_normalize_known_answers():  # arctic.zig:1047-1057
    v = oracle.l2_normalize(np.array([3, 4], np.float32))
    assert abs(v[0] - 0.6) < 1e-6 and abs(v[1] - 0.8) < 1e-6
    assert oracle.l2_normalize(np.zeros(5, np.float32)).tolist() == [0] * 5
    r = np.random.default_rng(3).standard_normal(384).astype(np.float32)
    np.testing.assert_allclose(oracle.l2_normalize(r), r / np.linalg.norm(r.astype(np.float64)), atol=1e-7)


# ------------------------------------------------------------------ A6 attention
@pytest.mark.parametrize("L", [1, 2, 7, 130])
def test_attention_head_vs_torch_float64(L):
    rng = np.random.default_rng(L)
    q, k, v = (rng.standard_normal((L, 32)).astype(np.float32) for _ in range(3))
    t = [torch.from_numpy(x).double() for x in (q, k, v)]
    p = torch.softmax(t[0] @ t[1].T / np.sqrt(32.0), dim=-1)
    ref = (p @ t[2]).numpy()
    np.testing.assert_allclose(oracle.attention_head(q, k, v), ref, atol=1e-5, rtol=1e-5)


def test_attention_padding_mask_equals_unpadded():
    """softmax.zig:423-441 masks keys with an additive -1e9; a padded,
    masked sequence gives the unpadded result (the reference forwards each
    sequence at its true length, arctic.zig:874-898)."""
    rng = np.random.default_rng(4)
    L, P = 9, 16
    q, k, v = (rng.standard_normal((P, 32)).astype(np.float64) for _ in range(3))
    mask = np.where(np.arange(P) < L, 0.0, -1e9)
    s = q @ k.T / np.sqrt(32.0) + mask
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    masked = (p @ v)[:L]
    got = oracle.attention_head(q[:L].astype(np.float32), k[:L].astype(np.float32), v[:L].astype(np.float32))
    np.testing.assert_allclose(got, masked, atol=1e-5)


# ------------------------------------------------------------------ A3 embeddings, full forward
def test_embeddings_vs_numpy_gather_and_torch_layernorm():
    cfg = synth.Config(num_hidden_layers=1)
    w = synth.make_arctic_f32(5, cfg, ln_random=True)
    hw = synth.HostWeights(synth.quantize(w), cfg)
    ids = np.array([101, 0, 30521, 2000, 2000, 17], np.uint32)
    got = oracle.arctic_hidden(hw, ids, 0)
    x = (w["embeddings.word_embeddings.weight"][ids].astype(np.float64)
         + w["embeddings.position_embeddings.weight"][: len(ids)] + w["embeddings.token_type_embeddings.weight"][0])
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (384,),
                                         torch.from_numpy(w["embeddings.LayerNorm.weight"]).double(),
                                         torch.from_numpy(w["embeddings.LayerNorm.bias"]).double(), eps=1e-12).numpy()
    np.testing.assert_allclose(got, ref, atol=2e-5)


def test_forward_vs_huggingface_bert_float64():
    """The int8 forward equals the f32 forward with dequantized weights;
    HuggingFace's BertModel (tanh GELU, eps 1e-12) built from a config and
    run in float64 is an independent implementation of it."""
    from tests.golden.gen_golden import hf_embeddings

    cfg = synth.Config(num_hidden_layers=2)
    w = synth.quantize(synth.make_arctic_f32(9, cfg, ln_random=True))
    hw = synth.HostWeights(w, cfg)
    lengths = np.array([1, 5, 40], np.int32)
    ids, _ = synth.make_batch(10, 3, seq_len=40)
    ours = np.stack([oracle.arctic_forward(hw, ids[b, :L]) for b, L in enumerate(lengths)])
    ref = hf_embeddings(synth.dequantize(w), cfg, ids, lengths)
    assert np.abs(ours - ref).max() < 1e-5


def test_linear_f32_vs_float64():
    """orc_linear_f32 (arctic.zig:609-621: sgemm, then += bias) against a
    float64 product, within the f32 summation bound: a transposed operand, a
    dropped or misplaced bias, or a wrong k stride exceed it by orders of
    magnitude."""
    rng = np.random.default_rng(21)
    for m, k, n in [(1, 384, 384), (7, 384, 1536), (33, 1536, 384), (3, 37, 5)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        b = rng.uniform(-0.1, 0.1, n).astype(np.float32)
        ref = a.astype(np.float64) @ w.astype(np.float64).T + b
        bound = (np.abs(a).astype(np.float64) @ np.abs(w).astype(np.float64).T) * (k + 2) * 2.0 ** -24 \
            + np.abs(ref) * 2.0 ** -24 + 1e-30
        got = oracle.linear_f32(a, w, b)
        assert (np.abs(got - ref) <= bound).all(), (m, k, n)
        # no bias: the product alone
        assert (np.abs(oracle.linear_f32(a, w) - (ref - b)) <= bound).all()
        # the bound is tight enough to see a dropped bias
        assert not (np.abs(got - b - ref) <= bound).all()


@pytest.mark.parametrize("lengths", [[128], [1, 7, 64]])
def test_f32_forward_vs_huggingface_bert_float64(lengths):
    """The f32 model (MatWeight.f32 linears, f32 tables; config 1 is batch 1
    x 128) against transformers' BertModel run in float64 on the same f32
    weights, not dequantised int8 ones: this pins orc_linear_f32 inside the
    whole forward."""
    from tests.golden.gen_golden import hf_embeddings

    cfg = synth.Config()
    w = synth.make_arctic_f32(3, cfg, ln_random=True)
    hw = synth.HostWeights(w, cfg)
    lengths = np.array(lengths, np.int32)
    ids, _ = synth.make_batch(31, len(lengths), seq_len=int(lengths.max()))
    ours = np.stack([oracle.arctic_forward(hw, ids[b, :L]) for b, L in enumerate(lengths)])
    ref = hf_embeddings(w, cfg, ids, lengths)
    assert np.abs(ours - ref).max() < 1e-5


def test_forward_golden_fixture_and_batch_threads():
    g = np.load(os.path.join(GOLDEN, "arctic_small.npz"))
    cfg = synth.Config()
    hw = synth.HostWeights(synth.quantize(synth.make_arctic_f32(int(g["seed"]), cfg, ln_random=True)), cfg)
    flat, offs = synth.packed(g["ids"], g["lengths"])
    for threads in (1, 3):
        got = oracle.arctic_forward_batch(hw, flat, offs, g["lengths"], nthreads=threads)
        assert np.array_equal(got, g["expected"])


# ------------------------------------------------------------------ A12-A15 executor
def _eval(expr, leaves_np, dtype=np.float32):
    nodes, _ = to_tape(expr)
    return oracle.eval_tape(nodes, leaves_np, dtype)


class _HostT:
    def __init__(self, a):
        self.a = np.asarray(a)
        self.shape = self.a.shape
        self.dtype = torch.float32 if self.a.dtype == np.float32 else torch.float64

    def is_contiguous(self):
        return True


def HT(a, dt=np.float32):
    return Tensor(_HostT(np.asarray(a, dt)))


def run(expr, dt=np.float32):
    nodes, leaves = to_tape(expr)
    return oracle.eval_tape(nodes, [l.data.a for l in leaves], dt)


def test_empty_operand_broadcast_is_an_error():
    """shape.zig:196-200 gives [0, 4] + scalar the shape [1, 4] (@max(0, 1));
    executor.zig:142-144 would then index the empty slice.  The restatement
    refuses the tape (the GPU planner does the same) instead of reading past
    the empty buffer; both operands empty stays a valid empty result."""
    e = HT(np.zeros((0, 4))).add(1.0)
    assert e.shape == (1, 4)
    assert run(e)[0] == _abi.ERR_SHAPE
    rc, out = run(HT(np.zeros((0, 4))).add(HT(np.zeros((0, 4)))))
    assert rc == 0 and out.shape == (0, 4)


def test_executor_known_answers():  # executor.zig:616-706, elementwise.zig:339-460, reduce.zig:241-350
    assert run(UnaryExpr("relu", HT([-2, -1, 1, 2])))[1].tolist() == [0, 0, 1, 2]
    assert run(BinaryExpr("add", HT([1, 2, 3, 4]), HT([10, 20, 30, 40])))[1].tolist() == [11, 22, 33, 44]
    assert run(UnaryExpr("relu", BinaryExpr("add", HT([-1, 2, -3, 4]), HT([1, 1, 1, 1]))))[1].tolist() == [0, 3, 0, 5]
    assert float(run(ReduceExpr("sum", HT([1, 2, 3, 4])))[1]) == 10
    assert float(run(ReduceExpr("sum", HT([1, 2, 3, 4, 5, 6, 7, 8])))[1]) == 36
    assert float(run(ReduceExpr("mean", HT([2, 4, 6, 8])))[1]) == 5
    assert float(run(ReduceExpr("reduce_max", HT([3, 1, 4, 1, 5, 9, 2, 6])))[1]) == 9
    assert float(run(ReduceExpr("prod", HT([1, 2, 3, 4])))[1]) == 24
    m = [[1, 2, 3], [4, 5, 6]]
    assert run(ReduceExpr("sum", HT(m), (1,)))[1].tolist() == [6, 15]
    assert run(ReduceExpr("sum", HT(m), (0,)))[1].tolist() == [5, 7, 9]
    assert run(ReduceExpr("mean", HT(m), (1,)))[1].tolist() == [2, 5]
    assert run(ReduceExpr("reduce_max", HT([[1, 5, 3], [4, 2, 6]]), (1,)))[1].tolist() == [5, 6]
    assert float(run(ReduceExpr("sum", HT(np.zeros(0))))[1]) == 0
    assert float(run(ReduceExpr("prod", HT(np.zeros(0))))[1]) == 1
    assert run(BinaryExpr("add", HT([1, 2, 3, 4]), ScalarExpr(10.0)))[1].tolist() == [11, 12, 13, 14]
    s = run(UnaryExpr("sigmoid", HT([-100, 0, 100, 1])))[1]
    assert abs(s[0]) < 1e-6 and abs(s[1] - 0.5) < 1e-6 and abs(s[2] - 1) < 1e-6 and abs(s[3] - 0.7310586) < 1e-5
    e = run(UnaryExpr("exp", HT([0.0, 1.0])))[1]
    assert abs(e[0] - 1) < 1e-6 and abs(e[1] - 2.71828) < 1e-4


def test_op_semantics_vs_numpy():
    x = np.linspace(-5, 5, 2001, dtype=np.float32)
    xp = np.abs(x) + np.float32(0.01)
    x64 = x.astype(np.float64)
    xp64 = xp.astype(np.float64)
    # correctly rounded references: float64 libm, rounded once to float32
    lib_ref = {
        "exp": (x, np.exp(x64)), "log": (xp, np.log(xp64)), "sqrt": (xp, np.sqrt(xp64)), "sin": (x, np.sin(x64)),
        "cos": (x, np.cos(x64)), "neg": (x, -x64), "abs": (x, np.abs(x64)), "floor": (x, np.floor(x64)),
        "ceil": (x, np.ceil(x64)), "relu": (x, np.maximum(x64, 0)),
    }
    for op, (inp, ref) in lib_ref.items():
        assert ulp_diff(oracle.unary(op, inp), ref.astype(np.float32)).max() <= 1, op
    approx = {
        "tanh": np.tanh(x64), "sigmoid": 1 / (1 + np.exp(-x64)), "silu": x64 / (1 + np.exp(-x64)),
        "softplus": np.logaddexp(0, x64),
        "gelu": torch.nn.functional.gelu(torch.from_numpy(x64), approximate="tanh").numpy(),
        "rsqrt": None,
    }
    for op, ref in approx.items():
        if ref is None:
            ref, inp = 1 / np.sqrt(xp.astype(np.float64)), xp
        else:
            inp = x
        np.testing.assert_allclose(oracle.unary(op, inp), ref, atol=3e-7, rtol=2e-6, err_msg=op)
    r = oracle.unary("round", np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997], np.float32))
    assert r.tolist() == [1, -1, 2, 3, -3, 0]  # half away from zero, not numpy's half-to-even
    a = np.linspace(0.1, 3, 101, dtype=np.float32)
    b = np.linspace(-2, 2, 101, dtype=np.float32)
    for op, ref in {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b, "max": np.maximum(a, b),
                    "min": np.minimum(a, b)}.items():
        assert ulp_diff(oracle.binary(op, a, b), ref).max() == 0, op
    assert ulp_diff(oracle.binary("pow", a, b), np.power(a.astype(np.float64), b).astype(np.float32)).max() <= 1


@pytest.mark.parametrize("ls,rs", [((4, 6), (6,)), ((4, 6), (4, 1)), ((2, 1, 5), (3, 1)), ((2, 3, 4, 5), (3, 1, 5))])
def test_broadcast_vs_numpy(ls, rs):
    rng = np.random.default_rng(5)
    a = rng.standard_normal(ls).astype(np.float32)
    b = rng.standard_normal(rs).astype(np.float32)
    rc, out = run(BinaryExpr("sub", HT(a), HT(b)).mul(HT(b)))
    assert rc == 0 and np.array_equal(out, (a - b) * b)


def test_chain_golden_and_three_pass_semantics():
    g = np.load(os.path.join(GOLDEN, "chain_small.npz"))
    out = oracle.chain_add_mul_exp(g["a"], g["b"], g["c"])
    assert np.array_equal(out, g["out"])
    rc, out2 = run(BinaryExpr("add", HT(g["a"]), HT(g["b"])).mul(HT(g["c"])).exp())
    assert rc == 0 and np.array_equal(out2, out)


def test_reduce_vs_numpy():
    rng = np.random.default_rng(6)
    x = rng.uniform(0.5, 1.5, (5, 7, 9)).astype(np.float32)
    x64 = x.astype(np.float64)
    for op, fn in {"sum": np.sum, "mean": np.mean, "prod": np.prod, "reduce_max": np.max, "reduce_min": np.min}.items():
        for ax in (0, 1, 2):
            np.testing.assert_allclose(run(ReduceExpr(op, HT(x), (ax,)))[1], fn(x64, axis=ax), rtol=1e-5)
        np.testing.assert_allclose(run(ReduceExpr(op, HT(x)))[1], fn(x64), rtol=1e-5)


def test_eval_errors():
    rc, _ = run(UnaryExpr("exp2", HT([1.0])))
    assert rc == _abi.ERR_UNSUPPORTED_OP
    rc, _ = run(ReduceExpr("variance", HT([1.0, 2.0])))
    assert rc == _abi.ERR_UNSUPPORTED_OP
    nodes, _ = to_tape(BinaryExpr("add", HT(np.zeros((2, 3))), HT(np.zeros(3))))
    nodes[-1].shape[1] = 4  # corrupt the result shape
    rc, _ = oracle.eval_tape(nodes, [np.zeros((2, 3), np.float32), np.zeros(3, np.float32)])
    assert rc == _abi.ERR_SHAPE


# ------------------------------------------------------------------ A12-A15 executor in f64
# The reference runs the same op set on f64 slices (elementwise.zig:13-207,
# simd.zig:107-315, reduce.zig:13-96).  The oracle's f64 mode (orc_eval with
# F64, orc_unary_f64 / orc_binary_f64) is pinned against numpy / torch in
# float64 with bounds a few f64 ulp wide: evaluating in f32 (errors near
# 2^-24), dropping a term or swapping an operand fails them.
def H64(a):
    return HT(np.asarray(a, np.float64), np.float64)


def run64(expr):
    return run(expr, np.float64)


def test_f64_unary_ops_vs_float64_references():
    x = np.linspace(-5, 5, 2001)
    xp = np.abs(x) + 0.01
    t = torch.from_numpy(x)
    exact = {  # correctly rounded (or one-rounding) float64 references
        "neg": (x, -x), "abs": (x, np.abs(x)), "sqrt": (xp, np.sqrt(xp)), "floor": (x, np.floor(x)),
        "ceil": (x, np.ceil(x)), "relu": (x, np.maximum(x, 0)),
    }
    for op, (inp, ref) in exact.items():
        rc, out = run64(UnaryExpr(op, H64(inp)))
        assert rc == 0 and out.dtype == np.float64 and np.array_equal(out, ref), op
    libm = {"exp": (x, np.exp(x)), "log": (xp, np.log(xp)), "sin": (x, np.sin(x)), "cos": (x, np.cos(x)),
            "rsqrt": (xp, 1 / np.sqrt(xp))}
    for op, (inp, ref) in libm.items():
        rc, out = run64(UnaryExpr(op, H64(inp)))
        assert rc == 0
        np.testing.assert_allclose(out, ref, rtol=4e-16, atol=0, err_msg=op)
    closed = {  # the reference's forms (2 sigmoid(2x) - 1 tanh, simd.zig) against torch / numpy
        "tanh": torch.tanh(t).numpy(), "sigmoid": torch.sigmoid(t).numpy(),
        "silu": torch.nn.functional.silu(t).numpy(), "softplus": np.logaddexp(0, x),
        "gelu": torch.nn.functional.gelu(t, approximate="tanh").numpy(),
    }
    for op, ref in closed.items():
        rc, out = run64(UnaryExpr(op, H64(x)))
        assert rc == 0
        np.testing.assert_allclose(out, ref, rtol=1e-14, atol=1e-15, err_msg=op)
    rc, r = run64(UnaryExpr("round", H64([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999999999999994])))
    assert rc == 0 and r.tolist() == [1, -1, 2, 3, -3, 0]  # half away from zero
    # f64 really is f64: 1 + 2^-40 survives, an f32 evaluation loses it
    rc, out = run64(BinaryExpr("add", H64([1.0]), H64([2.0 ** -40])))
    assert rc == 0 and out[0] == 1 + 2.0 ** -40


def test_f64_binary_ops_and_broadcasts_vs_numpy():
    rng = np.random.default_rng(71)
    a = rng.uniform(0.1, 3, 257)
    b = rng.uniform(-2, 2, 257)
    for op, ref in {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b, "max": np.maximum(a, b),
                    "min": np.minimum(a, b)}.items():
        rc, out = run64(BinaryExpr(op, H64(a), H64(b)))
        assert rc == 0 and np.array_equal(out, ref), op
    rc, out = run64(BinaryExpr("pow", H64(a), H64(b)))
    np.testing.assert_allclose(out, np.power(a, b), rtol=4e-16, atol=0)
    rc, out = run64(BinaryExpr("sub", H64(a), ScalarExpr(0.25, "float64")))
    assert rc == 0 and np.array_equal(out, a - 0.25)
    for ls, rs in [((4, 6), (6,)), ((4, 6), (4, 1)), ((2, 1, 5), (3, 1)), ((2, 3, 4, 5), (3, 1, 5))]:
        x = rng.standard_normal(ls)
        y = rng.standard_normal(rs)
        rc, out = run64(BinaryExpr("sub", H64(x), H64(y)).mul(H64(y)))
        assert rc == 0 and np.array_equal(out, (x - y) * y), (ls, rs)


def test_f64_reductions_and_chain_vs_numpy():
    rng = np.random.default_rng(72)
    x = rng.uniform(0.5, 1.5, (5, 7, 9))
    for op, fn in {"sum": np.sum, "mean": np.mean, "prod": np.prod, "reduce_max": np.max,
                   "reduce_min": np.min}.items():
        for ax in (0, 1, 2):
            rc, out = run64(ReduceExpr(op, H64(x), (ax,)))
            assert rc == 0
            np.testing.assert_allclose(out, fn(x, axis=ax), rtol=1e-14, atol=0, err_msg=f"{op} axis {ax}")
        rc, out = run64(ReduceExpr(op, H64(x)))
        np.testing.assert_allclose(out, fn(x), rtol=1e-13, atol=0, err_msg=op)
    # the config-2 chain in f64: exp((a + b) * c), b broadcast over rows
    a = rng.uniform(-1, 1, (33, 65))
    bb = rng.uniform(-1, 1, 65)
    c = rng.uniform(-1, 1, (33, 65))
    rc, out = run64(BinaryExpr("add", H64(a), H64(bb)).mul(H64(c)).exp())
    assert rc == 0
    np.testing.assert_allclose(out, np.exp((a + bb) * c), rtol=4e-16, atol=0)
    # a reduction feeding more elementwise work
    rc, out = run64(BinaryExpr("mul", ReduceExpr("sum", H64(a), (0,)), H64(bb)).exp())
    assert rc == 0
    np.testing.assert_allclose(out, np.exp(a.sum(axis=0) * bb), rtol=1e-14, atol=0)
