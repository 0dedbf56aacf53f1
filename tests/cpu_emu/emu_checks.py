"""TEST INFRASTRUCTURE ONLY: run the GPU test scenarios against the CPU
emulation build of libtenzor_hip (tests/cpu_emu), under AddressSanitizer.

Every kernel runs with its real launch shape on the CPU; an out-of-bounds
access aborts with an ASan report naming the kernel's source line, and a
barrier that some lane can never reach aborts with the kernel named.  Results
are also compared with the oracle, so kernel index logic is checked before
anything runs on a GPU.

Run (what tests/test_cpu_emulation.py does):
    LD_PRELOAD=<libclang_rt.asan-x86_64.so> ASAN_OPTIONS=detect_leaks=0 \
        python tests/cpu_emu/emu_checks.py [group ...]
"""
import ctypes as C
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tenzor_amd import _abi, synth  # noqa: E402
from tenzor_amd.expr import BinaryExpr, ReduceExpr, ScalarExpr, Tensor, UnaryExpr, to_tape  # noqa: E402

L = _abi.bind(C.CDLL(os.environ.get("TZH_EMU_LIB", os.path.join(HERE, "libtenzor_hip_emu.so"))))
CTX = C.c_void_p()


def check(rc):
    if rc != 0:
        raise RuntimeError(f"rc={rc}: {L.tzh_last_error().decode()}")


def ulp(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(2 ** 31) - ai, ai)
    bi = np.where(bi < 0, -(2 ** 31) - bi, bi)
    return np.abs(ai - bi)


class Host:
    """Stand-in for a device tensor: a numpy array whose address is passed."""

    def __init__(self, a):
        self.a = np.ascontiguousarray(a)
        self.shape = self.a.shape
        self.dtype = type("D", (), {"is_floating_point": True, "__str__": lambda s: "torch." + str(self.a.dtype)})()

    def is_contiguous(self):
        return True

    def data_ptr(self):
        return self.a.ctypes.data


def T(x, dt=np.float32):
    return Tensor(Host(np.asarray(x, dt)))


def eval_both(expr):
    nodes, leaves = to_tape(expr)
    dt = np.float64 if expr.dtype == "float64" else np.float32
    out = np.empty(expr.shape, dt)
    arr = (_abi.Leaf * max(1, len(leaves)))()
    for i, t in enumerate(leaves):
        arr[i].data = t.data.data_ptr()
        arr[i].ndim = len(t.shape)
        for j, d in enumerate(t.shape):
            arr[i].shape[j] = d
    tape = (_abi.Node * len(nodes))(*nodes)
    check(L.tzh_eval_into(CTX, tape, len(nodes), arr, len(leaves), _abi.F64 if dt == np.float64 else _abi.F32,
                          out.ctypes.data))
    rc, ref = oracle.eval_tape(nodes, [t.data.a for t in leaves], dt)
    assert rc == 0
    return out, ref


def group_eval():
    assert eval_both(UnaryExpr("relu", T([-2, -1, 1, 2])))[0].tolist() == [0, 0, 1, 2]
    assert eval_both(BinaryExpr("add", T([1, 2, 3, 4]), T([10, 20, 30, 40])))[0].tolist() == [11, 22, 33, 44]
    e = UnaryExpr("relu", BinaryExpr("add", T([-1, 2, -3, 4]), T([1, 1, 1, 1])))
    assert eval_both(e)[0].tolist() == [0, 3, 0, 5]
    for op, axis, data, exp in [("sum", 1, [[1, 2, 3], [4, 5, 6]], [6, 15]), ("sum", 0, [[1, 2, 3], [4, 5, 6]], [5, 7, 9]),
                                ("mean", 1, [[1, 2, 3], [4, 5, 6]], [2, 5]), ("reduce_max", 1, [[1, 5, 3], [4, 2, 6]], [5, 6])]:
        out, _ = eval_both(ReduceExpr(op, T(data), (axis,)))
        assert np.allclose(out, exp), (op, axis, out)
    rng = np.random.default_rng(1)
    x = rng.uniform(-4, 4, 203).astype(np.float32)
    for op in ["neg", "abs", "relu", "floor", "ceil", "round", "exp", "sin", "tanh", "sigmoid", "gelu", "silu",
               "softplus"]:
        out, ref = eval_both(UnaryExpr(op, T(x)))
        assert ((ulp(out, ref) <= 4) | (np.abs(out - ref) < 1e-6)).all(), op
    xp = np.abs(x) + np.float32(1e-3)
    for op in ["log", "sqrt", "rsqrt"]:
        out, ref = eval_both(UnaryExpr(op, T(xp)))
        assert ((ulp(out, ref) <= 4)).all(), op
    a = rng.uniform(-3, 3, (7, 29)).astype(np.float32)
    b = rng.uniform(-3, 3, (7, 29)).astype(np.float32)
    for op in ["add", "sub", "mul", "div", "max", "min"]:
        out, ref = eval_both(BinaryExpr(op, T(a), T(b)))
        assert ulp(out, ref).max() == 0, op
    for ls, rs in [((8, 12), (12,)), ((8, 12), (8, 1)), ((8, 12), ()), ((4, 1, 6), (3, 1)), ((2, 3, 4, 5), (3, 1, 5)),
                   ((7,), (5, 1)), ((3, 5), (3, 5))]:
        aa = rng.standard_normal(ls).astype(np.float32)
        bb = rng.standard_normal(rs).astype(np.float32)
        out, ref = eval_both(BinaryExpr("add", T(aa), T(bb)).mul(T(bb)).sub(T(aa)))
        assert ulp(out, ref).max() == 0, (ls, rs)
    # the GPU tests' exact shapes and seeds (test_gpu_eval.py)
    rng4 = np.random.default_rng(4)
    xs = [T(rng4.standard_normal((33, 65)).astype(np.float32)) for _ in range(8)]
    e = xs[0]
    for t in xs[1:]:
        e = BinaryExpr("add", t, UnaryExpr("tanh", e))
    out, ref = eval_both(e)
    assert ((ulp(out, ref) <= 8) | (np.abs(out - ref) < 1e-6)).all()
    xl = T(np.linspace(-1, 1, 4097, dtype=np.float32))
    e = xl
    for _ in range(20):
        e = e.mul(0.99).add(xl)
    out, ref = eval_both(e)
    assert ulp(out, ref).max() == 0
    xr = np.random.default_rng(5).uniform(0.9, 1.1, (6, 50, 33)).astype(np.float32)
    for op in ["sum", "mean", "prod", "reduce_max", "reduce_min"]:
        for axes, keep in [((), False), ((), True), ((0,), False), ((1,), True), ((2,), False)]:
            out, ref = eval_both(ReduceExpr(op, T(xr).mul(T(xr)), axes, keep))
            assert np.allclose(out, ref, rtol=1e-4), (op, axes, keep)
    xm = np.random.default_rng(6).standard_normal((40, 300)).astype(np.float32)
    out, ref = eval_both(T(xm).sub(ReduceExpr("mean", T(xm), (1,), True)).exp())
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)
    rng7 = np.random.default_rng(7)
    a64 = rng7.standard_normal((17, 31))
    b64 = rng7.standard_normal((31,))
    out, ref = eval_both(BinaryExpr("add", T(a64, np.float64), T(b64, np.float64)).exp().mul(T(a64, np.float64)))
    assert np.allclose(out, ref, rtol=1e-14)
    for n in (1, 3, 5, 255, 1027):
        out, ref = eval_both(T(np.arange(n, dtype=np.float32)).add(1.0).exp())
        assert (ulp(out, ref) <= 2).all()
    # leaf dtypes: 0 or the element type is a value leaf; another float type
    # or integers outside a gather are WRONG_DTYPE
    xv = T(np.arange(6, dtype=np.float32))
    nodes, leaves = to_tape(UnaryExpr("neg", xv))
    tape = (_abi.Node * len(nodes))(*nodes)
    yv = np.empty(6, np.float32)
    for dtc, want in [(0, 0), (_abi.F32, 0), (_abi.F64, _abi.ERR_WRONG_DTYPE), (_abi.I32, _abi.ERR_WRONG_DTYPE)]:
        arr = (_abi.Leaf * 1)()
        arr[0].data, arr[0].ndim, arr[0].shape[0], arr[0].dtype = leaves[0].data.data_ptr(), 1, 6, dtc
        assert L.tzh_eval_into(CTX, tape, len(nodes), arr, 1, _abi.F32, yv.ctypes.data) == want, dtc
    out, _ = eval_both(ReduceExpr("sum", T(np.zeros(0, np.float32))))
    assert float(out) == 0.0
    # regression: an empty operand under a scalar broadcast (shape.zig's
    # @max(0, 1) = 1 gives a 1 x 4 result) was read through its null data
    # pointer by the chain kernel; it is a shape error now, for the library
    # and the oracle alike
    class Null(Host):
        def data_ptr(self):
            return 0
    ez = Tensor(Null(np.zeros((0, 4), np.float32))).add(1.0)
    assert ez.shape == (1, 4)
    nodes, leaves = to_tape(ez)
    arr = (_abi.Leaf * 1)()
    arr[0].data, arr[0].ndim, arr[0].shape[0], arr[0].shape[1] = None, 2, 0, 4
    res = np.zeros(4, np.float32)
    assert L.tzh_eval_into(CTX, (_abi.Node * len(nodes))(*nodes), len(nodes), arr, 1, _abi.F32,
                           res.ctypes.data) == _abi.ERR_SHAPE
    assert oracle.eval_tape(nodes, [np.zeros((0, 4), np.float32)], np.float32)[0] == _abi.ERR_SHAPE
    assert eval_both(Tensor(Null(np.zeros((0, 4), np.float32))).add(Tensor(Null(np.zeros((0, 4), np.float32)))))[0].size == 0
    A = rng.uniform(-1, 1, (16, 64)).astype(np.float32)
    bb = rng.uniform(-1, 1, 64).astype(np.float32)
    c = rng.uniform(-1, 1, (16, 64)).astype(np.float32)
    out, _ = eval_both(BinaryExpr("add", T(A), T(bb)).mul(T(c)).exp())
    assert ulp(out, oracle.chain_add_mul_exp(A, bb, c)).max() <= 2


def problem(seed, m, k, n, scale=1.0):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((m, k)) * scale).astype(np.float32)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.001, 0.02, n).astype(np.float32)], np.uint16)
    bias = rng.uniform(-0.1, 0.1, n).astype(np.float32)
    return a, q, s, bias


def aligned_empty(shape, dt, align=64):
    """An uninitialised array whose data starts on an `align`-byte boundary
    (the library checks the 16-byte alignment of vector-stored operands;
    the sanitizer's allocator guarantees only 8)."""
    nbytes = int(np.prod(shape)) * np.dtype(dt).itemsize
    raw = np.empty(nbytes + align, np.uint8)
    off = -raw.ctypes.data % align
    return raw[off:off + nbytes].view(dt).reshape(shape)


def aligned(x):
    out = aligned_empty(x.shape, x.dtype)
    out[...] = x
    return out


def linear(a, q, s, bias, out_dt, epi, res=None, g=None, b=None):
    m, k = a.shape
    n = q.shape[0]
    c = aligned_empty((m, n), out_dt)
    a = aligned(a)
    res = None if res is None else aligned(res)
    adt = _abi.F16 if a.dtype == np.float16 else _abi.F32
    cdt = _abi.F16 if out_dt == np.float16 else _abi.F32
    ptr = lambda x: None if x is None else x.ctypes.data
    check(L.tzh_linear_w8(CTX, a.ctypes.data, adt, q.ctypes.data, s.ctypes.data, ptr(bias), c.ctypes.data, cdt, m, k,
                          n, epi, ptr(res), cdt, ptr(g), ptr(b), 1e-12))
    return c.astype(np.float32)


def group_gemm():
    for m, k, n in [(1, 64, 128), (5, 384, 384), (133, 384, 1152), (70, 1536, 384)]:
        a, q, s, bias = problem(m + n, m, k, n)
        c = np.empty((m, n), np.float32)
        check(L.tzh_matmul_w8a32(CTX, a.ctypes.data, q.ctypes.data, s.ctypes.data, bias.ctypes.data, c.ctypes.data, m,
                                 k, n))
        ref = oracle.matmul_w8a32(a, q, s, bias)
        sf = s.view(np.float16).astype(np.float64)
        bound = (np.abs(a) @ np.abs(q.astype(np.float64)).T) * sf * (2 ** -10 + k * 2 ** -23) + 1e-6
        assert (np.abs(c - ref) <= bound).all(), (m, k, n)
    a, q, s, bias = problem(5, 77, 384, 1152)
    a16 = a.astype(np.float16)
    c = linear(a16, q, s, bias, np.float16, _abi.EPI_BIAS)
    ref = oracle.matmul_w8a32(a16.astype(np.float32), q, s, bias)
    assert np.abs(c - ref).max() < 2e-2 * np.abs(ref).max()
    a, q, s, bias = problem(6, 40, 384, 1536, 0.05)
    c = linear(a, q, s, bias, np.float32, _abi.EPI_BIAS_GELU)
    lin = oracle.matmul_w8a32(a, q, s, bias)
    sf = s.view(np.float16).astype(np.float64)
    bound = (np.abs(a) @ np.abs(q.astype(np.float64)).T) * sf * (2 ** -10 + 384 * 2 ** -23) * 1.13 + 1e-6
    err = np.abs(c - oracle.gelu(lin))
    assert (err <= bound).all(), float((err / bound).max())
    for dt in (np.float32, np.float16):
        a, q, s, bias = problem(7, 67, 1536, 384, 0.1)
        rng = np.random.default_rng(8)
        res = rng.standard_normal((67, 384)).astype(dt)
        g = (1 + 0.1 * rng.standard_normal(384)).astype(np.float32)
        b = (0.1 * rng.standard_normal(384)).astype(np.float32)
        c = linear(a, q, s, bias, dt, _abi.EPI_BIAS_RES_LN, res, g, b)
        ref = oracle.layernorm(res.astype(np.float32) + oracle.matmul_w8a32(a, q, s, bias), g, b, 1e-12)
        assert np.abs(c - ref).max() < 2e-2, float(np.abs(c - ref).max())
    # f16 activations: the pipelined direct-to-LDS kernel (several units per
    # persistent block: the emulated device has 16 CUs, two per XCD)
    for m, k, n, epi, odt in [(1, 64, 384, _abi.EPI_BIAS, np.float16), (333, 384, 1152, _abi.EPI_BIAS, np.float16),
                              (200, 384, 1536, _abi.EPI_BIAS_GELU, np.float16), (129, 64, 256, _abi.EPI_BIAS, np.float32),
                              (130, 1536, 384, _abi.EPI_BIAS_RES_LN, np.float16),
                              (61, 384, 384, _abi.EPI_BIAS_RES_LN, np.float32)]:
        a, q, s, bias = problem(m + k + n, m, k, n, 0.1 if epi == _abi.EPI_BIAS_GELU else 1.0)
        a16 = a.astype(np.float16)
        lin = oracle.matmul_w8a32(a16.astype(np.float32), q, s, bias)
        if epi == _abi.EPI_BIAS_RES_LN:
            rng = np.random.default_rng(m)
            res = rng.standard_normal((m, n)).astype(odt)
            g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            b = (0.1 * rng.standard_normal(n)).astype(np.float32)
            c = linear(a16, q, s, bias, odt, epi, res, g, b)
            ref = oracle.layernorm(res.astype(np.float32) + lin, g, b, 1e-12)
            tol = 2e-2
        else:
            c = linear(a16, q, s, bias, odt, epi)
            ref = oracle.gelu(lin) if epi == _abi.EPI_BIAS_GELU else lin
            tol = 2e-3 * max(1.0, float(np.abs(ref).max()))
        err = float(np.abs(c - ref).max())
        assert err < tol, (m, k, n, epi, err)
    # f32 activations with several units per persistent block (64-row tiles,
    # two workgroups per CU: 32 slots on the emulated device), ragged last
    # panel, the three epilogues
    for m, k, n, epi in [(64 * 70 - 13, 64, 384, _abi.EPI_BIAS), (64 * 35 - 5, 128, 768, _abi.EPI_BIAS_GELU),
                         (64 * 40 - 31, 128, 384, _abi.EPI_BIAS_RES_LN)]:
        a, q, s, bias = problem(m + k, m, k, n, 0.1 if epi == _abi.EPI_BIAS_GELU else 1.0)
        lin = oracle.matmul_w8a32(a, q, s, bias)
        sf = s.view(np.float16).astype(np.float64)
        bound = (np.abs(a) @ np.abs(q.astype(np.float64)).T) * sf * (2 ** -20 + k * 2 ** -23) + 1e-6
        if epi == _abi.EPI_BIAS_RES_LN:
            rng = np.random.default_rng(m)
            res = rng.standard_normal((m, n)).astype(np.float32)
            g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            b = (0.1 * rng.standard_normal(n)).astype(np.float32)
            c = linear(a, q, s, bias, np.float32, epi, res, g, b)
            err = float(np.abs(c - oracle.layernorm(res + lin, g, b, 1e-12)).max())
            assert err < 1e-4, (m, k, n, err)
        else:
            c = linear(a, q, s, bias, np.float32, epi)
            ref = oracle.gelu(lin) if epi == _abi.EPI_BIAS_GELU else lin
            err = np.abs(c - ref)
            assert (err <= bound * (1.13 if epi == _abi.EPI_BIAS_GELU else 1.0) + 1e-6).all(), (m, k, n, epi)
    w = (np.random.default_rng(12).standard_normal((64, 384)) * 0.02).astype(np.float32)
    w[0] = 0
    qg = np.empty((64, 384), np.int8)
    sg = np.empty(64, np.uint16)
    check(L.tzh_quantize_rows(CTX, w.ctypes.data, 64, 384, qg.ctypes.data, sg.ctypes.data))
    qo, so = oracle.quantize_rows(w)
    assert np.array_equal(qg, qo) and np.array_equal(sg, so)
    x = np.random.default_rng(13).standard_normal((9, 384)).astype(np.float32)
    gg = np.ones(384, np.float32)
    bt = np.zeros(384, np.float32)
    y = x.copy()
    check(L.tzh_layernorm_last_dim(CTX, y.ctypes.data, gg.ctypes.data, bt.ctypes.data, y.ctypes.data, 9, 384, 1e-12))
    assert np.allclose(y, oracle.layernorm(x, gg, bt, 1e-12), atol=1e-4)


def group_gemm_ln():
    # LayerNorm tiles past the last whole round are split into pieces and
    # normalised by a separate kernel: those rows must match, bit for bit,
    # the same rows computed inside whole tiles (the emulated device has 16
    # CUs: 17 tiles = 16 whole + 1 split into 64 x 64 pieces; k > 384, since
    # tiled int8 weights with k <= 384 use two workgroups per CU unsplit)
    for odt, k in ((np.float16, 448), (np.float32, 448)):
        m, n = 16 * 128 + 100, 384
        a, q, s, bias = problem(21, m, k, n)
        a16 = a.astype(np.float16)
        rng = np.random.default_rng(22)
        res = rng.standard_normal((m, n)).astype(odt)
        g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        b = (0.1 * rng.standard_normal(n)).astype(np.float32)
        split = linear(a16, q, s, bias, odt, _abi.EPI_BIAS_RES_LN, res, g, b)
        whole = linear(np.ascontiguousarray(a16[100:]), q, s, bias, odt, _abi.EPI_BIAS_RES_LN,
                       np.ascontiguousarray(res[100:]), g, b)
        assert np.array_equal(split[2048:], whole[1948:]), odt
        assert np.array_equal(split[100:2048], whole[:1948]), odt
        ref = oracle.layernorm(res.astype(np.float32) + oracle.matmul_w8a32(a16.astype(np.float32), q, s, bias), g, b,
                               1e-12)
        assert np.abs(split - ref).max() < 2e-2
    # several LayerNorm tiles per persistent block (32 tiles on 16 CUs): the
    # stage ring runs across tile boundaries, where each epilogue's residual
    # loads and stores count in the stage waits
    for odt in (np.float16, np.float32):
        m, k, n = 32 * 128, 64, 384
        a, q, s, bias = problem(23, m, k, n)
        a16 = a.astype(np.float16)
        rng = np.random.default_rng(24)
        res = rng.standard_normal((m, n)).astype(odt)
        g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        b = (0.1 * rng.standard_normal(n)).astype(np.float32)
        two = linear(a16, q, s, bias, odt, _abi.EPI_BIAS_RES_LN, res, g, b)
        shifted = linear(np.ascontiguousarray(a16[128:]), q, s, bias, odt, _abi.EPI_BIAS_RES_LN,
                         np.ascontiguousarray(res[128:]), g, b)
        assert np.array_equal(two[128:], shifted), odt
        ref = oracle.layernorm(res.astype(np.float32) + oracle.matmul_w8a32(a16.astype(np.float32), q, s, bias), g, b,
                               1e-12)
        assert np.abs(two - ref).max() < 2e-2


def range_problem(seed, m, k, n, scale):
    a, q, s, _ = problem(seed, m, k, n)
    return (a.astype(np.float64) * scale).astype(np.float32), q, s


def normalised_error(c, a, q, s, bias=None):
    """max |c - exact| / (sum_k |a| |q| s): the error of an f32 matmul_w8a32
    relative to the magnitude of its terms (exact = float64)."""
    sf = s.view(np.float16).astype(np.float64)
    exact = (a.astype(np.float64) @ q.astype(np.float64).T) * sf
    if bias is not None:
        exact = exact + bias.astype(np.float64)
    mag = (np.abs(a.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * sf
    return float((np.abs(c.astype(np.float64) - exact) / mag).max())


def group_range():
    # f32 activations over the f32 range (row exponents scale each row into
    # the f16 split's range): at every input scale the error relative to the
    # terms' magnitude stays at the oracle's own f32 level
    m, k, n = 37, 384, 384
    for scale in (1e-6, 1e-3, 1.0, 3e4, 1e6):
        a, q, s = range_problem(31, m, k, n, scale)
        c = np.empty((m, n), np.float32)
        check(L.tzh_matmul_w8a32(CTX, a.ctypes.data, q.ctypes.data, s.ctypes.data, None, c.ctypes.data, m, k, n))
        ours = normalised_error(c, a, q, s)
        orc = normalised_error(oracle.matmul_w8a32(a, q, s, None), a, q, s)
        print(f"  scale {scale:g}: normalised error {ours:.2e} (oracle {orc:.2e})", flush=True)
        assert np.isfinite(c).all() and ours <= max(4 * orc, 2.0 ** -22), (scale, ours, orc)
        cn = np.empty((m, n), np.float32)
        check(L.tzh_matmul_w8a32_noalloc(CTX, a.ctypes.data, q.ctypes.data, s.ctypes.data, None, cn.ctypes.data, m, k,
                                         n))
        assert np.array_equal(c, cn), scale
    # rows of very different scales in one matrix, a zero row, a row of
    # subnormals, and the GELU and LayerNorm epilogues of tzh_linear_w8
    a, q, s = range_problem(32, 64 * 3 + 5, 128, 768, 1.0)
    a[0] = 0
    a[1] *= np.float32(2.0 ** -140)
    a[2:] *= np.logspace(-30, 30, a.shape[0] - 2).astype(np.float32)[:, None]
    bias = np.random.default_rng(33).uniform(-0.1, 0.1, 768).astype(np.float32)
    c = linear(a, q, s, bias, np.float32, _abi.EPI_BIAS)
    assert np.isfinite(c).all() and np.array_equal(c[0], bias)
    sf = s.view(np.float16).astype(np.float64)
    exact = (a.astype(np.float64) @ q.astype(np.float64).T) * sf
    mag = (np.abs(a.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * sf
    err = np.abs(c - (exact + bias)) / (mag + np.abs(exact + bias))
    assert err[1:].max() < 2.0 ** -21, float(err[1:].max())
    g = oracle.gelu(oracle.matmul_w8a32(a, q, s, bias))
    cg = linear(a, q, s, bias, np.float32, _abi.EPI_BIAS_GELU)
    assert np.isfinite(cg).all()
    assert (np.abs(cg - g) <= 1.13 * 2.0 ** -21 * (mag + np.abs(exact)) + 2.0 ** -20 * np.abs(g) + 1e-37).all()
    # rows whose scale changes along k (the row exponent drops at a later
    # stage, with the sums so far rescaled), rows that start with zeros, and
    # every epilogue
    m, k = 70, 448
    a, q, s = range_problem(36, m, k, 768, 1.0)
    prof = np.ones((m, k), np.float32)
    prof[0::5, :64] = 1e-3
    prof[0::5, 64:] = 1e3           # larger from the second stage on
    prof[1::5, :192] = 0.0          # zeros, then ordinary values
    prof[2::5, :] = np.logspace(-20, 20, k).astype(np.float32)  # growing all the way
    prof[3::5, 200:] = 1e-9         # large first, then tiny
    a *= prof
    bias = np.random.default_rng(37).uniform(-0.1, 0.1, 768).astype(np.float32)
    c = linear(a, q, s, bias, np.float32, _abi.EPI_BIAS)
    sf = s.view(np.float16).astype(np.float64)
    exact = (a.astype(np.float64) @ q.astype(np.float64).T) * sf
    mag = (np.abs(a.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * sf
    err = np.abs(c - (exact + bias)) / (mag + np.abs(exact + bias))
    print(f"  rows changing scale along k: relative error {err.max():.2e}", flush=True)
    assert np.isfinite(c).all() and err.max() < 2.0 ** -21, float(err.max())
    for k in (384, 448):  # the two-workgroup tiles (row-scaled LayerNorm GEMMs at any k)
        m = 16 * 128 + 100
        a, q, s = range_problem(34, m, k, 384, 1.0)
        a *= np.logspace(-20, 20, m).astype(np.float32)[:, None]
        rng = np.random.default_rng(35)
        res = (rng.standard_normal((m, 384)) * np.logspace(-20, 20, m)[:, None]).astype(np.float32)
        gm = (1 + 0.1 * rng.standard_normal(384)).astype(np.float32)
        bt = (0.1 * rng.standard_normal(384)).astype(np.float32)
        bias = np.zeros(384, np.float32)
        c = linear(a, q, s, bias, np.float32, _abi.EPI_BIAS_RES_LN, res, gm, bt)
        ref = oracle.layernorm(res + oracle.matmul_w8a32(a, q, s, bias), gm, bt, 1e-12)
        assert np.isfinite(c).all() and np.abs(c - ref).max() < 1e-4, (k, float(np.abs(c - ref).max()))


def group_attention():
    H, D = 384, 32
    for lengths in ([1], [2, 3], [15, 16, 17], [63, 64, 65], [100, 1, 130], [512], [300, 0]):
        # [300, 0]: key norms growing along the sequence (the row max moves
        # up block after block: lazy rescaling both skipped and taken)
        grow = lengths[-1] == 0
        lengths = [x for x in lengths if x]
        rng = np.random.default_rng(sum(lengths))
        Tn = sum(lengths)
        qkv = (rng.standard_normal((Tn, 3 * H)) * 1.5).astype(np.float32)
        if grow:
            qkv[:, H:2 * H] *= (0.2 + np.arange(Tn) / 30.0)[:, None]
        for dt in (np.float16, np.float32):
            x = qkv.astype(dt)
            cu = np.zeros(len(lengths) + 1, np.int32)
            cu[1:] = np.cumsum(lengths)
            out = np.zeros((Tn, H), dt)
            check(L.tzh_attention_varlen(CTX, x.ctypes.data, out.ctypes.data, _abi.F32 if dt == np.float32 else _abi.F16,
                                         cu.ctypes.data, len(lengths), 12, H))
            q32 = x.astype(np.float32)
            for bi, Ln in enumerate(lengths):
                s0 = cu[bi]
                for h in (0, 7, 11):
                    ref = oracle.attention_head(q32[s0:s0 + Ln, h * D:(h + 1) * D],
                                                q32[s0:s0 + Ln, H + h * D:H + (h + 1) * D],
                                                q32[s0:s0 + Ln, 2 * H + h * D:2 * H + (h + 1) * D])
                    got = out[s0:s0 + Ln, h * D:(h + 1) * D].astype(np.float32)
                    vmax = np.abs(q32[s0:s0 + Ln, 2 * H + h * D:2 * H + (h + 1) * D]).max()
                    if dt == np.float16:
                        tol = 2 ** -9 * vmax + 2 ** -10 * np.abs(ref)
                    else:
                        tol = (2 ** -14 if grow else 2 ** -16) * vmax + 2 ** -18 * np.abs(ref)
                    assert (np.abs(got - ref) <= tol).all(), (lengths, dt, bi, h, float(np.abs(got - ref).max()))


def arctic_model(seed=1234):
    cfg = synth.Config()
    hw = synth.HostWeights(synth.quantize(synth.make_arctic_f32(seed, cfg, ln_random=True)), cfg)
    m = C.c_void_p()
    check(L.tzh_arctic_upload(CTX, C.byref(hw.struct), C.byref(m)))
    return hw, m


def group_arctic():
    # the f32 forward (the fused O-projection + feed-forward kernel), its
    # hidden states, and on a small batch and the GEMM pair (cheaper to
    # emulate) packed = padded ids bit for bit and the bad-id count
    hw, m = arctic_model()
    ids, lengths = synth.make_batch(21, 3, seq_len=40, min_len=5)
    out = np.empty((3, 384), np.float32)
    check(L.tzh_arctic_forward_batch(m, out.ctypes.data, ids.ctypes.data, lengths.ctypes.data, 3, 40))
    ref = np.stack([oracle.arctic_forward(hw, ids[b, :Ln]) for b, Ln in enumerate(lengths)])
    err = np.abs(out - ref).max()
    print(f"  arctic emu (f32 activations) vs oracle max-abs {err:.2e}", flush=True)
    assert err < 1e-5
    hid = np.empty((int(lengths.sum()), 384), np.float32)
    check(L.tzh_arctic_hidden(m, hid.ctypes.data, ids.ctypes.data, lengths.ctypes.data, 3, 40, 1))
    r1 = oracle.arctic_hidden(hw, ids[0, :lengths[0]], 1)
    assert np.abs(hid[:lengths[0]] - r1).max() < 1e-4
    check(L.tzh_arctic_set_ffn_fusion(m, 0))
    ids, lengths = synth.make_batch(22, 3, seq_len=12, min_len=3)
    small = np.empty((3, 384), np.float32)
    check(L.tzh_arctic_forward_batch(m, small.ctypes.data, ids.ctypes.data, lengths.ctypes.data, 3, 12))
    flat, _ = synth.packed(ids, lengths)
    out2 = np.empty((3, 384), np.float32)
    check(L.tzh_arctic_forward_batch(m, out2.ctypes.data, flat.ctypes.data, lengths.ctypes.data, 3, 0))
    assert np.array_equal(small, out2)
    bad = ids.copy()
    bad[1, 2] = 99999
    check(L.tzh_arctic_forward_batch(m, out2.ctypes.data, bad.ctypes.data, lengths.ctypes.data, 3, 12))
    n = C.c_int32()
    check(L.tzh_arctic_bad_id_count(m, C.byref(n)))
    assert n.value == 1
    check(L.tzh_arctic_free(m))


def group_arctic_f16w():
    # the opt-in f16 activations, and the f32 model (MatWeight.f32 linears on
    # the f32 GEMM, two layers)
    hw, m = arctic_model()
    ids, lengths = synth.make_batch(21, 3, seq_len=40, min_len=5)
    ref = np.stack([oracle.arctic_forward(hw, ids[b, :Ln]) for b, Ln in enumerate(lengths)])
    r1 = oracle.arctic_hidden(hw, ids[0, :lengths[0]], 1)
    hid = np.empty((int(lengths.sum()), 384), np.float32)
    check(L.tzh_arctic_set_precision(m, _abi.F16))
    out16 = np.empty((3, 384), np.float32)
    check(L.tzh_arctic_forward_batch(m, out16.ctypes.data, ids.ctypes.data, lengths.ctypes.data, 3, 40))
    assert np.abs(out16 - ref).max() < 1e-3
    check(L.tzh_arctic_hidden(m, hid.ctypes.data, ids.ctypes.data, lengths.ctypes.data, 3, 40, 1))
    assert np.abs(hid[:lengths[0]] - r1).max() < 2e-2
    check(L.tzh_arctic_free(m))
    cfg2 = synth.Config(num_hidden_layers=2)
    w32 = synth.make_arctic_f32(77, cfg2, ln_random=True)
    hw32 = synth.HostWeights(w32, cfg2)
    m32 = C.c_void_p()
    check(L.tzh_arctic_upload(CTX, C.byref(hw32.struct), C.byref(m32)))
    d = C.c_int32()
    check(L.tzh_arctic_precision(m32, C.byref(d)))
    assert d.value == _abi.F32
    out32 = np.empty((3, 384), np.float32)
    check(L.tzh_arctic_forward_batch(m32, out32.ctypes.data, ids.ctypes.data, lengths.ctypes.data, 3, 40))
    ref32 = np.stack([oracle.arctic_forward(hw32, ids[b, :Ln]) for b, Ln in enumerate(lengths)])
    err = np.abs(out32 - ref32).max()
    print(f"  arctic emu (f32 weights) vs oracle max-abs {err:.2e}", flush=True)
    assert err < 1e-5
    check(L.tzh_arctic_free(m32))


def mixed_weights(w, f32_names):
    """The quantized weights of `w` with the linears named in f32_names kept
    f32 (a model that mixes MatWeight.f32 and MatWeight.q8 linears)."""
    out = synth.quantize(w)
    for name in f32_names:
        out[name] = w[name]
        del out[name + ".scale"]
    return out


def forward_vs_oracle(w, cfg, ids, lengths, what, tol=1e-5):
    hw = synth.HostWeights(w, cfg)
    m = C.c_void_p()
    check(L.tzh_arctic_upload(CTX, C.byref(hw.struct), C.byref(m)))
    try:
        d = C.c_int32()
        check(L.tzh_arctic_precision(m, C.byref(d)))
        out = np.empty((len(lengths), 384), np.float32)
        rc = L.tzh_arctic_forward_batch(m, out.ctypes.data, ids.ctypes.data, lengths.ctypes.data, len(lengths),
                                        ids.shape[1])
        if rc != 0:
            return rc, d.value
        ref = np.stack([oracle.arctic_forward(hw, ids[b, :Ln]) for b, Ln in enumerate(lengths)])
        err = float(np.abs(out - ref).max())
        print(f"  {what}: max-abs {err:.2e} vs oracle", flush=True)
        assert np.isfinite(out).all() and err < tol, (what, err)
        return rc, d.value
    finally:
        check(L.tzh_arctic_free(m))


def group_models():
    # models that mix f32 and int8 linears: each linear on its own format's
    # GEMM, the forward in f32 (f32 activations for the f32 GEMM)
    cfg = synth.Config(num_hidden_layers=2)
    w = synth.make_arctic_f32(91, cfg, ln_random=True)
    ids, lengths = synth.make_batch(92, 3, seq_len=40, min_len=5)
    att = [f"encoder.layer.0.attention.self.{x}.weight" for x in ("query", "key", "value")] + \
          ["encoder.layer.0.attention.output.dense.weight"]
    ffn = ["encoder.layer.1.intermediate.dense.weight", "encoder.layer.1.output.dense.weight"]
    rc, act = forward_vs_oracle(mixed_weights(w, att + ffn), cfg, ids, lengths, "f32 attention / int8 FFN, then reverse")
    assert rc == 0 and act == _abi.F32
    rc, act = forward_vs_oracle(mixed_weights(w, ["encoder.layer.1.attention.self.key.weight"]), cfg, ids, lengths,
                                "QKV with an f32 key among int8 query and value")
    assert rc == 0 and act == _abi.F32
    # activations past the f16 range: the embedding LayerNorm's gamma makes
    # layer 0's QKV input reach ~1e5 (the bound, sqrt(383) * 2e4, marks the
    # model row-scaled); small QKV weights keep the attention inside its range
    wr = dict(w)
    wr["embeddings.LayerNorm.weight"] = (w["embeddings.LayerNorm.weight"] * 2e4).astype(np.float32)
    for x in ("query", "key", "value"):
        wr[f"encoder.layer.0.attention.self.{x}.weight"] = (w[f"encoder.layer.0.attention.self.{x}.weight"] *
                                                           1e-4).astype(np.float32)
    rc, act = forward_vs_oracle(synth.quantize(wr), cfg, ids, lengths, "row-scaled int8 GEMMs (inputs ~1e5)")
    assert rc == 0 and act == _abi.F32
    # ... and with full-size QKV weights the attention's inputs could pass
    # its split's range: the forward refuses instead of returning NaN
    wr2 = dict(w)
    wr2["embeddings.LayerNorm.weight"] = wr["embeddings.LayerNorm.weight"]
    rc, _ = forward_vs_oracle(synth.quantize(wr2), cfg, ids, lengths, "attention past its range")
    assert rc == _abi.ERR_TOO_LARGE, rc


def ffn_oracle(w, layer, x, eps):
    """The reference's feedForward (arctic.zig:760-811) on the oracle's
    pieces: LayerNorm(x + (gelu(x W1^T s1 + b1) W2^T s2 + b2))."""
    p = f"encoder.layer.{layer}."
    h = oracle.matmul_w8a32(x, w[p + "intermediate.dense.weight"], w[p + "intermediate.dense.weight.scale"],
                            w[p + "intermediate.dense.bias"])
    y = oracle.matmul_w8a32(oracle.gelu(h), w[p + "output.dense.weight"], w[p + "output.dense.weight.scale"],
                            w[p + "output.dense.bias"])
    return oracle.layernorm(x + y, w[p + "output.LayerNorm.weight"], w[p + "output.LayerNorm.bias"], eps)


def group_mlp():
    # the feed-forward block as one kernel (mlp.hip) and as the GEMM pair,
    # through tzh_arctic_feed_forward, against the oracle.  Run with two
    # emulated CUs (TZH_EMU_CUS=2, as tests/test_cpu_emulation.py does),
    # 300 tokens make 5 panels of 64 on two blocks: two whole panels each
    # (the weight ring runs on across panels), then the fifth, holding 44
    # tokens (two full waves, one partial, one with none), split into two
    # parts of 12 chunks; 1 to 64 tokens make one panel, split the same way.
    cfg = synth.Config(num_hidden_layers=2)
    w = synth.quantize(synth.make_arctic_f32(5150, cfg, ln_random=True))
    hw = synth.HostWeights(w, cfg)
    m = C.c_void_p()
    check(L.tzh_arctic_upload(CTX, C.byref(hw.struct), C.byref(m)))
    rng = np.random.default_rng(5151)
    try:
        for t, layer in ((1, 0), (17, 1), (64, 0), (300, 1)):
            x = aligned_empty((t, 384), np.float32)
            x[...] = rng.standard_normal((t, 384), dtype=np.float32)
            x[t // 2] = 0.0  # a zero row
            ref = ffn_oracle(w, layer, x, cfg.layer_norm_eps)
            outs = []
            for fused in (1, 0):
                check(L.tzh_arctic_set_ffn_fusion(m, fused))
                y = aligned_empty((t, 384), np.float32)
                y[...] = np.nan
                check(L.tzh_arctic_feed_forward(m, layer, x.ctypes.data, y.ctypes.data, t))
                err = float(np.abs(y - ref).max())
                print(f"  feed-forward t={t} layer {layer} {'fused' if fused else 'GEMM pair'}: max-abs {err:.2e} "
                      f"vs oracle", flush=True)
                assert np.isfinite(y).all() and err < 2e-5, (t, fused, err)
                outs.append(y)
            assert float(np.abs(outs[0] - outs[1]).max()) < 2e-5
        # the forward, whose O-projection, LayerNorm and feed-forward block
        # run as one kernel (about 280 tokens: 5 panels on the two blocks),
        # and with the fusion off, against the oracle
        ids, lengths = synth.make_batch(5152, 6, seq_len=64, min_len=30)
        ref = np.stack([oracle.arctic_forward(hw, ids[b, :Ln]) for b, Ln in enumerate(lengths)])
        for fused in (1, 0):
            check(L.tzh_arctic_set_ffn_fusion(m, fused))
            out = np.empty((len(lengths), 384), np.float32)
            check(L.tzh_arctic_forward_batch(m, out.ctypes.data, ids.ctypes.data, lengths.ctypes.data, len(lengths),
                                             ids.shape[1]))
            err = float(np.abs(out - ref).max())
            print(f"  forward {int(lengths.sum())} tokens {'fused' if fused else 'unfused'}: max-abs {err:.2e} "
                  f"vs oracle", flush=True)
            assert np.isfinite(out).all() and err < 1e-5, (fused, err)
        check(L.tzh_arctic_set_ffn_fusion(m, 1))
        x = aligned_empty((32, 384), np.float32)
        x[...] = 1.0
        assert L.tzh_arctic_feed_forward(m, 0, x.ctypes.data, x.ctypes.data, 32) == _abi.ERR_INVALID_ARGS
        assert L.tzh_arctic_feed_forward(m, 2, x.ctypes.data, x.ctypes.data + 32 * 384 * 4, 1) == _abi.ERR_INVALID_ARGS
        check(L.tzh_arctic_feed_forward(m, 0, x.ctypes.data, None, 0))
    finally:
        check(L.tzh_arctic_free(m))


def group_mlp_split():
    # The fused kernel's split last round (mlp.hip, TailSplit) with 24
    # emulated CUs (TZH_EMU_CUS=24, as tests/test_cpu_emulation.py does):
    # 1, 2 and 3 panels split into 24, 12 and 8 parts (one, two and three
    # chunks each), through tzh_arctic_feed_forward and, with the
    # O-projection at the kernel's head, the forward; against the oracle.
    cfg = synth.Config(num_hidden_layers=2)
    w = synth.quantize(synth.make_arctic_f32(5160, cfg, ln_random=True))
    hw = synth.HostWeights(w, cfg)
    m = C.c_void_p()
    check(L.tzh_arctic_upload(CTX, C.byref(hw.struct), C.byref(m)))
    rng = np.random.default_rng(5161)
    try:
        for t, layer in ((1, 0), (100, 1), (130, 0)):
            x = aligned_empty((t, 384), np.float32)
            x[...] = rng.standard_normal((t, 384), dtype=np.float32)
            y = aligned_empty((t, 384), np.float32)
            y[...] = np.nan
            check(L.tzh_arctic_feed_forward(m, layer, x.ctypes.data, y.ctypes.data, t))
            err = float(np.abs(y - ffn_oracle(w, layer, x, cfg.layer_norm_eps)).max())
            print(f"  split feed-forward t={t}: max-abs {err:.2e} vs oracle", flush=True)
            assert np.isfinite(y).all() and err < 2e-5, (t, err)
        for seed, n, seq, lo in ((5162, 2, 30, 10), (5163, 3, 64, 40)):
            ids, lengths = synth.make_batch(seed, n, seq_len=seq, min_len=lo)
            ref = np.stack([oracle.arctic_forward(hw, ids[b, :Ln]) for b, Ln in enumerate(lengths)])
            out = np.empty((n, 384), np.float32)
            check(L.tzh_arctic_forward_batch(m, out.ctypes.data, ids.ctypes.data, lengths.ctypes.data, n, seq))
            err = float(np.abs(out - ref).max())
            print(f"  split forward {int(lengths.sum())} tokens: max-abs {err:.2e} vs oracle", flush=True)
            assert np.isfinite(out).all() and err < 1e-5, err
    finally:
        check(L.tzh_arctic_free(m))


def group_embed():
    # tokenizer -> chunks of every document -> one batched forward -> the
    # chunk pooling kernel, against the same forward on the oracle's chunks
    # and the oracle's pooling (one layer keeps the emulated forward short)
    from oracle import wordpiece as wp

    cfg = synth.Config(num_hidden_layers=1)
    hw = synth.HostWeights(synth.quantize(synth.make_arctic_f32(77, cfg)), cfg)
    m = C.c_void_p()
    check(L.tzh_arctic_upload(CTX, C.byref(hw.struct), C.byref(m)))
    data, words = synth.make_vocab(5)
    vocab = wp.load_vocab_bytes(data)
    tok = C.c_void_p()
    check(L.tzh_tokenizer_create(C.byref(tok)))
    check(L.tzh_tokenizer_load_vocab_bytes(tok, data, len(data)))
    docs = [synth.make_text(6, words, 925, plain=True), synth.make_text(7, words, 30), b""]
    arr = (C.c_char_p * 3)(*docs)
    lens = np.array([len(d) for d in docs], np.int64)
    out = np.empty((3, 384), np.float32)
    counts = np.zeros(3, np.int32)
    check(L.tzh_arctic_embed_documents(m, tok, arr, lens.ctypes.data_as(C.POINTER(C.c_int64)), 3, out.ctypes.data,
                                       counts.ctypes.data_as(C.POINTER(C.c_int32))))
    chunks = [wp.chunks(wp.encode_raw(vocab, d)) for d in docs]
    assert counts.tolist() == [len(c) for c in chunks] == [2, 1, 1], counts
    flat = np.array([i for c in chunks for ch in c for i in ch], np.uint32)
    clen = np.array([len(ch) for c in chunks for ch in c], np.int32)
    emb = np.empty((len(clen), 384), np.float32)
    check(L.tzh_arctic_forward_batch(m, emb.ctypes.data, flat.ctypes.data, clen.ctypes.data, len(clen), 0))
    ref = np.stack([wp.chunk_mean_l2(emb[0:2]), wp.chunk_mean_l2(emb[2:3]), wp.chunk_mean_l2(emb[3:4])])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    ntok = np.zeros(3, np.int32)
    check(L.tzh_arctic_embed_texts(m, tok, arr, lens.ctypes.data_as(C.POINTER(C.c_int64)), 3, out.ctypes.data,
                                   ntok.ctypes.data_as(C.POINTER(C.c_int32))))
    enc = [wp.encode(vocab, d, 512) for d in docs]
    assert ntok.tolist() == [len(e) for e in enc] and ntok[0] == 512
    flat = np.array([i for e in enc for i in e], np.uint32)
    check(L.tzh_arctic_forward_batch(m, emb.ctypes.data, flat.ctypes.data, ntok.ctypes.data, 3, 0))
    assert np.array_equal(out, emb[:3])
    check(L.tzh_tokenizer_free(tok))
    check(L.tzh_arctic_free(m))


def eval_lib(expr):
    nodes, leaves = to_tape(expr)
    dt = np.float64 if expr.dtype == "float64" else np.float32
    out = np.empty(expr.shape, dt)
    arr = (_abi.Leaf * max(1, len(leaves)))()
    for i, t in enumerate(leaves):
        arr[i].data = t.data.data_ptr()
        arr[i].ndim = len(t.shape)
        arr[i].dtype = {"int32": _abi.I32, "int64": _abi.I64}.get(t.dtype, 0)
        for j, d in enumerate(t.shape):
            arr[i].shape[j] = d
    tape = (_abi.Node * len(nodes))(*nodes)
    rc = L.tzh_eval_into(CTX, tape, len(nodes), arr, len(leaves), _abi.F64 if dt == np.float64 else _abi.F32,
                         out.ctypes.data)
    return rc, out


def group_nodes():
    # softmax / layernorm / transpose / reshape nodes, alone and read by
    # chains and reductions, against the numpy restatement
    from oracle import eval_nodes as en
    from tenzor_amd.expr import LayerNormExpr

    rng = np.random.default_rng(3)
    for dt in (np.float32, np.float64):
        x = (rng.standard_normal((3, 5, 70)) * 3).astype(dt)
        y = rng.standard_normal((5, 70)).astype(dt)
        g, b = rng.standard_normal(70).astype(dt), rng.standard_normal(70).astype(dt)
        tx, ty, tg, tb = T(x, dt), T(y, dt), T(g, dt), T(b, dt)
        host = {id(tx): x, id(ty): y, id(tg): g, id(tb): b}
        tol = 1e-5 if dt == np.float32 else 1e-12
        # rows of 68 take the vector-width kernels; softmax over a leading
        # axis of few columns runs through transposes
        x68, g68 = np.ascontiguousarray(x[:, :, :68]), np.ascontiguousarray(g[:68])
        tz, tg68 = T(x68, dt), T(g68, dt)
        host.update({id(tz): x68, id(tg68): g68})
        for e in [tx.softmax(-1), tx.softmax(1), tx.softmax(0), tx.transpose((2, 0, 1)), tx.transpose((1, 0, 2)),
                  tx.reshape((15, 70)), tx.softmax(-1).mul(2.0).add(ty), LayerNormExpr(tx, tg, tb, 1),
                  LayerNormExpr(tx.mul(ty), tg, tb, 1).transpose((0, 2, 1)), tx.softmax(-1).sum(),
                  ReduceExpr("sum", tx.transpose((2, 1, 0)), (0,)), tx.reshape((5, 3, 70)).add(ty.reshape((5, 1, 70))),
                  tz.softmax(-1), tz.softmax(0), LayerNormExpr(tz, tg68, tg68, 1)]:
            rc, out = eval_lib(e)
            assert rc == 0, L.tzh_last_error()
            ref = en.evaluate(e, host)
            assert np.abs(out - ref).max() <= tol * max(1.0, float(np.abs(ref).max())), (dt, type(e).__name__)
        g2 = rng.standard_normal((5, 70)).astype(dt)
        tg2, tb2 = T(g2, dt), T(g2, dt)
        host.update({id(tg2): g2, id(tb2): g2})
        e = LayerNormExpr(tx, tg2, tb2, 2)
        rc, out = eval_lib(e)
        assert rc == 0 and np.abs(out - en.evaluate(e, host)).max() <= 10 * tol
    # gather: int32 / int64 indices, a computed table, a chain after it,
    # and a row outside the table (NaN)
    from tenzor_amd.expr import GatherExpr

    tab = rng.standard_normal((50, 36)).astype(np.float32)
    tt = T(tab)
    for it in (np.int32, np.int64):
        idx = rng.integers(0, 50, size=(3, 7)).astype(it)
        idx[1, 2] = 50
        ti = T(idx, it)
        host = {id(tt): tab, id(ti): idx}
        for e in [GatherExpr(tt, ti), GatherExpr(tt.mul(2.0), ti).add(1.0)]:
            rc, out = eval_lib(e)
            assert rc == 0, L.tzh_last_error()
            ref = en.evaluate(e, host)
            assert np.array_equal(np.isnan(out), np.isnan(ref)) and np.array_equal(np.nan_to_num(out), np.nan_to_num(ref))
    # transposes that move the last axis (LDS tiles, partial edges) and
    # those that keep it, bit-exact
    xt = rng.standard_normal((3, 37, 5, 70)).astype(np.float32)
    tt4 = T(xt)
    for perm in [(0, 1, 3, 2), (3, 2, 1, 0), (1, 3, 0, 2), (0, 2, 1, 3), (2, 0, 1, 3)]:
        rc, out = eval_lib(tt4.transpose(perm))
        assert rc == 0 and np.array_equal(out, np.transpose(xt, perm)), perm
    # matmul: 1-D / 2-D / batched / broadcast batches, a chain after it,
    # softmax over its rows (executor.zig:675-970 shapes)
    for sa, sb in [((7,), (7,)), ((7,), (7, 5)), ((9, 7), (7,)), ((9, 7), (7, 20)), ((3, 9, 7), (3, 7, 20)),
                   ((3, 9, 7), (7, 20)), ((2, 1, 9, 7), (3, 7, 20)), ((33, 40), (40, 17))]:
        A = rng.standard_normal(sa).astype(np.float32)
        B = rng.standard_normal(sb).astype(np.float32)
        ta, tb2 = T(A), T(B)
        host = {id(ta): A, id(tb2): B}
        for e in [ta.matmul(tb2), ta.matmul(tb2).mul(2.0)] + ([ta.matmul(tb2).softmax(-1)] if len(sb) > 1 else []):
            rc, out = eval_lib(e)
            assert rc == 0, L.tzh_last_error()
            ref = en.evaluate(e, host)
            assert out.shape == ref.shape and np.abs(out - ref).max() <= 1e-5 * max(1.0, float(np.abs(ref).max())), (sa, sb)
    # errors the planner raises for malformed tapes
    nodes, leaves = to_tape(T(np.zeros((2, 3), np.float32)).transpose((1, 0)))
    nodes[1].perm[1] = 1  # not a permutation
    tape = (_abi.Node * 2)(*nodes)
    arr = (_abi.Leaf * 1)()
    arr[0].data, arr[0].ndim, arr[0].shape[0], arr[0].shape[1] = leaves[0].data.data_ptr(), 2, 2, 3
    out = np.empty((3, 2), np.float32)
    assert L.tzh_eval_into(CTX, tape, 2, arr, 1, _abi.F32, out.ctypes.data) == -10  # TZH_ERR_SHAPE


def group_gemm_fp():
    """The matrix-core f32/f64 GEMM (gemm_fp.hip): ONNX Gemm for every
    transpose flag and C shape, ONNX MatMul's shape branches, and the fused
    matmul epilogue of the eval planner."""
    from oracle import onnx_ops as oo

    rng = np.random.default_rng(21)
    for ta, tb in [(0, 0), (1, 0), (0, 1), (1, 1)]:
        for (m, n, k), cshape, al in [((5, 7, 3), None, True), ((130, 20, 17), (1, 1), False), ((33, 129, 40), (129,), True),
                                      ((64, 64, 16), (64, 1), True), ((9, 200, 0), (9, 200), False)]:
            A = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
            B = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
            Cm = None if cshape is None else rng.standard_normal(cshape).astype(np.float32)
            if al:
                A, B = aligned(A), aligned(B)
            y = aligned_empty((m, n), np.float32)
            cr, cc = (0, 0) if Cm is None else ((1, Cm.shape[0]) if Cm.ndim == 1 else Cm.shape)
            check(L.tzh_gemm_f32(CTX, ta, tb, m, n, k, 0.75, A.ctypes.data, A.shape[1], B.ctypes.data, B.shape[1], -1.5,
                                 None if Cm is None else Cm.ctypes.data, cr, cc, y.ctypes.data))
            ref = oo.gemm(A, B, Cm, 0.75, -1.5, bool(ta), bool(tb))
            bound = (0.75 * (np.abs(A.T if ta else A).astype(np.float64) @ np.abs(B.T if tb else B)) * (k + 2) * 2.0 ** -23
                     + 2.0 ** -22 * np.abs(ref) + 1e-30)
            assert (np.abs(y - ref) <= bound).all(), (ta, tb, m, n, k, cshape)
    # a padded row pitch (lda > k)
    A = rng.standard_normal((10, 24)).astype(np.float32)
    B = rng.standard_normal((13, 7)).astype(np.float32)
    y = np.empty((10, 7), np.float32)
    check(L.tzh_gemm_f32(CTX, 0, 0, 10, 7, 13, 1.0, A.ctypes.data, 24, B.ctypes.data, 7, 0.0, None, 0, 0, y.ctypes.data))
    assert np.allclose(y, A[:, :13].astype(np.float64) @ B, rtol=1e-5, atol=1e-5)
    # MatMul: the reference's test, its shape branches, f64, scalar B, zero dims
    for dt in (np.float32, np.float64):
        for sa, sb in [((2, 3), (3, 2)), ((7,), (7,)), ((7,), (7, 5)), ((9, 7), (7,)), ((3, 9, 7), (3, 7, 20)),
                       ((3, 9, 7), (7, 20)), ((9, 7), (3, 7, 20)), ((2, 3, 9, 7), (2, 3, 7, 20)), ((2, 3, 9, 7), (7, 20)),
                       ((2, 1, 9, 7), (3, 7, 20)), ((4, 6), ()), ((4, 6), (1,)), ((0, 5), (5, 3)), ((4, 0), (0, 3))]:
            A = (np.arange(1, 7, dtype=dt).reshape(2, 3) if sa == (2, 3) else rng.standard_normal(sa).astype(dt))
            B = (np.arange(1, 7, dtype=dt).reshape(3, 2) if sb == (3, 2) else rng.standard_normal(sb).astype(dt))
            ys, yn = (C.c_int64 * 8)(), C.c_int32()
            sha, shb = (C.c_int64 * 8)(*sa), (C.c_int64 * 8)(*sb)
            dcode = _abi.F64 if dt == np.float64 else _abi.F32
            check(L.tzh_matmul_nd(CTX, dcode, A.ctypes.data, sha, len(sa), B.ctypes.data, shb, len(sb), None, ys, C.byref(yn)))
            ref = oo.matmul(A, B)
            shape = tuple(ys[i] for i in range(yn.value))
            assert shape == ref.shape, (sa, sb, shape, ref.shape)
            y = np.full(shape, np.nan, dt)
            check(L.tzh_matmul_nd(CTX, dcode, A.ctypes.data, sha, len(sa), B.ctypes.data, shb, len(sb),
                                  y.ctypes.data if y.size else None, ys, C.byref(yn)))
            tol = 2e-6 if dt == np.float32 else 1e-14
            assert np.abs(y - ref).max(initial=0) <= tol * max(1.0, float(np.abs(ref).max(initial=0))) * np.sqrt(max(1, sa[-1]))
            if sa == (2, 3):
                assert y.tolist() == [[22, 28], [49, 64]]  # executor.zig:6288-6290
    # the fused epilogue: known answer (codegen.zig:330-347), then fused vs
    # the same ops over a materialised matmul, bit for bit
    a, i2, bias = T(np.array([[1, 2], [3, 4]], np.float32)), T(np.eye(2, dtype=np.float32)), T(np.array([-10, 10], np.float32))
    rc, out = eval_lib(UnaryExpr("relu", BinaryExpr("add", a.matmul(i2), bias)))
    assert rc == 0 and out.tolist() == [[0, 12], [0, 14]]
    for dt in (np.float32, np.float64):
        A = rng.standard_normal((3, 37, 20)).astype(dt)
        B = rng.standard_normal((20, 45)).astype(dt)
        bv = rng.standard_normal(45).astype(dt)
        ta_, tb_, tbias = T(A, dt), T(B, dt), T(bv, dt)
        mm = ta_.matmul(tb_)
        rc, mmv = eval_lib(mm)
        assert rc == 0
        tm = T(mmv, dt)
        for build in [lambda x: UnaryExpr("relu", BinaryExpr("add", x, tbias)), lambda x: UnaryExpr("gelu", x),
                      lambda x: UnaryExpr("silu", UnaryExpr("tanh", BinaryExpr("add", tbias, x)))]:
            rc1, fused = eval_lib(build(mm))
            rc2, split = eval_lib(build(tm))
            assert rc1 == 0 and rc2 == 0 and np.array_equal(fused, split), dt


GROUPS = {"eval": group_eval, "gemm_fp": group_gemm_fp, "gemm": group_gemm, "gemm_ln": group_gemm_ln, "range": group_range,
          "attention": group_attention,
          "arctic": group_arctic, "arctic_f16w": group_arctic_f16w, "embed": group_embed, "models": group_models, "mlp": group_mlp,
          "mlp_split": group_mlp_split,
          "nodes": group_nodes}

if __name__ == "__main__":
    check(L.tzh_init(0, None, C.byref(CTX)))
    names = sys.argv[1:] or list(GROUPS)
    for name in names:
        t0 = time.time()
        GROUPS[name]()
        print(f"emu {name}: ok ({time.time() - t0:.1f}s)", flush=True)
    check(L.tzh_destroy(CTX))
    print("EMU CHECKS PASSED", flush=True)
