"""GPU parity of the int8-weight GEMM (K3) and its epilogues against the
oracle's matmul_w8a32 (matmul_w8a32.zig:14-57), GELU (arctic.zig:750-756)
and LayerNorm (layernorm.zig:26-117).

Tolerance: each f32 activation row is scaled by the power of two 2^e that
puts its largest magnitude M in [2^14, 2^15) and enters the MFMA as an
exact f16 split a 2^e = hi + lo + r with |r| <= 2^-22 |a 2^e| (for |a| >=
2^-17 M) or 2^-25 (below), and the sums run in f32 in another order than
the oracle's, so every output is checked against the bound
    |gpu - oracle| <= s_j * sum_k (|a_ik| + 2^-36 M_i) |q_jk| * (2^-20 + k 2^-23) + 2^-22 |c_ij| + 1e-37
which a dropped lo half (2^-12 |a|), a wrong scale/bias index, a
transposed operand or a missing row scale (2^-25 |a|^-1 relative error for
small rows) exceeds.  f16 activations (the opt-in model path) are exact in
the MFMA; their outputs are compared with the oracle on the same f16
values."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import _abi, check, lib, quantize_rows_host

pytestmark = pytest.mark.gpu


def make_problem(seed, m, k, n, x_scale=1.0):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((m, k)) * x_scale).astype(np.float32)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.001, 0.02, n).astype(np.float32)], np.uint16)
    bias = rng.uniform(-0.1, 0.1, n).astype(np.float32)
    return a, q, s, bias


def bound(a, q, s, c, k):
    sf = s.view(np.float16).astype(np.float64)
    a64 = np.abs(a.astype(np.float64))
    mag = (a64 + 2.0 ** -36 * a64.max(axis=1, keepdims=True)) @ np.abs(q.astype(np.float64)).T * sf[None, :]
    return mag * (2.0 ** -20 + k * 2.0 ** -23) + 2.0 ** -22 * np.abs(c) + 1e-37


def normalised_error(c, a, q, s, bias=None):
    """max |c - exact| / (sum_k |a| |q| s): the error of an f32 matmul_w8a32
    relative to the magnitude of its terms (exact = float64)."""
    sf = s.view(np.float16).astype(np.float64)
    exact = (a.astype(np.float64) @ q.astype(np.float64).T) * sf
    if bias is not None:
        exact = exact + bias.astype(np.float64)
    mag = (np.abs(a.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * sf
    return float((np.abs(c.astype(np.float64) - exact) / mag).max())


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def gpu_linear(ctx, a, q, s, bias, out_dtype=torch.float32, epi=_abi.EPI_BIAS, res=None, g=None, b=None,
               eps=1e-12):
    m, k = a.shape
    n = q.shape[0]
    A = dev(a) if a.dtype != np.float16 else dev(a)
    Q, S, B = dev(q), dev(s.view(np.int16)), dev(bias)
    Cout = torch.empty((m, n), dtype=out_dtype, device="cuda")
    a_dt = _abi.F16 if A.dtype == torch.float16 else _abi.F32
    c_dt = _abi.F16 if out_dtype == torch.float16 else _abi.F32
    R = dev(res) if res is not None else None
    G = dev(g) if g is not None else None
    Bt = dev(b) if b is not None else None
    check(lib().tzh_linear_w8(ctx.handle, A.data_ptr(), a_dt, Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                              Cout.data_ptr(), c_dt, m, k, n, epi, R.data_ptr() if R is not None else None,
                              c_dt, G.data_ptr() if G is not None else None,
                              Bt.data_ptr() if Bt is not None else None, eps))
    return Cout.float().cpu().numpy()


@pytest.mark.parametrize("m,k,n", [(1, 64, 128), (5, 384, 384), (333, 384, 1152), (1000, 1536, 384),
                                   (129, 384, 1536), (4096, 384, 384),
                                   # k tails (matmul_w8a32.zig:50-52), odd n, n over one 1536-column chunk
                                   (37, 385, 384), (9, 7, 5), (130, 1000, 1537), (3, 40, 128)])
def test_matmul_w8a32_vs_oracle(ctx, m, k, n):
    a, q, s, bias = make_problem(m * 7 + n, m, k, n)
    A, Q, S, B = dev(a), dev(q), dev(s.view(np.int16)), dev(bias)
    Cg = torch.empty((m, n), device="cuda")
    check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                 Cg.data_ptr(), m, k, n))
    c = Cg.cpu().numpy()
    ref = oracle.matmul_w8a32(a, q, s, bias)
    err = np.abs(c.astype(np.float64) - ref)
    assert (err <= bound(a, q, s, ref, k)).all(), float((err / bound(a, q, s, ref, k)).max())


def test_matmul_w8a32_unaligned_operands(ctx):
    """Row pitches that are not multiples of 16 bytes and operands that start
    off 16-byte boundaries (views into larger buffers)."""
    m, k, n = 45, 130, 7
    a, q, s, bias = make_problem(17, m, k, n)
    Abuf = torch.zeros(m * k + 1, device="cuda")
    Abuf[1:] = dev(a).reshape(-1)
    Cbuf = torch.full((m * n + 1,), float("nan"), device="cuda")
    Q, S, B = dev(q), dev(s.view(np.int16)), dev(bias)
    check(lib().tzh_matmul_w8a32(ctx.handle, Abuf.data_ptr() + 4, Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                 Cbuf.data_ptr() + 4, m, k, n))
    c = Cbuf[1:].reshape(m, n).cpu().numpy()
    ref = oracle.matmul_w8a32(a, q, s, bias)
    assert (np.abs(c - ref) <= bound(a, q, s, ref, k)).all()
    assert np.isnan(Cbuf[0].item())  # nothing written before c


def test_matmul_w8a32_null_bias_and_zero_rows(ctx):
    a, q, s, _ = make_problem(3, 70, 128, 256)
    A, Q, S = dev(a), dev(q), dev(s.view(np.int16))
    Cg = torch.empty((70, 256), device="cuda")
    check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(),
                                 70, 128, 256))
    ref = oracle.matmul_w8a32(a, q, s, None)
    assert (np.abs(Cg.cpu().numpy() - ref) <= bound(a, q, s, ref, 128)).all()


def test_matmul_w8a32_empty_and_k0_edges(ctx):
    """matmul_w8a32.zig:24 returns for m == 0 or n == 0 before touching c;
    with k == 0 the sum is empty and c[i,j] = 0 * s[j] + bias[j] (40-55)."""
    a, q, s, bias = make_problem(4, 8, 40, 128)
    A, Q, S, B = dev(a), dev(q), dev(s.view(np.int16)), dev(bias)
    sentinel = torch.full((8 * 128,), 7.0, device="cuda")
    for m, k, n in [(0, 40, 128), (8, 40, 0), (0, 0, 0), (0, 65536, 65536)]:
        check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                     sentinel.data_ptr(), m, k, n))
        assert (sentinel == 7.0).all(), (m, k, n)
    Cg = torch.full((8, 128), float("nan"), device="cuda")
    check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(), Cg.data_ptr(),
                                 8, 0, 128))
    assert np.array_equal(Cg.cpu().numpy(), np.broadcast_to(bias, (8, 128)))
    check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(), 8, 0, 128))
    assert (Cg == 0).all()
    assert np.array_equal(oracle.matmul_w8a32(np.zeros((8, 0), np.float32), np.zeros((128, 0), np.int8), s, bias),
                          np.broadcast_to(bias, (8, 128)))


def test_matmul_w8a32_rejects_bad_arguments(ctx):
    a, q, s, bias = make_problem(4, 8, 40, 128)
    A, Q, S = dev(a), dev(q), dev(s.view(np.int16))
    Cg = torch.empty((8, 128), device="cuda")
    for m, k, n in [(-1, 40, 128), (8, -1, 128), (8, 40, -1)]:
        rc = lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(), m, k, n)
        assert rc == _abi.ERR_INVALID_ARGS, (m, k, n)
    rc = lib().tzh_matmul_w8a32(ctx.handle, None, Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(), 8, 40, 128)
    assert rc == _abi.ERR_INVALID_ARGS


SCALES = [1e-6, 1e-3, 1.0, 3e4, 1e6]


@pytest.mark.parametrize("scale", SCALES)
def test_matmul_w8a32_over_the_f32_range(ctx, scale):
    """Inputs N(0,1) * scale from 1e-6 to 1e6 (the f16 halves alone span
    2^-24 .. 65504): every output within the bound, no NaN, and the error
    relative to the terms' magnitude at the f32 oracle's own level, through
    tzh_matmul_w8a32, tzh_matmul_w8a32_noalloc and tzh_linear_w8."""
    m, k, n = 300, 384, 1152
    a, q, s, _ = make_problem(40, m, k, n)
    a = (a.astype(np.float64) * scale).astype(np.float32)
    A, Q, S = dev(a), dev(q), dev(s.view(np.int16))
    ref = oracle.matmul_w8a32(a, q, s, None)
    orc = normalised_error(ref, a, q, s)
    outs = {}
    for name in ("tzh_matmul_w8a32", "tzh_matmul_w8a32_noalloc"):
        Cg = torch.full((m, n), float("nan"), device="cuda")
        check(getattr(lib(), name)(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(), m, k, n))
        outs[name] = Cg.cpu().numpy()
    outs["tzh_linear_w8"] = gpu_linear(ctx, a, q, s, np.zeros(n, np.float32))
    for name, c in outs.items():
        ours = normalised_error(c, a, q, s)
        assert np.isfinite(c).all(), name
        assert (np.abs(c - ref) <= bound(a, q, s, ref, k)).all(), name
        assert ours <= max(4 * orc, 2.0 ** -22), (name, ours, orc)


@pytest.mark.parametrize("scale", SCALES)
def test_linear_w8_epilogues_over_the_f32_range(ctx, scale):
    """GELU and residual + LayerNorm epilogues of tzh_linear_w8 with f32
    activations of every scale (LayerNorm: its 128-row tiles with a split
    last round at k = 1536, the two-workgroup tiles at k = 384)."""
    m, k, n = 300, 384, 1536
    a, q, s, bias = make_problem(41, m, k, n)
    a = (a.astype(np.float64) * scale).astype(np.float32)
    bias = (bias * min(scale, 1.0)).astype(np.float32)
    lin = oracle.matmul_w8a32(a, q, s, bias)
    c = gpu_linear(ctx, a, q, s, bias, torch.float32, _abi.EPI_BIAS_GELU)
    ref = oracle.gelu(lin)
    tol = 1.13 * bound(a, q, s, lin, k) + 2.0 ** -20 * np.abs(ref) + 1e-37
    assert np.isfinite(c).all() and (np.abs(c - ref) <= tol).all(), float((np.abs(c - ref) / tol).max())
    rng = np.random.default_rng(42)
    # 40000 rows at k = 1536: whole rounds of 128-row tiles, then the
    # leftover tiles as pieces; 3000 rows: pieces only; k = 384: the
    # two-workgroup tiles.  Parity on sampled rows of every region.
    for m, k in ((40000, 1536), (3000, 1536), (777, 384)):
        a, q, s, bias = make_problem(43 + k, m, k, 384)
        a = (a.astype(np.float64) * scale).astype(np.float32)
        bias = (bias * scale).astype(np.float32)
        res = (rng.standard_normal((m, 384)) * scale).astype(np.float32)
        gamma = (1 + 0.1 * rng.standard_normal(384)).astype(np.float32)
        beta = (0.1 * rng.standard_normal(384)).astype(np.float32)
        c = gpu_linear(ctx, a, q, s, bias, torch.float32, _abi.EPI_BIAS_RES_LN, res, gamma, beta)
        rows = np.unique(np.concatenate([rng.choice(m, min(m, 400), replace=False), np.arange(m - 50, m)]))
        a, res, c = a[rows], res[rows], c[rows]
        pre = res + oracle.matmul_w8a32(a, q, s, bias)
        ref = oracle.layernorm(pre, gamma, beta, 1e-12)
        std = pre.astype(np.float64).std(axis=1, keepdims=True)
        tol = (bound(a, q, s, pre, k) + 2.0 ** -22 * np.abs(res)).max(axis=1, keepdims=True) * 4 * \
            np.abs(gamma)[None, :] / std + 1e-5
        assert np.isfinite(c).all() and (np.abs(c - ref) <= tol).all(), (m, k, float((np.abs(c - ref) / tol).max()))


@pytest.mark.parametrize("epi", [_abi.EPI_BIAS, _abi.EPI_BIAS_GELU])
def test_rows_changing_scale_along_k(ctx, epi):
    """Row scaling is chosen stage by stage: rows that grow by 1e6 after
    their first 64 values, rows of zeros then ordinary values, rows growing
    from 1e-20 to 1e20 along k, rows large then tiny; the sums accumulated
    so far are rescaled exactly when a row's exponent drops."""
    m, k, n = 700, 448, 768
    a, q, s, bias = make_problem(45, m, k, n)
    prof = np.ones((m, k), np.float32)
    prof[0::5, :64] = 1e-3
    prof[0::5, 64:] = 1e3
    prof[1::5, :192] = 0.0
    prof[2::5, :] = np.logspace(-20, 20, k).astype(np.float32)
    prof[3::5, 200:] = 1e-9
    a = a * prof
    c = gpu_linear(ctx, a, q, s, bias, torch.float32, epi)
    lin = oracle.matmul_w8a32(a, q, s, bias)
    sf = s.view(np.float16).astype(np.float64)
    exact = (a.astype(np.float64) @ q.astype(np.float64).T) * sf + bias
    mag = (np.abs(a.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * sf
    assert np.isfinite(c).all()
    if epi == _abi.EPI_BIAS:
        assert (np.abs(c - exact) / (mag + np.abs(exact))).max() < 2.0 ** -21
    else:
        ref = oracle.gelu(lin)
        tol = 1.13 * 2.0 ** -21 * (mag + np.abs(exact)) + 2.0 ** -20 * np.abs(ref) + 1e-37
        assert (np.abs(c - ref) <= tol).all()


def test_matmul_w8a32_rows_of_every_scale(ctx):
    """One matrix whose rows span 1e-30 .. 1e30, a zero row and a row of
    f32 subnormals: each row keeps its own relative accuracy."""
    m, k, n = 197, 128, 768
    a, q, s, bias = make_problem(44, m, k, n)
    a[0] = 0
    a[1] *= np.float32(2.0 ** -140)
    a[2:] *= np.logspace(-30, 30, m - 2).astype(np.float32)[:, None]
    A, Q, S, B = dev(a), dev(q), dev(s.view(np.int16)), dev(bias)
    Cg = torch.empty((m, n), device="cuda")
    check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(), Cg.data_ptr(),
                                 m, k, n))
    c = Cg.cpu().numpy()
    assert np.isfinite(c).all() and np.array_equal(c[0], bias)
    sf = s.view(np.float16).astype(np.float64)
    exact = (a.astype(np.float64) @ q.astype(np.float64).T) * sf + bias
    mag = (np.abs(a.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * sf
    assert (np.abs(c - exact) / (mag + np.abs(exact)))[1:].max() < 2.0 ** -21


def test_f16_activations_f16_out(ctx):
    m, k, n = 777, 384, 1152
    a, q, s, bias = make_problem(5, m, k, n)
    a16 = a.astype(np.float16)
    c = gpu_linear(ctx, a16, q, s, bias, torch.float16)
    ref = oracle.matmul_w8a32(a16.astype(np.float32), q, s, bias)
    tol = bound(a16.astype(np.float32), q, s, ref, k) + np.abs(ref) * 2.0 ** -11
    assert (np.abs(c - ref) <= tol).all()


def test_gelu_epilogue(ctx):
    m, k, n = 300, 384, 1536
    a, q, s, bias = make_problem(6, m, k, n, x_scale=0.05)
    c = gpu_linear(ctx, a, q, s, bias, torch.float32, _abi.EPI_BIAS_GELU)
    lin = oracle.matmul_w8a32(a, q, s, bias)
    ref = oracle.gelu(lin)
    # gelu is 1.13-Lipschitz; tanh differs from libm by a few ulp
    tol = 1.13 * bound(a, q, s, lin, k) + 1e-6 * (1 + np.abs(ref))
    assert (np.abs(c - ref) <= tol).all()


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_residual_layernorm_epilogue(ctx, out_dtype):
    m, k, n = 257, 1536, 384
    a, q, s, bias = make_problem(7, m, k, n, x_scale=0.1)
    rng = np.random.default_rng(8)
    res = rng.standard_normal((m, n)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
    if out_dtype == torch.float16:
        res = res.astype(np.float16)
    c = gpu_linear(ctx, a, q, s, bias, out_dtype, _abi.EPI_BIAS_RES_LN, res, gamma, beta)
    pre = res.astype(np.float32) + oracle.matmul_w8a32(a, q, s, bias)  # input + tmp (arctic.zig:720)
    ref = oracle.layernorm(pre, gamma, beta, 1e-12)
    # LN amplifies the pre-norm error by |gamma| / std(row)
    std = pre.std(axis=1, keepdims=True)
    tol = bound(a, q, s, pre, k).max(axis=1, keepdims=True) * 4 * np.abs(gamma)[None, :] / std + 1e-5
    if out_dtype == torch.float16:
        tol = tol + np.abs(ref) * 2.0 ** -11
    assert (np.abs(c - ref) <= tol).all(), float((np.abs(c - ref) / tol).max())


def test_config3_gemm_pair_full_size_row_sample(ctx):
    """Config 3 at full size (T = 65536): GELU GEMM then the residual + LN
    GEMM, f32 X, f32 intermediate and f32 output (the reference's
    arithmetic); parity on sampled rows."""
    T, K, N = 65536, 384, 1536
    rng = np.random.default_rng(9)
    X = torch.randn(T, K, generator=torch.Generator().manual_seed(9)).numpy()
    _, q1, s1, b1 = make_problem(10, 1, K, N)
    _, q2, s2, b2 = make_problem(11, 1, N, K)
    gamma, beta = np.ones(K, np.float32), np.zeros(K, np.float32)
    Xd, Hd, Yd = dev(X), torch.empty((T, N), device="cuda"), torch.empty((T, K), device="cuda")
    Q1, S1, B1 = dev(q1), dev(s1.view(np.int16)), dev(b1)
    Q2, S2, B2, G, Bt = dev(q2), dev(s2.view(np.int16)), dev(b2), dev(gamma), dev(beta)
    check(lib().tzh_linear_w8(ctx.handle, Xd.data_ptr(), _abi.F32, Q1.data_ptr(), S1.data_ptr(), B1.data_ptr(),
                              Hd.data_ptr(), _abi.F32, T, K, N, _abi.EPI_BIAS_GELU, None, _abi.F32, None, None, 0.0))
    check(lib().tzh_linear_w8(ctx.handle, Hd.data_ptr(), _abi.F32, Q2.data_ptr(), S2.data_ptr(), B2.data_ptr(),
                              Yd.data_ptr(), _abi.F32, T, N, K, _abi.EPI_BIAS_RES_LN, Xd.data_ptr(), _abi.F32,
                              G.data_ptr(), Bt.data_ptr(), 1e-12))
    Y = Yd.cpu().numpy()
    # exact properties on every row: LN output has mean ~0 and variance ~1
    assert np.abs(Y.mean(axis=1)).max() < 1e-4
    assert np.abs(Y.var(axis=1) - 1).max() < 1e-3
    rows = np.sort(rng.choice(T, 256, replace=False))
    h = oracle.gelu(oracle.matmul_w8a32(X[rows], q1, s1, b1))
    ref = oracle.layernorm(X[rows] + oracle.matmul_w8a32(h, q2, s2, b2), gamma, beta, 1e-12)
    err = np.abs(Y[rows] - ref)
    # f32 arithmetic end to end: errors of order 1e-6 (f16 activations gave 1e-3)
    assert err.max() < 1e-4, float(err.max())
    assert np.sqrt((err ** 2).mean()) < 1e-5


def test_quantize_rows_gpu_bit_exact(ctx):
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((1536, 384)) * 0.02).astype(np.float32)
    w[0] = 0.0                       # all-zero row -> scale 1, codes 0
    w[1, :5] = [1.0, -1.0, 0.5, -0.5, 0.25]
    w[2] = np.float32(3.0)
    W = dev(w)
    Q = torch.empty((1536, 384), dtype=torch.int8, device="cuda")
    S = torch.empty(1536, dtype=torch.int16, device="cuda")
    check(lib().tzh_quantize_rows(ctx.handle, W.data_ptr(), 1536, 384, Q.data_ptr(), S.data_ptr()))
    qo, so = oracle.quantize_rows(w)
    assert np.array_equal(Q.cpu().numpy(), qo)
    assert np.array_equal(S.cpu().numpy().view(np.uint16), so)
    qh, sh = quantize_rows_host(w)
    assert np.array_equal(qh, qo) and np.array_equal(sh, so)


def test_layernorm_entry_vs_oracle(ctx):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((300, 384)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(384).astype(np.float32)
    b = rng.standard_normal(384).astype(np.float32)
    ref = oracle.layernorm(x, g, b, 1e-12)
    X, G, B = dev(x), dev(g), dev(b)
    check(lib().tzh_layernorm_last_dim(ctx.handle, X.data_ptr(), G.data_ptr(), B.data_ptr(), X.data_ptr(), 300, 384,
                                       1e-12))  # in place (layernorm.zig:26-35 allows input == output)
    np.testing.assert_allclose(X.cpu().numpy(), ref, rtol=1e-5, atol=2e-5)
