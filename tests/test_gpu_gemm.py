"""GPU parity of the int8-weight GEMM (K3) and its epilogues against the
oracle's matmul_w8a32 (matmul_w8a32.zig:14-57), GELU (arctic.zig:750-756)
and LayerNorm (layernorm.zig:26-117).

Tolerance: f32 activations enter the MFMA as an exact f16 split a = hi +
lo + r with |r| <= 2^-22 |a| + 2^-25, and the sums run in f32 in another
order than the oracle's, so every output is checked against the bound
    |gpu - oracle| <= s_j * sum_k (|a_ik| + 2^-4) |q_jk| * (2^-20 + k 2^-23) + 2^-22 |c_ij| + 1e-30
which a dropped lo half (2^-12 |a|), a wrong scale/bias index or a
transposed operand exceeds by orders of magnitude.  f16 activations (the
opt-in model path) are exact in the MFMA; their outputs are compared with
the oracle on the same f16 values."""
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
    mag = (np.abs(a).astype(np.float64) + 2.0 ** -4) @ np.abs(q.astype(np.float64)).T * sf[None, :]
    return mag * (2.0 ** -20 + k * 2.0 ** -23) + 2.0 ** -22 * np.abs(c) + 1e-30


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
    # m == 0 is a no-op (matmul_w8a32.zig:24)
    check(lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(),
                                 0, 128, 256))


def test_matmul_w8a32_rejects_bad_arguments(ctx):
    a, q, s, bias = make_problem(4, 8, 40, 128)
    A, Q, S = dev(a), dev(q), dev(s.view(np.int16))
    Cg = torch.empty((8, 128), device="cuda")
    for m, k, n in [(8, 0, 128), (-1, 40, 128), (8, 40, 0)]:
        rc = lib().tzh_matmul_w8a32(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(), m, k, n)
        assert rc == _abi.ERR_INVALID_ARGS, (m, k, n)
    rc = lib().tzh_matmul_w8a32(ctx.handle, None, Q.data_ptr(), S.data_ptr(), None, Cg.data_ptr(), 8, 40, 128)
    assert rc == _abi.ERR_INVALID_ARGS


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
