"""GPU checks of the split partial round of the LayerNorm GEMM (K3 with the
bias + residual + LayerNorm epilogue, arctic.zig:716-746 / 779-809).

The 128-row tiles run in whole rounds of one tile per CU; the tiles left
for a partial last round are cut into 64 x 64, 128 x 64 or 128 x 128
pieces whose pre-normalisation rows a separate kernel normalises.  Those
rows must equal, bit for bit, the same rows computed inside whole tiles
(the model's batch-order invariance depends on it), and match the oracle:
|gpu - oracle| < 1e-4 on unit-variance LayerNorm outputs with f32
activations (the model's default), < 2e-2 stored as f16."""
import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import _abi, check, lib

pytestmark = pytest.mark.gpu
N = 384


def problem(seed, m, k, dtype=np.float16):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(dtype)
    q = rng.integers(-127, 128, size=(N, k)).astype(np.int8)
    s = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.001, 0.02, N).astype(np.float32)], np.uint16)
    bias = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    res = rng.standard_normal((m, N)).astype(dtype)
    g = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32)
    return a, q, s, bias, res, g, b


def ln_gemm(ctx, a, q, s, bias, res, g, b):
    """Activations, residual and output all f32 or all f16: the model's two
    precisions."""
    m, k = a.shape
    f32 = a.dtype == np.float32
    dt = _abi.F32 if f32 else _abi.F16
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    A, Q, S, B, R, G, Bt = dev(a), dev(q), dev(s.view(np.int16)), dev(bias), dev(res), dev(g), dev(b)
    out = torch.empty((m, N), dtype=torch.float32 if f32 else torch.float16, device="cuda")
    check(lib().tzh_linear_w8(ctx.handle, A.data_ptr(), dt, Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                              out.data_ptr(), dt, m, k, N, _abi.EPI_BIAS_RES_LN, R.data_ptr(), dt,
                              G.data_ptr(), Bt.data_ptr(), 1e-12))
    return out.cpu().numpy()


def bits(x):
    return x.view(np.uint32 if x.dtype == np.float32 else np.uint16)


def bar(dtype):
    return 1e-4 if dtype == np.float32 else 2e-2


# extra tiles past the whole rounds -> pieces per tile: 2 -> 12 (64 x 64),
# 30 -> 6 (128 x 64), 60 -> 3 (128 x 128), 100 -> no split; partial tiles
# too.  k = 384 takes the unsplit two-workgroups-per-CU configuration.
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("extra_rows,k", [(2 * 128 - 28, 448), (30 * 128, 1536), (60 * 128 - 5, 448),
                                          (100 * 128, 448), (1, 1536), (2 * 128 - 28, 384)])
def test_split_rows_match_whole_tiles(ctx, extra_rows, k, dtype):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    whole_rows = cus * 128
    m = whole_rows + extra_rows
    a, q, s, bias, res, g, b = problem(extra_rows + k, m, k, dtype)
    split = ln_gemm(ctx, a, q, s, bias, res, g, b)
    # the same rows again, shifted so that every one lies in a whole tile
    shift = m - whole_rows
    whole = ln_gemm(ctx, a[shift:], q, s, bias, res[shift:], g, b)
    assert np.array_equal(bits(split[shift:]), bits(whole))
    # the oracle on a sample of the tail rows and of the whole-round rows
    rows = np.unique(np.concatenate([np.arange(whole_rows, m, max(1, extra_rows // 16)), [0, 1, whole_rows - 1, m - 1]]))
    lin = oracle.matmul_w8a32(a[rows].astype(np.float32), q, s, bias)
    ref = oracle.layernorm(res[rows].astype(np.float32) + lin, g, b, 1e-12)
    err = np.abs(split[rows].astype(np.float32) - ref).max()
    assert err < bar(dtype), float(err)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_small_batch_is_all_pieces(ctx, dtype):
    """Fewer tiles than CUs (config-1-like sizes): every tile is split
    (k = 448), or the short-k configuration runs them (k = 384, f16)."""
    for m, k in ((1, 448), (7, 448), (128, 384), (1000, 448), (1000, 384)):
        a, q, s, bias, res, g, b = problem(m, m, k, dtype)
        got = ln_gemm(ctx, a, q, s, bias, res, g, b)
        ref = oracle.layernorm(res.astype(np.float32) + oracle.matmul_w8a32(a.astype(np.float32), q, s, bias), g, b,
                               1e-12)
        assert np.abs(got.astype(np.float32) - ref).max() < bar(dtype), m


def test_config3_gemm_pair_f16_boundaries(ctx):
    """BASELINE config 3 shapes (T = 65536) through the model's path: f16
    activations between the GELU GEMM (384 -> 1536) and the residual +
    LayerNorm GEMM (1536 -> 384), int8 weights in the tiled device format.
    The oracle runs in f32 on the same f16 inputs, with the intermediate
    rounded to f16 as the GPU stores it; parity on sampled rows, exact
    LayerNorm properties on every row."""
    T, K, N1 = 65536, 384, 1536
    rng = np.random.default_rng(9)
    x = rng.standard_normal((T, K)).astype(np.float16)
    q1 = rng.integers(-127, 128, size=(N1, K)).astype(np.int8)
    s1 = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.001, 0.02, N1).astype(np.float32)], np.uint16)
    b1 = rng.uniform(-0.1, 0.1, N1).astype(np.float32)
    q2 = rng.integers(-127, 128, size=(K, N1)).astype(np.int8)
    s2 = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.001, 0.02, K).astype(np.float32)], np.uint16)
    b2 = rng.uniform(-0.1, 0.1, K).astype(np.float32)
    g, bt = np.ones(K, np.float32), np.zeros(K, np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    X = dev(x)
    H = torch.empty((T, N1), dtype=torch.float16, device="cuda")
    Y = torch.empty((T, K), dtype=torch.float16, device="cuda")
    Q1, S1, B1, Q2, S2, B2, G, Bt = (dev(q1), dev(s1.view(np.int16)), dev(b1), dev(q2), dev(s2.view(np.int16)),
                                     dev(b2), dev(g), dev(bt))
    check(lib().tzh_linear_w8(ctx.handle, X.data_ptr(), _abi.F16, Q1.data_ptr(), S1.data_ptr(), B1.data_ptr(),
                              H.data_ptr(), _abi.F16, T, K, N1, _abi.EPI_BIAS_GELU, None, _abi.F16, None, None, 0.0))
    check(lib().tzh_linear_w8(ctx.handle, H.data_ptr(), _abi.F16, Q2.data_ptr(), S2.data_ptr(), B2.data_ptr(),
                              Y.data_ptr(), _abi.F16, T, N1, K, _abi.EPI_BIAS_RES_LN, X.data_ptr(), _abi.F16,
                              G.data_ptr(), Bt.data_ptr(), 1e-12))
    y = Y.cpu().numpy().astype(np.float32)
    assert np.abs(y.mean(axis=1)).max() < 2e-3
    assert np.abs(y.var(axis=1) - 1).max() < 5e-3
    rows = np.sort(rng.choice(T, 256, replace=False))
    xf = x[rows].astype(np.float32)
    h = oracle.gelu(oracle.matmul_w8a32(xf, q1, s1, b1)).astype(np.float16).astype(np.float32)
    ref = oracle.layernorm(xf + oracle.matmul_w8a32(h, q2, s2, b2), g, bt, 1e-12)
    err = np.abs(y[rows] - ref)
    assert err.max() < 1e-2, float(err.max())
    assert np.sqrt((err ** 2).mean()) < 1e-3
