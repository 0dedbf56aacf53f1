"""tzh_matmul_w8a32_noalloc (the entry point for callers that cannot
allocate device memory) against tzh_matmul_w8a32: the same kernels, so the
results must agree bit for bit, on two calls in a row (the second smaller,
so stale workspace contents from the first would show), through the C-ABI;
and its size limit."""
import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import _abi, check, lib

pytestmark = pytest.mark.gpu


def problem(seed, m, k, n):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(np.float32)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = np.array([oracle.f32_to_f16(v) for v in rng.uniform(0.001, 0.02, n).astype(np.float32)], np.uint16)
    b = rng.uniform(-0.1, 0.1, n).astype(np.float32)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return dev(a), dev(q), dev(s.view(np.int16)), dev(b)


def call(fn, ctx, A, Q, S, B, m, k, n):
    C = torch.full((m, n), float("nan"), device="cuda")
    check(fn(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(), C.data_ptr(), m, k, n))
    torch.cuda.synchronize()
    return C.cpu().numpy()


@pytest.mark.parametrize("shapes", [[(2048, 1536, 384), (70, 384, 1152)],   # k % 64 == 0: codes only
                                    [(1000, 385, 768), (33, 100, 5)]])       # k tails: padded rows too
def test_noalloc_matches_allocating_entry(ctx, shapes):
    for i, (m, k, n) in enumerate(shapes):
        A, Q, S, B = problem(100 + i, m, k, n)
        want = call(lib().tzh_matmul_w8a32, ctx, A, Q, S, B, m, k, n)
        got = call(lib().tzh_matmul_w8a32_noalloc, ctx, A, Q, S, B, m, k, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n)
        ref = oracle.matmul_w8a32(A.cpu().numpy(), Q.cpu().numpy(), S.cpu().numpy().view(np.uint16), B.cpu().numpy())
        assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())


def test_noalloc_rejects_oversized_workspace(ctx):
    m, k, n = 40000, 385, 384  # padded rows alone: 40000 * 448 * 4 bytes > 32 MiB
    A, Q, S, B = problem(7, m, k, n)
    C = torch.empty((m, n), device="cuda")
    rc = lib().tzh_matmul_w8a32_noalloc(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                        C.data_ptr(), m, k, n)
    assert rc == _abi.ERR_TOO_LARGE
    rc = lib().tzh_matmul_w8a32_noalloc(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                        C.data_ptr(), m, 0, n)
    assert rc == _abi.ERR_INVALID_ARGS
