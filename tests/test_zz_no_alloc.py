"""tzh_matmul_w8a32_noalloc (the entry point for callers that cannot
allocate device memory) against tzh_matmul_w8a32: the same kernels, so the
results must agree bit for bit, on two calls in a row (the second smaller,
so stale workspace contents from the first would show), through the C-ABI;
that its calls leave the context's own scratch unallocated (a context that
only ever ran the no-allocation entry point still reports 0 bytes and 0
allocations); and its size limit and empty shapes."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
import tenzor_amd
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
    Cg = torch.full((m, n), float("nan"), device="cuda")
    check(fn(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(), Cg.data_ptr(), m, k, n))
    torch.cuda.synchronize()
    return Cg.cpu().numpy()


def scratch_info(c):
    nbytes, allocs = C.c_int64(), C.c_int64()
    check(lib().tzh_ctx_scratch_info(c.handle, C.byref(nbytes), C.byref(allocs)))
    return nbytes.value, allocs.value


@pytest.mark.parametrize("shapes", [[(2048, 1536, 384), (70, 384, 1152)],   # k % 64 == 0: codes only
                                    [(1000, 385, 768), (33, 100, 5)]])       # k tails: padded rows too
def test_noalloc_matches_allocating_entry(ctx, shapes):
    own = tenzor_amd.Context(0)  # runs the no-allocation entry point only
    try:
        for i, (m, k, n) in enumerate(shapes):
            A, Q, S, B = problem(100 + i, m, k, n)
            want = call(lib().tzh_matmul_w8a32, ctx, A, Q, S, B, m, k, n)
            got = call(lib().tzh_matmul_w8a32_noalloc, own, A, Q, S, B, m, k, n)
            assert scratch_info(own) == (0, 0), (m, k, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n)
            ref = oracle.matmul_w8a32(A.cpu().numpy(), Q.cpu().numpy(), S.cpu().numpy().view(np.uint16),
                                      B.cpu().numpy())
            assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    finally:
        own.close()


def test_noalloc_empty_and_k0_shapes(ctx):
    """The reference's edges (matmul_w8a32.zig:24, 40-55): m == 0 or n == 0
    does nothing whatever k * n would need, k == 0 writes the bias."""
    A, Q, S, B = problem(8, 4, 40, 128)
    own = tenzor_amd.Context(0)
    try:
        c = torch.full((4 * 128,), 7.0, device="cuda")
        for m, k, n in [(0, 65536, 65536), (4, 40, 0), (0, 0, 0)]:
            check(lib().tzh_matmul_w8a32_noalloc(own.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                                 c.data_ptr(), m, k, n))
            assert (c == 7.0).all(), (m, k, n)
        check(lib().tzh_matmul_w8a32_noalloc(own.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                             c.data_ptr(), 4, 0, 128))
        assert torch.equal(c.reshape(4, 128), B[None, :].expand(4, 128))
        torch.cuda.synchronize()
        assert scratch_info(own) == (0, 0)
    finally:
        own.close()


def test_noalloc_rejects_oversized_workspace(ctx):
    m, k, n = 40000, 385, 384  # padded rows alone: 40000 * 448 * 4 bytes > 32 MiB
    A, Q, S, B = problem(7, m, k, n)
    Cg = torch.empty((m, n), device="cuda")
    rc = lib().tzh_matmul_w8a32_noalloc(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                        Cg.data_ptr(), m, k, n)
    assert rc == _abi.ERR_TOO_LARGE
    rc = lib().tzh_matmul_w8a32_noalloc(ctx.handle, A.data_ptr(), Q.data_ptr(), S.data_ptr(), B.data_ptr(),
                                        Cg.data_ptr(), m, -1, n)
    assert rc == _abi.ERR_INVALID_ARGS
