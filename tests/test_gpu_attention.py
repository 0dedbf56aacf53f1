"""GPU parity of the variable-length attention kernel (K4) against the
oracle's per-head attention (arctic.zig:660-713).

f32 Q/K/V (the model's default): every product is formed from exact f16
hi/lo splits and summed in f32, so the result agrees with the oracle's f32
attention to about 2^-20 relative; the bar is
    |gpu - oracle| <= 2^-16 max|V| + 2^-18 |O|
which dropping any of the split terms (errors near 2^-12 max|V|) exceeds.

f16 Q/K/V (the opt-in fast path): the oracle runs in f32 on the same f16
values; the GPU rounds P to f16 for the P*V MFMA and the output to f16, so
|gpu - oracle| <= 2^-9 max|V| + 2^-10 |O| is the bar."""
import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import TzhError, _abi, check, lib

pytestmark = pytest.mark.gpu
H, NH, D = 384, 12, 32


def run(ctx, qkv, lengths):
    """qkv: f16 or f32 [T, 3H] host array -> (out f32 [T, H], cu)."""
    cu = np.zeros(len(lengths) + 1, np.int32)
    cu[1:] = np.cumsum(lengths)
    f32 = qkv.dtype == np.float32
    Q = torch.from_numpy(qkv if f32 else qkv.view(np.int16)).cuda()
    O = torch.zeros((qkv.shape[0], H), dtype=torch.float32 if f32 else torch.int16, device="cuda")
    CU = torch.from_numpy(cu).cuda()
    check(lib().tzh_attention_varlen(ctx.handle, Q.data_ptr(), O.data_ptr(), _abi.F32 if f32 else _abi.F16,
                                     CU.data_ptr(), len(lengths), NH, H))
    out = O.cpu().numpy()
    return (out if f32 else out.view(np.float16).astype(np.float32)), cu


def tolerance(v, ref, f32, extra=0.0):
    if f32:
        return 2.0 ** -16 * np.abs(v).max() + 2.0 ** -18 * np.abs(ref) + 1e-30
    return 2.0 ** -9 * np.abs(v).max() + 2.0 ** -10 * np.abs(ref) + extra


def check_heads(out, qkv, lengths, cu, heads, f32, extra=0.0):
    q32 = qkv.astype(np.float32)
    for b, L in enumerate(lengths):
        s0 = cu[b]
        for h in heads:
            cols = slice(h * D, (h + 1) * D)
            q = q32[s0:s0 + L, cols]
            k = q32[s0:s0 + L, H + h * D: H + (h + 1) * D]
            v = q32[s0:s0 + L, 2 * H + h * D: 2 * H + (h + 1) * D]
            ref = oracle.attention_head(q, k, v)
            got = out[s0:s0 + L, cols]
            tol = tolerance(v, ref, f32, extra)
            assert (np.abs(got - ref) <= tol).all(), (b, h, float(np.abs(got - ref).max()))


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("lengths", [[1], [2, 3], [15, 16, 17], [63, 64, 65], [100, 1, 511], [512, 300]])
def test_attention_vs_oracle(ctx, lengths, dtype):
    rng = np.random.default_rng(sum(lengths))
    T = int(sum(lengths))
    qkv = (rng.standard_normal((T, 3 * H)) * 1.5).astype(dtype)
    out, cu = run(ctx, qkv, lengths)
    check_heads(out, qkv, lengths, cu, range(NH), dtype == np.float32)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_attention_sharp_softmax(ctx, dtype):
    """Large scores (peaked softmax) exercise the running-max rescaling."""
    rng = np.random.default_rng(5)
    L = 300
    qkv = rng.standard_normal((L, 3 * H)).astype(np.float32)
    qkv[:, :H] *= 8
    qkv[:, H:2 * H] *= 8
    qkv = qkv.astype(dtype)
    out, cu = run(ctx, qkv, [L])
    # f32: scores of a few hundred carry an error of about 2^-21 of their
    # magnitude (in both the oracle and the split products) into the
    # exponent, hence the looser f32 bar here
    f32 = dtype == np.float32
    if not f32:
        check_heads(out, qkv, [L], cu, (0, 5, 11), False, extra=1e-3)
    else:
        q32 = qkv
        for h in (0, 5, 11):
            v = q32[:, 2 * H + h * D:2 * H + (h + 1) * D]
            ref = oracle.attention_head(q32[:, h * D:(h + 1) * D], q32[:, H + h * D:H + (h + 1) * D], v)
            assert np.abs(out[:, h * D:(h + 1) * D] - ref).max() <= 2.0 ** -12 * np.abs(v).max()


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_attention_growing_scores(ctx, dtype):
    """Key norms that grow along the sequence push the row max up block after
    block, by less than and by more than the softmax's lazy-rescale slack."""
    rng = np.random.default_rng(9)
    L = 512
    qkv = rng.standard_normal((L, 3 * H)).astype(np.float32)
    qkv[:, H:2 * H] *= (0.2 + np.arange(L) / 48.0)[:, None]
    qkv = qkv.astype(dtype)
    out, cu = run(ctx, qkv, [L])
    f32 = dtype == np.float32
    if f32:
        q32 = qkv
        for h in (0, 6, 11):
            v = q32[:, 2 * H + h * D:2 * H + (h + 1) * D]
            ref = oracle.attention_head(q32[:, h * D:(h + 1) * D], q32[:, H + h * D:H + (h + 1) * D], v)
            assert np.abs(out[:, h * D:(h + 1) * D] - ref).max() <= 2.0 ** -14 * np.abs(v).max()
    else:
        check_heads(out, qkv, [L], cu, (0, 6, 11), False, extra=1e-3)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_sequences_are_independent(ctx, dtype):
    """Packing order must not change any sequence's result (bit-exact)."""
    rng = np.random.default_rng(6)
    lengths = [40, 200, 7]
    qkv = rng.standard_normal((sum(lengths), 3 * H)).astype(dtype)
    out, cu = run(ctx, qkv, lengths)
    alone, _ = run(ctx, np.ascontiguousarray(qkv[cu[1]:cu[2]]), [200])
    assert np.array_equal(out[cu[1]:cu[2]], alone)


def test_attention_rejects_bad_lengths(ctx):
    qkv = np.zeros((600, 3 * H), np.float16)
    with pytest.raises(TzhError) as ei:
        run(ctx, qkv, [600])
    assert ei.value.code == _abi.ERR_INVALID_ARGS
    with pytest.raises(TzhError):
        run(ctx, qkv[:10], [0, 10])
    with pytest.raises(TzhError) as ei:
        check(lib().tzh_attention_varlen(ctx.handle, None, None, _abi.I8, None, 1, NH, H))
    assert ei.value.code == _abi.ERR_UNSUPPORTED_DTYPE


def test_work_queue_across_launches(ctx):
    """f32 attention takes (sequence, head) items from a work queue that each
    launch returns to zero: more items than CUs, then a smaller batch, then
    the first batch again (bit-identical: the queue changes which block
    computes an item, not its sums)."""
    rng = np.random.default_rng(21)
    big = [int(x) for x in rng.integers(1, 513, 64)]
    small = [int(x) for x in rng.integers(1, 513, 5)]
    qb = rng.standard_normal((sum(big), 3 * H)).astype(np.float32)
    qs = rng.standard_normal((sum(small), 3 * H)).astype(np.float32)
    out1, cu1 = run(ctx, qb, big)
    out2, cu2 = run(ctx, qs, small)
    out3, _ = run(ctx, qb, big)
    check_heads(out1, qb, big, cu1, (0, 11), True)
    check_heads(out2, qs, small, cu2, range(NH), True)
    assert np.array_equal(out1, out3)
