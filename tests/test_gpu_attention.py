"""GPU parity of the variable-length attention kernel (K4) against the
oracle's per-head attention (arctic.zig:660-713).

Inputs are f16 (what the GEMM producing QKV stores); the oracle runs in f32
on the same f16 values.  The GPU rounds P to f16 for the P*V MFMA and the
output to f16, so |gpu - oracle| <= 2^-9 * max|V| + 2^-10 |O| is the bar."""
import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import TzhError, _abi, check, lib

pytestmark = pytest.mark.gpu
H, NH, D = 384, 12, 32


def run(ctx, qkv16, lengths):
    cu = np.zeros(len(lengths) + 1, np.int32)
    cu[1:] = np.cumsum(lengths)
    Q = torch.from_numpy(qkv16.view(np.int16)).cuda()
    O = torch.zeros((qkv16.shape[0], H), dtype=torch.int16, device="cuda")
    CU = torch.from_numpy(cu).cuda()
    check(lib().tzh_attention_varlen(ctx.handle, Q.data_ptr(), O.data_ptr(), CU.data_ptr(), len(lengths), NH, H))
    return O.cpu().numpy().view(np.float16).astype(np.float32), cu


@pytest.mark.parametrize("lengths", [[1], [2, 3], [15, 16, 17], [63, 64, 65], [100, 1, 511], [512, 300]])
def test_attention_vs_oracle(ctx, lengths):
    rng = np.random.default_rng(sum(lengths))
    T = int(sum(lengths))
    qkv = (rng.standard_normal((T, 3 * H)) * 1.5).astype(np.float16)
    out, cu = run(ctx, qkv, lengths)
    q32 = qkv.astype(np.float32)
    for b, L in enumerate(lengths):
        s0 = cu[b]
        for h in range(NH):
            cols = slice(h * D, (h + 1) * D)
            q = q32[s0:s0 + L, cols]
            k = q32[s0:s0 + L, H + h * D: H + (h + 1) * D]
            v = q32[s0:s0 + L, 2 * H + h * D: 2 * H + (h + 1) * D]
            ref = oracle.attention_head(q, k, v)
            got = out[s0:s0 + L, cols]
            tol = 2.0 ** -9 * np.abs(v).max() + 2.0 ** -10 * np.abs(ref)
            assert (np.abs(got - ref) <= tol).all(), (b, h, float(np.abs(got - ref).max()))


def test_attention_sharp_softmax(ctx):
    """Large scores (peaked softmax) exercise the running-max rescaling."""
    rng = np.random.default_rng(5)
    L = 300
    qkv = rng.standard_normal((L, 3 * H)).astype(np.float32)
    qkv[:, :H] *= 8
    qkv[:, H:2 * H] *= 8
    qkv = qkv.astype(np.float16)
    out, _ = run(ctx, qkv, [L])
    q32 = qkv.astype(np.float32)
    for h in (0, 5, 11):
        q = q32[:, h * D:(h + 1) * D]
        k = q32[:, H + h * D:H + (h + 1) * D]
        v = q32[:, 2 * H + h * D:2 * H + (h + 1) * D]
        ref = oracle.attention_head(q, k, v)
        tol = 2.0 ** -9 * np.abs(v).max() + 2.0 ** -10 * np.abs(ref) + 1e-3
        assert (np.abs(out[:, h * D:(h + 1) * D] - ref) <= tol).all()


def test_attention_growing_scores(ctx):
    """Key norms that grow along the sequence push the row max up block after
    block, by less than and by more than the softmax's lazy-rescale slack."""
    rng = np.random.default_rng(9)
    L = 512
    qkv = rng.standard_normal((L, 3 * H)).astype(np.float32)
    qkv[:, H:2 * H] *= (0.2 + np.arange(L) / 48.0)[:, None]
    qkv = qkv.astype(np.float16)
    out, _ = run(ctx, qkv, [L])
    q32 = qkv.astype(np.float32)
    for h in (0, 6, 11):
        q = q32[:, h * D:(h + 1) * D]
        k = q32[:, H + h * D:H + (h + 1) * D]
        v = q32[:, 2 * H + h * D:2 * H + (h + 1) * D]
        ref = oracle.attention_head(q, k, v)
        tol = 2.0 ** -9 * np.abs(v).max() + 2.0 ** -10 * np.abs(ref) + 1e-3
        assert (np.abs(out[:, h * D:(h + 1) * D] - ref) <= tol).all()


def test_sequences_are_independent(ctx):
    """Packing order must not change any sequence's result (bit-exact)."""
    rng = np.random.default_rng(6)
    lengths = [40, 200, 7]
    qkv = rng.standard_normal((sum(lengths), 3 * H)).astype(np.float16)
    out, cu = run(ctx, qkv, lengths)
    alone, _ = run(ctx, qkv[cu[1]:cu[2]], [200])
    assert np.array_equal(out[cu[1]:cu[2]], alone)


def test_attention_rejects_bad_lengths(ctx):
    qkv = np.zeros((600, 3 * H), np.float16)
    with pytest.raises(TzhError) as ei:
        run(ctx, qkv, [600])
    assert ei.value.code == _abi.ERR_INVALID_ARGS
    with pytest.raises(TzhError):
        run(ctx, qkv[:10], [0, 10])
