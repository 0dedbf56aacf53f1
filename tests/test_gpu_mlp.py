"""GPU parity of the encoder's feed-forward block (feedForward,
arctic.zig:760-811) run as one kernel (mlp.hip), against the oracle and
against the GEMM pair it replaces.

Bar: the reference's f32 arithmetic.  On LayerNorm-scale inputs the
fused block is within 2e-5 max-abs of the oracle's f32 feedForward (its
int8 sums, GELU and two-pass LayerNorm in the reference's order) and of
the GEMM pair at the forward's full size (67 590 tokens); every token's
row depends on that token alone (bit-exact under a permutation of the
tokens among whole panels, and among split ones)."""
import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import TzhError, synth
from tenzor_amd.arctic import ModelWeights, feedForward, forwardBatch

pytestmark = pytest.mark.gpu
CFG = synth.Config(num_hidden_layers=2)
TOL = 2e-5


@pytest.fixture(scope="module")
def weights():
    return synth.quantize(synth.make_arctic_f32(4242, CFG, ln_random=True))


@pytest.fixture(scope="module")
def model(ctx, weights):
    m = ModelWeights.fromHost(ctx, weights, CFG)
    yield m
    m.set_ffn_fusion(True)
    m.deinit()


def ffn_oracle(w, layer, x):
    """LayerNorm(x + (gelu(x W1^T s1 + b1) W2^T s2 + b2)) (arctic.zig:771-803)."""
    p = f"encoder.layer.{layer}."
    h = oracle.matmul_w8a32(x, w[p + "intermediate.dense.weight"], w[p + "intermediate.dense.weight.scale"],
                            w[p + "intermediate.dense.bias"])
    y = oracle.matmul_w8a32(oracle.gelu(h), w[p + "output.dense.weight"], w[p + "output.dense.weight.scale"],
                            w[p + "output.dense.bias"])
    return oracle.layernorm(x + y, w[p + "output.LayerNorm.weight"], w[p + "output.LayerNorm.bias"],
                            CFG.layer_norm_eps)


def gpu_ffn(model, layer, x, fused=True):
    model.set_ffn_fusion(fused)
    try:
        d_x = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x)).cuda()
        d_y = torch.full_like(d_x, float("nan"))
        feedForward(d_y, d_x, model, layer, d_x.shape[0])
        torch.cuda.synchronize()
        return d_y
    finally:
        model.set_ffn_fusion(True)


def inputs(seed, t):
    x = np.random.default_rng(seed).standard_normal((t, CFG.hidden_size), dtype=np.float32)
    if t > 2:
        x[t // 2] = 0.0  # a zero row
    return x


@pytest.mark.parametrize("t,layer", [(1, 0), (15, 1), (16, 0), (17, 1), (64, 0), (65, 1), (1000, 0), (4097, 1)])
def test_fused_feed_forward_matches_oracle(model, weights, t, layer):
    print(f"feed-forward t={t} layer={layer}", flush=True)
    x = inputs(t, t)
    got = gpu_ffn(model, layer, x).cpu().numpy()
    err = float(np.abs(got - ffn_oracle(weights, layer, x)).max())
    assert np.isfinite(got).all() and err < TOL, err


def test_fused_vs_gemm_pair_full_size(model, weights):
    """The forward's size (256 sequences, 67 590 real tokens: 1057 panels,
    the last partial; four whole rounds on 256 CUs, the last 33 panels split
    in six parts): fused against the GEMM pair over every row, and sampled
    rows (from the first, middle and last, split panels) against the
    oracle."""
    t = 67590
    print(f"feed-forward full size t={t}", flush=True)
    x = torch.from_numpy(inputs(7, t)).cuda()
    fused = gpu_ffn(model, 1, x, fused=True)
    pair = gpu_ffn(model, 1, x, fused=False)
    diff = float((fused - pair).abs().max())
    assert bool(torch.isfinite(fused).all()) and diff < TOL, diff
    rows = np.r_[0:40, 33770:33800, t - 70:t]
    ref = ffn_oracle(weights, 1, x[rows].cpu().numpy())
    err = float(np.abs(fused[rows].cpu().numpy() - ref).max())
    assert err < TOL, err


@pytest.mark.parametrize("t", [3001, 16384])
def test_rows_independent_of_placement(model, t):
    """A token's output is the same bits wherever it lands (panel, wave,
    lane) among whole panels (16 384 tokens: 256 panels, one round) and
    among the parts of split ones (3001 tokens: all 47 panels split in four
    parts).  Whole and split panels add the chunks' sums in different
    orders, so a token alone (split in 24 parts) is within the bound."""
    print(f"feed-forward permutation t={t}", flush=True)
    x = torch.from_numpy(inputs(11, t)).cuda()
    perm = torch.from_numpy(np.random.default_rng(12).permutation(t)).cuda()
    a = gpu_ffn(model, 0, x)
    b = gpu_ffn(model, 0, x[perm].contiguous())
    assert bool(torch.equal(a[perm], b))
    c = gpu_ffn(model, 0, x[:1].contiguous())  # alone in its panel
    assert float((a[:1] - c).abs().max()) < TOL


def test_feed_forward_edges(model):
    print("feed-forward edges", flush=True)
    x = torch.ones((32, CFG.hidden_size), device="cuda")
    y = torch.full_like(x, 7.0)
    feedForward(y, x, model, 0, 0)  # no tokens: nothing written
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    with pytest.raises(TzhError):
        feedForward(x, x, model, 0, 32)  # in place: the kernel needs distinct buffers
    with pytest.raises(TzhError):
        feedForward(y, x, model, CFG.num_hidden_layers, 32)


def test_forward_with_and_without_fusion(model):
    """The whole forward: embeddings with the fused block within 1e-5 of the
    GEMM pair's (both f32 arithmetic)."""
    print("forward fused vs GEMM pair", flush=True)
    ids, lengths = synth.make_batch(31, 6, seq_len=128, min_len=3)
    d_ids = torch.from_numpy(np.ascontiguousarray(ids).view(np.int32)).cuda()
    outs = []
    for fused in (True, False):
        model.set_ffn_fusion(fused)
        out = torch.empty((len(lengths), CFG.hidden_size), device="cuda")
        forwardBatch(out, d_ids, lengths, model)
        outs.append(out.cpu().numpy())
    model.set_ffn_fusion(True)
    assert float(np.abs(outs[0] - outs[1]).max()) < 1e-5
