"""GPU parity of the int8 Arctic-embed-xs forward against the oracle
(arctic.zig:543-1013 restated) and the committed golden embeddings.

Bar: final L2-normalised embeddings within 1e-3
max-abs and cosine >= 0.9999 of the reference path; token ids / packing /
int8 codes bit-exact.  The default f32 activations (the reference's
arithmetic) are held to a bar a hundred times tighter: 1e-5 max-abs on
the embeddings, 1e-4 on the hidden states after any number of layers."""
import contextlib
import os

import numpy as np
import pytest
import torch

import oracle
from tenzor_amd import TzhError, _abi, check, lib, synth
from tenzor_amd.arctic import ModelWeights, forward, forwardBatch
from tests.conftest import GOLDEN, cosine

pytestmark = pytest.mark.gpu
CFG = synth.Config()
# A sequence's embedding in two batch compositions (alone, in another order):
# the same to f32 rounding.  The fused feed-forward kernel splits its last
# round of 64-token panels over idle CUs and adds the parts' sums in another
# order than a whole panel's, so which tokens land there changes the
# rounding (about 3e-8 on these unit-norm embeddings).  A given batch is
# deterministic, bit for bit.
COMPOSITION_TOL = 1e-6


@pytest.fixture(scope="module")
def weights():
    w32 = synth.make_arctic_f32(1234, CFG, ln_random=True)
    return synth.quantize(w32)


@pytest.fixture(scope="module")
def model(ctx, weights):
    m = ModelWeights.fromHost(ctx, weights, CFG)
    yield m
    m.deinit()


@pytest.fixture(scope="module")
def host(weights):
    return synth.HostWeights(weights, CFG)


def gpu_embed(model, ids, lengths, packed=False):
    lengths = np.asarray(lengths, np.int32)
    if packed:
        flat, _ = synth.packed(ids, lengths)
        d_ids = torch.from_numpy(flat.view(np.int32)).cuda()
    else:
        d_ids = torch.from_numpy(np.ascontiguousarray(ids).view(np.int32)).cuda()
    out = torch.empty((len(lengths), CFG.hidden_size), device="cuda")
    forwardBatch(out, d_ids, lengths, model)
    return out.cpu().numpy()


def gpu_hidden(model, ids, lengths, n_layers):
    lengths = np.asarray(lengths, np.int32)
    d_ids = torch.from_numpy(np.ascontiguousarray(ids).view(np.int32)).cuda()
    out = torch.empty((int(lengths.sum()), CFG.hidden_size), device="cuda")
    check(lib().tzh_arctic_hidden(model.handle, out.data_ptr(), d_ids.data_ptr(), lengths.ctypes.data,
                                  len(lengths), ids.shape[1], n_layers))
    return out.cpu().numpy()


def assert_embedding_parity(got, ref, max_abs=1e-5):
    """max_abs: 1e-5 for the f32 forward, the north star's 1e-3 for f16."""
    assert got.shape == ref.shape
    for i in range(ref.shape[0]):
        err = np.abs(got[i] - ref[i]).max()
        cs = cosine(got[i], ref[i])
        assert err <= max_abs and cs >= 0.9999, (i, float(err), cs)


@contextlib.contextmanager
def precision(model, dtype):
    model.set_precision(dtype)
    try:
        yield
    finally:
        model.set_precision("float32")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
@pytest.mark.parametrize("n_layers", [0, 1, 3, 6])
def test_hidden_states_layerwise(model, host, n_layers, dtype):
    ids, lengths = synth.make_batch(21, 3, seq_len=96, min_len=5)
    with precision(model, dtype):
        assert model.precision == dtype
        got = gpu_hidden(model, ids, lengths, n_layers)
    off = 0
    for b, L in enumerate(lengths):
        ref = oracle.arctic_hidden(host, ids[b, :L], n_layers)
        err = np.abs(got[off:off + L] - ref)
        if dtype == "float32":
            # f32 activations: f32-rounding-level differences only
            assert err.max() < 1e-4 and np.sqrt((err ** 2).mean()) < 1e-5, (n_layers, b, float(err.max()))
        else:
            # f16 storage between kernels: ~2^-11 relative per rounding
            assert err.max() < 2e-2 and np.sqrt((err ** 2).mean()) < 3e-3, (n_layers, b, float(err.max()))
        off += L


def test_f16_forward_within_north_star(model, host):
    """The opt-in f16 activation path still meets the north star's bar."""
    ids, lengths = synth.make_batch(24, 8, seq_len=256)
    with precision(model, "float16"):
        got = gpu_embed(model, ids, lengths)
    ref = np.stack([oracle.arctic_forward(host, ids[b, :lengths[b]]) for b in range(8)])
    assert_embedding_parity(got, ref, max_abs=1e-3)


def test_forward_batch_edge_lengths(model, host):
    lengths = np.array([1, 2, 17, 64, 65, 200, 512], np.int32)
    ids, _ = synth.make_batch(22, len(lengths), seq_len=512)
    for b, L in enumerate(lengths):
        ids[b, L:] = 0
    got = gpu_embed(model, ids, lengths)
    ref = np.stack([oracle.arctic_forward(host, ids[b, :L]) for b, L in enumerate(lengths)])
    assert_embedding_parity(got, ref)
    np.testing.assert_allclose(np.linalg.norm(got, axis=1), 1.0, atol=1e-5)


def test_config4_batch32_seq128(model, host):
    ids, lengths = synth.make_batch(4, 32, seq_len=128, fixed=True)
    got = gpu_embed(model, ids, lengths)
    flat, offs = synth.packed(ids, lengths)
    ref = oracle.arctic_forward_batch(host, flat, offs, lengths, nthreads=16)
    assert_embedding_parity(got, ref)


def test_config5_headline_batch(model, host):
    """B=256, lengths U[16,512]: full batch on the GPU, oracle on a sample
    (incl. the longest and shortest), invariants on all of it."""
    ids, lengths = synth.make_batch(5, 256, seq_len=512)
    got = gpu_embed(model, ids, lengths)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(np.linalg.norm(got, axis=1), 1.0, atol=1e-5)
    sample = sorted({int(np.argmax(lengths)), int(np.argmin(lengths)), 0, 77, 128, 255})
    ref = np.stack([oracle.arctic_forward(host, ids[b, :lengths[b]]) for b in sample])
    assert_embedding_parity(got[sample], ref)
    # packed input == padded input, bit for bit
    assert np.array_equal(gpu_embed(model, ids, lengths, packed=True), got)
    # batch order invariance: within f32 rounding (another order puts other
    # tokens in the split last round of the fused feed-forward kernel, whose
    # parts' sums are added in another order)
    perm = np.random.default_rng(0).permutation(256)
    got_p = gpu_embed(model, ids[perm], lengths[perm])
    assert float(np.abs(got_p - got[perm]).max()) < COMPOSITION_TOL


def test_single_sequence_forward(model, host):
    ids, lengths = synth.make_batch(23, 1, seq_len=128)
    L = int(lengths[0])
    d_ids = torch.from_numpy(ids[0, :L].view(np.int32)).cuda()
    out = torch.empty(CFG.hidden_size, device="cuda")
    forward(out, d_ids, model)
    assert_embedding_parity(out.cpu().numpy()[None], oracle.arctic_forward(host, ids[0, :L])[None])


def test_host_slice_entry_points(model, host):
    """The reference's host arguments (arctic.zig:874-879, 902-907): host id
    slices of different lengths in, host embeddings out; equal bit for bit
    to the device-resident batch entry."""
    from tenzor_amd.arctic import forwardBatchHost

    ids, lengths = synth.make_batch(25, 5, seq_len=200)
    seqs = [ids[b, :lengths[b]].copy() for b in range(5)]
    out = np.zeros((5, CFG.hidden_size), np.float32)
    forwardBatchHost(out, seqs, model)
    assert np.array_equal(out, gpu_embed(model, ids, lengths))
    one = np.zeros(CFG.hidden_size, np.float32)
    check(lib().tzh_arctic_forward_host(model.handle, one.ctypes.data, seqs[2].ctypes.data, len(seqs[2])))
    assert float(np.abs(one - out[2]).max()) < COMPOSITION_TOL  # alone: another batch composition
    ref = np.stack([oracle.arctic_forward(host, s) for s in seqs[:2]])
    assert_embedding_parity(out[:2], ref)
    with pytest.raises(TzhError):
        forwardBatchHost(np.zeros((1, CFG.hidden_size), np.float32), [np.zeros(0, np.uint32)], model)


def test_golden_embeddings(model):
    """Committed fixture: embeddings computed in the container by the oracle
    and cross-checked there against HuggingFace BertModel (float64)."""
    g = np.load(os.path.join(GOLDEN, "arctic_small.npz"))
    w = synth.quantize(synth.make_arctic_f32(int(g["seed"]), CFG, ln_random=True))
    ctx = model.ctx
    m = ModelWeights.fromHost(ctx, w, CFG)
    try:
        got = gpu_embed(m, g["ids"], g["lengths"])
    finally:
        m.deinit()
    assert_embedding_parity(got, g["expected"])


def test_quantized_embedding_tables(ctx, host):
    """quantize_arctic_xs also quantizes word/position embeddings (F9);
    the q8 gather path (arctic.zig:490-537) must match the oracle."""
    w = synth.quantize(synth.make_arctic_f32(77, CFG, ln_random=True), embeddings=True)
    assert w["embeddings.word_embeddings.weight"].dtype == np.int8
    m = ModelWeights.fromHost(ctx, w, CFG)
    hw = synth.HostWeights(w, CFG)
    try:
        ids, lengths = synth.make_batch(24, 4, seq_len=64, min_len=3)
        got = gpu_embed(m, ids, lengths)
        ref = np.stack([oracle.arctic_forward(hw, ids[b, :L]) for b, L in enumerate(lengths)])
        assert_embedding_parity(got, ref)
        h0 = gpu_hidden(m, ids, lengths, 0)
        r0 = oracle.arctic_hidden(hw, ids[0, :lengths[0]], 0)
        assert np.abs(h0[:lengths[0]] - r0).max() < 1e-4
    finally:
        m.deinit()


def test_out_of_range_ids_are_clamped_and_counted(ctx, weights):
    m = ModelWeights.fromHost(ctx, weights, CFG)
    try:
        ids = np.zeros((2, 8), np.uint32)
        ids[:, 0] = 101
        ids[1, 3] = 40000
        before = m.bad_id_count()
        out = gpu_embed(m, ids, [8, 8])
        assert np.isfinite(out).all()
        assert m.bad_id_count() == before + 1
    finally:
        m.deinit()


def test_length_validation(model):
    ids = np.zeros((1, 600), np.uint32)
    with pytest.raises(TzhError) as ei:
        gpu_embed(model, ids, [600])
    assert ei.value.code == _abi.ERR_INVALID_ARGS
    with pytest.raises(TzhError):
        gpu_embed(model, ids[:, :10], [0])


def test_safetensors_loader_variants(ctx, weights, tmp_path):
    """fromSafeTensors (arctic.zig:113-166): with/without "bert." prefix and
    LayerNorm gamma/beta names give the same model; errors map to the
    reference's error names."""
    from safetensors.numpy import save_file

    ids, lengths = synth.make_batch(25, 3, seq_len=40, min_len=4)
    m0 = ModelWeights.fromHost(ctx, weights, CFG)
    base = gpu_embed(m0, ids, lengths)
    m0.deinit()

    def to_file(d, name):
        p = str(tmp_path / name)
        save_file({k: (v.view(np.float16) if k.endswith(".scale") else v) for k, v in d.items()}, p)
        return p

    bert = {"bert." + k: v for k, v in weights.items()}
    gb = {k.replace("LayerNorm.weight", "LayerNorm.gamma").replace("LayerNorm.bias", "LayerNorm.beta"): v
          for k, v in weights.items()}
    for d, name in ((bert, "bert.safetensors"), (gb, "gb.safetensors")):
        m = ModelWeights.fromSafeTensors(ctx, to_file(d, name), CFG)
        try:
            assert np.array_equal(gpu_embed(m, ids, lengths), base)
        finally:
            m.deinit()

    missing = dict(weights)
    del missing["encoder.layer.3.output.dense.bias"]
    with pytest.raises(TzhError) as ei:
        ModelWeights.fromSafeTensors(ctx, to_file(missing, "missing.safetensors"), CFG)
    assert ei.value.code == _abi.ERR_MISSING_WEIGHT

    wrong = dict(weights)
    wrong["encoder.layer.0.attention.self.query.bias"] = wrong["encoder.layer.0.attention.self.query.bias"].astype(np.float16)
    with pytest.raises(TzhError) as ei:
        ModelWeights.fromSafeTensors(ctx, to_file(wrong, "wrong.safetensors"), CFG)
    assert ei.value.code == _abi.ERR_WRONG_DTYPE

    noscale = dict(weights)
    del noscale["encoder.layer.2.intermediate.dense.weight.scale"]
    with pytest.raises(TzhError) as ei:
        ModelWeights.fromSafeTensors(ctx, to_file(noscale, "noscale.safetensors"), CFG)
    assert ei.value.code == _abi.ERR_MISSING_WEIGHT

    unsup = dict(weights)
    unsup["encoder.layer.1.output.dense.weight"] = unsup["encoder.layer.1.output.dense.weight"].astype(np.int16)
    with pytest.raises(TzhError) as ei:
        ModelWeights.fromSafeTensors(ctx, to_file(unsup, "unsup.safetensors"), CFG)
    assert ei.value.code == _abi.ERR_UNSUPPORTED_DTYPE


def test_f32_model_config1(ctx):
    """Config 1: the f32 model (MatWeight.f32 linears and tables), batch 1 x
    seq 128, and a ragged batch, against the oracle's f32 forward (pinned
    against HuggingFace in float64).  The linears stay f32 and run on the
    f32 GEMM (exact products, f32 sums), so the bar is the f32 one."""
    w = synth.make_arctic_f32(3, CFG, ln_random=True)
    m = ModelWeights.fromHost(ctx, w, CFG)
    try:
        hw = synth.HostWeights(w, CFG)
        assert m.precision == "float32"
        m.set_precision("float16")  # f32 weights run in f32 whatever is set
        assert m.precision == "float32"
        ids, lengths = synth.make_batch(31, 1, seq_len=128, fixed=True)
        got = gpu_embed(m, ids, lengths)
        assert_embedding_parity(got, oracle.arctic_forward(hw, ids[0, :128])[None], max_abs=1e-5)
        ids, lengths = synth.make_batch(32, 6, seq_len=300)
        got = gpu_embed(m, ids, lengths)
        ref = np.stack([oracle.arctic_forward(hw, ids[b, :lengths[b]]) for b in range(6)])
        assert_embedding_parity(got, ref, max_abs=1e-5)
        hid = gpu_hidden(m, ids, lengths, 6)
        off = 0
        for b, L in enumerate(lengths):
            assert np.abs(hid[off:off + L] - oracle.arctic_hidden(hw, ids[b, :L], 6)).max() < 1e-4
            off += L
    finally:
        m.deinit()




def mixed_weights(w, f32_names):
    """The quantized weights of `w` with the linears named in f32_names kept
    f32: a model that mixes MatWeight.f32 and MatWeight.q8 linears, which the
    reference loads matrix by matrix (arctic.zig:55-58, 258-287)."""
    out = synth.quantize(w)
    for name in f32_names:
        out[name] = w[name]
        del out[name + ".scale"]
    return out


ATT = ["attention.self.query.weight", "attention.self.key.weight", "attention.self.value.weight",
       "attention.output.dense.weight"]
FFN = ["intermediate.dense.weight", "output.dense.weight"]


@pytest.mark.parametrize("f32_names", [
    [f"encoder.layer.{l}.{n}" for l in (0, 2, 4) for n in ATT] + [f"encoder.layer.{l}.{n}" for l in (1, 3, 5) for n in FFN],
    [f"encoder.layer.{l}.{n}" for l in (1, 3) for n in FFN],
    ["encoder.layer.2.attention.self.key.weight"]])
def test_mixed_f32_int8_models(ctx, f32_names):
    """Each linear on its own format's GEMM (f32 weights on the f32 GEMM,
    int8 on the int8 GEMM), the forward in f32 whatever precision is set;
    a QKV that mixes dtypes runs as one f32 matrix."""
    w = mixed_weights(synth.make_arctic_f32(51, CFG, ln_random=True), f32_names)
    m = ModelWeights.fromHost(ctx, w, CFG)
    try:
        hw = synth.HostWeights(w, CFG)
        m.set_precision("float16")
        assert m.precision == "float32"
        ids, lengths = synth.make_batch(52, 7, seq_len=200, min_len=1)
        got = gpu_embed(m, ids, lengths)
        ref = np.stack([oracle.arctic_forward(hw, ids[b, :L]) for b, L in enumerate(lengths)])
        assert_embedding_parity(got, ref, max_abs=1e-5)
        hid = gpu_hidden(m, ids, lengths, 6)
        assert np.abs(hid[:lengths[0]] - oracle.arctic_hidden(hw, ids[0, :lengths[0]], 6)).max() < 1e-4
    finally:
        m.deinit()


def test_activations_past_the_f16_range(ctx):
    """The embedding LayerNorm's gamma (2e4) puts layer 0's QKV input near
    1e5, past f16: the weights' bound marks the model row-scaled and its
    int8 GEMMs scale each row into the split's range, so the forward stays
    the f32 one.  With full-size QKV weights the attention's inputs could
    pass its split's range too, and the forward refuses (TooLarge) instead
    of returning NaN."""
    w = synth.make_arctic_f32(61, CFG, ln_random=True)
    w["embeddings.LayerNorm.weight"] = (w["embeddings.LayerNorm.weight"] * 2e4).astype(np.float32)
    small = dict(w)
    for n in ATT[:3]:
        small[f"encoder.layer.0.{n}"] = (w[f"encoder.layer.0.{n}"] * 1e-4).astype(np.float32)
    q = synth.quantize(small)
    m = ModelWeights.fromHost(ctx, q, CFG)
    try:
        hw = synth.HostWeights(q, CFG)
        ids, lengths = synth.make_batch(62, 5, seq_len=128, min_len=4)
        h0 = gpu_hidden(m, ids, lengths, 0)
        assert np.abs(h0).max() > 65504  # the QKV input really is past f16
        got = gpu_embed(m, ids, lengths)
        ref = np.stack([oracle.arctic_forward(hw, ids[b, :L]) for b, L in enumerate(lengths)])
        assert np.isfinite(got).all()
        assert_embedding_parity(got, ref, max_abs=1e-5)
    finally:
        m.deinit()
    m = ModelWeights.fromHost(ctx, synth.quantize(w), CFG)
    try:
        with pytest.raises(TzhError) as ei:
            gpu_embed(m, ids, lengths)
        assert ei.value.code == _abi.ERR_TOO_LARGE
    finally:
        m.deinit()
