"""GPU parity of the embed command's text paths (main.zig:718-1021):
tokenizer -> chunks -> one batched forward -> chunk mean + L2.

Bars: chunk plans, token ids and the pooling bit-exact (the pooling against
the oracle's f32 restatement applied to the same chunk embeddings); the
final embeddings against the full oracle (its tokenizer, its forward, its
pooling) within the forward's bar, 1e-3 max-abs and cosine >= 0.9999."""
import numpy as np
import pytest
import torch

import oracle
from oracle import wordpiece as wp
from tenzor_amd import TzhError, synth
from tenzor_amd.arctic import ModelWeights, embedDocuments, embedTexts, forwardBatch
from tenzor_amd.tokenizer import Tokenizer
from tests.conftest import cosine

pytestmark = pytest.mark.gpu
CFG = synth.Config()


@pytest.fixture(scope="module")
def weights():
    return synth.quantize(synth.make_arctic_f32(4321, CFG, ln_random=True))


@pytest.fixture(scope="module")
def host(weights):
    return synth.HostWeights(weights, CFG)


@pytest.fixture(scope="module")
def model(ctx, weights):
    m = ModelWeights.fromHost(ctx, weights, CFG)
    yield m
    m.deinit()


@pytest.fixture(scope="module")
def vocab():
    data, words = synth.make_vocab(11)
    tok = Tokenizer.init()
    tok.loadVocabFromBytes(data)
    return tok, wp.load_vocab_bytes(data), words


def forward_ids(model, seqs):
    """The library's batched forward on given id lists (packed)."""
    flat = np.array([i for s in seqs for i in s], np.uint32)
    out = torch.empty((len(seqs), CFG.hidden_size), device="cuda")
    forwardBatch(out, torch.from_numpy(flat.view(np.int32)).cuda(), [len(s) for s in seqs], model)
    return out.cpu().numpy()


def embed_docs(model, tok, docs):
    out = torch.empty((len(docs), CFG.hidden_size), device="cuda")
    counts = embedDocuments(out, docs, tok, model)
    return out.cpu().numpy(), counts


def test_documents_pool_bit_exact(model, vocab):
    tok, v, words = vocab
    # pieces: 0, 1 chunk short, exactly 510, 921 (2 chunks), 1381 (3), ~4700
    # (10, with a dropped tail), and mixed text with [UNK]s and punctuation
    docs = [b"", synth.make_text(1, words, 37, plain=True), synth.make_text(2, words, 510, plain=True),
            synth.make_text(3, words, 921, plain=True), synth.make_text(4, words, 1381, plain=True),
            synth.make_text(5, words, 4700, plain=True), synth.make_text(6, words, 1500)]
    got, counts = embed_docs(model, tok, docs)
    chunks = [wp.chunks(wp.encode_raw(v, d)) for d in docs]
    assert counts.tolist() == [len(c) for c in chunks]
    assert counts.tolist()[:6] == [1, 1, 1, 2, 3, 10]
    emb = forward_ids(model, [ch for c in chunks for ch in c])
    off = 0
    for d, c in enumerate(chunks):
        ref = wp.chunk_mean_l2(emb[off:off + len(c)])
        assert np.array_equal(got[d].view(np.uint32), ref.view(np.uint32)), d
        off += len(c)


def test_documents_batch_equals_single(model, vocab):
    tok, _, words = vocab
    docs = [synth.make_text(20 + i, words, n) for i, n in enumerate((5, 1000, 300, 2500))]
    together, _ = embed_docs(model, tok, docs)
    for d, doc in enumerate(docs):
        alone, _ = embed_docs(model, tok, [doc])
        # another batch composition: the same to f32 rounding (the fused
        # feed-forward kernel's split last round adds its parts' sums in
        # another order than a whole panel's)
        assert float(np.abs(alone[0] - together[d]).max()) < 1e-6, d


def test_document_end_to_end_vs_oracle(model, host, vocab):
    """Two chunks through the oracle's own forward (C restatement of
    arctic.zig) and pooling."""
    tok, v, words = vocab
    doc = synth.make_text(31, words, 940, plain=True)
    got, counts = embed_docs(model, tok, [doc])
    chunks = wp.chunks(wp.encode_raw(v, doc))
    assert counts[0] == len(chunks) == 2
    flat = np.array([i for ch in chunks for i in ch], np.uint32)
    lens = np.array([len(ch) for ch in chunks], np.int32)
    emb = oracle.arctic_forward_batch(host, flat, np.concatenate([[0], np.cumsum(lens)[:-1]]), lens, nthreads=2)
    ref = wp.chunk_mean_l2(emb)
    err = np.abs(got[0] - ref).max()
    assert err <= 1e-3 and cosine(got[0], ref) >= 0.9999, float(err)


def test_single_chunk_overrun_is_an_error(model, vocab):
    """511..920 pieces: the reference copies them into one 512-id chunk
    buffer (main.zig:903-906); here it is an error, and 921 is fine."""
    tok, _, words = vocab
    for n in (511, 700, 920):
        with pytest.raises(TzhError):
            embed_docs(model, tok, [synth.make_text(n, words, n, plain=True)])
    _, counts = embed_docs(model, tok, [synth.make_text(921, words, 921, plain=True)])
    assert counts[0] == 2


def test_texts_path(model, host, vocab):
    tok, v, words = vocab
    texts = [b"", b"HELLO, world!", synth.make_text(41, words, 100), synth.make_text(42, words, 700),
             synth.make_text(43, words, 509, plain=True)]
    out = torch.empty((len(texts), CFG.hidden_size), device="cuda")
    n_tokens = embedTexts(out, texts, tok, model)
    enc = [wp.encode(v, t, 512) for t in texts]
    assert n_tokens.tolist() == [len(e) for e in enc]
    assert n_tokens[3] == 512 and n_tokens[4] == 511
    got = out.cpu().numpy()
    assert np.array_equal(got, forward_ids(model, enc))
    for i in (1, 2):
        ref = oracle.arctic_forward(host, np.array(enc[i], np.uint32))
        assert np.abs(got[i] - ref).max() <= 1e-3 and cosine(got[i], ref) >= 0.9999, i
