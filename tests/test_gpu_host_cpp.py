"""GPU parity of the C++ host API (tenzor_amd/host/tenzor.hpp): runs the
compiled tests/cpp/test_host_api, whose cases mirror the reference's
executor tests (executor.zig:605-740) and the Arctic integration flow
(arctic_integration_test.zig: a safetensors file and a token file in,
embeddings out).  The fixture written here: int8 weights from a seed
(synth.quantize), a ragged packed batch of u32 ids, and the oracle's
embeddings for it; the bar is the north star's (max-abs <= 1e-3,
cosine >= 0.9999)."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from tenzor_amd import synth

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "test_host_api")


def test_cpp_host_api(tmp_path):
    from safetensors.numpy import save_file

    assert os.path.exists(EXE), "tests/cpp/test_host_api is built by __graft_entry__.build()"
    cfg = synth.Config()
    w = synth.quantize(synth.make_arctic_f32(4321, cfg, ln_random=True))
    save_file({k: (v.view(np.float16) if k.endswith(".scale") else v) for k, v in w.items()},
              str(tmp_path / "model.safetensors"))
    ids, lengths = synth.make_batch(77, 5, seq_len=96, min_len=3)
    flat, offs = synth.packed(ids, lengths)
    flat.astype(np.uint32).tofile(tmp_path / "ids.bin")
    lengths.astype(np.int32).tofile(tmp_path / "lengths.bin")
    hw = synth.HostWeights(w, cfg)
    expected = oracle.arctic_forward_batch(hw, flat, offs, lengths, nthreads=4)
    np.asarray(expected, np.float32).tofile(tmp_path / "expected.bin")
    # the embed command's document path: a synthetic vocab.txt, a document
    # of two chunks, and the oracle's chunk ids for it
    from oracle import wordpiece as wp

    vocab, words = synth.make_vocab(12)
    (tmp_path / "vocab.txt").write_bytes(vocab)
    doc = synth.make_text(13, words, 1000)
    (tmp_path / "doc.txt").write_bytes(doc)
    chunks = wp.chunks(wp.encode_raw(wp.load_vocab_bytes(vocab), doc))
    np.array([i for c in chunks for i in c], np.uint32).tofile(tmp_path / "chunk_ids.bin")
    np.array([len(c) for c in chunks], np.int32).tofile(tmp_path / "chunk_lens.bin")
    res = subprocess.run([EXE, str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "ALL PASSED" in res.stdout
    assert "PASS arctic integration" in res.stdout
    assert "PASS embed documents" in res.stdout
