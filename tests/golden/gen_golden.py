"""Writes the small golden fixtures under tests/golden/ (run in the build
container; the fixtures are committed, this script is not needed on the GPU
box).

Every fixture is computed by the C oracle AND checked here against an
independent implementation before it is written:
  - arctic_small.npz: final embeddings of a small int8 Arctic batch.  The
    int8 forward equals the f32 forward with dequantized weights
    (sum(a*q)*s == sum(a*(q*s)) exactly in real arithmetic), so it is pinned
    against HuggingFace transformers' BertModel built from a BertConfig
    (tanh GELU, eps 1e-12, absolute positions), run in float64 on the CPU
    with the same weights, CLS-pooled and L2-normalised.  No network access:
    the model is constructed from the config, never downloaded.
  - quantize_cases.npz: constructed rows (zero row, ties, clamp) with codes
    and scales; checked against numpy's float16 conversion and the closed
    form of quantize_arctic_xs.zig:94-115.
  - chain_small.npz: exp((a + b) * c) inputs/outputs; checked against numpy
    float64 within 2 f32 ulp.

Usage: python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tenzor_amd import synth  # noqa: E402


def hf_embeddings(w32: dict, cfg: synth.Config, ids, lengths):
    """CLS + L2 embeddings from transformers' BertModel in float64."""
    import torch
    from transformers import BertConfig, BertModel

    bc = BertConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, num_hidden_layers=cfg.num_hidden_layers,
                    num_attention_heads=cfg.num_attention_heads, intermediate_size=cfg.intermediate_size,
                    hidden_act="gelu_pytorch_tanh", max_position_embeddings=cfg.max_position_embeddings,
                    type_vocab_size=cfg.type_vocab_size, layer_norm_eps=cfg.layer_norm_eps,
                    hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0, attn_implementation="eager")
    model = BertModel(bc, add_pooling_layer=False).double().eval()
    sd = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in w32.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("position_ids" in m or "token_type_ids" in m for m in missing), missing
    out = []
    with torch.no_grad():
        for b, L in enumerate(lengths):
            t = torch.from_numpy(ids[b, :L].astype(np.int64))[None]
            h = model(input_ids=t, token_type_ids=torch.zeros_like(t)).last_hidden_state[0, 0]
            out.append((h / h.norm()).numpy())
    return np.stack(out)


def arctic_fixture():
    cfg = synth.Config()
    seed = 20241201
    w = synth.quantize(synth.make_arctic_f32(seed, cfg, ln_random=True))
    hw = synth.HostWeights(w, cfg)
    lengths = np.array([1, 2, 7, 33, 128], np.int32)
    ids, _ = synth.make_batch(seed + 1, len(lengths), seq_len=128)
    for b, L in enumerate(lengths):
        ids[b, 0] = 101
        ids[b, L:] = 0
    emb = np.stack([oracle.arctic_forward(hw, ids[b, :L]) for b, L in enumerate(lengths)])
    ref = hf_embeddings(synth.dequantize(w), cfg, ids, lengths)
    err = np.abs(emb - ref).max()
    print(f"arctic_small: oracle vs HF BertModel(f64) max-abs {err:.3e}")
    assert err < 1e-5, err
    np.savez_compressed(os.path.join(HERE, "arctic_small.npz"), seed=seed, ids=ids, lengths=lengths, expected=emb)


def quantize_fixture():
    rows = []
    rows.append(np.zeros(64, np.float32))                                  # zero row -> scale 1.0
    r = np.zeros(64, np.float32); r[:6] = [127, -63.5, 0.5, -0.5, 1.5, 2.5]  # ties away from zero
    rows.append(r)
    r = np.linspace(-1, 1, 64, dtype=np.float32); rows.append(r)
    r = np.full(64, 3.0e-3, np.float32); r[7] = -0.9; rows.append(r)
    rng = np.random.default_rng(3)
    for _ in range(12):
        rows.append((rng.standard_normal(64) * rng.uniform(1e-3, 10)).astype(np.float32))
    w = np.stack(rows)
    q, s = oracle.quantize_rows(w)
    # independent checks: numpy's float16 for the scale, closed form for codes
    mx = np.abs(w).max(axis=1)
    s_np = np.where(mx == 0, np.float32(1), mx / np.float32(127)).astype(np.float32).astype(np.float16)
    assert np.array_equal(s, s_np.view(np.uint16))
    x = w * (np.float32(1) / s_np.astype(np.float32))[:, None]
    q_np = np.clip(np.sign(x) * np.floor(np.abs(x) + np.float32(0.5)), -127, 127).astype(np.int8)
    assert np.array_equal(q, q_np)
    assert q[0].tolist() == [0] * 64 and s[0] == 0x3C00
    assert q[1, :6].tolist() == [127, -64, 1, -1, 2, 3]
    np.savez_compressed(os.path.join(HERE, "quantize_cases.npz"), w=w, q=q, scale=s)
    print("quantize_cases: ok")


def chain_fixture():
    rng = np.random.default_rng(8)
    a = rng.uniform(-1, 1, (64, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, 256).astype(np.float32)
    c = rng.uniform(-1, 1, (64, 256)).astype(np.float32)
    out = oracle.chain_add_mul_exp(a, b, c)
    t = (a + b) * c  # f32 add then f32 mul (numpy keeps float32)
    ref = np.exp(t.astype(np.float64)).astype(np.float32)
    from tests.conftest import ulp_diff

    assert ulp_diff(out, ref).max() <= 1
    np.savez_compressed(os.path.join(HERE, "chain_small.npz"), a=a, b=b, c=c, out=out)
    print("chain_small: ok")


if __name__ == "__main__":
    quantize_fixture()
    chain_fixture()
    arctic_fixture()
