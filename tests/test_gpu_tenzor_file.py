"""The Arctic weights from a .tenzor file (io/tenzor_format.zig) on the
GPU: converted from the safetensors file, loaded from the mapping, the
embeddings are bit-identical to the safetensors-loaded model's (same
codes, same kernels); missing names keep the loader's errors."""
import numpy as np
import pytest
import torch

from oracle import tenzor_file as tf
from tenzor_amd import TzhError, synth
from tenzor_amd.arctic import ModelWeights, forwardBatch
from tenzor_amd.tenzor_format import convertFromSafetensors

pytestmark = pytest.mark.gpu
CFG = synth.Config()


def test_tenzor_model_matches_safetensors_model(ctx, tmp_path):
    from safetensors.numpy import save_file

    w = synth.quantize(synth.make_arctic_f32(99, CFG, ln_random=True))
    st = tmp_path / "model.safetensors"
    save_file({"bert." + k: (v.view(np.float16) if k.endswith(".scale") else v) for k, v in w.items()}, str(st))
    tz = tmp_path / "model.tenzor"
    convertFromSafetensors(str(st), str(tz))
    assert tz.read_bytes() == tf.convert_safetensors(st.read_bytes())
    ids, lengths = synth.make_batch(7, 6, seq_len=200, min_len=2)
    d_ids = torch.from_numpy(ids.view(np.int32)).cuda()
    outs = []
    for load in (ModelWeights.fromSafeTensors, ModelWeights.fromTenzor):
        m = load(ctx, str(st if load is ModelWeights.fromSafeTensors else tz), CFG)
        out = torch.empty((len(lengths), CFG.hidden_size), device="cuda")
        forwardBatch(out, d_ids, lengths, m)
        outs.append(out.cpu().numpy())
        m.deinit()
    assert np.array_equal(outs[0], outs[1])


def test_tenzor_missing_weight(ctx, tmp_path):
    blob = tf.write([(b"embeddings.word_embeddings.weight", 0, (2, 384), np.zeros((2, 384), np.float32).tobytes())])
    p = tmp_path / "partial.tenzor"
    p.write_bytes(blob)
    with pytest.raises(TzhError) as e:
        ModelWeights.fromTenzor(ctx, str(p), CFG)
    assert e.value.code == -4  # MissingWeight
