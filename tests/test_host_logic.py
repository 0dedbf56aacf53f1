"""CPU: the C-ABI library loads and exports its header, host-side logic
(expression tapes, quantizer tool, safetensors writer, synthetic inputs)
behaves as the reference's, and compute entry points fail cleanly with no
GPU present."""
import ctypes as C
import json
import os
import re
import struct

import numpy as np
import pytest
import torch

import oracle
import tenzor_amd
from tenzor_amd import _abi, synth
from tenzor_amd.expr import BinaryExpr, ReduceExpr, ScalarExpr, Tensor, UnaryExpr, broadcast_shape, reduce_shape, to_tape
from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "tenzor_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tzh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = tenzor_amd.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_abi.PROTOTYPES), set(names) ^ set(_abi.PROTOTYPES)
    assert lib.tzh_abi_version() == 2


def test_init_without_gpu_fails_cleanly():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = tenzor_amd.lib().tzh_init(0, None, C.byref(h))
    assert rc == _abi.ERR_DEVICE and h.value is None
    assert b"HIP device" in tenzor_amd.lib().tzh_last_error()


class _HostT:
    def __init__(self, shape, dtype=torch.float32):
        self.shape, self.dtype = tuple(shape), dtype

    def is_contiguous(self):
        return True


def test_tape_is_post_order_with_leaf_sharing():
    a, b, c = Tensor(_HostT((4, 8))), Tensor(_HostT((8,))), Tensor(_HostT((4, 8)))
    e = BinaryExpr("add", a, b).mul(c).exp()  # config-2 chain (expr.zig:395, 461, 408)
    nodes, leaves = to_tape(e)
    kinds = [n.kind for n in nodes]
    assert kinds == [_abi.NODE_TENSOR, _abi.NODE_TENSOR, _abi.NODE_BINARY, _abi.NODE_TENSOR, _abi.NODE_BINARY,
                     _abi.NODE_UNARY]
    assert [nodes[i].op for i in (2, 4, 5)] == [_abi.OP["add"], _abi.OP["mul"], _abi.OP["exp"]]
    assert nodes[2].lhs == 0 and nodes[2].rhs == 1 and nodes[4].lhs == 2 and nodes[4].rhs == 3 and nodes[5].lhs == 4
    assert [leaves.index(x) for x in (a, b, c)] == [0, 1, 2]
    nodes, leaves = to_tape(a.add(a))
    assert len(leaves) == 1 and nodes[0].leaf == nodes[1].leaf == 0


def test_shape_algebra_matches_reference():
    assert broadcast_shape((4, 1, 6), (3, 1)) == (4, 3, 6)
    assert broadcast_shape((), (2, 3)) == (2, 3)
    with pytest.raises(ValueError):
        broadcast_shape((2, 3), (4,))
    # shape.zig:588-610 ReduceShape tests
    assert reduce_shape((2, 3, 4), (1,), False) == (2, 4)
    assert reduce_shape((2, 3, 4), (1,), True) == (2, 1, 4)
    assert reduce_shape((2, 3, 4), (), False) == ()
    assert reduce_shape((2, 3, 4), (), True) == (1, 1, 1)
    with pytest.raises(TypeError):
        BinaryExpr("add", Tensor(_HostT((3,))), Tensor(_HostT((3,), torch.float64)))
    with pytest.raises(TypeError):
        UnaryExpr("add", Tensor(_HostT((3,))))
    s = Tensor(_HostT((3,))).mul(2)
    assert isinstance(s.rhs, ScalarExpr) and s.rhs.dtype == "float32" and s.rhs.value == 2.0


def test_host_quantizer_bit_exact_with_oracle():
    rng = np.random.default_rng(0)
    for shape, scale in (((384, 384), 0.02), ((1536, 384), 0.02), ((7, 1536), 3.0), ((5, 9), 1e-3)):
        w = (rng.standard_normal(shape) * scale).astype(np.float32)
        w[0] = 0
        q, s = tenzor_amd.quantize_rows_host(w)
        qo, so = oracle.quantize_rows(w)
        assert np.array_equal(q, qo) and np.array_equal(s, so)


def _read_header(path):
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        return f.read(n), n


def test_quantize_tool_matches_reference_contract(tmp_path):
    """quantize_arctic_xs.zig:42-145: the 36 encoder linears and the word and
    position embeddings become I8 + F16 `.scale`; everything else is copied."""
    from safetensors.numpy import load_file, save_file

    cfg = synth.Config(num_hidden_layers=2)
    w = synth.make_arctic_f32(3, cfg)
    src, dst = str(tmp_path / "in.safetensors"), str(tmp_path / "out.safetensors")
    save_file(w, src)
    n = tenzor_amd.quantize_safetensors(src, dst)
    assert n == 2 * 6 + 2  # linears + word/position embeddings (token_type has 768 < 4096 elements)
    out = load_file(dst)
    for name, arr in w.items():
        if synth.should_quantize(name, arr):
            assert out[name].dtype == np.int8 and out[name + ".scale"].dtype == np.float16
            qo, so = oracle.quantize_rows(arr)
            assert np.array_equal(out[name], qo) and np.array_equal(out[name + ".scale"].view(np.uint16), so)
        else:
            assert out[name].dtype == arr.dtype and np.array_equal(out[name], arr)
    header, size = _read_header(dst)
    assert size % 8 == 0 and header.rstrip(b" ") == header[: len(header.rstrip(b" "))]
    meta = json.loads(header)
    assert b", " not in header.rstrip(b" ") and b": " not in header  # compact writer (safetensors.zig:350-409)
    ends = sorted(v["data_offsets"] for v in meta.values())
    assert ends[0][0] == 0 and all(ends[i][1] == ends[i + 1][0] for i in range(len(ends) - 1))


def test_quantize_tool_errors(tmp_path):
    with pytest.raises(tenzor_amd.TzhError) as ei:
        tenzor_amd.quantize_safetensors(str(tmp_path / "missing.safetensors"), str(tmp_path / "o.safetensors"))
    assert ei.value.code == _abi.ERR_IO
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(tenzor_amd.TzhError) as ei:
        tenzor_amd.quantize_safetensors(str(bad), str(tmp_path / "o.safetensors"))
    assert ei.value.code == _abi.ERR_INVALID_FORMAT


def test_synthetic_batches_follow_the_config():
    ids, lengths = synth.make_batch(5, 256, seq_len=512)
    assert lengths.min() >= 16 and lengths.max() <= 512
    assert (ids[:, 0] == 101).all()
    for b in range(0, 256, 37):
        L = lengths[b]
        assert (ids[b, 1:L] >= 1000).all() and (ids[b, 1:L] <= 30521).all() and (ids[b, L:] == 0).all()
    flat, offs = synth.packed(ids, lengths)
    assert flat.size == lengths.sum() and offs[-1] + lengths[-1] == flat.size
    w = synth.quantize(synth.make_arctic_f32(1, synth.Config(num_hidden_layers=1)))
    assert sum(1 for k, v in w.items() if v.dtype == np.int8) == 6


def test_build_rejects_scratch_spills():
    # the build refuses kernels that spill to scratch (their vector memory
    # traffic would not be in the pipelined GEMM's vmcnt plan)
    from tenzor_amd.build import scratch_spills
    remarks = "\n".join([
        "a.hip:1:1: remark: Function Name: k_ok [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark: Function Name: k_spill [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 40 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert scratch_spills(remarks) == [("k_spill", 40)]
