"""The .tenzor format (io/tenzor_format.zig): the oracle's restatement
pinned by the reference's own tests and FNV-1a test vectors, then the
library's reader and converter against it, byte for byte.  CPU only."""
import numpy as np
import pytest

from oracle import tenzor_file as tf
from tenzor_amd import TzhError
from tenzor_amd.tenzor_format import TenzorFile, convertFromSafetensors, hashName


def test_reference_layout_tests():
    """tenzor_format.zig:490-510, 563-575: header 64 bytes, entry 48, hash
    equal for equal names and not for different ones, dtype byte sizes,
    numel of a [2, 3, 4] entry."""
    assert tf.HEADER.size == 64 and tf.ENTRY.size == 48
    assert hashName("conv1.weight") == hashName("conv1.weight") != hashName("conv1.bias")
    assert tf.DTYPE_SIZE[0] == 4 and tf.DTYPE_SIZE[1] == 2 and tf.DTYPE_SIZE[3] == 8
    e = tf.ENTRY.pack(0, 0, 3, 2, 3, 4, 0, 0, 0, 96)
    dims = tf.ENTRY.unpack(e)[3:8]
    assert int(np.prod(dims[:3])) == 24


def test_fnv1a_vectors():
    """Published 64-bit FNV-1a test vectors, through the oracle and the library."""
    for s, h in [(b"", 0xcbf29ce484222325), (b"a", 0xaf63dc4c8601ec8c), (b"foobar", 0x85944171f73967e8)]:
        assert tf.hash_name(s) == h and hashName(s) == h


def test_write_and_read(tmp_path):
    """tenzor_format.zig:515-561: two f32 tensors written, read back by name."""
    d1 = np.array([1, 2, 3, 4, 5, 6], np.float32)
    d2 = np.array([0.1, 0.2, 0.3], np.float32)
    blob = tf.write([(b"tensor1", 0, (2, 3), d1.tobytes()), (b"tensor2", 0, (3,), d2.tobytes())])
    assert len(blob) == 4096 + 36  # data page-aligned after header, metadata, index
    p = tmp_path / "t.tenzor"
    p.write_bytes(blob)
    f = TenzorFile.open(str(p))
    assert f.tensor_count == 2 and f.metadata_json == b"{}"
    e1 = f.getTensor("tensor1")
    assert e1[0].ndim == 2 and list(e1[0].shape)[:2] == [2, 3]
    assert np.array_equal(f.getData(np.float32, e1), d1)
    assert np.array_equal(f.getF32("tensor2"), d2)
    assert f.getTensor("missing") is None
    meta, entries = tf.read(blob)
    assert meta == b"{}" and tf.get(entries, b"tensor2")["data"] == d2.tobytes()


def test_convert_is_byte_identical(tmp_path):
    """The library's converter against the restated writer, over every
    safetensors dtype (BOOL stored as u8) and ranks 0..3."""
    from safetensors.numpy import save_file

    rng = np.random.default_rng(0)
    tensors = {
        "a.f32": rng.standard_normal((3, 5)).astype(np.float32),
        "b.f16": rng.standard_normal(7).astype(np.float16),
        "c.i8": rng.integers(-128, 127, (4, 4, 2)).astype(np.int8),
        "d.i64": rng.integers(0, 99, 3).astype(np.int64),
        "e.u8": rng.integers(0, 255, 9).astype(np.uint8),
        "f.bool": rng.random(5) < 0.5,
        "g.f64": np.array(3.5),
        "h.u16": rng.integers(0, 9, (2, 2)).astype(np.uint16),
    }
    st = tmp_path / "m.safetensors"
    save_file(tensors, str(st))
    out = tmp_path / "m.tenzor"
    convertFromSafetensors(str(st), str(out))
    assert out.read_bytes() == tf.convert_safetensors(st.read_bytes())
    f = TenzorFile.open(str(out))
    for name, v in tensors.items():
        dt = np.uint8 if v.dtype == bool else v.dtype
        assert np.array_equal(f.getData(dt, f.getTensor(name)), v.astype(dt).ravel()), name


def test_bad_files_are_rejected(tmp_path):
    good = tf.write([(b"x", 0, (4,), np.zeros(4, np.float32).tobytes())])
    cases = {
        "magic": b"TENZOX" + good[6:],
        "version": good[:8] + (2).to_bytes(4, "little") + good[12:],
        "short": good[:40],
        "index_out_of_file": good[:16] + (1 << 20).to_bytes(4, "little") + good[20:],
        "data_out_of_file": good[:4096],
    }
    for name, blob in cases.items():
        p = tmp_path / f"{name}.tenzor"
        p.write_bytes(blob)
        with pytest.raises(TzhError):
            TenzorFile.open(str(p))
    with pytest.raises(TzhError):
        TenzorFile.open(str(tmp_path / "absent.tenzor"))
