"""The .tenzor file format: the mirror of io/tenzor_format.zig over the C ABI
(tenzor_file.cpp in the library).

    f = TenzorFile.open("model.tenzor")          # tenzor_format.zig:140-197
    e = f.getTensor("tensor1")                    # tenzor_format.zig:225-227
    x = f.getData(np.float32, e)                  # tenzor_format.zig:230-235 (a view of the mapping)
    convertFromSafetensors("m.safetensors", "m.tenzor")   # tenzor_format.zig:440-484
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi, check, lib

DTYPES = [np.float32, np.float16, None, np.float64, np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16,
          np.uint32, np.uint64]  # tenzor_format.DType order; bf16 has no numpy type


def hashName(name) -> int:
    b = name.encode() if isinstance(name, str) else bytes(name)
    return int(lib().tzh_tenzor_name_hash(b, len(b)))


class TenzorFile:
    def __init__(self, handle: C.c_void_p):
        self.handle = handle

    @staticmethod
    def open(path: str) -> "TenzorFile":
        h = C.c_void_p()
        check(lib().tzh_tenzor_open(str(path).encode(), C.byref(h)))
        return TenzorFile(h)

    def close(self) -> None:
        if self.handle:
            lib().tzh_tenzor_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def tensor_count(self) -> int:
        n = C.c_uint32()
        check(lib().tzh_tenzor_info(self.handle, C.byref(n), None, None))
        return n.value

    @property
    def metadata_json(self) -> bytes:
        p, n = C.c_void_p(), C.c_int64()
        check(lib().tzh_tenzor_info(self.handle, None, C.byref(p), C.byref(n)))
        return C.string_at(p, n.value) if n.value else b""

    def getTensor(self, name):
        """(entry, address of its bytes), or None when no entry has the name's hash."""
        e, p = _abi.TenzorEntry(), C.c_void_p()
        rc = lib().tzh_tenzor_get(self.handle, name.encode() if isinstance(name, str) else name, C.byref(e),
                                  C.byref(p))
        if rc == -4:  # TZH_ERR_MISSING_WEIGHT
            return None
        check(rc)
        return e, p.value

    def getData(self, dtype, tensor) -> np.ndarray:
        """The tensor's bytes as a read-only array (a copy: the mapping
        lives only as long as the file)."""
        e, addr = tensor
        raw = C.string_at(addr, e.data_size) if e.data_size else b""
        return np.frombuffer(raw, dtype=dtype)

    def getF32(self, name):
        t = self.getTensor(name)
        if t is None or t[0].dtype != 0:
            return None
        return self.getData(np.float32, t)


def convertFromSafetensors(input_path: str, output_path: str) -> None:
    check(lib().tzh_tenzor_convert_safetensors(str(input_path).encode(), str(output_path).encode()))
