"""TEST INFRASTRUCTURE ONLY: a pytest plugin that runs a GPU test module's
whole sequence, in file order and in one process, against the CPU emulation
of libtenzor_hip (tests/cpu_emu) instead of a GPU, so that state carried
from call to call (the generated-kernel cache, the context scratch, the
planner's temporaries, the attention work queue) is exercised the way a GPU
run exercises it, under the emulation's sanitizers.

    LD_PRELOAD=<libclang_rt.asan-x86_64.so> ASAN_OPTIONS=detect_leaks=0 \\
    TZH_EMU_LIB=tests/cpu_emu/libtenzor_hip_emu_ub.so \\
    python -m pytest -p tests.cpu_emu.replay_plugin -m gpu tests/test_gpu_eval.py

Tensors the tests place on "cuda" are made host tensors (the emulated
device's memory is host memory): a module's `DEV` is set to "cpu" and
torch's CUDA queries are answered for one device.  Skip marks are removed,
so cases kept off the GPU run here too.  Nothing here runs on a GPU."""
import ctypes as C
import os
import types

import pytest
import torch

import tenzor_amd
from tenzor_amd import _abi


def pytest_configure(config):
    path = os.environ.get("TZH_EMU_LIB")
    if not path:
        raise pytest.UsageError("TZH_EMU_LIB must name the emulation library")
    tenzor_amd._lib = _abi.bind(C.CDLL(os.path.abspath(path), mode=os.RTLD_NOW | os.RTLD_GLOBAL))
    torch.cuda.is_available = lambda: True
    torch.cuda.current_device = lambda: 0
    torch.cuda.synchronize = lambda *a, **k: None
    torch.cuda.current_stream = lambda *a, **k: types.SimpleNamespace(cuda_stream=0)


def pytest_collection_modifyitems(config, items):
    for item in items:
        mod = getattr(item, "module", None)
        if mod is not None and hasattr(mod, "DEV"):
            mod.DEV = "cpu"
        item.own_markers = [m for m in item.own_markers if m.name != "skip"]
