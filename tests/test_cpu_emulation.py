"""Every kernel of libtenzor_hip run on the CPU (tests/cpu_emu): each lane a
fiber, wave operations and MFMA in software, AddressSanitizer on every
buffer and LDS array, barrier deadlock detection, direct-to-LDS loads as
deferred writes retired only by the issuing lane's vmcnt wait.  The
scenarios are the GPU tests' (emu_checks.py) and the C++ host API test;
results are compared with the oracle.  This is how index arithmetic,
launch shapes and synchronisation are checked before anything runs on a
GPU, and it covers the GPU cases that are kept off the GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EMU = os.path.join(ROOT, "tests", "cpu_emu")
CLANG = "/opt/rocm/llvm/bin/clang++"


def _asan_runtime():
    res = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return res.stdout.strip()


@pytest.fixture(scope="module")
def emu_env():
    if not os.path.exists(CLANG):
        pytest.skip("ROCm clang not available")
    res = subprocess.run(["make", "-s", "-j8", "-C", EMU], capture_output=True, text=True, timeout=900)
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ)
    # the sanitizer runtime must come first; anything already preloaded stays
    env["LD_PRELOAD"] = " ".join(filter(None, [_asan_runtime(), os.environ.get("LD_PRELOAD")]))
    env["ASAN_OPTIONS"] = "detect_leaks=0"
    return env


GROUPS = ["eval", "attention", "gemm", "gemm_ln", "range", "models", "nodes", "gemm_fp", "mlp", "mlp_split", "arctic",
          "arctic_f16w"]
# emulated CU count per group (default 16): two CUs give the fused
# feed-forward kernel blocks of several panels at a size the emulation
# runs in about a minute (and a last round split in two); 24 CUs split
# one to three panels into 24, 12 and 8 parts; with four, the small
# forwards of group arctic split their two panels in two, not eight (each
# part repeats its panel's O-projection, which the emulation pays for)
GROUP_ENV = {"mlp": {"TZH_EMU_CUS": "2"}, "mlp_split": {"TZH_EMU_CUS": "24"}, "arctic": {"TZH_EMU_CUS": "4"}}


# test_gpu_eval.py's whole sequence in one process, in file order, with the
# generated kernels and the cases kept off the GPU (replay_plugin.py)
REPLAY = ["python", "-m", "pytest", "-p", "tests.cpu_emu.replay_plugin", "-m", "gpu", "-q", "-p", "no:cacheprovider",
          "tests/test_gpu_eval.py", "--deselect", "tests/test_gpu_eval.py::test_config2_chain_full_size"]


@pytest.fixture(scope="module")
def emu_runs(emu_env):
    """All groups started at once (each is single-threaded), so the module
    takes as long as the slowest group."""
    procs = {g: subprocess.Popen(["python", os.path.join(EMU, "emu_checks.py"), g], stdout=subprocess.PIPE,
                                 stderr=subprocess.STDOUT, text=True, env=dict(emu_env, **GROUP_ENV.get(g, {})),
                                 cwd=ROOT)
             for g in GROUPS}
    procs["replay_eval"] = subprocess.Popen(REPLAY, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                                            env=dict(emu_env, TZH_EMU_LIB=os.path.join(EMU, "libtenzor_hip_emu.so")),
                                            cwd=ROOT)
    yield procs
    for p in procs.values():
        if p.poll() is None:
            p.kill()
            p.wait()


@pytest.mark.parametrize("group", GROUPS)
def test_kernels_under_emulation(emu_runs, group):
    out, _ = emu_runs[group].communicate(timeout=1200)
    assert emu_runs[group].returncode == 0, out[-4000:]
    assert "EMU CHECKS PASSED" in out


def test_gpu_eval_sequence_replayed_under_emulation(emu_runs):
    """Every test of test_gpu_eval.py (the deep-tree case included, which
    stays off the GPU) in one process against the emulation."""
    out, _ = emu_runs["replay_eval"].communicate(timeout=1200)
    assert emu_runs["replay_eval"].returncode == 0, out[-4000:]


def test_cpp_host_api_under_emulation(emu_env, tmp_path):
    exe = str(tmp_path / "test_host_api_emu")
    asan = emu_env["LD_PRELOAD"]
    build = subprocess.run(
        ["g++", "-std=c++17", "-O1", os.path.join(ROOT, "tests", "cpp", "test_host_api.cpp"), "-o", exe,
         f"-L{EMU}", "-ltenzor_hip_emu", f"-L{os.path.join(ROOT, 'oracle')}", "-loracle", asan,
         f"-Wl,-rpath,{EMU}:{os.path.join(ROOT, 'oracle')}:{os.path.dirname(asan)}"],
        capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr[-3000:]
    res = subprocess.run([exe], capture_output=True, text=True, env=emu_env, timeout=900)
    assert res.returncode == 0, (res.stdout + res.stderr)[-4000:]
    assert "ALL PASSED" in res.stdout
