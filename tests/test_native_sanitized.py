"""Host code of libaegkv under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): the native planner (aegaeon_amd/csrc/plan.cpp) driven with
random block tables by tests/native/plan_fuzz.cpp."""

import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_transfer_entries_under_sanitizers(tmp_path):
    exe = tmp_path / "plan_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__HIP_PLATFORM_AMD__", f"-I{REPO / 'include'}", "-I/opt/rocm/include",
           f"-I{REPO / 'aegaeon_amd' / 'csrc'}",
           str(REPO / "tests" / "native" / "plan_fuzz.cpp"),
           str(REPO / "aegaeon_amd" / "csrc" / "plan.cpp"), "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe), "20000"], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "clean" in run.stdout


def _asan_runtime():
    for root in sorted(Path("/opt/rocm/lib/llvm/lib/clang").glob("*"), reverse=True):
        lib = root / "lib" / "linux" / "libclang_rt.asan-x86_64.so"
        if lib.exists():
            return lib
    return None


@pytest.mark.skipif(_asan_runtime() is None or shutil.which("hipcc") is None
                    and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc or the clang AddressSanitizer runtime is missing")
def test_library_host_code_under_asan(tmp_path):
    """libaegkv built with AddressSanitizer on its host code only (the GPU
    code is unchanged), then the CPU tests that call into it: every
    argument-validation path of the C ABI and the native planner."""
    import os
    import sys

    from aegaeon_amd import build as lib_build

    so = tmp_path / "libaegkv_asan.so"
    csrc = REPO / "aegaeon_amd" / "csrc"
    cmd = [lib_build.hipcc(), *lib_build.HIPCC_FLAGS, "-O1", "-g",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
           "-shared-libasan", f"-I{REPO / 'include'}", str(csrc / "aegkv.hip"),
           str(csrc / "fence.hip"), str(csrc / "plan.cpp"),
           "-o", str(so)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr
    env = dict(os.environ, AEGKV_LIBRARY=str(so), LD_PRELOAD=str(_asan_runtime()),
               ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:halt_on_error=1")
    run = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                          "tests/test_host.py", "tests/test_planner.py"],
                         capture_output=True, text=True, timeout=900, env=env, cwd=str(REPO))
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]
    assert "ERROR: AddressSanitizer" not in run.stderr
