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
