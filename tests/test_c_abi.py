"""libaegkv from C: tests/c_abi/abi_check links the library and the HIP
runtime with no Python or torch in the process (the boundary a C or C++
runtime binds). The CPU test checks the program loads the library and reads
its ABI version; the GPU test runs its swap-out, swap-in, copy_blocks and
rejection checks against plain host loops."""

import subprocess
import sys
from pathlib import Path

import pytest

C_ABI = Path(__file__).resolve().parent / "c_abi"


@pytest.fixture(scope="module")
def abi_check(aegkv_lib):
    binary = C_ABI / "abi_check"
    if not binary.exists():
        import importlib.util

        spec = importlib.util.spec_from_file_location("aegkv_c_abi_build", C_ABI / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return binary


def test_c_program_loads_the_library(abi_check, aegkv_lib):
    res = subprocess.run([str(abi_check), "--version"], capture_output=True, text=True,
                         timeout=60)
    assert res.returncode == 0, res.stderr
    assert res.stdout.strip() == f"aegkv ABI {aegkv_lib.aegkv_abi_version()}"


@pytest.mark.gpu
def test_c_program_moves_blocks_bit_exact(gpu, abi_check):
    print("running tests/c_abi/abi_check", file=sys.stderr, flush=True)
    res = subprocess.run([str(abi_check)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().splitlines()[-1] == "c-abi ok"
    assert "rejected as expected" in res.stdout
