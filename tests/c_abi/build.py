"""Build tests/c_abi/abi_check, a C caller of libaegkv (gcc, no Python or
torch at run time). It links the in-tree libaegkv.so (found through an
$ORIGIN-relative rpath, so the tree can move) and the HIP runtime."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
BIN = HERE / "abi_check"
ROCM = Path("/opt/rocm")


def build() -> Path:
    cc = shutil.which("gcc")
    if cc is None:
        raise RuntimeError("gcc not found")
    cmd = [cc, "-std=c99", "-O2", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           f"-I{REPO / 'include'}", f"-I{ROCM / 'include'}", str(HERE / "abi_check.c"),
           f"-L{REPO / 'aegaeon_amd'}", "-l:libaegkv.so", "-Wl,-rpath,$ORIGIN/../../aegaeon_amd",
           f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(BIN)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building {BIN.name} failed:\n{res.stderr}")
    return BIN


if __name__ == "__main__":
    print(build())
