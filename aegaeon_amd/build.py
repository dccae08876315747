"""Build libaegkv.so (HIP, gfx950) in-tree with hipcc.

The library is a plain C-ABI shared object; it links against the HIP
runtime by SONAME (libamdhip64.so.7), so inside a process that has already
imported torch it binds to the runtime torch loaded.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libaegkv.so"
ARCH = os.environ.get("AEGKV_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed FP32 instructions stay disabled in every HIP build here
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libaegkv")


def build(verbose: bool = False) -> Path:
    """Compile csrc/aegkv.hip, csrc/fence.hip and csrc/plan.cpp into
    aegaeon_amd/libaegkv.so (always rebuilds)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [
        hipcc(),
        *HIPCC_FLAGS,
        f"-I{REPO_DIR / 'include'}",
        str(CSRC / "aegkv.hip"),
        str(CSRC / "fence.hip"),
        str(CSRC / "plan.cpp"),
        "-o",
        str(tmp),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
