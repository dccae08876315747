"""Build recipe for the oracle's C restatement (gcc, output next to it).

Test infrastructure only. The reference's own native code for this path
(ops/swap.cu) needs nvcc and a CUDA build of torch, so there is no
oracle/_ref build of it here.
"""

from __future__ import annotations

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from oracle.oracle import build  # noqa: E402

if __name__ == "__main__":
    print(build())
