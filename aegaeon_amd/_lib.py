"""ctypes binding of libaegkv.so (declared in include/aegkv.h).

torch is imported first on purpose: torch ships its own HIP runtime with the
same SONAME (libamdhip64.so.7) as the system one, and loading torch first
makes libaegkv bind to that runtime, so torch's streams and device pointers
are valid inside the library.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede loading libaegkv, see module doc)

LIB_PATH = Path(__file__).resolve().parent / "libaegkv.so"

ABI_VERSION = 3

OK = 0
EINVAL = -1
ERANGE = -2
EDUP = -3
EEXTENT = -4
EOVERLAP = -5
ENOMEM = -6

MODE_AUTO = 0
MODE_DIRECT = 1
MODE_STAGED = 2

TUNE_SWAP_OUT_WORKGROUPS = 1
TUNE_STAGING_BYTES = 2
TUNE_AUTO_D2H = 3
TUNE_AUTO_H2D = 4
TUNE_NT_STORES = 5
TUNE_COPY_WGS_PER_CU = 6
TUNE_COPY_UNROLL = 7
TUNE_SWAP_SHAPE_AUTO = 8
TUNE_SWAP_IN_WORKGROUPS = 9
TUNE_STAGED_DMA_STREAMS = 10
TUNE_COPY_LDS_BYTES = 11
TUNE_SWAP_UNROLL = 12
TUNE_STAGED_WORKGROUPS = 13
TUNE_STAGED_OVERLAP = 14
TUNE_SWAP_OUT_WORKGROUPS_UNCACHED = 15
TUNE_COPY_LANES = 17
TUNE_COPY_ORDER = 18
HOST_UNCACHED = 1
HOST_COHERENT = 2
PROBE_READ = 1
PROBE_WRITE = 2
#: bit 62 of a fence word: the move behind it (or one before it on the same
#: stream) failed
FENCE_FAILED = 1 << 62

#: every symbol include/aegkv.h declares
EXPORTED_SYMBOLS = (
    "aegkv_abi_version",
    "aegkv_init",
    "aegkv_last_error",
    "aegkv_tune",
    "aegkv_swap",
    "aegkv_swap_blocks",
    "aegkv_copy_blocks",
    "aegkv_copy_blocks_noalloc",
    "aegkv_copy_probe",
    "aegkv_migrate_blocks",
    "aegkv_load_slices",
    "aegkv_transfer_entries",
    "aegkv_host_alloc",
    "aegkv_host_alloc_flags",
    "aegkv_host_free",
    "aegkv_host_usage",
    "aegkv_fence_signal",
    "aegkv_fence_wait",
    "aegkv_fence_publish",
    "aegkv_fence_host_wait",
    "aegkv_guard_merge",
    "aegkv_stream_create",
    "aegkv_stream_create_masked",
    "aegkv_stream_destroy",
    "aegkv_stream_release",
)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int
_I64P = ctypes.POINTER(ctypes.c_int64)
_I32P = ctypes.POINTER(ctypes.c_int32)
_U64P = ctypes.POINTER(ctypes.c_uint64)
_PP = ctypes.POINTER(ctypes.c_void_p)

_SIGNATURES = {
    "aegkv_abi_version": (_INT, []),
    "aegkv_init": (_INT, []),
    "aegkv_last_error": (ctypes.c_char_p, []),
    "aegkv_tune": (_I64, [_INT, _I64]),
    "aegkv_swap": (_INT, [_I64P, _I64P, _I64, _INT, _P, _I64, _P, _I64, _I64, _INT, _P]),
    "aegkv_swap_blocks": (
        _INT,
        [_I32, _PP, _I64P, _I64P, _U64P, _I64, _I32, _I64P, _P, _I64, _I64, _I64, _I64,
         _I64P, _I64P, _I32P, _I64P, _I64P, _INT, _INT, _P, _P],
    ),
    "aegkv_copy_blocks": (_INT, [_I32, _PP, _I64P, _I64, _I64, _I64P, _I64P, _P]),
    "aegkv_copy_blocks_noalloc": (_INT, [_I32, _PP, _I64P, _I64, _I64, _I64P, _I64P, _P]),
    "aegkv_copy_probe": (_INT, [_INT, _I32, _PP, _I64P, _I64, _I64, _I64P, _I64P, _P,
                                ctypes.c_uint32, _P]),
    "aegkv_migrate_blocks": (_INT, [_I32, _PP, _PP, _I64P, _I64, _I64, _I64, _I64P, _I64P, _P,
                                    _P]),
    "aegkv_load_slices": (_INT, [_I64, _PP, _PP, _I64P, _INT, _P]),
    "aegkv_transfer_entries": (
        _INT,
        [_I32, _I32P, _I64P, _I64P, _I64P, _I64, _I64P, _I64P, _I64P, _I64, _I64P, _I32P,
         _I64P, _I64P, _I64P, _I64P, _I64P],
    ),
    "aegkv_host_alloc": (_INT, [_PP, _I64]),
    "aegkv_host_alloc_flags": (_INT, [_PP, _I64, _INT]),
    "aegkv_host_free": (_INT, [_P]),
    "aegkv_host_usage": (_INT, [_I64P, _I64P]),
    "aegkv_fence_signal": (_INT, [_P, ctypes.c_uint64, _P, _P]),
    "aegkv_fence_wait": (_INT, [_P, ctypes.c_uint64, _I64, _P, _P]),
    "aegkv_fence_publish": (_INT, [_P, ctypes.c_uint64, _P, _P]),
    "aegkv_fence_host_wait": (_INT, [_P, ctypes.c_uint64, _I64]),
    "aegkv_guard_merge": (_INT, [_P, _P, _P]),
    "aegkv_stream_create": (_INT, [_PP]),
    "aegkv_stream_create_masked": (_INT, [_PP, ctypes.POINTER(ctypes.c_uint32), ctypes.c_int32]),
    "aegkv_stream_destroy": (_INT, [_P]),
    "aegkv_stream_release": (_INT, [_P]),
}

_lib = None
_lock = threading.Lock()


class AegkvError(RuntimeError):
    """A HIP runtime failure inside libaegkv (positive status)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libaegkv status {status}: {message}")
        self.status = status


class MoveFailedError(RuntimeError):
    """A move's completion carries the failure mark: a fence wait on its
    stream gave up, or a move it waited for had failed, so it moved nothing
    (or, for a STAGED swap-out, left its target host pages undefined). The
    reference stops the worker in that case (aegaeon/worker.py:2364-2368)."""


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libaegkv.so once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if path is None:
            path = os.environ.get("AEGKV_LIBRARY") or None   # another build, e.g. sanitized
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise ImportError(
                f"{p} is missing: build the HIP library first "
                "(python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.aegkv_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"libaegkv ABI {ver} != expected {ABI_VERSION}")
        # per-device set-up before any call can be captured into a graph
        # (a no-op without a device)
        if torch.cuda.is_available():
            rc = lib.aegkv_init()
            if rc != 0:
                raise AegkvError(rc, lib.aegkv_last_error().decode(errors="replace"))
        _lib = lib
        return lib


def check(status: int) -> None:
    """Map a libaegkv status to the reference's Python exception types.

    Invalid metadata raises ValueError (as aegaeon/worker.py:2237-2246 does),
    HIP failures raise RuntimeError (as torch does for CUDA errors).
    """
    if status == OK:
        return
    msg = load().aegkv_last_error().decode(errors="replace")
    if status < 0:
        raise ValueError(msg)
    raise AegkvError(status, msg)


def tune(key: int, value: int = -1) -> int:
    """Set a tuning knob (value >= 0) and return its previous value."""
    prev = load().aegkv_tune(key, value)
    if prev < 0:
        check(int(prev))
    return int(prev)
