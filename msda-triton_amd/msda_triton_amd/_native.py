"""ctypes binding of libmsda_hip.so, the C ABI declared in include/msda_hip.h.

The library is loaded lazily, on the first call that needs it, so that the
package imports on machines without ROCm or without a built library (the
reference likewise imports without its GPU backend and raises at call time,
src/msda_triton/ops.py:11-16,170-171).  There is no fallback: every device
computation goes through this library or raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libmsda_hip.so"
LIB_PATH = Path(os.environ.get("MSDA_HIP_LIB", Path(__file__).resolve().parent / LIB_NAME))

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

MSDA_OK = 0

# Every symbol the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
SIGNATURES = {
    "msda_forward": (_INT, [_P, _P, _P, _P, _P, _P] + [_I64] * 7 + [_INT, _P]),
    "msda_backward": (_INT, [_P] * 10 + [_I64] * 7 + [_INT, _P]),
    "msda_fused_forward": (_INT, [_P] * 8 + [_I64] * 7 + [_INT, _INT, _P]),
    "msda_fused_backward": (_INT, [_P] * 14 + [_I64] * 7 + [_INT, _INT, _P]),
    "msda_deterministic_workspace_bytes": (_I64, [_I64] * 7 + [_INT]),
    "msda_backward_deterministic": (_INT, [_P] * 10 + [_I64] * 7 + [_INT, _P]),
    "msda_fused_backward_deterministic": (_INT, [_P] * 14 + [_I64] * 7 + [_INT, _INT, _P]),
    "msda_projection_forward": (_INT, [_P] * 8 + [_I64] * 4 + [_INT, _P]),
    "msda_projection_workspace_bytes": (_I64, [_I64] * 3 + [_INT]),
    "msda_projection_backward": (_INT, [_P] * 12 + [_I64] * 4 + [_INT, _P]),
    "msda_projection_backward_noalloc": (_INT, [_P] * 11 + [_I64] * 4 + [_INT, _P]),
    "msda_error_string": (ctypes.c_char_p, [_INT]),
    "msda_abi_version": (_INT, []),
    "msda_backward_plan": (_INT, [_I64] * 7 + [_INT, _INT]),
    "msda_set_launch_override": (_INT, [_INT, _INT]),
}

# msda_set_launch_override knobs (MSDA_KNOB_* in the header).
KNOBS = {
    "FWD_TS": 0, "FWD_CB": 1, "BWD_TS": 2, "BWD_CB": 3, "BWD_PRIV": 4, "BWD_OWNER": 5,
    "BWD_BIN": 6, "OWN_MIX": 7, "OWN_ROWS": 8, "OWN_ENTRIES": 9,
}
OVERRIDE_AUTO = -(2 ** 31)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryError(RuntimeError):
    """libmsda_hip.so is missing or failed to load."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"the HIP path requires {LIB_PATH}, which is not built; run "
                    "`python msda-triton_amd/build.py` (or __graft_entry__.build())"
                )
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:  # e.g. no ROCm runtime on this machine
                raise NativeLibraryError(f"failed to load {LIB_PATH}: {exc}") from exc
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


@contextlib.contextmanager
def launch_overrides(**knobs: int):
    """Set launch-shape / path overrides (``BWD_OWNER=0``, ``FWD_TS=4``, ...)
    for the calls inside the block; every knob named is reset to the
    automatic choice on exit.  Process-wide: for sweeps and tests."""
    lib = load()
    codes = []
    try:
        for name, value in knobs.items():
            code = KNOBS[name]
            codes.append(code)
            check(lib.msda_set_launch_override(code, int(value)), "msda_set_launch_override")
        yield
    finally:
        for code in codes:
            lib.msda_set_launch_override(code, OVERRIDE_AUTO)


def check(rc: int, what: str) -> None:
    if rc != MSDA_OK:
        msg = load().msda_error_string(rc).decode()
        raise RuntimeError(f"{what} failed with code {rc}: {msg}")
