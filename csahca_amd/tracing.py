"""roctx ranges around the op calls, the counterpart of the reference's NVTX
ranges around its timed loop (hybrid_attention/benchmark.py:144-151) and
around each backend call of its SGLang hook
(integrations/sglang_dsv4/csahca_sglang_dsv4_patch/patch.py:285-297).

With ``CSAHCA_ROCTX=1`` in the environment when the package is imported, every
op of ``csahca_amd.native`` pushes a range named after it (``csahca.<op>``)
around its call, and ``op_range(name)`` marks a region (bench.py marks its
timed loops); ``rocprofv3 --marker-trace`` then shows them beside the kernels.
Without it the ops are the undecorated functions and ``op_range`` does
nothing, so the default path pays nothing.
"""
from __future__ import annotations

import contextlib
import ctypes
import functools
import os

ENABLED = os.environ.get("CSAHCA_ROCTX", "0") == "1"
_LIB = None
# rocprofv3's marker API first, the roctracer one as a fallback.
_CANDIDATES = ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so", "libroctx64.so.4", "libroctx64.so")


def _roctx():
    global _LIB
    if _LIB is None:
        errors = []
        for name in _CANDIDATES:
            for path in (name, os.path.join("/opt/rocm/lib", name)):
                try:
                    lib = ctypes.CDLL(path)
                except OSError as e:
                    errors.append(str(e))
                    continue
                lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
                lib.roctxRangePushA.restype = ctypes.c_int
                lib.roctxRangePop.argtypes = []
                lib.roctxRangePop.restype = ctypes.c_int
                _LIB = lib
                return _LIB
        raise RuntimeError("CSAHCA_ROCTX=1 but no roctx library loads: " + "; ".join(errors[-2:]))
    return _LIB


def push(name: str) -> int:
    """Open a roctx range (nesting depth, or a negative status)."""
    return _roctx().roctxRangePushA(name.encode())


def pop() -> int:
    """Close the innermost roctx range."""
    return _roctx().roctxRangePop()


@contextlib.contextmanager
def op_range(name: str):
    """A roctx range around the block when tracing is on; nothing otherwise."""
    if not ENABLED:
        yield
        return
    push(name)
    try:
        yield
    finally:
        pop()


def traced(fn):
    """``fn`` inside a ``csahca.<name>`` range when tracing is on at import;
    ``fn`` itself otherwise."""
    if not ENABLED:
        return fn
    label = "csahca." + fn.__name__

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        push(label)
        try:
            return fn(*args, **kwargs)
        finally:
            pop()

    return wrapper
