"""Optional roctx ranges around the steps of a paged layer.

With VLLM_EXPERT_PAGER_ROCTX=1 (not a reference setting) each eager layer
call marks its acquire, gather, decode, SSD wait and expert FFN as roctx
ranges, which `rocprofv3 --marker-trace` shows beside the kernels. The
ranges are host markers: inside a captured hipGraph they mark the capture,
not the replays. Unset, `range` costs one dictionary lookup.
"""

from __future__ import annotations

import contextlib
import ctypes
import os

_ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
_lib = None
_loaded = False


def _roctx():
    global _lib, _loaded
    if _loaded:
        return _lib
    _loaded = True
    if os.environ.get("VLLM_EXPERT_PAGER_ROCTX") != "1":
        return None
    for name in ("librocprofiler-sdk-roctx.so.1", "libroctx64.so"):
        try:
            lib = ctypes.CDLL(os.path.join(_ROCM, "lib", name))
        except OSError:
            continue
        lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
        lib.roctxRangePushA.restype = ctypes.c_int
        lib.roctxRangePop.argtypes = []
        lib.roctxRangePop.restype = ctypes.c_int
        _lib = lib
        break
    else:
        raise RuntimeError("VLLM_EXPERT_PAGER_ROCTX=1 but no roctx library was found under "
                           f"{os.path.join(_ROCM, 'lib')}")
    return _lib


@contextlib.contextmanager
def range(name: str):  # noqa: A001 - the roctx term
    """A roctx range named ``name`` around the block, when enabled."""
    lib = _roctx()
    if lib is None:
        yield
        return
    lib.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        lib.roctxRangePop()
