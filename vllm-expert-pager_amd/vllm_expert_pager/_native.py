"""ctypes binding of libxp.so, the gfx950 HIP kernels and host C++ of this package.

The library is built in-tree by ``csrc/build.py`` (``__graft_entry__.build()``)
and loaded from next to this file. There is no fallback: if it is missing or
a call fails, an exception says so.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

# The library next to this file; VLLM_EXPERT_PAGER_LIBRARY names another
# build (the sanitizer builds of the host code that the CPU tests load).
LIB_PATH = os.environ.get("VLLM_EXPERT_PAGER_LIBRARY") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libxp.so")

XP_OK, XP_E_ARG, XP_E_PITCH, XP_E_SHAPE, XP_E_HIP, XP_E_LIMIT = range(6)

c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p


class XpTable(ctypes.Structure):
    _fields_ = [
        ("slot_of", c_ptr),
        ("expert_in", c_ptr),
        ("last_used", c_ptr),
        ("step", c_ptr),
        ("hits", c_ptr),
        ("misses", c_ptr),
        ("num_experts", c_i64),
        ("num_slots", c_i64),
    ]


class XpGatherName(ctypes.Structure):
    _fields_ = [
        ("src", c_ptr),
        ("src_pitch", c_i64),
        ("src_rows", c_i64),
        ("cache", c_ptr),
        ("cache_rows", c_i64),
        ("dst", c_ptr),
        ("dst_rows", c_i64),
        ("row_bytes", c_i64),
        ("stg", c_ptr),
        ("stg_rows", c_i64),
        ("scale", c_ptr),
        ("scale_dst", c_ptr),
        ("scale_bytes", c_i64),
    ]


class XpRing(ctypes.Structure):
    _fields_ = [
        ("req", c_ptr),
        ("done", c_ptr),
        ("seq", c_ptr),
        ("block", c_i64),
        ("ring", c_i64),
    ]


class XpDecodeName(ctypes.Structure):
    _fields_ = [
        ("stg", c_ptr),
        ("pitch", c_i64),
        ("stg_rows", c_i64),
        ("dst", c_ptr),
        ("dst_rows", c_i64),
        ("row_bytes", c_i64),
    ]


class XpDecodeScale(ctypes.Structure):
    _fields_ = [
        ("scale", c_ptr),
        ("scale_dst", c_ptr),
        ("scale_bytes", c_i64),
        ("scale_rows", c_i64),
        ("scale_dst_rows", c_i64),
    ]


_P = c_ptr
_I = ctypes.c_int
_L = c_i64
_SIGNATURES = {
    "xp_last_error": (ctypes.c_char_p, []),
    "xp_version": (ctypes.c_char_p, []),
    "xp_acquire_pair": (_I, [_P, _I, _L, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "xp_table_acquire": (_I, [_P, _I, _L, _P, _P, _P, _P, _P, _P]),
    "xp_need_mask": (_I, [_P, _I, _L, _L, _P, _P]),
    "xp_pack": (_I, [_P, _L, _P, _P]),
    "xp_table_seed": (_I, [_P, _P, _P, _I, _L, _P, _P]),
    "xp_plan_chunks": (_I, [_P, _P, _P, _P, _L, _L, _L, _P, _P, _P, _P, _P, _P, _P]),
    "xp_table_acquire_host": (_I, [_P, _I, _L, _P, _P, _P, _P, _P]),
    "xp_need_mask_host": (_I, [_P, _I, _L, _L, _P]),
    "xp_pack_host": (_I, [_P, _L, _P]),
    "xp_table_seed_host": (_I, [_P, _P, _P, _I, _L, _P]),
    "xp_plan_chunks_host": (_I, [_P, _P, _P, _P, _L, _L, _L, _P, _P, _P, _P, _P, _P]),
    "xp_gather_rows": (_I, [_P, _L, _L, _P, _P, _P, _L, _P, _I, _P, _L, _P, _P]),
    "xp_gather_set_blocks": (_I, [_I]),
    "xp_fetch_rows": (_I, [_P, _L, _L, _P, _L, _L, _P, _P]),
    "xp_fetch_publish_rows": (_I, [_P, _L, _L, _P, _L, _L, _P, _P, _P]),
    "xp_fetch_wait_rows": (_I, [_P, _L, _P, _P, _P]),
    "xp_fetch_set_timing": (_I, [_L, _L]),
    "xp_decode_rows": (_I, [_P, _L, _L, _P, _P, _P, _P, _I, _P, _L, _P]),
    "xp_decode_rows_from_ram": (_I, [_P, _L, _L, _P, _P, _P, _L, _P, _P, _I, _P, _P, _L, _P]),
    "xp_encode_row": (_I, [_P, _L, _L, _P, _L, _P, _P]),
    "xp_code_build": (_I, [_P, _P, _P, _P]),
    "xp_host_alloc": (_I, [_P, _L, _I]),
    "xp_host_free": (_I, [_P]),
    "xp_host_device_pointer": (_I, [_P, _P]),
    "ssd_start": (_P, [_I, _P, _P, ctypes.c_long, ctypes.c_long, ctypes.c_long, ctypes.c_long,
                       ctypes.c_long, ctypes.c_long, _I, _P, _P, _I]),
    "ssd_stop": (None, [_P]),
    "ssd_stats": (None, [_P, _P, _P, _P, _P]),
    "ssd_error": (ctypes.c_char_p, [_P]),
    "ssd_test_delay": (None, [_P, ctypes.c_double]),
    "xp_ssd_phase_stats": (None, [_P, _P, _P, _P, _P, _P, _P, _P]),
    "xp_ssd_test_bounce": (None, [_P]),
    "xp_quant_tokens": (_I, [_P, _L, _L, _P, _P, _P]),
    "xp_moe_max_tiles": (_L, [_L, _L]),
    "xp_moe_route": (_I, [_P, _I, _L, _L, _P, _L, _L, _P, _P, _P, _P]),
    "xp_moe_quant_route": (_I, [_P, _L, _L, _P, _P, _P, _I, _L, _P, _L, _L, _P, _P, _P, _P]),
    "xp_moe_workspace_bytes": (_L, [_L, _L]),
    "xp_moe_experts": (_I, [_P, _P, _L, _L, _P, _L, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _L, _P, _I, _P]),
    "xp_ssd_read_probe": (_I, [_I, _L, _P, _L, _I, _I, _P]),
    "xp_moe_decode_experts": (_I, [_P, _L, _L, _P, _I, _L, _P, _P, _P, _L, _L, _P, _P, _P, _P, _L, _P, _L, _P, _I,
                                   _P]),
    "xp_moe_experts_noalloc": (_I, [_P, _P, _L, _L, _P, _L, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _I, _P]),
    "xp_encode_rows": (_I, [_P, _L, _L, _L, _L, _P, _L, _P, _L, _P, _P]),
    "xp_moe_topk_sum": (_I, [_P, _L, _L, _L, _P, _I, _L, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class NativeError(RuntimeError):
    """A libxp call failed in the HIP runtime or hit a kernel limit."""


def lib() -> ctypes.CDLL:
    """The loaded library. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build the HIP extension first "
                    "(python vllm-expert-pager_amd/csrc/build.py)"
                )
            so = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(so, name, None)
                if fn is None:
                    continue
                fn.restype = res
                fn.argtypes = args
            _lib = so
    return _lib


def check(rc: int, what: str) -> None:
    if rc == XP_OK:
        return
    msg = (lib().xp_last_error() or b"").decode(errors="replace")
    if rc in (XP_E_ARG, XP_E_PITCH, XP_E_SHAPE):
        raise ValueError(msg or f"{what} failed ({rc})")
    raise NativeError(f"{what}: {msg} (status {rc})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def stream() -> int:
    """Raw hipStream_t of torch's current stream."""
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} must be a GPU tensor (got {t.device})")


def device_pointer(host_ptr: int) -> int:
    """Device-visible address of pinned host memory."""
    out = ctypes.c_void_p()
    call("xp_host_device_pointer", ctypes.byref(out), ctypes.c_void_p(host_ptr))
    return out.value or 0


def table_struct(t) -> XpTable:
    return XpTable(
        t.slot_of.data_ptr(),
        t.expert_in.data_ptr(),
        t.last_used.data_ptr(),
        t.step.data_ptr(),
        t.hits.data_ptr(),
        t.misses.data_ptr(),
        t.num_experts,
        t.num_slots,
    )


def ids_arg(topk_ids: torch.Tensor) -> tuple[torch.Tensor, int]:
    """A contiguous int32 or int64 id tensor and its element size."""
    ids = topk_ids.reshape(-1)
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    if not ids.is_contiguous():
        ids = ids.contiguous()
    return ids, ids.element_size()
