"""Copy expert rows into the slab and request SSD reads from the host (replaces gather.py's Triton kernels).

``gather_rows`` copies the rows and scales of the experts in ``todo`` with a
fixed number of persistent workgroups that keep a bounded number of 16-byte
loads in flight over the host link (csrc/gather.hip). Sources are the RAM
tier (pinned host memory read directly by the GPU) or the cache slab (raw);
which experts to copy is passed as device index tensors, so the launches can
be captured in a hipGraph. The fetch functions are the device half of the
host request ring (store.py).

Semantics and argument order follow the reference (gather.py:314-439).
"""

from __future__ import annotations

import ctypes

import torch

from vllm_expert_pager import _native as nat


class DeviceRows:
    """A (rows, row_bytes) block of pinned host memory, addressed from the GPU.

    Stands where the reference passes a device view of the pinned RAM tier
    (store.py:430-432): ``shape`` is ``(rows, words)`` of int32 like the
    ``as_rows`` views, ``device_ptr`` the device-visible address.
    """

    def __init__(self, host_tensor: torch.Tensor, device_ptr: int | None = None) -> None:
        if host_tensor.dim() != 2 or not host_tensor.is_contiguous():
            raise ValueError("RAM-tier rows must be a contiguous 2-D tensor")
        self.host = host_tensor
        self.device_ptr = device_ptr if device_ptr is not None else nat.device_pointer(host_tensor.data_ptr())
        self.rows = host_tensor.shape[0]
        self.row_bytes = host_tensor.shape[1] * host_tensor.element_size()
        self.shape = (self.rows, self.row_bytes // 4)


def as_rows(t: torch.Tensor) -> torch.Tensor:
    """View a tensor whose leading axis is the expert axis as ``(E, W)`` int32 (gather.py:314-325)."""
    if not t.is_contiguous():
        raise ValueError("expert weights must be contiguous")
    row_bytes = t[0].numel() * t.element_size()
    if row_bytes % 4:
        raise ValueError(f"row size {row_bytes} B is not a multiple of 4")
    return t.view(torch.int32).reshape(t.shape[0], -1)


def _rows(x) -> tuple[int, int, int]:
    """(device pointer, rows, bytes per row) of a 2-D row block."""
    if isinstance(x, DeviceRows):
        return x.device_ptr, x.rows, x.row_bytes
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("row blocks must be contiguous 2-D tensors")
    if x.device.type == "cpu":
        if not x.is_pinned():
            raise ValueError("host rows must be pinned")
        p = nat.device_pointer(x.data_ptr())
    else:
        p = x.data_ptr()
    return p, x.shape[0], x.shape[1] * x.element_size()


def _index(t: torch.Tensor, what: str) -> torch.Tensor:
    nat.require_device(t, what)
    if t.dtype != torch.int64 or not t.is_contiguous():
        t = t.to(torch.int64).contiguous()
    return t


def gather_rows(
    todo: torch.Tensor,
    dst_row: torch.Tensor,
    cache_row: torch.Tensor,
    src_row: torch.Tensor,
    base: int,
    src: list,
    cache: list[torch.Tensor],
    dst: list[torch.Tensor],
    stg: list[torch.Tensor] | None,
    scale: list[torch.Tensor],
    scale_dst: list[torch.Tensor],
    fetch: tuple[torch.Tensor, int, object] | None = None,
    cached_only: bool = False,
) -> None:
    """Copy the rows and scales of the experts in ``todo`` (gather.py:328-393).

    Lists are per name (w13, w2), each an int32 row view (``as_rows``) or,
    for ``src``, a ``DeviceRows``/pinned tensor of the RAM tier. Experts with
    ``cache_row[e] >= 0`` are copied raw from ``cache`` to ``dst[dst_row[e]]``;
    the others from RAM-tier row ``src_row[e] + base`` to staging row j
    (compressed, ``stg`` given) or to ``dst[dst_row[e]]`` (raw). Scales go to
    ``scale_dst[dst_row[e]]``. With ``fetch=(ssd_todo, layer, store)`` the
    same launch publishes ``ssd_todo`` to the host and waits for it while
    copying the experts of ``todo`` that are not in ``ssd_todo``. With
    ``cached_only`` (``stg`` given, for its pitch) only the experts with
    ``cache_row[e] >= 0`` are copied: the launch gets zero staging rows, so
    the RAM-tier experts are skipped, for ``decode_rows_from_ram`` to expand.
    """
    todo = _index(todo, "todo")
    dst_row = _index(dst_row, "dst_row")
    cache_row = _index(cache_row, "cache_row")
    src_row = _index(src_row, "src_row")
    K = todo.shape[0]
    E = dst_row.shape[0]
    n = len(dst)
    W = [d.shape[1] * d.element_size() for d in dst]
    srcs = [_rows(s) for s in src]
    P = [s[2] for s in srcs]
    compress = stg is not None
    if cached_only and not compress:
        raise ValueError("cached_only needs stg (its rows give the tier's pitch)")
    if compress:
        if tuple(P) != tuple(s.shape[1] * s.element_size() for s in stg):
            raise ValueError("staging rows must have the RAM tier's pitch")
    elif tuple(P) != tuple(W):
        raise ValueError("uncompressed RAM rows must have the slab's row size")
    for i in range(n):
        if scale[i].shape[0] < E:
            raise ValueError(f"scale[{i}] has {scale[i].shape[0]} rows, fewer than the {E} experts")
        if scale_dst[i].shape[0] < dst[i].shape[0]:
            raise ValueError(f"scale_dst[{i}] has fewer rows than dst[{i}]")
    names = (nat.XpGatherName * n)()
    for i in range(n):
        sp, srows, spitch = srcs[i]
        names[i] = nat.XpGatherName(
            sp, spitch, srows,
            cache[i].data_ptr(), cache[i].shape[0],
            dst[i].data_ptr(), dst[i].shape[0], W[i],
            stg[i].data_ptr() if compress else None, stg[i].shape[0] if compress and not cached_only else 0,
            scale[i].data_ptr(), scale_dst[i].data_ptr(), scale[i].shape[1] * scale[i].element_size(),
        )
    ring = None
    ssd_ptr = None
    layer = 0
    if fetch is not None:
        ssd, layer, store = fetch
        ssd = _index(ssd, "ssd_todo")
        if ssd.shape[0] != K:
            raise ValueError(f"ssd_todo has {ssd.shape[0]} entries, todo has {K}")
        ring = store.ring_struct()
        ssd_ptr = ssd.data_ptr()
    nat.call(
        "xp_gather_rows", todo.data_ptr(), K, E, dst_row.data_ptr(), cache_row.data_ptr(), src_row.data_ptr(),
        int(base), names, n, ssd_ptr, int(layer), ctypes.byref(ring) if ring is not None else None, nat.stream(),
    )


def fetch_rows(todo: torch.Tensor, row: torch.Tensor, base: int, layer: int, store) -> None:
    """Ask the host to read the experts in ``todo`` from SSD and wait (gather.py:396-407)."""
    todo = _index(todo, "todo")
    row = _index(row, "row")
    ring = store.ring_struct()
    nat.call("xp_fetch_rows", todo.data_ptr(), todo.shape[0], row.shape[0], row.data_ptr(), int(base),
             int(layer), ctypes.byref(ring), nat.stream())


def fetch_publish_rows(todo: torch.Tensor, row: torch.Tensor, base: int, layer: int, store,
                       ticket: torch.Tensor) -> None:
    """Publish the request of ``fetch_rows`` without waiting (gather.py:410-431)."""
    todo = _index(todo, "todo")
    row = _index(row, "row")
    ring = store.ring_struct()
    nat.call("xp_fetch_publish_rows", todo.data_ptr(), todo.shape[0], row.shape[0], row.data_ptr(), int(base),
             int(layer), ctypes.byref(ring), ticket.data_ptr(), nat.stream())


def fetch_wait_rows(todo: torch.Tensor, store, ticket: torch.Tensor) -> None:
    """Wait for done to reach the seq in ``ticket`` (gather.py:434-439)."""
    todo = _index(todo, "todo")
    ring = store.ring_struct()
    nat.call("xp_fetch_wait_rows", todo.data_ptr(), todo.shape[0], ctypes.byref(ring), ticket.data_ptr(),
             nat.stream())
