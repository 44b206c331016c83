"""Expert -> slot table for one layer, kept in HBM and updated by HIP kernels.

Same API and state layout as the reference's ``ExpertTable``
(table.py:19-247): int64 tensors with a trailing sink element, LRU
replacement, graph-safe fixed-shape outputs. On a GPU every operation is one
launch of a single-workgroup kernel (csrc/table.hip); the host never reads a
value, so all of it can be captured in a hipGraph. A table made on the CPU
keeps its tensors in host memory and runs the same rules as sequential host
code (csrc/table_host.cpp), as the reference's device-agnostic table does on
CPU tensors (table.py:1-9).
"""

from __future__ import annotations

import torch

from vllm_expert_pager import _native as nat

# Added to the victim-selection key to push slots used in this step last
# (table.py:16).
_PROTECT = 1 << 40


class ExpertTable:
    """Expert -> slot table for one layer (LRU), on a GPU or on the CPU."""

    def __init__(self, num_experts: int, num_slots: int, device: torch.device) -> None:
        if num_slots < 1:
            raise ValueError(f"num_slots must be >= 1, got {num_slots}")
        device = torch.device(device)
        if device.type not in ("cuda", "cpu"):
            raise ValueError(f"ExpertTable runs on a GPU or the CPU; got device {device}")
        self._host = device.type == "cpu"
        self.num_experts = num_experts
        self.num_slots = num_slots
        self.device = device
        i64 = {"dtype": torch.int64, "device": device}
        self.slot_of = torch.full((num_experts + 1,), -1, **i64)
        self.expert_in = torch.full((num_slots + 1,), -1, **i64)
        self.last_used = torch.zeros((num_slots + 1,), **i64)
        self.step = torch.ones((), **i64)
        self.hits = torch.zeros((), **i64)
        self.misses = torch.zeros((), **i64)
        self.experts = torch.arange(num_experts, **i64)
        self.no_cache = torch.full((num_experts,), -1, **i64)

    def _struct(self) -> nat.XpTable:
        return nat.table_struct(self)

    def _local(self, t: torch.Tensor, what: str) -> None:
        """Refuse a tensor on another device: the kernels and the host code
        dereference its pointer directly."""
        if t.device.type != self.device.type:
            raise ValueError(f"{what} is on {t.device}; this table lives on {self.device}")

    def _call(self, name: str, *args) -> None:
        """The table operation ``name``: its host variant for a CPU table,
        else the kernel launch on torch's current stream."""
        if self._host:
            nat.call(name + "_host", *args)
        else:
            nat.call(name, *args, nat.stream())

    def need_mask(self, topk_ids: torch.Tensor) -> torch.Tensor:
        """The experts needed in this step as a bool mask (table.py:63-71)."""
        self._local(topk_ids, "topk_ids")
        ids, eb = nat.ids_arg(topk_ids)
        need = torch.empty((self.num_experts,), dtype=torch.bool, device=self.device)
        self._call("xp_need_mask", nat.ptr(ids), eb, ids.numel(), self.num_experts, need.data_ptr())
        return need

    def acquire(self, topk_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Assign a slot to every needed expert; returns ``(expert_map, slot, todo)`` (table.py:75-128).

        Requires ``topk_ids.numel() <= num_slots``.
        """
        self._local(topk_ids, "topk_ids")
        ids, eb = nat.ids_arg(topk_ids)
        K = ids.numel()
        E = self.num_experts
        expert_map = torch.empty((E,), dtype=torch.int64, device=self.device)
        slot = torch.empty((E,), dtype=torch.int64, device=self.device)
        todo = torch.empty((K,), dtype=torch.int64, device=self.device)
        st = self._struct()
        self._call(
            "xp_table_acquire", nat.ptr(ids), eb, K, nat.ctypes.byref(st), expert_map.data_ptr(), None,
            slot.data_ptr(), todo.data_ptr() if K else None,
        )
        return expert_map, slot, todo

    def pack(self, mask: torch.Tensor) -> torch.Tensor:
        """The experts set in ``mask`` packed from the front, padded with -1 (table.py:132-138)."""
        self._local(mask, "mask")
        m = mask.to(torch.bool).contiguous()
        out = torch.empty((self.num_experts,), dtype=torch.int64, device=self.device)
        self._call("xp_pack", m.data_ptr(), self.num_experts, out.data_ptr())
        return out

    def seed(self, vram: "ExpertTable", topk_ids: torch.Tensor, need: torch.Tensor) -> None:
        """Seed this RAM-tier table from a prefill's routing (table.py:140-171).

        Acquires the max(R - S, 1) most referenced experts (ties: lower
        expert id), then the VRAM tier's readable experts; hits and misses are
        not counted.
        """
        for t, what in ((vram.slot_of, "vram table"), (topk_ids, "topk_ids"), (need, "need")):
            self._local(t, what)
        ids, eb = nat.ids_arg(topk_ids)
        n = need.to(torch.bool).contiguous()
        a, b = self._struct(), vram._struct()
        self._call("xp_table_seed", nat.ctypes.byref(a), nat.ctypes.byref(b), nat.ptr(ids), eb, ids.numel(),
                   n.data_ptr())

    def plan_chunks(
        self,
        before: torch.Tensor,
        need: torch.Tensor,
        cached_row: torch.Tensor,
        rows: int,
        ram_base: int,
        working_base: int,
    ) -> tuple[torch.Tensor, ...]:
        """Arrange a working-slab step's experts into chunks of ``rows`` (table.py:173-247).

        Returns ``(dst_row, src_row, maps, todo, ssd, late)``.
        """
        for t, what in ((before, "before"), (need, "need"), (cached_row, "cached_row")):
            self._local(t, what)
        E, W = self.num_experts, rows
        N = -(-E // W) + 1
        i64 = {"dtype": torch.int64, "device": self.device}
        dst_row = torch.empty((E,), **i64)
        src_row = torch.empty((E,), **i64)
        maps = torch.empty((N, E), **i64)
        todo = torch.empty((N * W,), **i64)
        ssd = torch.empty((N * W,), **i64)
        late = torch.empty((N * W,), **i64)
        bf = before.to(torch.int64).contiguous()
        nd = need.to(torch.bool).contiguous()
        cr = cached_row.to(torch.int64).contiguous()
        st = self._struct()
        self._call(
            "xp_plan_chunks", nat.ctypes.byref(st), bf.data_ptr(), nd.data_ptr(), cr.data_ptr(), W, ram_base,
            working_base, dst_row.data_ptr(), src_row.data_ptr(), maps.data_ptr(), todo.data_ptr(),
            ssd.data_ptr(), late.data_ptr(),
        )
        return dst_row, src_row, maps, todo, ssd, late
