"""One-launch acquire of the VRAM and RAM tables (replaces acquire.py's Triton AcquirePair).

``AcquirePair(vram, ram)(topk_ids)`` updates both tables with one launch of
two workgroups (csrc/table.hip, ``xp_acquire_pair``) and writes the int32
``expert_map`` at a fixed device address, plus the per-expert slots and the
miss lists. Same contract as the reference (acquire.py:144-185). It also
writes ``pair_slot``, each id's VRAM slot in step order, which the decode
step's expert FFN reads instead of looking the ids up in ``expert_map``.
"""

from __future__ import annotations

import torch

from vllm_expert_pager import _native as nat
from vllm_expert_pager.table import ExpertTable

# Largest table the kernel accepts (slots per table).
MAX_SLOTS = 1024


class AcquirePair:
    """Update the VRAM and RAM tables in one launch. Outputs go to buffers at fixed addresses."""

    def __init__(self, vram: ExpertTable, ram: ExpertTable) -> None:
        if vram.num_experts != ram.num_experts:
            raise ValueError("both tables must have the same number of experts")
        if max(vram.num_slots, ram.num_slots) > MAX_SLOTS:
            raise ValueError(f"at most {MAX_SLOTS} slots per table")
        E, device = vram.num_experts, vram.device
        self.vram, self.ram = vram, ram
        i64 = {"dtype": torch.int64, "device": device}
        # Values of unneeded experts are never read.
        self.expert_map = torch.full((E,), -1, dtype=torch.int32, device=device)
        self.vram_slot = torch.zeros((E,), **i64)
        self.ram_slot = torch.zeros((E,), **i64)
        # Each id's VRAM slot in step order (K <= vram.num_slots ids).
        self.pair_slot = torch.full((vram.num_slots,), -1, dtype=torch.int32, device=device)
        self._vram_todo = torch.full((vram.num_slots,), -1, **i64)
        self._ram_todo = torch.full((ram.num_slots,), -1, **i64)
        self._a = vram._struct()
        self._b = ram._struct()

    def __call__(self, topk_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Update both tables; returns ``(vram_todo, ram_todo)`` of length K.

        ``expert_map``, ``vram_slot``, ``ram_slot`` and ``pair_slot[:K]`` are
        written in place. Requires ``topk_ids.numel() <= vram.num_slots``.
        """
        ids, eb = nat.ids_arg(topk_ids)
        K = ids.numel()
        nat.call(
            "xp_acquire_pair", nat.ptr(ids), eb, K, nat.ctypes.byref(self._a), nat.ctypes.byref(self._b),
            self.expert_map.data_ptr(), self.vram_slot.data_ptr(), self._vram_todo.data_ptr(),
            self.ram_slot.data_ptr(), self._ram_todo.data_ptr(), self.pair_slot.data_ptr(), nat.stream(),
        )
        return self._vram_todo[:K], self._ram_todo[:K]
