"""Oracle of ExpertTable (table.py:28-247) in numpy -- test infrastructure only.

Every function restates the reference's torch ops on int64 numpy arrays with
the same sink elements, so table state, expert_map, slot, todo and the chunk
plan can be compared bit for bit with the GPU kernels.

Pinning:
  acquire     -- pinned by LruRef (the reference's own plain-Python LRU,
                 tests/test_table.py:13-51, restated independently below), by
                 the invariants of tests/test_table.py:58-96 and its known
                 answers (121-144).
  need_mask, pack -- closed forms (tests/test_table.py:152-156).
  seed        -- set semantics pinned by tests/test_table.py:159-197 and by
                 golden vectors of the reference (tests/golden). The order
                 of torch.topk among equal counts is unspecified
                 (table.py:161); this oracle and the GPU kernel break ties by
                 lower expert id, so parity on ties at the cut is UNPINNED.
  plan_chunks -- pinned by the layout checks and the chunk-loop simulator of
                 tests/test_table.py:200-351 and by golden vectors.
"""

from __future__ import annotations

import numpy as np

PROTECT = 1 << 40  # table.py:16


class TableRef:
    """One layer's expert->slot LRU table (table.py:19-54)."""

    def __init__(self, num_experts: int, num_slots: int) -> None:
        if num_slots < 1:
            raise ValueError(f"num_slots must be >= 1, got {num_slots}")
        self.num_experts = num_experts
        self.num_slots = num_slots
        self.slot_of = np.full(num_experts + 1, -1, np.int64)
        self.expert_in = np.full(num_slots + 1, -1, np.int64)
        self.last_used = np.zeros(num_slots + 1, np.int64)
        self.step = 1
        self.hits = 0
        self.misses = 0
        self.experts = np.arange(num_experts, dtype=np.int64)

    def copy(self) -> "TableRef":
        t = TableRef(self.num_experts, self.num_slots)
        t.slot_of = self.slot_of.copy()
        t.expert_in = self.expert_in.copy()
        t.last_used = self.last_used.copy()
        t.step, t.hits, t.misses = self.step, self.hits, self.misses
        return t

    def warm(self, count: int) -> None:
        """Experts e < count sit in slot e (experts.py:256-259)."""
        self.slot_of[:count] = np.arange(count)
        self.expert_in[:count] = np.arange(count)

    # table.py:58-61
    def _ids(self, topk_ids) -> np.ndarray:
        ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
        return np.where(ids >= 0, ids, self.num_experts)

    # table.py:63-71
    def need_mask(self, topk_ids) -> np.ndarray:
        need = np.zeros(self.num_experts + 1, bool)
        need[self._ids(topk_ids)] = True
        return need[: self.num_experts]

    # table.py:75-128. `current` is a view of slot_of in the reference, so the
    # returned slot of an evicted expert reads -1 after the update (the slot
    # of every expert equals slot_of after the update). pair_slots=True gives
    # the fused kernel's output instead (acquire.py:309-341): slots loaded
    # before the update for experts that did not miss.
    def acquire(self, topk_ids, pair_slots: bool = False):
        E, S = self.num_experts, self.num_slots
        K = np.asarray(topk_ids).size
        need = self.need_mask(topk_ids)
        current = self.slot_of[:E].copy()
        hit = need & (current >= 0)
        miss = need & (current < 0)
        occupant = self.expert_in[:S]
        slot_used = (occupant >= 0) & hit[np.clip(occupant, 0, None)]
        key = self.last_used[:S] + slot_used.astype(np.int64) * PROTECT
        order = np.argsort(key, kind="stable")
        rank = np.cumsum(miss.astype(np.int64)) - 1
        victim = order[np.clip(rank, 0, S - 1)]
        evicted = self.expert_in[victim]
        self.slot_of[np.where(miss & (evicted >= 0), evicted, E)] = -1
        self.slot_of[np.where(miss, self.experts, E)] = victim
        self.expert_in[np.where(miss, victim, S)] = self.experts
        slot = np.where(miss, victim, current if pair_slots else self.slot_of[:E])
        self.last_used[np.where(need, slot, S)] = self.step
        self.step += 1
        self.hits += int(hit.sum())
        self.misses += int(miss.sum())
        expert_map = np.where(need, slot, -1)
        todo = np.full(K + 1, -1, np.int64)
        todo[np.where(miss, rank, K)] = self.experts
        return expert_map, slot, todo[:K]

    # table.py:132-138
    def pack(self, mask) -> np.ndarray:
        E = self.num_experts
        mask = np.asarray(mask, bool)
        rank = np.cumsum(mask.astype(np.int64)) - 1
        out = np.full(E + 1, -1, np.int64)
        out[np.where(mask, rank, E)] = self.experts
        return out[:E]

    # table.py:140-171, with ties of the count ranking broken by lower id
    def seed(self, vram: "TableRef", topk_ids, need) -> None:
        E, R, S = self.num_experts, self.num_slots, vram.num_slots
        hits, misses = self.hits, self.misses
        ids = self._ids(topk_ids)
        counts = np.zeros(E + 1, np.int64)
        np.add.at(counts, ids, 1)
        counts = counts[:E]
        ntop = max(R - S, 1)
        top = np.lexsort((np.arange(E), -counts))[:ntop]
        top = np.where(counts[top] > 0, top, top[:1])
        if R > S:
            self.acquire(top)
        v = vram.expert_in[:S]
        vc = np.clip(v, 0, None)
        ok = (v >= 0) & ((self.slot_of[vc] >= 0) | np.asarray(need, bool)[vc])
        self.acquire(np.where(ok, v, top[:1]))
        self.hits, self.misses = hits, misses

    # table.py:173-247
    def plan_chunks(self, before, need, cached_row, rows, ram_base, working_base):
        E, W = self.num_experts, rows
        N = -(-E // W) + 1
        before = np.asarray(before, np.int64)
        need = np.asarray(need, bool)
        cached_row = np.asarray(cached_row, np.int64)
        after = self.slot_of[:E]
        old_ok = (before >= 0) & ((after < 0) | (after == before))
        ssd = ~old_ok & (need | (before >= 0))
        first = need & ~ssd
        a = np.cumsum(first.astype(np.int64))
        b = np.cumsum(ssd.astype(np.int64))
        boundary = (a[-1] + W - 1) // W * W
        pos = np.where(first, a - 1, boundary + b - 1)
        dst_row = pos % W  # numpy % is floor mod, as torch's
        shared = working_base + (pos // W % 2) * W + dst_row
        src_row = np.where(old_ok, before + ram_base, np.where(after >= 0, after + ram_base, shared))
        chunk = np.where(need, pos // W, -1)
        maps = np.where(chunk[None, :] == np.arange(N)[:, None], dst_row[None, :], -1)

        def listing(mask):
            out = np.full(N * W + 1, -1, np.int64)
            out[np.where(mask, pos, N * W)] = self.experts
            return out[: N * W]

        return (
            dst_row,
            src_row,
            maps,
            listing(need & (~ssd | (cached_row >= 0))),
            listing(ssd),
            listing(need & ssd & (cached_row < 0)),
        )


class LruRef:
    """Plain LRU used to pin TableRef.acquire (tests/test_table.py:13-51).

    Recency is a per-step stamp; among equal stamps the lower slot is evicted
    first; slots hit in the step are protected.
    """

    def __init__(self, num_slots: int) -> None:
        self.num_slots = num_slots
        self.slot_of: dict[int, int] = {}
        self.stamp = [0] * num_slots
        self.step = 1
        self.hits = 0
        self.misses = 0

    def acquire(self, experts: set[int]) -> None:
        present = {e for e in experts if e in self.slot_of}
        missing = sorted(experts - present)
        self.hits += len(present)
        self.misses += len(missing)
        keep = {self.slot_of[e] for e in present}
        for e in missing:
            free = [s for s in range(self.num_slots) if s not in keep]
            victim = min(free, key=lambda s: (self.stamp[s], s))
            for old in [x for x, s in self.slot_of.items() if s == victim]:
                del self.slot_of[old]
            self.slot_of[e] = victim
            keep.add(victim)
        for e in experts:
            self.stamp[self.slot_of[e]] = self.step
        self.step += 1

    def cached(self) -> set[int]:
        return set(self.slot_of)


# ---- timing helper for the CPU baseline (bench.py) ----

def acquire_trace_rate(ids: np.ndarray, E: int, S: int, R: int, seconds: float,
                       start_at: float | None = None) -> tuple[int, float]:
    """Replay a routing trace ids (steps, layers, topk) through TableRef.acquire
    of both tables of each layer (a VRAM table of S slots, a RAM table of R
    warm slots), step after step, for about `seconds` from `start_at` (a
    time.time() value, so that several processes overlap). Returns (layer
    acquires done, seconds taken)."""
    import time

    steps, layers = ids.shape[:2]
    refs = []
    for _ in range(layers):
        v, r = TableRef(E, S), TableRef(E, R)
        r.warm(R)
        refs.append((v, r))
    if start_at is not None:
        time.sleep(max(0.0, start_at - time.time()))
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        row = ids[n % steps]
        for layer in range(layers):
            refs[layer][0].acquire(row[layer], pair_slots=True)
            refs[layer][1].acquire(row[layer], pair_slots=True)
        n += 1
    return n * layers, time.perf_counter() - t0


if __name__ == "__main__":
    # python -m oracle.table_ref IDS.npy E S R SECONDS START_AT: one process of
    # the all-cores acquire baseline; prints "<layer acquires> <seconds>".
    import sys

    _ids = np.load(sys.argv[1])
    _E, _S, _R = (int(x) for x in sys.argv[2:5])
    _n, _dt = acquire_trace_rate(_ids, _E, _S, _R, float(sys.argv[5]), float(sys.argv[6]))
    print(_n, _dt)
