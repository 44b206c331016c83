"""CPU checks of the table oracle (oracle/table_ref.py), and of the product's
ExpertTable on CPU tensors against the same expectations.

Pins the oracle with (1) the reference's own golden traces, (2) an
independent plain LRU (the reference's ReferenceLRU rule), (3) the invariants
and known answers of the reference's tests/test_table.py, and (4) the chunk
loop simulator. A planted mistake in the oracle fails at least one of them.
The tests of (2)-(4) also run on the product's table kept in CPU tensors
(csrc/table_host.cpp through vllm_expert_pager.table), through a thin
adapter with the oracle's numpy interface.
"""

import os
import random

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import gather_ref
from oracle.table_ref import LruRef, TableRef

E = 16


class CpuTable:
    """The product's ExpertTable on CPU tensors with the oracle's numpy interface."""

    def __init__(self, num_experts: int, num_slots: int) -> None:
        from vllm_expert_pager.table import ExpertTable

        self.t = ExpertTable(num_experts, num_slots, torch.device("cpu"))
        self.num_experts, self.num_slots = num_experts, num_slots
        # numpy views of the table's tensors: the host code updates them in place
        self.slot_of = self.t.slot_of.numpy()
        self.expert_in = self.t.expert_in.numpy()
        self.last_used = self.t.last_used.numpy()

    step = property(lambda self: int(self.t.step))
    hits = property(lambda self: int(self.t.hits))
    misses = property(lambda self: int(self.t.misses))

    @staticmethod
    def _ids(ids) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(np.asarray(ids), dtype=np.int64))

    def need_mask(self, ids) -> np.ndarray:
        return self.t.need_mask(self._ids(ids)).numpy()

    def acquire(self, ids):
        return tuple(x.numpy() for x in self.t.acquire(self._ids(ids)))

    def pack(self, mask) -> np.ndarray:
        return self.t.pack(torch.from_numpy(np.asarray(mask, bool))).numpy()

    def seed(self, vram: "CpuTable", ids, need) -> None:
        self.t.seed(vram.t, self._ids(ids), torch.from_numpy(np.asarray(need, bool)))

    def plan_chunks(self, before, need, cached_row, rows, ram_base, working_base):
        out = self.t.plan_chunks(torch.from_numpy(np.asarray(before, np.int64)),
                                 torch.from_numpy(np.asarray(need, bool)),
                                 torch.from_numpy(np.asarray(cached_row, np.int64)), rows, ram_base, working_base)
        return tuple(x.numpy() for x in out)


@pytest.fixture(params=["oracle", "cpu_table"])
def Table(request):
    """The table under test: the oracle, or the product's CPU table."""
    return TableRef if request.param == "oracle" else CpuTable


def cached(t: TableRef) -> set[int]:
    return {e for e in range(t.num_experts) if t.slot_of[e] >= 0}


def check_invariants(t: TableRef) -> None:
    """slot_of and expert_in are inverse maps; no slot is shared (tests/test_table.py:58-71)."""
    Ev, S = t.num_experts, t.num_slots
    used = [s for s in t.slot_of[:Ev] if s >= 0]
    assert len(used) == len(set(used))
    for e, s in enumerate(t.slot_of[:Ev]):
        if s >= 0:
            assert 0 <= s < S and t.expert_in[s] == e
    for s, e in enumerate(t.expert_in[:S]):
        if e >= 0:
            assert t.slot_of[e] == s


def check_acquire_result(t, ids, emap, slot, todo, before) -> None:
    """tests/test_table.py:74-96."""
    need = {int(x) for x in np.asarray(ids).reshape(-1) if x >= 0}
    for e in range(t.num_experts):
        if e in need:
            assert 0 <= emap[e] < t.num_slots and slot[e] == emap[e] == t.slot_of[e]
        else:
            assert emap[e] == -1
    assert len({emap[e] for e in need}) == len(need)
    misses = sorted(e for e in need if e not in before)
    todo = list(todo)
    assert len(todo) == np.asarray(ids).size
    assert todo[: len(misses)] == misses and all(x == -1 for x in todo[len(misses):])
    assert need <= cached(t)


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.mark.parametrize("fixture", ["table_vectors_small.npz", "table_vectors_big.npz"])
def test_oracle_matches_reference_traces(fixture):
    d = _load(fixture)
    Ev, S, R, W, L, layer = (int(d[k]) for k in "E S R W L layer".split())
    vram, ram = TableRef(Ev, S), TableRef(Ev, R)
    ram.warm(R)
    for i in range(int(d["steps"])):
        p = f"s{i}_"
        ids = d[p + "ids"]
        if int(d[p + "kind"]) == 0:
            emap, slot, todo = vram.acquire(ids)
            _, rslot, rtodo = ram.acquire(ids)
            for got, key in ((emap, "emap"), (slot, "slot"), (todo, "todo"), (rslot, "rslot"), (rtodo, "rtodo")):
                np.testing.assert_array_equal(got, d[p + key], err_msg=f"step {i} {key}")
        else:
            need = ram.need_mask(ids)
            np.testing.assert_array_equal(need, d[p + "need"])
            cached_row = vram.slot_of[:Ev].copy()
            before = ram.slot_of[:Ev].copy()
            if int(d[p + "kind"]) == 1:
                ram.acquire(ids)
            else:
                ram.seed(vram, ids, need)
            plan = ram.plan_chunks(before, need, cached_row, W, layer * R, L * R)
            for got, key in zip(plan, ("dst_row", "src_row", "maps", "todo", "ssd", "late")):
                np.testing.assert_array_equal(got, d[p + key], err_msg=f"step {i} {key}")
        for pre, t in (("vram_", vram), ("ram_", ram)):
            np.testing.assert_array_equal(t.slot_of[:Ev], d[p + pre + "slot_of"])
            np.testing.assert_array_equal(t.expert_in[: t.num_slots], d[p + pre + "expert_in"])
            np.testing.assert_array_equal(t.last_used[: t.num_slots], d[p + pre + "last_used"])
            assert [t.step, t.hits, t.misses] == list(d[p + pre + "counters"])


@pytest.mark.parametrize("num_slots", [1, 4, 8])
def test_acquire_matches_plain_lru(Table, num_slots):
    rng = random.Random(0)
    t = Table(E, num_slots)
    ref = LruRef(num_slots)
    for _ in range(300):
        k = rng.randint(1, num_slots)
        ids = np.array([[rng.randrange(E) for _ in range(k)]], np.int32)
        before = cached(t)
        assert before == ref.cached()
        emap, slot, todo = t.acquire(ids)
        check_invariants(t)
        check_acquire_result(t, ids, emap, slot, todo, before)
        ref.acquire({int(x) for x in ids.reshape(-1)})
        assert (t.hits, t.misses) == (ref.hits, ref.misses)
        assert cached(t) == ref.cached()


def test_acquire_known_answers(Table):
    t = Table(E, 2)
    for e in (0, 1, 0, 2):
        t.acquire(np.array([[e]]))
    assert cached(t) == {0, 2} and t.hits == 1 and t.misses == 3
    t = Table(E, 4)
    t.acquire(np.array([[0, 1, 2, 3]]))
    emap, _, todo = t.acquire(np.array([[2, 3, 4, 5]]))
    check_invariants(t)
    assert cached(t) == {2, 3, 4, 5}
    assert sorted(x for x in todo if x >= 0) == [4, 5]
    assert emap[0] == emap[1] == -1 and sorted(emap[[2, 3, 4, 5]]) == [0, 1, 2, 3]


def test_pair_slots_differ_only_for_evicted_experts():
    t1, t2 = TableRef(E, 2), TableRef(E, 2)
    for ids in ([[0, 1]], [[2]], [[3, 2]]):
        _, s1, _ = t1.acquire(np.array(ids))
        _, s2, _ = t2.acquire(np.array(ids), pair_slots=True)
        need = t1.need_mask(np.array(ids))
        np.testing.assert_array_equal(s1[need], s2[need])
        evicted = (s2 >= 0) & (s1 < 0)
        assert np.array_equal(s1 != s2, evicted)


def test_rejects_zero_slots(Table):
    with pytest.raises(ValueError):
        Table(E, 0)


def test_pack_and_negative_ids(Table):
    t = Table(E, 2)
    mask = np.zeros(E, bool)
    mask[[3, 7, 12]] = True
    assert list(t.pack(mask)) == [3, 7, 12] + [-1] * (E - 3)
    ram, vram = Table(E, 4), Table(E, 2)
    ids = np.array([[3, -1], [3, -1], [5, -1]])
    need = ram.need_mask(ids)
    assert list(np.nonzero(need)[0]) == [3, 5]
    ram.seed(vram, ids, need)
    check_invariants(ram)
    assert cached(ram) == {3, 5}


def test_seed_known_answers(Table):
    ram, vram = Table(E, 6), Table(E, 2)
    ram.acquire(np.array([[0, 1, 2, 3, 4, 5]]))
    vram.acquire(np.array([[4, 9]]))
    ids = np.array([[8, 7, 6, 5], [8, 7, 6, 5], [8, 7, 0, 9]])
    need = ram.need_mask(ids)
    before = ram.slot_of[:E].copy()
    ram.seed(vram, ids, need)
    check_invariants(ram)
    assert cached(ram) == {8, 7, 6, 5, 4, 9}
    assert ram.last_used[ram.slot_of[4]] > ram.last_used[ram.slot_of[8]]
    assert ram.last_used[ram.slot_of[9]] > ram.last_used[ram.slot_of[8]]
    assert ram.slot_of[4] == before[4] and ram.slot_of[5] == before[5]
    assert ram.hits == 0 and ram.misses == 6
    ram, vram = Table(E, 4), Table(E, 2)
    ram.acquire(np.array([[0, 1, 2, 3]]))
    vram.acquire(np.array([[0, 9]]))
    ids = np.array([[5, 6], [5, 6], [7, 0]])
    ram.seed(vram, ids, ram.need_mask(ids))
    assert 9 not in cached(ram) and {5, 6, 0} <= cached(ram)


def test_plan_chunks_known_answers(Table):
    R, S, L, W, layer = 4, 2, 3, 2, 1
    ram, vram = Table(E, R), Table(E, S)
    rows = np.full(L * R + 2 * W, -1)
    ram.acquire(np.array([[0, 1, 2, 3]]))
    for e in range(4):
        rows[layer * R + ram.slot_of[e]] = e
    vram.acquire(np.array([[0, 9]]))
    ids = np.array([[5, 6], [5, 6], [5, 0], [7, 1]])
    ssd, src_row = gather_ref.simulate_working_step(ram, vram, ids, rows, W, layer * R, L * R)
    check_invariants(ram)
    gather_ref.check_ram_rows(ram, rows, layer * R)
    assert cached(ram) == {5, 6, 0, 3}
    assert sorted(ssd) == [0, 5, 6, 7]
    assert L * R <= src_row[7] < L * R + 2 * W and rows[src_row[7]] == 7

    ram, vram = Table(E, 4), Table(E, 2)
    rows = np.full(2 * 4 + 2 * 4, -1)
    ram.acquire(np.array([[0, 1, 2, 3]]))
    for e in range(4):
        rows[ram.slot_of[e]] = e
    vram.acquire(np.array([[2, 3]]))
    ssd, _ = gather_ref.simulate_working_step(ram, vram, np.array([[2, 5], [3, 3]]), rows, 4, 0, 8)
    assert ssd == [5]

    ram, vram = Table(E, 4), Table(E, 2)
    rows = np.full(4 + 6, -1)
    ssd, src_row = gather_ref.simulate_working_step(ram, vram, np.arange(12).reshape(3, 4), rows, 3, 0, 4)
    assert sorted(ssd) == list(range(12))
    shared = [src_row[e] - 4 for e in ssd if src_row[e] >= 4]
    assert len(shared) == 10 and {r // 3 for r in shared} == {0, 1}


@pytest.mark.parametrize("W", [1, 3, 4])
def test_plan_chunks_random_steps(Table, W):
    rng = random.Random(W)
    R, S, L, layer = 6, 3, 2, 1
    ram, vram = Table(E, R), Table(E, S)
    rows = np.full(L * R + 2 * W, -1)
    for _ in range(200):
        k = rng.randint(1, 2 * E)
        ids = np.array([[rng.randrange(E) for _ in range(k)]])
        if k <= S:
            _, _, todo = ram.acquire(ids)
            for e in todo:
                if e >= 0:
                    rows[layer * R + ram.slot_of[e]] = e
            vram.acquire(ids)
        else:
            gather_ref.simulate_working_step(ram, vram, ids, rows, W, layer * R, L * R)
        check_invariants(ram)
        check_invariants(vram)
        gather_ref.check_ram_rows(ram, rows, layer * R)
