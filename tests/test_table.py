"""ExpertTable against the oracle, bit-exact, on both devices.

On a GPU each operation is a kernel launch (csrc/table.hip); on the CPU it is
the host code of csrc/table_host.cpp. Both are checked against the oracle on
random traces (invalid ids included), on the reference's recorded decode and
prefill steps (acquire, seed, plan_chunks; tests/golden), and on the closed
forms of need_mask and pack (the reference's tests/test_table.py:152-156).
"""

import os
import random

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle.table_ref import TableRef

DEVICES = [pytest.param("cpu", id="cpu"), pytest.param("cuda", id="gpu", marks=pytest.mark.gpu)]


def _table():
    from vllm_expert_pager.table import ExpertTable

    return ExpertTable


def _sync(dev):
    if dev.type == "cuda":
        torch.cuda.synchronize()


def assert_state(t, ref, what):
    E, S = ref.num_experts, ref.num_slots
    np.testing.assert_array_equal(t.slot_of[:E].cpu().numpy(), ref.slot_of[:E], err_msg=f"{what} slot_of")
    np.testing.assert_array_equal(t.expert_in[:S].cpu().numpy(), ref.expert_in[:S], err_msg=f"{what} expert_in")
    np.testing.assert_array_equal(t.last_used[:S].cpu().numpy(), ref.last_used[:S], err_msg=f"{what} last_used")
    assert [int(t.step), int(t.hits), int(t.misses)] == [ref.step, ref.hits, ref.misses], what


def zipf_steps(E, steps, topk, seed, s=1.1):
    """Top-k distinct experts per step from Zipf(s) over a seeded permutation."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p = (np.arange(1, E + 1, dtype=np.float64)) ** -s
    p /= p.sum()
    for _ in range(steps):
        yield perm[rng.choice(E, size=topk, replace=False, p=p)].astype(np.int64)


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_table_acquire_matches_oracle(device, dtype):
    dev = torch.device(device)
    for E, S in ((16, 1), (16, 5), (256, 32), (300, 200)):
        t, ref = _table()(E, S, dev), TableRef(E, S)
        rng = random.Random(E + S)
        for step in range(120):
            k = rng.randint(0, S)
            ids = [rng.randrange(-1, E) for _ in range(k)]
            emap, slot, todo = t.acquire(torch.tensor(ids, dtype=dtype, device=dev))
            r_emap, r_slot, r_todo = ref.acquire(np.array(ids, np.int64))
            np.testing.assert_array_equal(emap.cpu().numpy(), r_emap, err_msg=f"{E},{S} step {step}")
            np.testing.assert_array_equal(slot.cpu().numpy(), r_slot, err_msg=f"{E},{S} step {step}")
            np.testing.assert_array_equal(todo.cpu().numpy(), r_todo)
        assert_state(t, ref, f"{E},{S}")


@pytest.mark.parametrize("device", DEVICES)
def test_acquire_rejects_more_ids_than_slots(device):
    dev = torch.device(device)
    t = _table()(16, 2, dev)
    with pytest.raises(ValueError):
        t.acquire(torch.tensor([1, 2, 3], device=dev))


@pytest.mark.parametrize("device", DEVICES)
def test_need_mask_and_pack(device):
    dev = torch.device(device)
    t = _table()(300, 4, dev)
    ids = torch.tensor([[3, -1, 299], [3, 7, -5]], dtype=torch.int32, device=dev)
    need = t.need_mask(ids)
    assert need.dtype == torch.bool and need.nonzero().flatten().tolist() == [3, 7, 299]
    assert t.pack(need).tolist() == [3, 7, 299] + [-1] * 297
    g = torch.Generator().manual_seed(5)
    big = torch.randint(-1, 300, (4096,), generator=g).to(dev)
    ref = TableRef(300, 4)
    np.testing.assert_array_equal(t.need_mask(big).cpu().numpy(), ref.need_mask(big.cpu().numpy()))
    m = (torch.rand(300, generator=g) < 0.3).to(dev)
    np.testing.assert_array_equal(t.pack(m).cpu().numpy(), ref.pack(m.cpu().numpy()))
    assert t.pack(torch.zeros(300, dtype=torch.bool, device=dev)).tolist() == [-1] * 300


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("fixture", ["table_vectors_small.npz", "table_vectors_big.npz"])
def test_reference_traces_with_seed_and_plan(device, fixture):
    """Replay the reference's recorded decode / prefill steps through the tables."""
    d = np.load(os.path.join(GOLDEN, fixture), allow_pickle=False)
    E, S, R, W, L, layer = (int(d[k]) for k in "E S R W L layer".split())
    dev = torch.device(device)
    vram, ram = _table()(E, S, dev), _table()(E, R, dev)
    ram.slot_of[:R] = ram.experts[:R]
    ram.expert_in[:R] = ram.experts[:R]
    for i in range(int(d["steps"])):
        p = f"s{i}_"
        ids = torch.from_numpy(d[p + "ids"]).to(dev)
        if int(d[p + "kind"]) == 0:
            emap, slot, todo = vram.acquire(ids)
            _, rslot, rtodo = ram.acquire(ids)
            for got, key in ((emap, "emap"), (slot, "slot"), (todo, "todo"), (rslot, "rslot"), (rtodo, "rtodo")):
                np.testing.assert_array_equal(got.cpu().numpy(), d[p + key], err_msg=f"step {i} {key}")
        else:
            need = ram.need_mask(ids)
            np.testing.assert_array_equal(need.cpu().numpy(), d[p + "need"])
            cached_row = vram.slot_of[:E].clone()
            before = ram.slot_of[:E].clone()
            if ids.numel() <= R:
                ram.acquire(ids)
            else:
                ram.seed(vram, ids, need)
            plan = ram.plan_chunks(before, need, cached_row, W, layer * R, L * R)
            for got, key in zip(plan, ("dst_row", "src_row", "maps", "todo", "ssd", "late")):
                np.testing.assert_array_equal(got.cpu().numpy(), d[p + key], err_msg=f"step {i} {key}")
        for pre, t in (("vram_", vram), ("ram_", ram)):
            np.testing.assert_array_equal(t.slot_of[:E].cpu().numpy(), d[p + pre + "slot_of"], err_msg=f"{i}")
            np.testing.assert_array_equal(t.expert_in[: t.num_slots].cpu().numpy(), d[p + pre + "expert_in"])
            np.testing.assert_array_equal(t.last_used[: t.num_slots].cpu().numpy(), d[p + pre + "last_used"])
            assert [int(t.step), int(t.hits), int(t.misses)] == list(d[p + pre + "counters"])


@pytest.mark.parametrize("device", DEVICES)
def test_seed_with_ties_matches_oracle_rule(device):
    """Near-uniform prefill routing (ties at the cut): table and oracle follow the same lower-id rule."""
    dev = torch.device(device)
    E, S, R = 256, 32, 128
    vram, ram = _table()(E, S, dev), _table()(E, R, dev)
    ref_v, ref_r = TableRef(E, S), TableRef(E, R)
    ram.slot_of[:R] = ram.experts[:R]
    ram.expert_in[:R] = ram.experts[:R]
    ref_r.warm(R)
    for ids in zipf_steps(E, 30, 8, seed=3):
        t = torch.from_numpy(ids).to(dev)
        vram.acquire(t), ram.acquire(t)
        ref_v.acquire(ids), ref_r.acquire(ids)
    rng = np.random.default_rng(4)
    ids = np.stack([rng.permutation(E)[:8] for _ in range(2048)]).astype(np.int64)
    t = torch.from_numpy(ids).to(dev)
    need = ram.need_mask(t)
    ram.seed(vram, t, need)
    ref_r.seed(ref_v, ids, ref_r.need_mask(ids))
    _sync(dev)
    assert_state(ram, ref_r, "seeded ram")


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("E,S,R,W", [(64, 8, 32, 8), (256, 32, 128, 48), (300, 16, 200, 7)])
def test_prefill_steps_match_oracle(device, E, S, R, W):
    """Random prefills after random decode steps: acquire or seed, then the chunk plan."""
    dev = torch.device(device)
    vram, ram = _table()(E, S, dev), _table()(E, R, dev)
    ref_v, ref_r = TableRef(E, S), TableRef(E, R)
    rng = np.random.default_rng(E * W)
    L, layer = 3, 1
    for step in range(12):
        for ids in zipf_steps(E, int(rng.integers(1, 20)), min(8, S), seed=int(rng.integers(1 << 30))):
            t = torch.from_numpy(ids).to(dev)
            vram.acquire(t), ram.acquire(t)
            ref_v.acquire(ids), ref_r.acquire(ids)
        n = int(rng.choice([1, 4, R // 8 + 1, 2 * R, 600]))
        ids = rng.integers(-1, E, size=(n, min(8, S))).astype(np.int64)
        t = torch.from_numpy(ids).to(dev)
        need = ram.need_mask(t)
        r_need = ref_r.need_mask(ids)
        cached_row, r_cached = vram.slot_of[:E].clone(), ref_v.slot_of[:E].copy()
        before, r_before = ram.slot_of[:E].clone(), ref_r.slot_of[:E].copy()
        if t.numel() <= R:
            ram.acquire(t)
            ref_r.acquire(ids)
        else:
            ram.seed(vram, t, need)
            ref_r.seed(ref_v, ids, r_need)
        plan = ram.plan_chunks(before, need, cached_row, W, layer * R, L * R)
        want = ref_r.plan_chunks(r_before, r_need, r_cached, W, layer * R, L * R)
        for got, w, key in zip(plan, want, ("dst_row", "src_row", "maps", "todo", "ssd", "late")):
            np.testing.assert_array_equal(got.cpu().numpy(), w, err_msg=f"step {step} {key}")
        assert_state(ram, ref_r, f"step {step} ram")
        assert_state(vram, ref_v, f"step {step} vram")


def test_cpu_table_refuses_tensors_of_another_device():
    """A CPU table never hands a device pointer to host code (checked without a GPU: meta tensors)."""
    t = _table()(16, 4, torch.device("cpu"))
    meta = torch.empty((1, 2), dtype=torch.int64, device="meta")
    for op in (t.need_mask, t.acquire):
        with pytest.raises(ValueError, match="lives on cpu"):
            op(meta)
    with pytest.raises(ValueError, match="lives on cpu"):
        t.pack(torch.empty(16, dtype=torch.bool, device="meta"))


def test_cpu_table_argument_errors_surface():
    """Host code checks its arguments like the kernels' launchers (error text from the library)."""
    from vllm_expert_pager import _native as nat

    t = _table()(16, 4, torch.device("cpu"))
    st = t._struct()
    ids = torch.tensor([1], dtype=torch.int64)
    with pytest.raises(ValueError, match="element size"):
        nat.call("xp_table_acquire_host", ids.data_ptr(), 2, 1, nat.ctypes.byref(st), None, None, None, None)
    with pytest.raises(ValueError, match="W=0"):
        z = torch.zeros(16, dtype=torch.int64)
        nat.call("xp_plan_chunks_host", nat.ctypes.byref(st), z.data_ptr(), z.data_ptr(), z.data_ptr(), 0, 0, 0,
                 z.data_ptr(), z.data_ptr(), z.data_ptr(), z.data_ptr(), z.data_ptr(), z.data_ptr())


@pytest.mark.gpu
def test_gpu_table_refuses_host_tensors():
    """A GPU table never hands a host pointer to a kernel: inputs on the CPU are refused before any launch."""
    t = _table()(16, 4, torch.device("cuda"))
    host_ids = torch.tensor([[1, 2]], dtype=torch.int64)
    for op in (t.need_mask, t.acquire):
        with pytest.raises(ValueError, match="lives on cuda"):
            op(host_ids)
    with pytest.raises(ValueError, match="lives on cuda"):
        t.pack(torch.zeros(16, dtype=torch.bool))
    vram = _table()(16, 2, torch.device("cuda"))
    with pytest.raises(ValueError, match="lives on cuda"):
        t.seed(vram, host_ids, torch.zeros(16, dtype=torch.bool))
    with pytest.raises(ValueError, match="lives on cuda"):
        z = torch.zeros(16, dtype=torch.int64)
        t.plan_chunks(z, z.bool(), z, 4, 0, 0)
