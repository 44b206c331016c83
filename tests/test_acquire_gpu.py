"""GPU parity of the table kernels against the oracle (bit-exact).

Mirrors the reference's tests/test_acquire.py (AcquirePair == torch
ExpertTable.acquire on the full state) with the oracle as the checker, plus
the decode trace of the single-layer workload (256 experts, 32 VRAM slots,
256 RAM slots, 1000 steps of top-8 Zipf(1.1) routing), the seed/plan traces
of the reference, and hipGraph replay.
"""

import random

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle.table_ref import TableRef

pytestmark = pytest.mark.gpu


def _mods():
    from vllm_expert_pager.acquire import AcquirePair
    from vllm_expert_pager.table import ExpertTable

    return AcquirePair, ExpertTable


def make_pair(E, S, R, warm):
    AcquirePair, ExpertTable = _mods()
    dev = torch.device("cuda")
    vram, ram = ExpertTable(E, S, dev), ExpertTable(E, R, dev)
    ref_v, ref_r = TableRef(E, S), TableRef(E, R)
    if warm:
        ram.slot_of[:R] = ram.experts[:R]
        ram.expert_in[:R] = ram.experts[:R]
        ref_r.warm(R)
    return vram, ram, ref_v, ref_r, AcquirePair(vram, ram)


def assert_state(gpu, ref, what):
    E, S = ref.num_experts, ref.num_slots
    np.testing.assert_array_equal(gpu.slot_of[:E].cpu().numpy(), ref.slot_of[:E], err_msg=f"{what} slot_of")
    np.testing.assert_array_equal(gpu.expert_in[:S].cpu().numpy(), ref.expert_in[:S], err_msg=f"{what} expert_in")
    np.testing.assert_array_equal(gpu.last_used[:S].cpu().numpy(), ref.last_used[:S], err_msg=f"{what} last_used")
    assert [int(gpu.step), int(gpu.hits), int(gpu.misses)] == [ref.step, ref.hits, ref.misses], what


def zipf_steps(E, steps, topk, seed, s=1.1, reuse=0.0):
    """Top-k distinct experts per step from Zipf(s) over a seeded permutation."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p = (np.arange(1, E + 1, dtype=np.float64)) ** -s
    p /= p.sum()
    prev = None
    for _ in range(steps):
        if prev is not None and rng.random() < reuse:
            ids = prev
        else:
            ids = perm[rng.choice(E, size=topk, replace=False, p=p)]
        prev = ids
        yield ids.astype(np.int64)


@pytest.mark.parametrize("E,S,R,warm", [(16, 4, 8, False), (16, 4, 4, True), (256, 102, 256, True),
                                        (256, 32, 128, True)])
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_pair_matches_oracle(E, S, R, warm, dtype):
    vram, ram, ref_v, ref_r, pair = make_pair(E, S, R, warm)
    rng = random.Random(0)
    for step in range(200):
        k = rng.randint(1, S)
        ids = [rng.randrange(E) for _ in range(k)]
        if rng.random() < 0.1:
            ids[rng.randrange(k)] = -1
        t = torch.tensor([ids], dtype=dtype, device="cuda")
        emap, vslot, vtodo = ref_v.acquire(ids, pair_slots=True)
        _, rslot, rtodo = ref_r.acquire(ids, pair_slots=True)
        todo, ssd = pair(t)
        torch.cuda.synchronize()
        assert_state(vram, ref_v, f"step {step} vram")
        assert_state(ram, ref_r, f"step {step} ram")
        np.testing.assert_array_equal(pair.expert_map.cpu().numpy(), emap.astype(np.int32))
        np.testing.assert_array_equal(pair.vram_slot.cpu().numpy(), vslot)
        np.testing.assert_array_equal(pair.ram_slot.cpu().numpy(), rslot)
        np.testing.assert_array_equal(todo.cpu().numpy(), vtodo)
        np.testing.assert_array_equal(ssd.cpu().numpy(), rtodo)
        # Each id's VRAM slot in step order: the oracle's expert_map at the id, -1 for an invalid id.
        want_pairs = np.array([emap[i] if 0 <= i < E else -1 for i in ids], np.int32)
        np.testing.assert_array_equal(pair.pair_slot[:k].cpu().numpy(), want_pairs, err_msg=f"step {step}")


def test_pair_single_layer_decode_trace():
    """256 experts, CACHE_SLOTS=32, RAM_SLOTS=256 (warm), 1000 steps of top-8 Zipf(1.1)."""
    vram, ram, ref_v, ref_r, pair = make_pair(256, 32, 256, True)
    for step, ids in enumerate(zipf_steps(256, 1000, 8, seed=1)):
        t = torch.from_numpy(ids.astype(np.int32)).view(1, 8).cuda()
        emap, vslot, vtodo = ref_v.acquire(ids, pair_slots=True)
        _, rslot, rtodo = ref_r.acquire(ids, pair_slots=True)
        todo, ssd = pair(t)
        out = torch.cat([pair.expert_map.long(), pair.vram_slot, pair.ram_slot, todo, ssd]).cpu().numpy()
        want = np.concatenate([emap, vslot, rslot, vtodo, rtodo])
        np.testing.assert_array_equal(out, want, err_msg=f"step {step}")
    assert_state(vram, ref_v, "vram")
    assert_state(ram, ref_r, "ram")
    hit = ref_v.hits / (ref_v.hits + ref_v.misses)
    assert 0.3 < hit < 0.8  # the trace is the intended mix of hits and misses


def test_table_acquire_matches_oracle():
    _, ExpertTable = _mods()
    for E, S in ((16, 1), (16, 5), (256, 32), (300, 200)):
        t, ref = ExpertTable(E, S, torch.device("cuda")), TableRef(E, S)
        rng = random.Random(E + S)
        for step in range(120):
            k = rng.randint(0, S)
            ids = [rng.randrange(-1, E) for _ in range(k)]
            emap, slot, todo = t.acquire(torch.tensor(ids, dtype=torch.int64, device="cuda"))
            r_emap, r_slot, r_todo = ref.acquire(np.array(ids, np.int64))
            np.testing.assert_array_equal(emap.cpu().numpy(), r_emap, err_msg=f"{E},{S} step {step}")
            np.testing.assert_array_equal(slot.cpu().numpy(), r_slot, err_msg=f"{E},{S} step {step}")
            np.testing.assert_array_equal(todo.cpu().numpy(), r_todo)
        assert_state(t, ref, f"{E},{S}")


def test_acquire_rejects_more_ids_than_slots():
    _, ExpertTable = _mods()
    t = ExpertTable(16, 2, torch.device("cuda"))
    with pytest.raises(ValueError):
        t.acquire(torch.tensor([1, 2, 3], device="cuda"))


def test_need_mask_and_pack():
    _, ExpertTable = _mods()
    t = ExpertTable(300, 4, torch.device("cuda"))
    ids = torch.tensor([[3, -1, 299], [3, 7, -5]], dtype=torch.int32, device="cuda")
    need = t.need_mask(ids)
    assert need.dtype == torch.bool and need.nonzero().flatten().tolist() == [3, 7, 299]
    assert t.pack(need).tolist() == [3, 7, 299] + [-1] * 297
    big = torch.randint(-1, 300, (4096,), device="cuda")
    ref = TableRef(300, 4)
    np.testing.assert_array_equal(t.need_mask(big).cpu().numpy(), ref.need_mask(big.cpu().numpy()))
    m = torch.rand(300, device="cuda") < 0.3
    np.testing.assert_array_equal(t.pack(m).cpu().numpy(), ref.pack(m.cpu().numpy()))


@pytest.mark.parametrize("fixture", ["table_vectors_small.npz", "table_vectors_big.npz"])
def test_reference_traces_with_seed_and_plan(fixture):
    """Replay the reference's recorded decode / prefill steps through the GPU tables."""
    import os

    _, ExpertTable = _mods()
    d = np.load(os.path.join(GOLDEN, fixture), allow_pickle=False)
    E, S, R, W, L, layer = (int(d[k]) for k in "E S R W L layer".split())
    dev = torch.device("cuda")
    vram, ram = ExpertTable(E, S, dev), ExpertTable(E, R, dev)
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


def test_seed_with_ties_matches_oracle_rule():
    """Near-uniform prefill routing (ties at the cut): GPU and oracle follow the same lower-id rule."""
    _, ExpertTable = _mods()
    dev = torch.device("cuda")
    E, S, R = 256, 32, 128
    vram, ram = ExpertTable(E, S, dev), ExpertTable(E, R, dev)
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
    assert_state(ram, ref_r, "seeded ram")


def test_pair_in_graph():
    vram, ram, ref_v, ref_r, pair = make_pair(256, 32, 128, True)
    ids_buf = torch.zeros((1, 8), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    steps = list(zipf_steps(256, 40, 8, seed=7))
    with torch.cuda.stream(s):
        ids_buf.copy_(torch.from_numpy(steps[0].astype(np.int32)).view(1, 8))
        todo, ssd = pair(ids_buf)  # eager warm-up step
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            todo_g, ssd_g = pair(ids_buf)
    torch.cuda.synchronize()
    ref_v.acquire(steps[0], pair_slots=True)
    ref_r.acquire(steps[0], pair_slots=True)
    for i, ids in enumerate(steps[1:]):
        ids_buf.copy_(torch.from_numpy(ids.astype(np.int32)).view(1, 8))
        g.replay()
        torch.cuda.synchronize()
        emap, _, vtodo = ref_v.acquire(ids, pair_slots=True)
        _, _, rtodo = ref_r.acquire(ids, pair_slots=True)
        np.testing.assert_array_equal(pair.expert_map.cpu().numpy(), emap.astype(np.int32), err_msg=f"replay {i}")
        np.testing.assert_array_equal(todo_g.cpu().numpy(), vtodo)
        np.testing.assert_array_equal(ssd_g.cpu().numpy(), rtodo)
    assert_state(vram, ref_v, "vram")
    assert_state(ram, ref_r, "ram")
