"""GPU parity of the fused two-table acquire against the oracle (bit-exact).

Mirrors the reference's tests/test_acquire.py (AcquirePair == torch
ExpertTable.acquire on the full state) with the oracle as the checker, plus
the decode trace of the single-layer workload (256 experts, 32 VRAM slots,
256 RAM slots, 1000 steps of top-8 Zipf(1.1) routing) and hipGraph replay.
The single-table operations are covered on both devices by test_table.py.
"""

import random

import numpy as np
import pytest
import torch

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
