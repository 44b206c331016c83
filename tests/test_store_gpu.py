"""The RAM tier, the paging file and the request ring, driven from the GPU.

Covers store.py (tier layout, loading, validation), the fetch kernels of
gather.py and the host server (csrc/ssd.cpp) together. A request, seen from
the GPU, is:

  1. a fetch kernel writes the experts and their RAM-tier rows into ring
     slot ``seq % ring`` and publishes ``seq`` last, with a system-scope
     release store; an empty request publishes nothing;
  2. the host server reads each expert's record from the paging file into
     its row and writes ``done = seq``, also when a read fails (the failure
     is kept and reported on the next eager forward);
  3. the waiting kernel returns once ``done >= seq``; it re-publishes the
     slot every retry interval and counts it, and after ``giveup``
     re-publishes it stops and counts a give-up, so a host that never answers
     cannot hold the GPU;
  4. the host writes ``done`` again when the re-publish count moves.

Rows come from tests/_tiers.py; the expected record of a compressed row is
the oracle's encoding (oracle/codec_ref.py), independent of the product's
encoders.
"""

from __future__ import annotations

import os
import time

import numpy as np
import pytest
import torch

import _tiers
from oracle import codec_ref

pytestmark = pytest.mark.gpu

GROUP = 512 * 32  # one codec group: rows are whole groups
NAMES = {"w13_weight": 3 * GROUP, "w2_weight": GROUP}
L, E, R, W = 3, 10, 4, 3  # layers, experts, RAM slots per layer, working rows per face


class Tiers:
    """A Store loaded with deterministic rows, and what each of its rows should hold."""

    def __init__(self, tmp_path, compress: bool, layers=L, experts=E, ram=R, names=NAMES, fname="tiers.bin"):
        from vllm_expert_pager.store import Store

        self.layers, self.experts, self.ram = layers, experts, ram
        self.names = dict(names)
        self.path = str(tmp_path / fname)
        self.store = Store(layers, experts, ram, 2 * W, self.names, compress, 1.0, self.path, torch.device("cuda"))
        for layer in range(layers):
            for i, (name, nbytes) in enumerate(self.names.items()):
                rows = np.stack([_tiers.expert_row(layer, e, i, nbytes) for e in range(experts)])
                self.store.write_rows(layer, name, torch.from_numpy(rows))
        self._records: dict[tuple[int, int, int], np.ndarray] = {}

    def raw(self, layer: int, expert: int, i: int) -> np.ndarray:
        return _tiers.expert_row(layer, expert, i, list(self.names.values())[i])

    def record(self, layer: int, expert: int, i: int) -> np.ndarray:
        """The bytes a RAM row or paging-file record of this expert holds."""
        key = (layer, expert, i)
        if key not in self._records:
            raw = self.raw(layer, expert, i)
            name = list(self.names)[i]
            self._records[key] = codec_ref.encode(raw, self.store.pitch[name])[0] if self.store.compress else raw
        return self._records[key]

    def row(self, i: int, row: int) -> np.ndarray:
        return self.store.pinned[list(self.names)[i]][row].view(torch.uint8).numpy()

    def assert_slot_holds(self, layer: int, slot: int, expert: int) -> None:
        for i in range(len(self.names)):
            got = self.row(i, layer * self.ram + slot)
            assert np.array_equal(got, self.record(layer, expert, i)), f"layer {layer} slot {slot} is not expert {expert}"

    def close(self) -> None:
        self.store.close()


@pytest.fixture
def tiers(tmp_path):
    made: list[Tiers] = []

    def make(compress=True, **kw):
        t = Tiers(tmp_path, compress, fname=f"tiers{len(made)}.bin", **kw)
        made.append(t)
        return t

    yield make
    for t in made:
        t.close()


@pytest.fixture
def fast_timing():
    """Re-publish every 50 ms (default 500 ms), give up after 8 (the default)."""
    from vllm_expert_pager import _native as nat

    nat.call("xp_fetch_set_timing", 50_000, 8)
    yield
    nat.call("xp_fetch_set_timing", 500_000, 8)


class Fetch:
    """A fetch of up to ``width`` experts into the RAM slots of one layer,
    captured once in a hipGraph and replayed per request."""

    def __init__(self, t: Tiers, width: int, layer: int):
        from vllm_expert_pager import gather

        self.t, self.layer, self.width = t, layer, width
        self.todo = torch.full((width,), -1, dtype=torch.int64, device="cuda")
        self.slot = torch.zeros((t.experts,), dtype=torch.int64, device="cuda")
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            gather.fetch_rows(self.todo, self.slot, layer * t.ram, layer, t.store)  # empty: publishes nothing
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=side):
                gather.fetch_rows(self.todo, self.slot, layer * t.ram, layer, t.store)
        torch.cuda.synchronize()

    def __call__(self, placement: dict[int, int]) -> float:
        """Read each expert into its RAM slot; returns the seconds the replay took."""
        todo = np.full(self.width, -1, np.int64)
        todo[: len(placement)] = sorted(placement)
        slot = np.zeros(self.t.experts, np.int64)
        for e, s in placement.items():
            slot[e] = s
        self.todo.copy_(torch.from_numpy(todo))
        self.slot.copy_(torch.from_numpy(slot))
        t0 = time.perf_counter()
        self.graph.replay()
        torch.cuda.synchronize()
        return time.perf_counter() - t0


@pytest.mark.parametrize("compress", [True, False], ids=["compressed", "raw"])
def test_loading_fills_the_first_slots_and_the_paging_file(tiers, compress):
    """RAM slot s of layer l holds expert s (s < R); the paging file holds every
    expert's record at ((l * E + e) * record + offset[name]) (store.py:576-599)."""
    t = tiers(compress)
    st = t.store
    with open(t.path, "rb") as f:
        data = f.read()
    assert len(data) == L * E * st.record_bytes
    for layer in range(L):
        for e in range(E):
            if e < R:
                t.assert_slot_holds(layer, e, e)
            for i, name in enumerate(NAMES):
                at = (layer * E + e) * st.record_bytes + st.offset[name]
                rec = np.frombuffer(data, np.uint8, st.pitch[name], at)
                assert np.array_equal(rec, t.record(layer, e, i)), (layer, e, name)


@pytest.mark.parametrize("compress", [True, False], ids=["compressed", "raw"])
def test_replayed_requests_land_in_their_slots(tiers, compress):
    t = tiers(compress)
    rng = np.random.default_rng(4)
    fetch = Fetch(t, R, layer=2)
    reads = 0
    for _ in range(24):
        n = int(rng.integers(1, R + 1))
        experts = rng.choice(np.arange(R, E), size=n, replace=False)
        slots = rng.permutation(R)[:n]
        fetch(dict(zip(experts.tolist(), slots.tolist())))
        assert t.store.failed is None, t.store.failed
        for e, s in zip(experts.tolist(), slots.tolist()):
            t.assert_slot_holds(2, s, e)
        reads += n
    assert (t.store.fetches, t.store.reads, t.store.missed) == (24, reads, 0)
    assert int(t.store.req[t.store.retry_at]) == 0 and int(t.store.req[t.store.giveup_at]) == 0


def test_empty_requests_stay_on_the_device(tiers):
    t = tiers()
    fetch = Fetch(t, R, layer=0)
    seq = int(t.store.seq)
    for _ in range(5):
        fetch({})
    assert int(t.store.seq) == seq and t.store.fetches == 0
    fetch({7: 1})  # and the ring still works after them
    assert int(t.store.seq) == seq + 1 and t.store.fetches == 1
    t.assert_slot_holds(0, 1, 7)


def test_one_request_uses_every_reader(tiers):
    """A request of twice as many experts as the most reader threads the
    server sizes itself to (8)."""
    n = 16
    t = tiers(layers=1, experts=3 * n, ram=n)
    fetch = Fetch(t, n, layer=0)
    placement = {e: e - 2 * n for e in range(2 * n, 3 * n)}
    fetch(placement)
    assert t.store.failed is None, t.store.failed
    assert (t.store.fetches, t.store.reads) == (1, n)
    for e, s in placement.items():
        t.assert_slot_holds(0, s, e)


def test_readers_are_sized_from_the_disk_after_sync(tiers, monkeypatch):
    """sync() probes the paging file at 1, 2, 4 and 8 reads in flight and
    restarts the server with the smallest depth of at least 2 within 10% of
    the fastest (1 when no deeper one is); it still serves the ring
    afterwards. VLLM_EXPERT_PAGER_READ_WORKERS fixes the count instead."""
    monkeypatch.delenv("VLLM_EXPERT_PAGER_READ_WORKERS", raising=False)
    t = tiers(layers=2, experts=12, ram=4)
    st = t.store
    assert st.readers == 2 and st.reader_probe is None
    st.sync()
    assert set(st.reader_probe) == {"1", "2", "4", "8"} and st.readers in (1, 2, 4, 8)
    assert all(r > 0 for r in st.reader_probe.values())
    best = max(st.reader_probe.values())
    # the probe's rates are rounded to 3 decimals
    assert st.reader_probe[str(st.readers)] >= 0.9 * best - 1e-3
    assert all(st.reader_probe[str(d)] < 0.9 * best + 1e-3 for d in (2, 4, 8) if d < st.readers)
    if st.readers == 1:  # only when no deeper depth is within 10%
        assert all(st.reader_probe[str(d)] < 0.9 * best + 1e-3 for d in (2, 4, 8))
    fetch = Fetch(t, 4, layer=1)
    fetch({5: 0, 9: 3, 11: 1})
    assert st.failed is None and (st.fetches, st.reads) == (1, 3)
    for e, slot in ((5, 0), (9, 3), (11, 1)):
        t.assert_slot_holds(1, slot, e)
    assert st.size_readers() is None  # requests were made: the server keeps its seq

    monkeypatch.setenv("VLLM_EXPERT_PAGER_READ_WORKERS", "3")
    t2 = tiers(layers=1, experts=6, ram=2)
    assert t2.store.readers == 3
    t2.store.sync()
    assert t2.store.readers == 3 and t2.store.reader_probe is None


@pytest.mark.parametrize("compress", [True, False], ids=["compressed", "raw"])
def test_decode_step_copies_ram_rows_while_the_host_reads(tiers, compress):
    """The decode sequence of one layer (experts.py:427-446) in a hipGraph:
    gather the experts in RAM while the same launch publishes and waits for
    the SSD read, expand them, then gather and expand the ones read. Every
    slab row ends up the expert's raw row and every scale row its scales."""
    from vllm_expert_pager import codec, gather

    t = tiers(compress)
    st = t.store
    layer, S = 1, 3
    dev = torch.device("cuda")
    src = [st.view[name] for name in NAMES]
    cache = [torch.zeros((S, n // 4), dtype=torch.int32, device=dev) for n in NAMES.values()]
    slab = [torch.zeros((S, n), dtype=torch.uint8, device=dev) for n in NAMES.values()]
    staging = [torch.zeros((S, st.pitch[name]), dtype=torch.uint8, device=dev) for name in NAMES]
    scales = [torch.arange(E * 8, dtype=torch.int32, device=dev).view(E, 8) * (i + 3) for i in range(2)]
    scale_slab = [torch.zeros((S, 8), dtype=torch.int32, device=dev) for _ in range(2)]
    todo = torch.full((S,), -1, dtype=torch.int64, device=dev)
    ssd = torch.full((S,), -1, dtype=torch.int64, device=dev)
    dst_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    no_cache = torch.full((E,), -1, dtype=torch.int64, device=dev)
    src_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    lut = st.layer_lut(layer)
    rows = (src, cache, [s.view(torch.int32) for s in slab],
            [s.view(torch.int32) for s in staging] if compress else None, scales, scale_slab)

    def step():
        gather.gather_rows(todo, dst_row, no_cache, src_row, layer * R, *rows, fetch=(ssd, layer, st))
        if compress:
            codec.decode_rows(todo, dst_row, no_cache, staging, slab, lut, skip=ssd)
        gather.gather_rows(ssd, dst_row, no_cache, src_row, layer * R, *rows)
        if compress:
            codec.decode_rows(ssd, dst_row, no_cache, staging, slab, lut)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        step()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step()
    torch.cuda.synchronize()
    rng = np.random.default_rng(9)
    for i in range(6):
        # Two experts in RAM (warm-start slots hold experts 0..R-1) and one
        # read from the paging file into a third slot.
        in_ram = rng.choice(R, size=2, replace=False).tolist()
        free = int(rng.choice([s for s in range(R) if s not in in_ram]))
        from_ssd = int(rng.integers(R, E))
        experts = [in_ram[0], from_ssd, in_ram[1]]
        slab_row = {in_ram[0]: 2, from_ssd: 0, in_ram[1]: 1}
        ram_slot = {in_ram[0]: in_ram[0], from_ssd: free, in_ram[1]: in_ram[1]}
        todo.copy_(torch.tensor(experts, device=dev))
        ssd.copy_(torch.tensor([from_ssd, -1, -1], device=dev))
        for e in experts:
            dst_row[e] = slab_row[e]
            src_row[e] = ram_slot[e]
        for s in slab:
            s.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert st.failed is None, st.failed
        for k in range(2):
            for e in experts:
                r = slab_row[e]
                assert np.array_equal(slab[k][r].cpu().numpy(), t.raw(layer, e, k)), f"step {i} name {k} expert {e}"
                assert torch.equal(scale_slab[k][r], scales[k][e])
        t.assert_slot_holds(layer, free, from_ssd)
        for e in in_ram:
            t.assert_slot_holds(layer, e, e)
        # Give the slot back its warm-start expert for the next step.
        for k, name in enumerate(NAMES):
            st.pinned[name][layer * R + free].view(torch.uint8).copy_(torch.from_numpy(t.record(layer, free, k)))
    assert st.fetches == 6 and st.reads == 6


def test_a_failed_read_is_reported_and_releases_the_wait(tiers):
    t = tiers()
    fetch = Fetch(t, R, layer=1)
    fetch.todo.copy_(torch.tensor([5, 6, -1, -1], device="cuda"))
    fetch.slot[5] = 2
    fetch.slot[6] = 10**6  # outside the RAM tier
    fetch.graph.replay()
    torch.cuda.synchronize()
    assert t.store.failed is not None and "outside the RAM tier" in t.store.failed, t.store.failed
    t.assert_slot_holds(1, 2, 5)  # the good read of the same request still landed
    assert t.store.fetches == 1


def test_a_slow_host_sees_the_request_again(tiers, fast_timing):
    t = tiers()
    fetch = Fetch(t, R, layer=0)
    t.store.test_delay(0.15)  # three re-publish intervals, well short of the give-up
    try:
        fetch({8: 3})
    finally:
        t.store.test_delay(0.0)
    assert t.store.failed is None, t.store.failed
    republished = int(t.store.req[t.store.retry_at])
    assert 1 <= republished < 8 and int(t.store.req[t.store.giveup_at]) == 0
    assert (t.store.fetches, t.store.reads) == (1, 1)  # served once, however often it was re-published
    t.assert_slot_holds(0, 3, 8)


def test_a_host_that_never_answers_cannot_hold_the_gpu(tiers, fast_timing):
    t = tiers()
    fetch = Fetch(t, R, layer=0)
    t.store.test_delay(30.0)
    try:
        waited = fetch({9: 0})
    finally:
        t.store.test_delay(0.0)
    assert waited < 5.0, f"the fetch waited {waited:.1f} s"
    assert int(t.store.req[t.store.giveup_at]) == 1 and int(t.store.req[t.store.retry_at]) == 8
    deadline = time.time() + 10
    while t.store.fetches < 1 and time.time() < deadline:  # the host serves it once its delay is cleared
        time.sleep(0.01)
    assert t.store.fetches == 1 and t.store.missed == 0


def test_the_host_rewrites_done_when_the_republish_count_moves(tiers):
    t = tiers()
    fetch = Fetch(t, R, layer=0)
    fetch({4: 0})
    served = int(t.store.done[0])
    assert served == int(t.store.seq)
    t.store.done[0] = 0  # as if the GPU had never seen the write
    t.store.req[t.store.retry_at] += 1
    deadline = time.time() + 2.0
    while int(t.store.done[0]) != served and time.time() < deadline:
        time.sleep(0.005)
    assert int(t.store.done[0]) == served


def test_prefill_tickets_publish_ahead_of_the_wait(tiers):
    """The overflow path's order (experts.py:538-560): chunk k+1's read is
    published before chunk k's wait, alternating two tickets."""
    from vllm_expert_pager import gather

    t = tiers(layers=1)
    st = t.store
    row = torch.zeros((E,), dtype=torch.int64, device="cuda")
    row[torch.tensor([4, 5, 6, 7], device="cuda")] = torch.tensor([0, 1, 2, 3], device="cuda")
    chunks = [torch.tensor(c, device="cuda") for c in ([4, -1], [-1, -1], [5, 6], [7, -1])]
    ticket = lambda k: st.ticket_chunk[k % 2 : k % 2 + 1]  # noqa: E731
    gather.fetch_publish_rows(chunks[0], row, 0, 0, st, ticket(0))
    for k in range(len(chunks)):
        if k + 1 < len(chunks):
            gather.fetch_publish_rows(chunks[k + 1], row, 0, 0, st, ticket(k + 1))
        gather.fetch_wait_rows(chunks[k], st, ticket(k))
    torch.cuda.synchronize()
    assert st.failed is None, st.failed
    assert (st.fetches, st.reads) == (3, 4)  # the empty chunk published nothing
    for e, s in ((4, 0), (5, 1), (6, 2), (7, 3)):
        t.assert_slot_holds(0, s, e)


def test_a_request_longer_than_a_ring_slot(tiers):
    """A prefill chunk lists W entries, which may exceed the ring's slot of
    next_pow2(E) entries; its experts sit below E, and only the first
    `block` entries are published (the reference's kernels mask to BLOCK,
    gather.py:216)."""
    from vllm_expert_pager import gather

    t = tiers(layers=1)
    st = t.store
    assert st.block == 16
    todo = torch.full((40,), -1, dtype=torch.int64, device="cuda")
    todo[:3] = torch.tensor([5, 8, 9], device="cuda")
    todo[30] = 6  # past the slot: not published
    row = torch.zeros((E,), dtype=torch.int64, device="cuda")
    row[torch.tensor([5, 8, 9, 6], device="cuda")] = torch.tensor([1, 2, 3, 0], device="cuda")
    gather.fetch_publish_rows(todo, row, 0, 0, st, st.ticket_chunk[:1])
    gather.fetch_wait_rows(todo, st, st.ticket_chunk[:1])
    torch.cuda.synchronize()
    assert st.failed is None and (st.fetches, st.reads) == (1, 3)
    for e, s in ((5, 1), (8, 2), (9, 3), (0, 0)):
        t.assert_slot_holds(0, s, e)


def test_the_pinned_tier_is_exactly_rows_times_pitch():
    """Each weight's RAM tier is one hipHostMalloc of rows x pitch bytes (a
    1.5 GiB tier is not rounded up to 2 GiB, unlike a caching host
    allocator's block), and the GPU reads its last row."""
    from vllm_expert_pager import gather
    from vllm_expert_pager.store import Store

    dev = torch.device("cuda")
    nbytes = 3 * 2**20
    experts = 511  # 511 expert rows + 1 working row = 512 rows of 3 MiB
    st = Store(1, experts, experts, 1, {"w13_weight": nbytes}, False, 1.0, None, dev)
    try:
        assert [b.nbytes for b in st._buffers if b.nbytes >= nbytes] == [512 * nbytes]
        last = experts - 1
        want = _tiers.expert_row(0, last, 0, nbytes)
        st.write(0, last, "w13_weight", torch.from_numpy(want))
        todo = torch.tensor([last], dtype=torch.int64, device=dev)
        slab = [torch.zeros((1, nbytes // 4), dtype=torch.int32, device=dev)]
        scales = [torch.ones((experts, 4), dtype=torch.int32, device=dev)]
        gather.gather_rows(todo, torch.zeros((experts,), dtype=torch.int64, device=dev),
                           torch.full((experts,), -1, dtype=torch.int64, device=dev),
                           torch.arange(experts, dtype=torch.int64, device=dev), 0, [st.view["w13_weight"]],
                           slab, slab, None, scales, [torch.zeros((1, 4), dtype=torch.int32, device=dev)])
        torch.cuda.synchronize()
        assert np.array_equal(slab[0][0].view(torch.uint8).cpu().numpy(), want)
    finally:
        st.close()


def test_gpu_rows_are_encoded_as_the_host_encodes_them(tmp_path):
    """write_rows of GPU rows (the GPU encoder) leaves the RAM tier, the LUTs
    and the paging file byte-equal to per-expert writes of host rows (the
    host encoder)."""
    from vllm_expert_pager.store import Store

    dev = torch.device("cuda")
    stores = [Store(1, E, R, 2, NAMES, True, 1.0, str(tmp_path / f"{k}.bin"), dev) for k in "ab"]
    try:
        for i, (name, nbytes) in enumerate(NAMES.items()):
            rows = np.stack([_tiers.expert_row(0, e, i, nbytes) for e in range(E)])
            for e in range(E):
                stores[0].write(0, e, name, torch.from_numpy(rows[e]))
            stores[1].write_rows(0, name, torch.from_numpy(rows).to(dev))
        torch.cuda.synchronize()
        for name in NAMES:
            assert torch.equal(stores[0].pinned[name][:R], stores[1].pinned[name][:R]), name
        assert torch.equal(stores[0].lut.cpu(), stores[1].lut.cpu())
        assert (tmp_path / "a.bin").read_bytes() == (tmp_path / "b.bin").read_bytes()
    finally:
        for st in stores:
            st.close()


def test_the_store_refuses_bad_layouts(tmp_path):
    from vllm_expert_pager.store import Store

    dev = torch.device("cuda")
    path = str(tmp_path / "paging.bin")
    with pytest.raises(ValueError, match="RAM_SLOTS must be in"):
        Store(1, 4, 5, 2, NAMES, True, 1.0, None, dev)
    with pytest.raises(ValueError, match="SSD_PATH is required"):
        Store(1, 4, 2, 2, NAMES, True, 1.0, None, dev)
    with pytest.raises(ValueError, match="not a multiple"):
        Store(1, 4, 4, 2, {"w2_weight": 1000}, True, 1.0, None, dev)
    with open(path, "wb") as f:
        f.write(b"something else")
    with pytest.raises(FileExistsError):
        Store(1, 4, 2, 2, NAMES, True, 1.0, path, dev)
    os.remove(path)


@pytest.mark.parametrize("where", ["host", "gpu"])
def test_a_row_over_its_pitch_names_the_ratio_it_needs(tmp_path, where):
    from vllm_expert_pager.store import Store

    st = Store(1, 2, 1, 2, NAMES, True, 0.5, str(tmp_path / "p.bin"), torch.device("cuda"))
    try:
        noise = torch.from_numpy(np.random.default_rng(0).integers(0, 256, NAMES["w2_weight"], dtype=np.uint8))
        row = noise.cuda() if where == "gpu" else noise
        with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
            st.write(0, 0, "w2_weight", row)
        if where == "gpu":
            with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
                st.write_rows(0, "w2_weight", row.view(1, -1))
    finally:
        st.close()
