"""GPU round trip of the Store, the fetch ring and the host server.

Restates the reference's tests/test_store.py: the GPU publishes a request
into pinned memory, the C++ server preadv's records from the paging file
into RAM-tier rows, the GPU sees done; driven through hipGraph replay, and
combined with the gather + decode launches of the decode step. A slow host
(test delay) makes the fetch re-publish; a host that never answers makes it
give up after a bounded wait (the kernel's own deadline, never a hang).
"""

import os
import time

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

L, E, R = 2, 8, 4
GROUP = 512 * 32
ROW_BYTES = {"w13_weight": 2 * GROUP, "w2_weight": GROUP}
PITCH = 1.0
WORKING_ROWS = 2


def _mods():
    from vllm_expert_pager import codec, gather
    from vllm_expert_pager.store import _READ_WORKERS, Store

    return codec, gather, Store, _READ_WORKERS


def pattern(layer, expert, name):
    return torch.full((ROW_BYTES[name] // 4,), layer * 1000 + expert * 10 + len(name), dtype=torch.int32)


def encoded(store, layer, expert, name):
    codec = _mods()[0]
    row = pattern(layer, expert, name)
    if not store.compress:
        return row
    rec, _ = codec.encode(row.view(torch.uint8), store.pitch[name])
    return rec.view(torch.int32)


def make_store(tmp_path, num_layers, num_experts, ram_slots, compress=True):
    Store = _mods()[2]
    s = Store(num_layers, num_experts, ram_slots, WORKING_ROWS, ROW_BYTES, compress, PITCH,
              str(tmp_path / "expert_pager.bin"), torch.device("cuda"))
    for layer in range(num_layers):
        for e in range(num_experts):
            for name in ROW_BYTES:
                s.write(layer, e, name, pattern(layer, e, name))
    return s


@pytest.fixture
def make(tmp_path):
    made = []

    def _make(*args, **kwargs):
        s = make_store(tmp_path, *args, **kwargs)
        made.append(s)
        return s

    yield _make
    for s in made:
        s.close()


@pytest.fixture(params=[True, False], ids=["compressed", "raw"])
def store(make, request):
    return make(L, E, R, compress=request.param)


def capture_fetch(store, todo, row, layer):
    gather = _mods()[1]
    base = layer * store.ram_slots
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        gather.fetch_rows(todo, row, base, layer, store)  # warm-up (empty request)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            gather.fetch_rows(todo, row, base, layer, store)
    torch.cuda.synchronize()
    return g


def test_warm_start_rows(store):
    for layer in range(L):
        for e in range(R):
            for name in ROW_BYTES:
                assert torch.equal(store.pinned[name][layer * R + e], encoded(store, layer, e, name))


def test_fetch_reads_missing_experts_in_graph(store):
    dev = torch.device("cuda")
    todo = torch.full((R,), -1, dtype=torch.int64, device=dev)
    row = torch.zeros((E,), dtype=torch.int64, device=dev)
    layer = 1
    g = capture_fetch(store, todo, row, layer)
    for i in range(20):
        a, b = 4 + i % 4, 4 + (i + 1) % 4
        sa, sb = i % R, (i + 1) % R
        todo.copy_(torch.tensor([a, b, -1, -1], device=dev))
        row[a], row[b] = sa, sb
        g.replay()
        torch.cuda.synchronize()
        assert store.failed is None, store.failed
        for name in ROW_BYTES:
            assert torch.equal(store.pinned[name][layer * R + sa], encoded(store, layer, a, name))
            assert torch.equal(store.pinned[name][layer * R + sb], encoded(store, layer, b, name))
    assert store.fetches == 20 and store.reads == 40
    seq_before = int(store.seq)
    todo.fill_(-1)
    g.replay()
    torch.cuda.synchronize()
    assert int(store.seq) == seq_before and store.fetches == 20  # an empty request never reaches the host


def test_fetch_gathers_ram_hits_while_reading_ssd(store):
    codec, gather, _, _ = _mods()
    dev = torch.device("cuda")
    layer, S = 1, 3
    base = layer * R
    src = [store.view[name] for name in ROW_BYTES]
    cache = [torch.zeros((S, n // 4), dtype=torch.int32, device=dev) for n in ROW_BYTES.values()]
    dst = [torch.zeros((S, n), dtype=torch.uint8, device=dev) for n in ROW_BYTES.values()]
    dst_rows = [d.view(torch.int32) for d in dst]
    staging = [torch.zeros((S, store.pitch[name]), dtype=torch.uint8, device=dev) for name in ROW_BYTES]
    stg = [t.view(torch.int32) for t in staging]
    scale = [torch.arange(E * 8, dtype=torch.int32, device=dev).view(E, 8) * (i + 1) for i in range(2)]
    scale_dst = [torch.zeros((S, 8), dtype=torch.int32, device=dev) for _ in range(2)]
    todo = torch.full((S,), -1, dtype=torch.int64, device=dev)
    ssd = torch.full((S,), -1, dtype=torch.int64, device=dev)
    dst_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    src_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    lut = store.layer_lut(layer)

    def step():
        stg_or_none = stg if store.compress else None
        gather.gather_rows(todo, dst_row, cache_row, src_row, base, src, cache, dst_rows, stg_or_none, scale,
                           scale_dst, fetch=(ssd, layer, store))
        if store.compress:
            codec.decode_rows(todo, dst_row, cache_row, staging, dst, lut, skip=ssd)
        gather.gather_rows(ssd, dst_row, cache_row, src_row, base, src, cache, dst_rows, stg_or_none, scale,
                           scale_dst)
        if store.compress:
            codec.decode_rows(ssd, dst_row, cache_row, staging, dst, lut)

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    for i in range(6):
        a, b, c = i % 2, 2, R + i % (E - R)
        todo.copy_(torch.tensor([a, c, b], device=dev))
        ssd.copy_(torch.tensor([c, -1, -1], device=dev))
        src_row[a], src_row[b], src_row[c] = a, b, R - 1
        dst_row[a], dst_row[c], dst_row[b] = 0, 1, 2
        dst[0].zero_(), dst[1].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert store.failed is None, store.failed
        for k, name in enumerate(ROW_BYTES):
            raw = [pattern(layer, x, name).view(torch.uint8).to(dev) for x in (a, c, b)]
            for rr in range(3):
                assert torch.equal(dst[k][rr], raw[rr]), f"iteration {i} name {name} row {rr}"
            assert torch.equal(scale_dst[k][0], scale[k][a])
            assert torch.equal(scale_dst[k][1], scale[k][c])
            assert torch.equal(scale_dst[k][2], scale[k][b])
    assert store.fetches == 6 and store.reads == 6


def test_fetch_reads_many_experts_at_once(make):
    _, _, _, workers = _mods()
    E2, R2 = 4 * workers, 2 * workers
    store = make(1, E2, R2)
    dev = torch.device("cuda")
    todo = torch.full((R2,), -1, dtype=torch.int64, device=dev)
    row = torch.zeros((E2,), dtype=torch.int64, device=dev)
    g = capture_fetch(store, todo, row, 0)
    missing = list(range(R2, E2))
    todo.copy_(torch.tensor(missing, device=dev))
    row[R2:] = torch.arange(R2, device=dev)
    g.replay()
    torch.cuda.synchronize()
    assert store.failed is None, store.failed
    assert store.fetches == 1 and store.reads == R2
    for s, e in enumerate(missing):
        for name in ROW_BYTES:
            assert torch.equal(store.pinned[name][s], encoded(store, 0, e, name))


def test_failed_read_releases_gpu(store):
    dev = torch.device("cuda")
    todo = torch.full((R,), -1, dtype=torch.int64, device=dev)
    row = torch.zeros((E,), dtype=torch.int64, device=dev)
    layer = 1
    g = capture_fetch(store, todo, row, layer)
    todo.copy_(torch.tensor([4, 5, -1, -1], device=dev))
    row[4], row[5] = 10**6, 0
    g.replay()
    torch.cuda.synchronize()
    assert store.failed is not None and "outside the RAM tier" in store.failed, store.failed
    for name in ROW_BYTES:
        assert torch.equal(store.pinned[name][layer * R + 0], encoded(store, layer, 5, name))


def test_slow_host_makes_the_fetch_republish_the_request(store):
    dev = torch.device("cuda")
    todo = torch.full((R,), -1, dtype=torch.int64, device=dev)
    row = torch.zeros((E,), dtype=torch.int64, device=dev)
    layer = 1
    g = capture_fetch(store, todo, row, layer)
    store.test_delay(1.5)  # longer than the re-publish interval (0.5 s)
    todo.copy_(torch.tensor([4, -1, -1, -1], device=dev))
    row[4] = 0
    g.replay()
    torch.cuda.synchronize()
    store.test_delay(0.0)
    assert store.failed is None, store.failed
    assert int(store.req[store.retry_at]) >= 1
    assert store.fetches == 1 and store.reads == 1
    for name in ROW_BYTES:
        assert torch.equal(store.pinned[name][layer * R], encoded(store, layer, 4, name))


def test_fetch_gives_up_when_the_host_never_answers(store):
    dev = torch.device("cuda")
    todo = torch.full((R,), -1, dtype=torch.int64, device=dev)
    row = torch.zeros((E,), dtype=torch.int64, device=dev)
    g = capture_fetch(store, todo, row, 1)
    store.test_delay(60.0)
    todo.copy_(torch.tensor([4, -1, -1, -1], device=dev))
    row[4] = 0
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    waited = time.perf_counter() - t0
    store.test_delay(0.0)
    assert waited < 30, f"the fetch waited {waited:.1f} s"
    assert int(store.req[store.giveup_at]) == 1
    assert int(store.req[store.retry_at]) >= 1
    for _ in range(500):
        if store.fetches == 1:
            break
        time.sleep(0.01)
    assert store.fetches == 1 and store.missed == 0


def test_serve_resends_done_when_the_fetch_is_still_spinning(store):
    dev = torch.device("cuda")
    todo = torch.full((R,), -1, dtype=torch.int64, device=dev)
    row = torch.zeros((E,), dtype=torch.int64, device=dev)
    g = capture_fetch(store, todo, row, 1)
    todo.copy_(torch.tensor([4, -1, -1, -1], device=dev))
    row[4] = 0
    g.replay()
    torch.cuda.synchronize()
    served = int(store.done[0])
    assert served > 0
    store.done[0] = 0
    store.req[store.retry_at] += 1
    for _ in range(200):
        if int(store.done[0]) == served:
            break
        time.sleep(0.01)
    assert int(store.done[0]) == served


def test_publish_and_wait_with_two_tickets(store):
    """The prefill order: publish chunk k+1's read before waiting for chunk k's."""
    gather = _mods()[1]
    dev = torch.device("cuda")
    layer = 0
    tickets = store.ticket_chunk
    row = torch.zeros((E,), dtype=torch.int64, device=dev)
    row[4], row[5], row[6] = 0, 1, 2
    chunks = [torch.tensor([4, -1], device=dev), torch.tensor([5, 6], device=dev), torch.tensor([-1, -1], device=dev)]
    gather.fetch_publish_rows(chunks[0], row, 0, layer, store, tickets[0:1])
    for k in range(3):
        if k + 1 < 3:
            gather.fetch_publish_rows(chunks[k + 1], row, 0, layer, store, tickets[(k + 1) % 2:(k + 1) % 2 + 1])
        gather.fetch_wait_rows(chunks[k], store, tickets[k % 2:k % 2 + 1])
    torch.cuda.synchronize()
    assert store.failed is None, store.failed
    assert store.fetches == 2 and store.reads == 3
    for e, r in ((4, 0), (5, 1), (6, 2)):
        for name in ROW_BYTES:
            assert torch.equal(store.pinned[name][r], encoded(store, layer, e, name))


def test_large_pinned_tier_is_allocated_at_its_size():
    """Counterpart of the reference's test_large_pinned_is_not_rounded_to_pow2
    (tests/test_store.py:360-371). There the RAM tier came from torch's
    caching host allocator, which rounds large blocks up to a power of two.
    Here each name's tier is one hipHostMalloc of exactly rows x pitch bytes:
    a 1.5 GiB tier reports 1.5 GiB, and the GPU reads its last row."""
    _, gather, Store, _ = _mods()
    dev = torch.device("cuda")
    row = 3 * 2**20
    E = 511  # 511 RAM rows + 1 working row = 512 rows of 3 MiB
    s = Store(1, E, E, 1, {"w13_weight": row}, False, 1.0, None, dev)
    try:
        assert [b.nbytes for b in s._buffers if b.nbytes >= row] == [3 * 2**29]
        e = E - 1
        want = torch.arange(row // 4, dtype=torch.int32) * 7 + 3
        s.write(0, e, "w13_weight", want)
        todo = torch.tensor([e], dtype=torch.int64, device=dev)
        dst_row = torch.zeros((E,), dtype=torch.int64, device=dev)
        cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
        src_row = torch.arange(E, dtype=torch.int64, device=dev)
        cache = [torch.zeros((1, row // 4), dtype=torch.int32, device=dev)]
        dst = [torch.zeros((1, row // 4), dtype=torch.int32, device=dev)]
        scale = [torch.ones((E, 4), dtype=torch.int32, device=dev)]
        sdst = [torch.zeros((1, 4), dtype=torch.int32, device=dev)]
        gather.gather_rows(todo, dst_row, cache_row, src_row, 0, [s.view["w13_weight"]], cache, dst, None, scale,
                           sdst)
        torch.cuda.synchronize()
        assert torch.equal(dst[0][0].cpu(), want)
    finally:
        s.close()


def test_rejects_foreign_file(tmp_path):
    Store = _mods()[2]
    path = tmp_path / "expert_pager.bin"
    path.write_bytes(b"not a paging file")
    with pytest.raises(FileExistsError):
        Store(L, E, R, WORKING_ROWS, ROW_BYTES, True, PITCH, str(path), torch.device("cuda"))


def test_rejects_rows_over_pitch(tmp_path):
    Store = _mods()[2]
    s = Store(1, 2, 1, WORKING_ROWS, ROW_BYTES, True, 0.5, str(tmp_path / "expert_pager.bin"), torch.device("cuda"))
    try:
        row = torch.randint(-(2**31), 2**31 - 1, (ROW_BYTES["w2_weight"] // 4,), dtype=torch.int32)
        with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
            s.write(0, 0, "w2_weight", row)
    finally:
        s.close()


def test_rows_over_pitch_on_the_gpu(tmp_path):
    Store = _mods()[2]
    s = Store(1, 2, 1, WORKING_ROWS, ROW_BYTES, True, 0.5, str(tmp_path / "expert_pager.bin"), torch.device("cuda"))
    try:
        row = torch.randint(-(2**31), 2**31 - 1, (ROW_BYTES["w2_weight"] // 4,), dtype=torch.int32).cuda()
        with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
            s.write(0, 0, "w2_weight", row)
        with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
            s.write_rows(0, "w2_weight", row.view(1, -1))
    finally:
        s.close()


def test_gpu_rows_store_the_host_encoding(tmp_path):
    """write_rows of GPU rows (GPU encoder) leaves the RAM tier, the LUTs and the
    paging file byte-equal to per-expert writes of host rows (host encoder)."""
    Store = _mods()[2]
    dev = torch.device("cuda")
    rng = np.random.default_rng(3)
    rows = {}
    for name, nb in ROW_BYTES.items():
        exp = rng.choice(16, size=(E, nb), p=np.array([0] * 8 + [1, 2, 4, 8, 16, 32, 24, 13], float) / 100)
        rows[name] = torch.from_numpy((exp.astype(np.uint8) << 3) | (rng.integers(0, 256, (E, nb), dtype=np.uint8) & 0x87))
    a = Store(1, E, R, WORKING_ROWS, ROW_BYTES, True, PITCH, str(tmp_path / "a.bin"), dev)
    b = Store(1, E, R, WORKING_ROWS, ROW_BYTES, True, PITCH, str(tmp_path / "b.bin"), dev)
    try:
        for name in ROW_BYTES:
            for e in range(E):
                a.write(0, e, name, rows[name][e])
            b.write_rows(0, name, rows[name].to(dev))
        torch.cuda.synchronize()
        for name in ROW_BYTES:
            assert torch.equal(a.pinned[name][:R].cpu(), b.pinned[name][:R].cpu()), name
        assert torch.equal(a.lut.cpu(), b.lut.cpu())
        assert (tmp_path / "a.bin").read_bytes() == (tmp_path / "b.bin").read_bytes()
    finally:
        a.close()
        b.close()


def test_settings_validation(tmp_path):
    Store = _mods()[2]
    with pytest.raises(ValueError, match="RAM_SLOTS"):
        Store(1, 4, 5, 2, ROW_BYTES, True, 1.0, None, torch.device("cuda"))
    with pytest.raises(ValueError, match="SSD_PATH"):
        Store(1, 4, 2, 2, ROW_BYTES, True, 1.0, None, torch.device("cuda"))
    with pytest.raises(ValueError, match="not a multiple"):
        Store(1, 4, 4, 2, {"w2_weight": 1000}, True, 1.0, None, torch.device("cuda"))
