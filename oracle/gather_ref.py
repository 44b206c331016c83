"""Oracle of the row movement on the paging path -- test infrastructure only.

  gather_rows_ref  byte semantics of gather_rows (gather.py:328-393): which
                   source row goes to which destination row, and the scale
                   copy; pinned by the reference's known answer
                   (tests/test_gather.py:19-61) restated in tests.
  decode_rows_ref  which staging row is expanded where (codec.py:297-327),
                   expanding with codec_ref; pinned by
                   tests/test_codec.py:118-154 restated in tests.
  simulate_working_step, check_layout, check_ram_rows
                   the reference's CPU simulator of the prefill chunk loop
                   (tests/test_table.py:200-281), over a TableRef.
"""

from __future__ import annotations

import numpy as np

from oracle import codec_ref


def gather_rows_ref(todo, dst_row, cache_row, src_row, base, src, cache, dst, stg, scale, scale_dst, skip=None):
    """Apply gather_rows to numpy byte arrays in place (lists per name)."""
    skip_set = set() if skip is None else {int(x) for x in skip if x >= 0}
    for j, e in enumerate(np.asarray(todo).tolist()):
        if e < 0 or e in skip_set:
            continue
        # The reference clamps a negative row to 0 (gather.py:130); the
        # listings acquire and plan_chunks hand over never carry one, and this
        # build skips such an expert (and a row past the destination) instead.
        drow = int(dst_row[e])
        if drow < 0 or drow >= dst[0].shape[0]:
            continue
        for n in range(len(dst)):
            if cache_row[e] >= 0:
                dst[n][drow] = cache[n][cache_row[e]]
            elif stg is not None:
                stg[n][j] = src[n][src_row[e] + base]
            else:
                dst[n][drow] = src[n][src_row[e] + base]
            scale_dst[n][drow] = scale[n][e]


def decode_rows_ref(todo, dst_row, cache_row, staging, dst, lut, skip=None, chunk=codec_ref.CHUNK):
    """Apply decode_rows to numpy byte arrays in place."""
    skip_set = set() if skip is None else {int(x) for x in skip if x >= 0}
    for j, e in enumerate(np.asarray(todo).tolist()):
        if e < 0 or e in skip_set or cache_row[e] >= 0:
            continue
        drow = int(dst_row[e])  # clamped to 0 by the reference (codec.py:272); skipped here
        if drow < 0 or drow >= dst[0].shape[0]:
            continue
        for n in range(len(dst)):
            N = dst[n].shape[1]
            dst[n][drow] = codec_ref.decode_fast(staging[n][j], lut[e, n], N, chunk)[0]


def check_layout(todo, ssd, W):
    """Experts with no wait are packed from the front; SSD reads start at the next chunk boundary."""
    ssd_set = {int(e) for e in ssd if e >= 0}
    first = [i for i, e in enumerate(np.asarray(todo).tolist()) if e >= 0 and e not in ssd_set]
    assert first == list(range(len(first)))
    at = [i for i, e in enumerate(np.asarray(ssd).tolist()) if e >= 0]
    boundary = -(-len(first) // W) * W
    assert at == list(range(boundary, boundary + len(at)))


def check_ram_rows(ram, rows, ram_base):
    for e in range(ram.num_experts):
        s = int(ram.slot_of[e])
        if s >= 0:
            assert rows[ram_base + s] == e, f"RAM row of expert {e} is stale"


def simulate_working_step(ram, vram, ids, rows, W, ram_base, working_base):
    """Run one working-slab step's chunk order on the CPU (tests/test_table.py:200-263).

    ``rows`` holds which expert each RAM-tier / shared row contains. Reads are
    assumed to land as soon as they are published (the harshest case for a
    read overwriting a copy source). Checks each chunk's working slab and
    expert_map; returns the experts read from SSD and src_row.
    """
    E = ram.num_experts
    need = ram.need_mask(ids)
    cached_row = vram.slot_of[:E].copy()
    before = ram.slot_of[:E].copy()
    if np.asarray(ids).size <= ram.num_slots:
        ram.acquire(ids)
    else:
        ram.seed(vram, ids, need)
    dst_row, src_row, maps, todo, ssd, late = ram.plan_chunks(before, need, cached_row, W, ram_base, working_base)
    N = maps.shape[0]
    assert N == -(-E // W) + 1
    assert todo.shape == ssd.shape == late.shape == (N * W,)
    check_layout(todo, ssd, W)

    def chunk(t, k):
        return [int(e) for e in t[k * W : (k + 1) * W] if e >= 0]

    working = np.full(W, -1)

    def copy(experts):
        for e in experts:
            working[dst_row[e]] = e if cached_row[e] >= 0 else rows[src_row[e]]

    def read(experts):
        for e in experts:
            rows[src_row[e]] = e

    read(chunk(ssd, 0))
    mapped = set()
    for k in range(N):
        copy(chunk(todo, k))
        if k + 1 < N:
            read(chunk(ssd, k + 1))
        copy(chunk(late, k))
        emap = maps[k]
        for e, r in enumerate(emap.tolist()):
            if r < 0:
                continue
            assert need[e], f"expert {e} is mapped in chunk {k} but not needed"
            assert r == dst_row[e] and working[r] == e, f"working row of expert {e} in chunk {k} is wrong"
            assert e not in mapped
            mapped.add(e)
        used = [r for r in emap.tolist() if r >= 0]
        assert len(used) == len(set(used))
    assert mapped == set(np.nonzero(need)[0].tolist())
    return [int(e) for e in ssd if e >= 0], src_row
