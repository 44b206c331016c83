"""GPU parity of the slot gather (bit-exact bytes) against the oracle.

Restates the reference's known answer (tests/test_gather.py) and adds random
traces in both modes (compressed -> staging, raw -> slab), RAM-tier rows in
pinned host memory, cache-slab sources, and out-of-range rows that must be
skipped without touching memory.
"""

import numpy as np
import pytest
import torch

from oracle import gather_ref

pytestmark = pytest.mark.gpu


def _gather():
    from vllm_expert_pager import gather

    return gather


def test_known_answer():
    gather = _gather()
    dev = torch.device("cuda")
    E, S = 8, 4
    WORDS, PITCH, SCALE_WORDS = (8192, 4096), (6144, 3072), (32, 16)
    g = torch.Generator(device=dev).manual_seed(0)

    def rand(*shape):
        return torch.randint(-(2**31), 2**31 - 1, shape, dtype=torch.int32, device=dev, generator=g)

    src = [rand(16, p) for p in PITCH]
    cache = [rand(S, w) for w in WORDS]
    dst = [torch.zeros((S, w), dtype=torch.int32, device=dev) for w in WORDS]
    stg = [torch.zeros((S, p), dtype=torch.int32, device=dev) for p in PITCH]
    scale = [rand(E, w) for w in SCALE_WORDS]
    scale_dst = [torch.zeros((S, w), dtype=torch.int32, device=dev) for w in SCALE_WORDS]
    todo = torch.tensor([3, 5, -1, -1], dtype=torch.int64, device=dev)
    dst_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    dst_row[3], dst_row[5] = 1, 2
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    cache_row[5] = 0
    src_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    src_row[3] = 7
    gather.gather_rows(todo, dst_row, cache_row, src_row, 2, src, cache, dst, stg, scale, scale_dst)
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(stg[i][0], src[i][9])
        assert torch.equal(dst[i][2], cache[i][0])
        assert torch.equal(scale_dst[i][1], scale[i][3])
        assert torch.equal(scale_dst[i][2], scale[i][5])
        assert not dst[i][0].any() and not dst[i][1].any() and not dst[i][3].any()
        assert not stg[i][1:].any()
        assert not scale_dst[i][0].any() and not scale_dst[i][3].any()


@pytest.mark.parametrize("compress", [True, False])
@pytest.mark.parametrize("blocks", [1, 7, 32])
def test_random_against_oracle(compress, blocks):
    gather = _gather()
    from vllm_expert_pager import _native as nat

    nat.call("xp_gather_set_blocks", blocks)
    rng = np.random.default_rng(10 + blocks + compress)
    E, S, R, base = 64, 12, 40, 40
    N = (49152, 20480)  # bytes per raw row (w13, w2)
    P = (36864, 16384) if compress else N
    SB = (512, 256)
    src_np = [rng.integers(0, 256, (2 * R, p), dtype=np.uint8) for p in P]
    src = [torch.from_numpy(a).pin_memory() for a in src_np]  # pinned host RAM tier
    cache_np = [rng.integers(0, 256, (S, n), dtype=np.uint8) for n in N]
    scale_np = [rng.integers(0, 256, (E, sb), dtype=np.uint8) for sb in SB]
    try:
        for trial in range(6):
            K = int(rng.integers(1, S + 1))
            todo_np = np.full(K, -1, np.int64)
            experts = rng.choice(E, size=K, replace=False)
            live = rng.random(K) < 0.8
            todo_np[live] = experts[live]
            dst_row_np = rng.integers(0, S, E).astype(np.int64)
            dst_row_np[experts] = rng.permutation(S)[:K]
            cache_row_np = np.where(rng.random(E) < 0.3, rng.integers(0, S, E), -1).astype(np.int64)
            src_row_np = rng.integers(0, R, E).astype(np.int64)
            dst_np = [rng.integers(0, 256, (S, n), dtype=np.uint8) for n in N]
            stg_np = [rng.integers(0, 256, (S, p), dtype=np.uint8) for p in P] if compress else None
            sdst_np = [rng.integers(0, 256, (S, sb), dtype=np.uint8) for sb in SB]
            d = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
            dst = [d(a) for a in dst_np]
            stg = [d(a) for a in stg_np] if compress else None
            sdst = [d(a) for a in sdst_np]
            gather.gather_rows(
                d(todo_np), d(dst_row_np), d(cache_row_np), d(src_row_np), base,
                src, [d(a) for a in cache_np], dst, stg, [d(a) for a in scale_np], sdst,
            )
            torch.cuda.synchronize()
            gather_ref.gather_rows_ref(todo_np, dst_row_np, cache_row_np, src_row_np, base, src_np, cache_np,
                                       dst_np, stg_np, scale_np, sdst_np)
            for i in range(2):
                np.testing.assert_array_equal(dst[i].cpu().numpy(), dst_np[i], err_msg=f"trial {trial} dst {i}")
                np.testing.assert_array_equal(sdst[i].cpu().numpy(), sdst_np[i], err_msg=f"trial {trial} scale {i}")
                if compress:
                    np.testing.assert_array_equal(stg[i].cpu().numpy(), stg_np[i], err_msg=f"trial {trial} stg {i}")
    finally:
        nat.call("xp_gather_set_blocks", 32)


def test_out_of_range_rows_are_skipped():
    gather = _gather()
    dev = torch.device("cuda")
    E, S = 4, 2
    src = [torch.arange(4 * 64, dtype=torch.int32, device=dev).view(4, 64)]
    cache = [torch.zeros((S, 64), dtype=torch.int32, device=dev)]
    dst = [torch.zeros((S, 64), dtype=torch.int32, device=dev)]
    scale = [torch.ones((E, 4), dtype=torch.int32, device=dev)]
    sdst = [torch.zeros((S, 4), dtype=torch.int32, device=dev)]
    todo = torch.tensor([0, 1], dtype=torch.int64, device=dev)
    dst_row = torch.tensor([5, 1, 0, 0], dtype=torch.int64, device=dev)  # expert 0 -> row 5 (out of range)
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    src_row = torch.tensor([0, 100, 0, 0], dtype=torch.int64, device=dev)  # expert 1 -> RAM row 100 (out of range)
    gather.gather_rows(todo, dst_row, cache_row, src_row, 0, src, cache, dst, None, scale, sdst)
    torch.cuda.synchronize()
    assert not dst[0].any()


@pytest.mark.parametrize("compress", [True, False])
def test_negative_destination_rows_are_skipped(compress):
    """An expert whose dst_row is negative is skipped whole: no slab row, no
    staging row and no scale row is written (the reference clamps it to row
    0; a listing from acquire or plan_chunks never carries one). Both the
    gather and the decode launch follow the rule."""
    gather = _gather()
    from vllm_expert_pager import codec

    from oracle import codec_ref

    dev = torch.device("cuda")
    E, S, N = 4, 3, 16384
    rng = np.random.default_rng(2)
    raw = [(rng.integers(0, 256, N, dtype=np.uint8) & 0x87) | (rng.integers(9, 14, N, dtype=np.uint8) << 3)
           for _ in range(E)]
    P = codec_ref.pitch_of(N, 1.0, 4096) if compress else N
    recs = [codec_ref.encode(r, P) for r in raw] if compress else None
    src = [torch.from_numpy(np.stack([rc for rc, _ in recs] if compress else raw)).pin_memory()]
    cache = [torch.zeros((S, N), dtype=torch.uint8, device=dev)]
    dst = [torch.full((S, N), 0x5A, dtype=torch.uint8, device=dev)]
    stg = [torch.full((S, P), 0x5A, dtype=torch.uint8, device=dev)] if compress else None
    scale = [torch.arange(E * 4, dtype=torch.int32, device=dev).view(E, 4) + 1]
    sdst = [torch.zeros((S, 4), dtype=torch.int32, device=dev)]
    todo = torch.tensor([2, 0, 3], dtype=torch.int64, device=dev)
    dst_row = torch.tensor([-1, 0, 2, -7], dtype=torch.int64, device=dev)  # experts 0 and 3: negative
    no_cache = torch.full((E,), -1, dtype=torch.int64, device=dev)
    src_row = torch.arange(E, dtype=torch.int64, device=dev)
    gather.gather_rows(todo, dst_row, no_cache, src_row, 0, src, cache,
                       [t.view(torch.int32) for t in dst] if not compress else dst,
                       [t.view(torch.int32) for t in stg] if compress else None, scale, sdst)
    if compress:
        lut = torch.from_numpy(np.stack([l for _, l in recs])).view(E, 1, 512).to(dev)
        codec.decode_rows(todo, dst_row, no_cache, stg, dst, lut)
    torch.cuda.synchronize()
    got = dst[0].cpu().numpy()
    assert np.array_equal(got[2], raw[2])                      # expert 2 -> row 2
    assert (got[0] == 0x5A).all() and (got[1] == 0x5A).all()   # rows 0 and 1 untouched
    assert torch.equal(sdst[0][2], scale[0][2]) and not sdst[0][:2].any()
    if compress:
        s = stg[0].cpu().numpy()
        assert np.array_equal(s[0], recs[2][0])                # todo entry 0 staged
        assert (s[1] == 0x5A).all() and (s[2] == 0x5A).all()   # entries 1 and 2 (negative rows) not staged


def test_cached_only_copies_cached_experts():
    """gather_rows(cached_only=True) (zero staging rows) copies the experts
    with cache_row >= 0 raw from the cache slab, with their scales, and
    leaves every RAM-tier expert to the decoder: no slab, staging or scale
    row of those is written. With the RAM-tier ones expanded by
    decode_rows_from_ram, the slab matches a staging gather + decode."""
    gather = _gather()
    from vllm_expert_pager import codec

    from oracle import codec_ref

    dev = torch.device("cuda")
    E, S, N = 6, 5, 16384
    rng = np.random.default_rng(5)
    raw = [(rng.integers(0, 256, N, dtype=np.uint8) & 0x87) | (rng.integers(9, 14, N, dtype=np.uint8) << 3)
           for _ in range(E)]
    P = codec_ref.pitch_of(N, 1.0, 4096)
    recs = [codec_ref.encode(r, P) for r in raw]
    src = [torch.from_numpy(np.stack([rc for rc, _ in recs])).pin_memory()]
    lut = torch.from_numpy(np.stack([l for _, l in recs])).view(E, 1, 512).to(dev)
    cache = [torch.from_numpy(np.stack([raw[4], raw[1]])).to(dev)]  # experts 4 and 1 cached in rows 0, 1
    scale = [torch.arange(E * 4, dtype=torch.int32, device=dev).view(E, 4) + 1]
    todo = torch.tensor([1, 3, 4, 0], dtype=torch.int64, device=dev)
    dst_row = torch.tensor([1, 4, 9, 2, 0, 9], dtype=torch.int64, device=dev)  # 2 and 5 are not listed
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    cache_row[4], cache_row[1] = 0, 1
    src_row = torch.arange(E, dtype=torch.int64, device=dev)
    pitch_rows = [torch.zeros((1, P), dtype=torch.uint8, device=dev).view(torch.int32)]

    def fresh():
        return ([torch.full((S, N), 0x5A, dtype=torch.uint8, device=dev)],
                [torch.zeros((S, 4), dtype=torch.int32, device=dev)])

    dst, sdst = fresh()
    gather.gather_rows(todo, dst_row, cache_row, src_row, 0, src, cache, dst, pitch_rows, scale, sdst,
                       cached_only=True)
    torch.cuda.synchronize()
    got = dst[0].cpu().numpy()
    assert np.array_equal(got[0], raw[4]) and np.array_equal(got[4], raw[1])  # the cached experts
    for r in (1, 2, 3):
        assert (got[r] == 0x5A).all() and not sdst[0][r].any(), r              # RAM-tier ones untouched
    assert torch.equal(sdst[0][0], scale[0][4]) and torch.equal(sdst[0][4], scale[0][1])
    assert not pitch_rows[0].any()                                              # never written
    codec.decode_rows_from_ram(todo, dst_row, cache_row, src_row, 0, src, dst, lut, scale, sdst)
    ref, rsdst = fresh()
    stg = [torch.zeros((len(todo), P), dtype=torch.uint8, device=dev)]
    gather.gather_rows(todo, dst_row, cache_row, src_row, 0, src, cache, ref, [stg[0].view(torch.int32)], scale,
                       rsdst)
    codec.decode_rows(todo, dst_row, cache_row, stg, ref, lut)
    torch.cuda.synchronize()
    assert torch.equal(dst[0], ref[0]) and torch.equal(sdst[0], rsdst[0])
    assert np.array_equal(dst[0][2].cpu().numpy(), raw[3]) and np.array_equal(dst[0][1].cpu().numpy(), raw[0])
