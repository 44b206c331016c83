"""GPU parity of the Huffman row expansion (bit-exact bytes).

Checks the decoder against the reference encoder's golden records, against
the oracle (round trips for the reference's four distributions), the
todo/skip/cache_row rules of the reference's tests/test_codec.py, full-size
synthetic expert rows (w13 2 MiB + w2 1 MiB of N(0, 0.02) weights quantised to
fp8 e4m3 with 128x128 block scales) in batches, and hipGraph replay.
"""

import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import codec_ref

pytestmark = pytest.mark.gpu

CHUNK = 64
N = 2 * CHUNK * 32
EXP_P = [0.0] * 4 + [0.001, 0.002, 0.004, 0.008, 0.016, 0.032, 0.064, 0.125, 0.228, 0.315, 0.188, 0.015]


def _codec():
    from vllm_expert_pager import codec

    return codec


def rows(seed, n=N, p=EXP_P):
    rng = np.random.default_rng(seed)
    p = np.asarray(p, np.float64)
    exp = rng.choice(16, size=n, p=p / p.sum()).astype(np.uint8)
    sm = rng.integers(0, 256, size=n, dtype=np.uint8) & 0x87
    return sm | (exp << 3)


def fp8_expert(seed, shape):
    """N(0, 0.02) weights quantised to e4m3 with 128x128 block scales, as uint8."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(shape, generator=g) * 0.02
    r, c = shape
    blk = w.view(r // 128, 128, c // 128, 128)
    s = blk.abs().amax(dim=(1, 3), keepdim=True).clamp(min=1e-12) / 448.0
    q = (blk / s).to(torch.float8_e4m3fn).view(r, c)
    return q.view(torch.uint8).numpy().reshape(-1)


def decode_one(codec, rec, lut, n, chunk, dst_row=0):
    dev = torch.device("cuda")
    stg = [torch.from_numpy(rec.reshape(1, -1)).to(dev)]
    dst = [torch.zeros((1, n), dtype=torch.uint8, device=dev)]
    lut_t = torch.from_numpy(lut.reshape(1, 1, -1)).to(dev)
    todo = torch.zeros((1,), dtype=torch.int64, device=dev)
    rowmap = torch.zeros((1,), dtype=torch.int64, device=dev)
    cache_row = torch.full((1,), -1, dtype=torch.int64, device=dev)
    codec.decode_rows(todo, rowmap, cache_row, stg, dst, lut_t, chunk=chunk)
    torch.cuda.synchronize()
    return dst[0][0].cpu().numpy()


def test_golden_records():
    codec = _codec()
    g = np.load(os.path.join(GOLDEN, "codec_vectors.npz"), allow_pickle=False)
    for name in g["cases"]:
        raw = g[f"{name}_raw"]
        out = decode_one(codec, g[f"{name}_record"], g[f"{name}_lut"], raw.size, int(g[f"{name}_chunk"]))
        np.testing.assert_array_equal(out, raw, err_msg=str(name))


@pytest.mark.parametrize("dist", ["realistic", "uniform", "geometric", "constant", "long_codes"])
# 128-byte stores for chunks of 128, 512 and 4096 (the largest chunk a
# record may use), 64-byte for 64 and 192, plain for 32 and 96
@pytest.mark.parametrize("chunk", [32, 64, 96, 128, 192, 512, 4096])
def test_round_trip(dist, chunk):
    codec = _codec()
    n = 2 * chunk * 32
    raw = {
        "realistic": lambda: rows(0, n),
        "uniform": lambda: rows(1, n, [1.0] * 16),
        "geometric": lambda: rows(2, n, [2.0**k for k in range(16)]),
        "constant": lambda: np.full(n, 13 << 3, np.uint8),
        # first half one exponent, second half uniform: the second half's codes
        # are long, so its groups carry more Huffman words than the LDS stage
        # holds at chunk 512
        "long_codes": lambda: np.concatenate([np.full(n // 2, 13 << 3, np.uint8), rows(5, n // 2, [1.0] * 16)]),
    }[dist]()
    pitch = codec_ref.pitch_of(n, 1.6, 4096)
    rec, lut = codec_ref.encode(raw, pitch, chunk)
    np.testing.assert_array_equal(decode_one(codec, rec, lut, n, chunk), raw)


@pytest.mark.parametrize("chunk", [64, 128, 512])
@pytest.mark.parametrize("groups", [1, 3, 5, 9])
def test_odd_group_counts(chunk, groups):
    """A wave decodes two groups side by side; with an odd group count the
    last wave's second group is a spare that must store nothing (the rows
    around the decoded one stay zero)."""
    codec = _codec()
    n = groups * chunk * 32
    raw = rows(20 + groups, n)
    pitch = codec_ref.pitch_of(n, 1.6, 4096)
    rec, lut = codec_ref.encode(raw, pitch, chunk)
    dev = torch.device("cuda")
    stg = [torch.from_numpy(rec.reshape(1, -1)).to(dev)]
    dst = [torch.zeros((3, n), dtype=torch.uint8, device=dev)]
    lut_t = torch.from_numpy(lut.reshape(1, 1, -1)).to(dev)
    todo = torch.zeros((1,), dtype=torch.int64, device=dev)
    rowmap = torch.ones((1,), dtype=torch.int64, device=dev)  # expert 0 -> row 1
    cache_row = torch.full((1,), -1, dtype=torch.int64, device=dev)
    codec.decode_rows(todo, rowmap, cache_row, stg, dst, lut_t, chunk=chunk)
    torch.cuda.synchronize()
    got = dst[0].cpu().numpy()
    np.testing.assert_array_equal(got[1], raw)
    assert not got[0].any() and not got[2].any()


def test_follows_todo_and_skips():
    """tests/test_codec.py:118-154 of the reference, restated."""
    codec = _codec()
    dev = torch.device("cuda")
    E = 8
    ns = (N, N // 2)
    pitches = [codec_ref.pitch_of(n, 1.25, 4096) for n in ns]
    raws = {e: [rows(10 * e + k, n) for k, n in enumerate(ns)] for e in (3, 5, 6)}
    staging = [torch.zeros((3, p), dtype=torch.uint8, device=dev) for p in pitches]
    lut = torch.zeros((E, 2, 512), dtype=torch.uint8, device=dev)
    for j, e in enumerate((3, 5, 6)):
        for k in range(2):
            rec, lt = codec_ref.encode(raws[e][k], pitches[k], CHUNK)
            staging[k][j] = torch.from_numpy(rec).to(dev)
            lut[e, k] = torch.from_numpy(lt).to(dev)
    dst = [torch.zeros((2, n), dtype=torch.uint8, device=dev) for n in ns]
    todo = torch.tensor([3, 5, 6], dtype=torch.int64, device=dev)
    dst_row = torch.zeros((E,), dtype=torch.int64, device=dev)
    dst_row[3], dst_row[5], dst_row[6] = 1, 0, 0
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    cache_row[5] = 2
    skip = torch.tensor([6, -1, -1], dtype=torch.int64, device=dev)
    codec.decode_rows(todo, dst_row, cache_row, staging, dst, lut, skip=skip, chunk=CHUNK)
    torch.cuda.synchronize()
    for k in range(2):
        assert np.array_equal(dst[k][1].cpu().numpy(), raws[3][k])
        assert not dst[k][0].any()
    codec.decode_rows(todo, dst_row, cache_row, staging, dst, lut, chunk=CHUNK)
    torch.cuda.synchronize()
    for k in range(2):
        assert np.array_equal(dst[k][0].cpu().numpy(), raws[6][k])


def _ram_tier(records_by_row, rows, pitch):
    """A pinned RAM tier of `rows` records of `pitch` bytes (random bytes
    where no record is placed) and its device view."""
    from vllm_expert_pager.gather import DeviceRows
    from vllm_expert_pager.store import PinnedBuffer

    buf = PinnedBuffer(rows * pitch, coherent=False)
    host = buf.tensor(torch.uint8, (rows, pitch))
    host.copy_(torch.from_numpy(np.random.default_rng(rows).integers(0, 256, (rows, pitch), dtype=np.uint8)))
    for r, rec in records_by_row.items():
        host[r] = torch.from_numpy(rec)
    return buf, DeviceRows(host, buf.device_ptr)


# 128-byte runs (512), 64-byte (64), plain stores (32, 96)
@pytest.mark.parametrize("chunk", [32, 64, 96, 512])
def test_decode_from_ram_follows_rows_and_copies_scales(chunk):
    """xp_decode_rows_from_ram: expert e's record is RAM-tier row
    src_row[e] + base and its scale row goes to scale_dst[dst_row[e]];
    todo -1 entries, cached experts, listed skips and record or destination
    rows outside their tensors are skipped (records and scales alike)."""
    codec = _codec()
    dev = torch.device("cuda")
    E, rows_ram, base = 10, 16, 4
    ns = (2 * chunk * 32, chunk * 32)
    pitches = [codec_ref.pitch_of(n, 1.25, 4096) for n in ns]
    src_row = torch.tensor([0, 3, 7, -9, 9, 12, 2, 5, 8, 1], dtype=torch.int64)  # row - base per expert
    dst_row = torch.tensor([0, 3, 1, 0, 5, 2, 0, 4, 0, 0], dtype=torch.int64)  # dst_rows = 5: expert 4 is outside
    used = (1, 2, 4, 5, 7, 9)
    raws = {e: [rows(200 + 10 * e + k, n) for k, n in enumerate(ns)] for e in used}
    lut = torch.zeros((E, 2, 512), dtype=torch.uint8, device=dev)
    placed = [{}, {}]
    for e in used:
        for k in range(2):
            rec, lt = codec_ref.encode(raws[e][k], pitches[k], chunk)
            lut[e, k] = torch.from_numpy(lt).to(dev)
            r = base + int(src_row[e])
            if 0 <= r < rows_ram:
                placed[k][r] = rec
    tiers = [_ram_tier(placed[k], rows_ram, pitches[k]) for k in range(2)]
    words = (8, 4)
    scale = [torch.randint(1, 2**30, (E, w), dtype=torch.int32, device=dev) for w in words]
    scale_dst = [torch.zeros((5, w), dtype=torch.int32, device=dev) for w in words]
    dst = [torch.zeros((5, n), dtype=torch.uint8, device=dev) for n in ns]
    # 5: base + 12 = 16 is past the tier; 4: dst row 5 is past dst; 9: cached; 1: listed as skipped.
    todo = torch.tensor([2, 7, 4, -1, 9, 1, 5], dtype=torch.int64, device=dev)
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    cache_row[9] = 0
    skip = torch.tensor([1, -1, -1, -1, -1, -1, -1], dtype=torch.int64, device=dev)
    src, ram = [t[1] for t in tiers], (src_row.to(dev), base)

    def run(sk):
        codec.decode_rows_from_ram(todo, dst_row.to(dev), cache_row, ram[0], ram[1], src, dst, lut, scale, scale_dst,
                                   skip=sk, chunk=chunk)
        torch.cuda.synchronize()

    run(skip)
    done = {2: 1, 7: 4}
    for k in range(2):
        for e, d in done.items():
            np.testing.assert_array_equal(dst[k][d].cpu().numpy(), raws[e][k])
            assert torch.equal(scale_dst[k][d], scale[k][e])
        for d in set(range(5)) - set(done.values()):
            assert not dst[k][d].any() and not scale_dst[k][d].any(), (k, d)
    run(None)  # now expert 1 too
    for k in range(2):
        np.testing.assert_array_equal(dst[k][3].cpu().numpy(), raws[1][k])
        assert torch.equal(scale_dst[k][3], scale[k][1])
        for d in (0, 2):
            assert not dst[k][d].any() and not scale_dst[k][d].any(), (k, d)


def test_decode_from_ram_matches_staging_full_size():
    """Full-size expert records read from shuffled RAM-tier rows give the
    bytes the staging decoder gives (and the raw rows)."""
    codec = _codec()
    dev = torch.device("cuda")
    count, base = 6, 3
    raws, stg_np, luts_np = _expert_batch(codec, count, 41)
    order = [4, 0, 5, 2, 1, 3]  # expert j's record sits at RAM row base + order[j]
    rows_ram = base + count
    tiers = [_ram_tier({base + order[j]: stg_np[k][j] for j in range(count)}, rows_ram, stg_np[k].shape[1])
             for k in range(2)]
    lut = torch.from_numpy(luts_np).to(dev)
    todo = torch.arange(count, dtype=torch.int64, device=dev)
    dst_row = torch.tensor([5, 3, 1, 0, 2, 4], dtype=torch.int64, device=dev)
    cache_row = torch.full((count,), -1, dtype=torch.int64, device=dev)
    src_row = torch.tensor(order, dtype=torch.int64, device=dev)
    scale = [torch.arange(count * w, dtype=torch.int32, device=dev).view(count, w) for w in (128, 64)]
    scale_dst = [torch.zeros_like(c) for c in scale]
    a = [torch.zeros((count, r.shape[1]), dtype=torch.uint8, device=dev) for r in raws]
    b = [torch.zeros_like(t) for t in a]
    codec.decode_rows_from_ram(todo, dst_row, cache_row, src_row, base, [t[1] for t in tiers], a, lut, scale,
                               scale_dst)
    stg = [torch.from_numpy(s).to(dev) for s in stg_np]
    codec.decode_rows(todo, dst_row, cache_row, stg, b, lut)
    torch.cuda.synchronize()
    for k in range(2):
        assert torch.equal(a[k], b[k])
        for j in range(count):
            np.testing.assert_array_equal(a[k][int(dst_row[j])].cpu().numpy(), raws[k][j])
            assert torch.equal(scale_dst[k][int(dst_row[j])], scale[k][j])


@pytest.mark.parametrize("chunk", [32, 64, 96, 512, 4096])
def test_decode_from_ram_single_row(chunk):
    """A launch with a single row to expand from the RAM tier takes the
    kernel's latency path (both nibble words of an iteration fetched an
    iteration ahead). A valid record gives its raw bytes alone, in a two-row
    launch (the paced path) and from staging. Records of random bytes with
    a table of 9-bit codes (a refill every 3 symbols: the most ring traffic,
    with the stream outrunning its requests) or a random table expand to the
    same bytes alone as in a two-row launch, and to nothing outside their
    own row."""
    codec = _codec()
    dev = torch.device("cuda")
    ns = (4 * chunk * 32, 2 * chunk * 32)
    pitches = [codec_ref.pitch_of(n, 1.25, 4096) for n in ns]
    E, rows_ram = 4, 6
    rng = np.random.default_rng(chunk)
    raw = [rows(300 + k, n) for k, n in enumerate(ns)]
    lut_np = rng.integers(0, 256, (E, 2, 512), dtype=np.uint8)
    lut_np[1] = 0x09
    recs = [rng.integers(0, 256, (E, p), dtype=np.uint8) for p in pitches]
    for k in range(2):
        recs[k][0], lut_np[0, k] = codec_ref.encode(raw[k], pitches[k], chunk)
    src_row = torch.tensor([3, 0, 5, 2], dtype=torch.int64, device=dev)  # RAM row of each expert
    tiers = [_ram_tier({int(src_row[e]): recs[k][e] for e in range(E)}, rows_ram, pitches[k]) for k in range(2)]
    lut = torch.from_numpy(lut_np).to(dev)
    scale = [torch.randint(1, 2**30, (E, 4), dtype=torch.int32, device=dev) for _ in range(2)]
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    dst_row = torch.arange(E, dtype=torch.int64, device=dev)

    def from_ram(todo):
        dst = [torch.zeros((E, n), dtype=torch.uint8, device=dev) for n in ns]
        sdst = [torch.zeros_like(s) for s in scale]
        codec.decode_rows_from_ram(torch.tensor(todo, dtype=torch.int64, device=dev), dst_row, cache_row, src_row,
                                   0, [t[1] for t in tiers], dst, lut, scale, sdst, chunk=chunk)
        torch.cuda.synchronize()
        return dst, sdst

    stg = [torch.from_numpy(r).to(dev) for r in recs]
    want = [torch.zeros((E, n), dtype=torch.uint8, device=dev) for n in ns]
    codec.decode_rows(torch.arange(E, dtype=torch.int64, device=dev), dst_row, cache_row, stg, want, lut,
                      chunk=chunk)
    torch.cuda.synchronize()
    for k in range(2):
        np.testing.assert_array_equal(want[k][0].cpu().numpy(), raw[k])
    for e in range(E):
        alone, sdst = from_ram([e, -1])
        pair, _ = from_ram([e, (e + 1) % E])
        for k in range(2):
            assert torch.equal(alone[k][e], pair[k][e]), (e, k)
            if e == 0:
                assert torch.equal(alone[k][e], want[k][e]), k
            assert torch.equal(sdst[k][e], scale[k][e])
            others = [d for d in range(E) if d != e]
            assert not alone[k][others].any() and not sdst[k][others].any(), (e, k)


# 4096: a table of 9-bit codes makes a group consume its most words (about
# 36900), and random start words give header counts above 65535, which the
# decoder clamps
@pytest.mark.parametrize("chunk", [64, 512, 4096])
def test_garbage_records_stay_in_bounds(chunk):
    """Records and LUTs of random bytes (start words out of range, code
    lengths 0-15) expand to arbitrary bytes in their own rows only: the
    valid experts of the same launch are exact and a spare row stays zero."""
    codec = _codec()
    dev = torch.device("cuda")
    ns = (4 * chunk * 32, 2 * chunk * 32)
    pitches = [codec_ref.pitch_of(n, 1.25, 4096) for n in ns]
    E = 6
    rng = np.random.default_rng(7)
    raws = {e: [rows(100 + 10 * e + k, n) for k, n in enumerate(ns)] for e in (0, 3)}
    staging = [torch.from_numpy(rng.integers(0, 256, (E, p), dtype=np.uint8)).to(dev) for p in pitches]
    lut_np = rng.integers(0, 256, (E, 2, 512), dtype=np.uint8)
    lut_np[4] = 0x09  # every window a 9-bit code: a refill every 3 symbols
    lut_np[5] = 0x00  # length 0, read as 1
    for e in (0, 3):
        for k in range(2):
            rec, lt = codec_ref.encode(raws[e][k], pitches[k], chunk)
            staging[k][e] = torch.from_numpy(rec).to(dev)
            lut_np[e, k] = lt
    lut = torch.from_numpy(lut_np).to(dev)
    dst = [torch.zeros((E + 1, n), dtype=torch.uint8, device=dev) for n in ns]
    todo = torch.arange(E, dtype=torch.int64, device=dev)
    dst_row = torch.arange(E, dtype=torch.int64, device=dev)
    cache_row = torch.full((E,), -1, dtype=torch.int64, device=dev)
    codec.decode_rows(todo, dst_row, cache_row, staging, dst, lut, chunk=chunk)
    torch.cuda.synchronize()
    for k in range(2):
        for e in (0, 3):
            np.testing.assert_array_equal(dst[k][e].cpu().numpy(), raws[e][k])
        assert not dst[k][E].any()


def _expert_batch(codec, count, seed):
    """Compressed staging (count rows per name) for synthetic full-size experts, plus the raw rows."""
    shapes = ((1024, 2048), (2048, 512))
    raws = [np.stack([fp8_expert(seed * 1000 + 2 * j + k, shapes[k]) for j in range(count)]) for k in range(2)]
    pitches = [codec.pitch_of(r.shape[1], 0.89, 4096) for r in raws]
    stg = [np.empty((count, p), np.uint8) for p in pitches]
    luts = np.empty((count, 2, 512), np.uint8)
    for k in range(2):
        for j in range(count):
            codec.encode_into(raws[k][j], stg[k][j], luts[j, k])
    return raws, stg, luts


def test_full_size_expert_rows():
    codec = _codec()
    dev = torch.device("cuda")
    count = 12
    raws, stg_np, luts_np = _expert_batch(codec, count, seed=1)
    stg = [torch.from_numpy(s).to(dev) for s in stg_np]
    lut = torch.from_numpy(luts_np).to(dev)
    dst = [torch.zeros((count, r.shape[1]), dtype=torch.uint8, device=dev) for r in raws]
    todo = torch.arange(count, dtype=torch.int64, device=dev)
    dst_row = torch.arange(count - 1, -1, -1, dtype=torch.int64, device=dev)  # reversed rows
    cache_row = torch.full((count,), -1, dtype=torch.int64, device=dev)
    codec.decode_rows(todo, dst_row, cache_row, stg, dst, lut)
    torch.cuda.synchronize()
    for k in range(2):
        got = dst[k].cpu().numpy()[::-1]
        np.testing.assert_array_equal(got, raws[k])
        # and the oracle decodes the same records to the same bytes
        np.testing.assert_array_equal(codec_ref.decode_fast(stg_np[k][:2], luts_np[:2, k], raws[k].shape[1]),
                                      raws[k][:2])


def test_headline_launch_256_experts():
    """The headline decode launch at its full size: 256 experts (w13 1024x2048
    and w2 2048x512 fp8 rows, N(0, 0.02) weights with 128x128 block scales),
    encoded on the GPU at pitch 0.89 and expanded in one launch of 6144
    workgroups; every byte equals the raw rows. On a sample the GPU records
    equal the host encoder's and the oracle decodes them to the same rows."""
    codec = _codec()
    dev = torch.device("cuda")
    count = 256
    g = torch.Generator(device=dev).manual_seed(1234)
    raws = []
    for r, c in ((1024, 2048), (2048, 512)):
        rows = torch.empty((count, r * c), dtype=torch.uint8, device=dev)
        for j in range(count):
            w = torch.randn((r, c), generator=g, device=dev) * 0.02
            blk = w.view(r // 128, 128, c // 128, 128)
            scale = blk.abs().amax(dim=(1, 3), keepdim=True).clamp(min=1e-12) / 448.0
            rows[j] = (blk / scale).to(torch.float8_e4m3fn).view(torch.uint8).reshape(-1)
        raws.append(rows)
    stg, luts = [], []
    for r in raws:
        rec, lut, _ = codec.encode_rows(r, codec.pitch_of(r.shape[1], 0.89, 4096))
        stg.append(rec)
        luts.append(lut)
    lut = torch.stack(luts, dim=1).contiguous()  # (E, names, 512)
    dst = [torch.zeros_like(r) for r in raws]
    todo = torch.arange(count, dtype=torch.int64, device=dev)
    cache_row = torch.full((count,), -1, dtype=torch.int64, device=dev)
    codec.decode_rows(todo, todo.clone(), cache_row, stg, dst, lut)
    torch.cuda.synchronize()
    for k in range(2):
        assert torch.equal(dst[k], raws[k]), f"name {k}"
    for k in range(2):
        for j in (0, 137, count - 1):
            raw = raws[k][j].cpu().numpy()
            rec = np.empty(stg[k].shape[1], np.uint8)
            lut_h = np.empty(512, np.uint8)
            codec.encode_into(raw, rec, lut_h)
            np.testing.assert_array_equal(stg[k][j].cpu().numpy(), rec)
            np.testing.assert_array_equal(luts[k][j].cpu().numpy(), lut_h)
            np.testing.assert_array_equal(codec_ref.decode_fast(rec[None], lut_h[None], raw.size)[0], raw)


def test_decode_in_graph_replays():
    codec = _codec()
    dev = torch.device("cuda")
    count = 4
    raws, stg_np, luts_np = _expert_batch(codec, count, seed=2)
    stg = [torch.from_numpy(s).to(dev) for s in stg_np]
    lut = torch.from_numpy(luts_np).to(dev)
    dst = [torch.zeros((count, r.shape[1]), dtype=torch.uint8, device=dev) for r in raws]
    todo = torch.full((count,), -1, dtype=torch.int64, device=dev)
    dst_row = torch.arange(count, dtype=torch.int64, device=dev)
    cache_row = torch.full((count,), -1, dtype=torch.int64, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        codec.decode_rows(todo, dst_row, cache_row, stg, dst, lut)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            codec.decode_rows(todo, dst_row, cache_row, stg, dst, lut)
    torch.cuda.synchronize()
    for rep in range(3):
        pick = [(rep + i) % count for i in range(2)]
        for d in dst:
            d.zero_()
        # staging row j holds expert j's record, so expert j stays at position j
        todo.copy_(torch.tensor([j if j in pick else -1 for j in range(count)], device=dev))
        g.replay()
        torch.cuda.synchronize()
        for k in range(2):
            got = dst[k].cpu().numpy()
            for j in range(count):
                if j in pick:
                    np.testing.assert_array_equal(got[j], raws[k][j], err_msg=f"replay {rep}")
                else:
                    assert not got[j].any()
