"""CPU tests of the SSD request server (host C++ in libxp.so).

The ring protocol is plain memory, so a Python thread plays the GPU: it
writes a request slot, publishes its seq, and polls `done`. Covers in-order
serving, the worker pool, read failures that still release the waiter, the
re-publish and idle resend of `done`, gaps in seq counted as missed, and the
test delay (the behaviours of store.py:83-308 and tests/test_store.py).

The protocol tests run against both servers: this build's (``xp``) and the
reference's own C server compiled from its source text by
``oracle/build_ref.py`` (``ref``, skipped where no reference tree is
present), which pins ``ssd.cpp`` to the reference's behaviour.
"""

import ctypes
import os
import time

import numpy as np
import pytest

import _tiers

RING, BLOCK = 4, 64
L, E, R, W = 2, 40, 8, 2
PITCH = (4096, 8192)
RECORD = sum(PITCH)


_SSD_SIGS = {
    "ssd_start": (ctypes.c_void_p, [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_long] * 6
                  + [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]),
    "ssd_stop": (None, [ctypes.c_void_p]),
    "ssd_stats": (None, [ctypes.c_void_p] * 5),
    "ssd_error": (ctypes.c_char_p, [ctypes.c_void_p]),
    "ssd_test_delay": (None, [ctypes.c_void_p, ctypes.c_double]),
}
_REF = {}


def _ref_lib():
    """The reference's C server (built once per session), or a skip without a reference tree."""
    if "lib" not in _REF:
        from oracle import build_ref

        path = build_ref.build_ssd_ref()
        lib = None
        if path:
            lib = ctypes.CDLL(path)
            for name, (res, args) in _SSD_SIGS.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
        _REF["lib"] = lib
    if _REF["lib"] is None:
        pytest.skip("no reference tree to build its C server from")
    return _REF["lib"]


def _lib(which="xp"):
    if which == "ref":
        return _ref_lib()
    from vllm_expert_pager import _native

    return _native.lib()


# The sanitizer runs instrument this build's server only.
SERVERS = ["xp"] if os.environ.get("XP_SSD_TEST_OWN_ONLY") else ["xp", "ref"]


def aligned(nbytes, dtype=np.uint8):
    raw = np.zeros(nbytes + 4096, np.uint8)
    off = (-raw.ctypes.data) % 4096
    return raw[off : off + nbytes].view(dtype)


def pattern(layer, e, name):
    return _tiers.expert_row(layer, e, name, PITCH[name]).view(np.int32)


class Server:
    def __init__(self, path, nworkers=7, which="xp", pitches=PITCH):
        self.lib = _lib(which)
        self.pitches = pitches
        with open(path, "wb") as f:
            for layer in range(L):
                for e in range(E):
                    f.write(b"".join(self.expected(layer, e, n).tobytes() for n in range(len(pitches))))
        self.fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
        self.rows = L * R + 2 * W
        self.req = aligned(8 * (2 + RING * (2 + 2 * BLOCK)), np.int64)
        self.done = aligned(4096, np.int64)[:1]
        self.pinned = [aligned(self.rows * p).view(np.int32).reshape(self.rows, -1) for p in pitches]
        ptrs = (ctypes.c_void_p * len(pitches))(*(a.ctypes.data for a in self.pinned))
        pitch = (ctypes.c_long * len(pitches))(*pitches)
        self.h = self.lib.ssd_start(self.fd, self.req.ctypes.data, self.done.ctypes.data, RING, BLOCK, L, E,
                                    self.rows, sum(pitches), len(pitches), ptrs, pitch, nworkers)
        assert self.h
        self.seq = 0

    def expected(self, layer, e, name):
        if self.pitches == PITCH:
            return pattern(layer, e, name)
        return _tiers.expert_row(layer, e, name, self.pitches[name]).view(np.int32)

    def publish(self, layer, experts, rows, seq=None):
        seq = self.seq + 1 if seq is None else seq
        self.seq = seq
        slot = 2 + (seq % RING) * (2 + 2 * BLOCK)
        self.req[slot + 2 : slot + 2 + BLOCK] = -1
        self.req[slot + 2 + BLOCK : slot + 2 + 2 * BLOCK] = -1
        self.req[slot + 2 : slot + 2 + len(experts)] = experts
        self.req[slot + 2 + BLOCK : slot + 2 + BLOCK + len(rows)] = rows
        self.req[slot + 1] = layer
        self.req[slot] = seq  # published last (x86 stores are not reordered)
        return seq

    def wait(self, seq, timeout=10.0):
        t0 = time.time()
        while int(self.done[0]) < seq:
            assert time.time() - t0 < timeout, f"done stuck at {int(self.done[0])} < {seq}"
            time.sleep(0.001)

    def stats(self):
        f, r, m = ctypes.c_long(), ctypes.c_long(), ctypes.c_long()
        io = ctypes.c_double()
        self.lib.ssd_stats(self.h, ctypes.byref(f), ctypes.byref(r), ctypes.byref(io), ctypes.byref(m))
        return f.value, r.value, io.value, m.value

    def error(self):
        e = self.lib.ssd_error(self.h)
        return None if e is None else e.decode()

    def close(self):
        if self.h:
            self.lib.ssd_stop(self.h)
            self.h = None
            os.close(self.fd)


@pytest.fixture(params=SERVERS)
def which(request):
    return request.param


@pytest.fixture
def server(tmp_path, which):
    s = Server(str(tmp_path / "paging.bin"), which=which)
    yield s
    s.close()


def test_serves_requests_in_order(server):
    for i in range(12):
        layer = i % L
        experts = [(3 * i) % E, (3 * i + 1) % E]
        rows = [layer * R + (i % R), layer * R + ((i + 1) % R)]
        seq = server.publish(layer, experts, rows)
        server.wait(seq)
        for e, row in zip(experts, rows):
            for n in range(2):
                np.testing.assert_array_equal(server.pinned[n][row], pattern(layer, e, n))
    f, r, io, missed = server.stats()
    assert (f, r, missed) == (12, 24, 0) and io > 0
    assert server.error() is None


def test_many_jobs_in_one_request(server):
    """More reads than threads in one request; done is written once all are in."""
    seq = server.publish(1, list(range(20, 36)), list(range(16)))
    server.wait(seq)
    for k in range(16):
        for n in range(2):
            np.testing.assert_array_equal(server.pinned[n][k], pattern(1, 20 + k, n))
    assert server.stats()[:2] == (1, 16)


def test_read_failure_still_releases(server):
    seq = server.publish(1, [4, 5], [10**6, 0])
    server.wait(seq)
    assert "outside the RAM tier" in server.error()
    np.testing.assert_array_equal(server.pinned[0][0], pattern(1, 5, 0))
    seq = server.publish(1, [E + 3], [0])
    server.wait(seq)
    assert "outside the RAM tier" in server.error()  # the first failure is kept


def test_expert_out_of_range(tmp_path, which):
    s = Server(str(tmp_path / "p.bin"), which=which)
    try:
        s.wait(s.publish(5, [1], [0]))
        assert "out of range" in s.error()
    finally:
        s.close()


def test_gap_in_seq_counts_missed(server):
    server.wait(server.publish(0, [1], [0]))
    # seqs 2..5 were given up by the GPU before the host saw them; seq 6
    # lands in the slot the host watches (6 % RING == 2 % RING).
    server.wait(server.publish(0, [2], [1], seq=6))
    assert server.stats()[3] == 4
    np.testing.assert_array_equal(server.pinned[0][1], pattern(0, 2, 0))


def test_done_is_resent_when_the_republish_count_moves(server):
    seq = server.publish(0, [3], [0])
    server.wait(seq)
    server.done[0] = 0
    server.req[0] += 1
    server.wait(seq, timeout=2.0)


def test_done_is_resent_after_idling(server):
    seq = server.publish(0, [3], [0])
    server.wait(seq)
    server.done[0] = 0
    server.wait(seq, timeout=5.0)


def test_test_delay_holds_requests(server):
    server.lib.ssd_test_delay(server.h, 0.3)
    t0 = time.time()
    server.wait(server.publish(0, [3], [0]))
    assert time.time() - t0 >= 0.29
    server.lib.ssd_test_delay(server.h, 0.0)


def test_stop_while_delaying(tmp_path, which):
    s = Server(str(tmp_path / "p.bin"), which=which)
    s.lib.ssd_test_delay(s.h, 60.0)
    s.publish(0, [1], [0])
    time.sleep(0.05)
    t0 = time.time()
    s.close()
    assert time.time() - t0 < 5.0


def test_start_rejects_bad_arguments(tmp_path, which):
    lib = _lib(which)
    req = aligned(8 * 64, np.int64)
    done = aligned(4096, np.int64)
    ptrs = (ctypes.c_void_p * 5)()
    pitch = (ctypes.c_long * 5)()
    assert not lib.ssd_start(0, req.ctypes.data, done.ctypes.data, RING, BLOCK, 1, 1, 1, 4096, 5, ptrs, pitch, 1)


@pytest.mark.parametrize("use_uring", [0, 1], ids=["threads", "io_uring"])
@pytest.mark.parametrize("depth", [1, 3, 8])
def test_read_probe_reads_every_record(tmp_path, use_uring, depth):
    """The disk probe reads whole records with O_DIRECT at any depth, through
    the thread pool and through io_uring, and refuses misaligned offsets."""
    lib = _lib()
    rec = 3 * 4096
    path = tmp_path / "records.bin"
    path.write_bytes(bytes(range(256)) * (rec * 12 // 256))
    fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
    try:
        offs = (ctypes.c_int64 * 10)(*[rec * i for i in (3, 0, 11, 5, 5, 7, 1, 9, 2, 10)])
        sec = ctypes.c_double(-1.0)
        rc = lib.xp_ssd_read_probe(fd, rec, offs, 10, depth, use_uring, ctypes.byref(sec))
        if rc and use_uring and b"io_uring" in (lib.xp_last_error() or b""):
            pytest.skip(f"io_uring unavailable here: {lib.xp_last_error().decode()}")
        assert rc == 0, lib.xp_last_error()
        assert sec.value >= 0.0
        bad = (ctypes.c_int64 * 1)(100)
        assert lib.xp_ssd_read_probe(fd, rec, bad, 1, depth, use_uring, ctypes.byref(sec)) != 0
        assert b"aligned" in lib.xp_last_error()
        past = (ctypes.c_int64 * 1)(rec * 40)  # beyond the end: a short read is an error
        assert lib.xp_ssd_read_probe(fd, rec, past, 1, depth, use_uring, ctypes.byref(sec)) != 0
    finally:
        os.close(fd)


@pytest.mark.parametrize("bounce", [False, True], ids=["direct", "bounce"])
def test_records_larger_than_a_copy_chunk(tmp_path, which, bounce):
    """Records whose names are longer than a copy chunk (258 and 515 pages,
    so a bounced copy is cut into 256 KiB chunks with short last ones, spread
    over the copiers and readers) land whole in their rows, one preadv per
    record."""
    if bounce and which != "xp":
        pytest.skip("the bounce hook is this build's")
    pitches = (258 * 4096, 515 * 4096)
    s = Server(str(tmp_path / "big.bin"), nworkers=3, which=which, pitches=pitches)
    if bounce:
        s.lib.xp_ssd_test_bounce(s.h)
    try:
        for i in range(3):
            experts, rows = [5 + i, 30 - i, 17], [i, R + i, 2 * R + 1]
            s.wait(s.publish(i % L, experts, rows))
            for e, row in zip(experts, rows):
                for n in range(2):
                    np.testing.assert_array_equal(s.pinned[n][row], s.expected(i % L, e, n))
        assert s.error() is None and s.stats()[:2] == (3, 9)
        if which == "xp":
            bounce_on = bounce
            b, q, r, c = (ctypes.c_double() for _ in range(4))
            preads, readers, bounce = ctypes.c_long(), ctypes.c_int(), ctypes.c_int()
            s.lib.xp_ssd_phase_stats(s.h, ctypes.byref(b), ctypes.byref(q), ctypes.byref(r), ctypes.byref(c),
                                     ctypes.byref(preads), ctypes.byref(readers), ctypes.byref(bounce))
            # One read per record; plain host memory takes O_DIRECT, so only the hook bounces.
            assert preads.value == 9 and readers.value == 4 and bounce.value == int(bounce_on)
            assert r.value > 0 and q.value >= 0 and (c.value > 0) == bounce_on
            # Requests one at a time: the busy time is the summed request time.
            assert abs(b.value - s.stats()[2]) < 1e-3 * max(1.0, b.value)
    finally:
        s.close()


@pytest.mark.parametrize("bounce", [False, True], ids=["direct", "bounce"])
def test_requests_published_together_answer_in_order(server, which, bounce):
    """A long request and a short one published back to back: done reaches
    the short one's seq only once every row of the long one is in."""
    if bounce:
        if which != "xp":
            pytest.skip("the bounce hook is this build's")
        server.lib.xp_ssd_test_bounce(server.h)
    for rep in range(4):
        a = server.publish(1, list(range(rep, rep + 16)), list(range(16)))
        b = server.publish(0, [30 + rep], [16 + rep])  # rows 16-19: past the long request's
        server.wait(b)
        assert int(server.done[0]) == b
        for k in range(16):
            for n in range(2):
                np.testing.assert_array_equal(server.pinned[n][k], pattern(1, rep + k, n))
        np.testing.assert_array_equal(server.pinned[0][16 + rep], pattern(0, 30 + rep, 0))
        assert a == b - 1
    assert server.stats()[:2] == (8, 4 * 17) and server.error() is None


def test_one_reader_bounced_requests_back_to_back(tmp_path):
    """One reader with bounced reads: it rotates through its bounce buffers
    while the copier empties them (45 records, more than it has buffers, so
    each is reused), and requests of several records published back to back
    still land whole and answer in order; a stop with reads and copies still
    queued waits for the copies out of the buffers it frees (the sanitizer
    runs repeat this test)."""
    pitches = (258 * 4096, 515 * 4096)
    s = Server(str(tmp_path / "one.bin"), nworkers=0, which="xp", pitches=pitches)
    s.lib.xp_ssd_test_bounce(s.h)
    try:
        for rep in range(3):
            want = {}
            seqs = []
            for i in range(3):
                experts = [(11 * rep + 5 * i + k) % E for k in range(5)]
                rows = [5 * i + k for k in range(5)]
                layer = (rep + i) % L
                seqs.append(s.publish(layer, experts, rows))
                want.update({row: (layer, e) for e, row in zip(experts, rows)})
            s.wait(seqs[-1])
            assert int(s.done[0]) == seqs[-1]
            for row, (layer, e) in want.items():
                for n in range(2):
                    np.testing.assert_array_equal(s.pinned[n][row], s.expected(layer, e, n))
        assert s.error() is None and s.stats()[:2] == (9, 45)
        s.publish(0, list(range(8)), list(range(8)))
        s.publish(1, list(range(8, 16)), list(range(8, 16)))
    finally:
        s.close()  # stops with these two still being read and copied
