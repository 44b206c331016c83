"""Oracle of the fp8 exponent Huffman row codec -- test infrastructure only.

Restates codec.py (monochromegane/vllm-expert-pager v0.1.1):
  huffman_lengths / code_lengths  codec.py:61-87   (heapq, ties by node id)
  Code                            codec.py:90-114  (canonical, bit-reversed, LUT)
  pitch_of                        codec.py:117-119
  encode                          codec.py:125-193 (numpy version of the torch ops:
                                                    bincount, cumsum, searchsorted,
                                                    scatter-add, argsort by refill key)
  decode_ref                      tests/test_codec.py:49-79 (sequential, lane by lane)
  decode_fast                     the same rule in C (codec_ref.c), threaded over groups

Pinning: decoded bytes are pinned by the round trip decode(encode(x)) == x and
by decode_ref, which restates the reference's own sequential decoder. The
exact record bytes and LUT of encode are pinned against vectors produced by
the reference's encoder (tests/golden/codec_vectors.npz). Kraft sum == 1 and
length <= LIMIT pin code_lengths (tests/test_codec.py:104-107).
"""

from __future__ import annotations

import ctypes
import heapq
import os

import numpy as np

LIMIT = 9
LUT_BYTES = 1 << LIMIT
CHUNK = 512
LANES = 32
GROUP = CHUNK * LANES

_HERE = os.path.dirname(os.path.abspath(__file__))
# XP_ORACLE_LIBRARY names another build of codec_ref.c (a sanitizer build).
_LIB = os.environ.get("XP_ORACLE_LIBRARY") or os.path.join(_HERE, "liboracle.so")


def huffman_lengths(counts):
    heap = [(c, i, (i,)) for i, c in enumerate(counts)]
    heapq.heapify(heap)
    lengths = [0] * len(counts)
    nid = len(counts)
    while len(heap) > 1:
        c1, _, s1 = heapq.heappop(heap)
        c2, _, s2 = heapq.heappop(heap)
        for s in s1 + s2:
            lengths[s] += 1
        heapq.heappush(heap, (c1 + c2, nid, s1 + s2))
        nid += 1
    return lengths


def code_lengths(hist, limit: int = LIMIT):
    counts = [float(max(int(c), 1)) for c in hist]
    k = 0
    while True:
        lengths = huffman_lengths(counts)
        if max(lengths) <= limit:
            return lengths
        k += 1
        floor = sum(counts) / 2 ** (limit - k)
        counts = [max(c, floor) for c in counts]


class Code:
    def __init__(self, hist) -> None:
        self.lengths = code_lengths(hist)
        order = sorted(range(16), key=lambda s: (self.lengths[s], s))
        canon = [0] * 16
        code = 0
        for i, s in enumerate(order):
            if i:
                code = (code + 1) << (self.lengths[s] - self.lengths[order[i - 1]])
            canon[s] = code
        self.codes = [
            int(format(canon[s], f"0{self.lengths[s]}b")[::-1], 2) for s in range(16)
        ]
        self.lut = [-1] * LUT_BYTES
        for s in range(16):
            n = self.lengths[s]
            for hi in range(1 << (LIMIT - n)):
                x = self.codes[s] | (hi << n)
                assert self.lut[x] < 0, "codes are not prefix-free"
                self.lut[x] = (s << 4) | n
        assert min(self.lut) >= 0, "codes do not fill the LUT (Kraft sum < 1)"


def pitch_of(n_values: int, ratio: float, align: int) -> int:
    return -(-int(n_values * ratio) // align) * align


def groups(n_bytes: int, chunk: int = CHUNK) -> int:
    return n_bytes // (chunk * LANES)


def _u32_bytes(x: np.ndarray) -> np.ndarray:
    return (x.astype(np.int64) & 0xFFFFFFFF).astype("<u4").view(np.uint8)


def encode(raw: np.ndarray, pitch: int, chunk: int = CHUNK):
    """(record uint8[pitch], lut uint8[512]); ValueError like codec.py:133-166."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    N = raw.size
    if N % (chunk * LANES):
        raise ValueError(f"row of {N} values is not a multiple of {chunk * LANES}")
    C, G = N // chunk, N // (chunk * LANES)
    exp = ((raw >> 3) & 15).astype(np.int64)
    sm = ((raw >> 7) << 3) | (raw & 7)
    fixed = (sm[0::2] | (sm[1::2] << 4)).astype(np.uint8).reshape(G, LANES, chunk // 8, 4)
    fixed = np.ascontiguousarray(fixed.transpose(0, 2, 1, 3)).reshape(-1)

    code = Code(np.bincount(exp, minlength=16).tolist())
    lengths = np.array(code.lengths, np.int64)
    codes = np.array(code.codes, np.int64)
    n = lengths[exp].reshape(C, chunk)
    before = np.cumsum(n, 1) - n
    nw = (before[:, -1] + (LIMIT - 1)) // 32 + 1
    kmax = int(nw.max())
    thr = 32 * np.arange(kmax) - (LIMIT - 1)
    at = np.stack([np.searchsorted(before[c], thr, side="left") for c in range(C)])
    valid = at < chunk
    total_words = int(nw.sum())
    head = 4 * (G + 1) + N // 2
    nbytes = head + 4 * total_words
    if nbytes > pitch:
        raise ValueError(
            f"compressed row is {nbytes} B, pitch is {pitch} B; "
            f"VLLM_EXPERT_PAGER_PITCH must be at least {nbytes / N:.4f}"
        )
    wbase = np.cumsum(nw) - nw
    start = (wbase * 32)[:, None] + before
    v = codes[exp].reshape(C, chunk)
    w, sh = start >> 5, start & 31
    # Code bit ranges never overlap, so adding equals OR; float64 sums of
    # values below 2**32 are exact.
    words = np.bincount(
        w.reshape(-1), weights=((v << sh) & 0xFFFFFFFF).reshape(-1), minlength=total_words + 1
    ).astype(np.int64)
    words += np.bincount(
        (w + 1).reshape(-1), weights=(v >> (32 - sh)).reshape(-1), minlength=total_words + 1
    ).astype(np.int64)
    c = np.broadcast_to(np.arange(C)[:, None], (C, kmax))
    key = ((c // LANES) * chunk + at) * LANES + (c % LANES)
    src = (wbase[:, None] + np.arange(kmax))[valid]
    interleaved = words[src[np.argsort(key[valid], kind="stable")]]
    per_group = nw.reshape(G, LANES).sum(1)
    gstart = np.concatenate([np.cumsum(per_group) - per_group, [per_group.sum()]])

    out = np.zeros(pitch, np.uint8)
    out[: 4 * (G + 1)] = _u32_bytes(gstart)
    out[4 * (G + 1) : head] = fixed
    out[head:nbytes] = _u32_bytes(interleaved)
    return out, np.array(code.lut, np.uint8)


def decode_ref(rec: bytes, lut: bytes, n: int, chunk: int) -> list[int]:
    """Sequential decoder, one lane at a time (tests/test_codec.py:49-79)."""
    G = n // (chunk * LANES)

    def i32(off: int) -> int:
        return int.from_bytes(rec[off : off + 4], "little", signed=True)

    nib_off = 4 * (G + 1)
    huff_off = nib_off + n // 2
    out = [0] * n
    for g in range(G):
        rp = i32(4 * g)
        buf, level = [0] * LANES, [0] * LANES
        for i in range(chunk):
            m, k = divmod(i, 8)
            for lane in range(LANES):
                if level[lane] < LIMIT:
                    buf[lane] |= (i32(huff_off + 4 * rp) & 0xFFFFFFFF) << level[lane]
                    level[lane] += 32
                    rp += 1
                ent = lut[buf[lane] & 511]
                buf[lane] >>= ent & 15
                level[lane] -= ent & 15
                nib = i32(nib_off + 4 * ((g * (chunk // 8) + m) * LANES + lane))
                s = (nib >> (4 * k)) & 15
                out[(g * LANES + lane) * chunk + i] = ((s & 8) << 4) | ((ent >> 4) << 3) | (s & 7)
        assert rp <= i32(4 * (g + 1))
    return out


# ---- C build of the decoder rule (codec_ref.c) ----

_lib = None


def build_lib(out: str | None = None, sanitize: bool = False) -> str:
    """Compile codec_ref.c into `out` (default: the library _load() uses);
    with `sanitize`, under AddressSanitizer and UndefinedBehaviorSanitizer."""
    import subprocess

    out = out or _LIB
    src = os.path.join(_HERE, "codec_ref.c")
    tmp = out + f".tmp{os.getpid()}"
    opt = (["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
            "-fno-sanitize-recover=undefined"] if sanitize else ["-O3"])
    subprocess.run(["gcc", *opt, "-std=c11", "-fPIC", "-shared", "-pthread", src, "-o", tmp], check=True)
    os.replace(tmp, out)
    return out


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build_lib()
        lib = ctypes.CDLL(_LIB)
        lib.oracle_decode_rows.restype = ctypes.c_int
        lib.oracle_decode_rows.argtypes = [
            ctypes.c_void_p, ctypes.c_long, ctypes.c_long,  # records, rows, pitch
            ctypes.c_void_p,                                # luts (rows x 512)
            ctypes.c_void_p, ctypes.c_long,                 # out, n
            ctypes.c_long, ctypes.c_int,                    # chunk, threads
        ]
        _lib = lib
    return _lib


def decode_fast(records: np.ndarray, luts: np.ndarray, n: int, chunk: int = CHUNK,
                threads: int = 1) -> np.ndarray:
    """Decode rows (rows, pitch) with luts (rows, 512) into (rows, n) uint8."""
    records = np.ascontiguousarray(records, np.uint8)
    luts = np.ascontiguousarray(luts, np.uint8)
    if records.ndim == 1:
        records = records[None]
        luts = luts.reshape(1, -1)
    rows, pitch = records.shape
    out = np.empty((rows, n), np.uint8)
    rc = _load().oracle_decode_rows(
        records.ctypes.data, rows, pitch, luts.ctypes.data, out.ctypes.data, n, chunk, threads
    )
    if rc:
        raise ValueError(f"oracle decode failed ({rc}): malformed record")
    return out
