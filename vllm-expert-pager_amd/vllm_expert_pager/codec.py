"""Lossless fp8 e4m3 row codec: host encoder and batched GPU decoder (replaces codec.py).

Format (codec.py:1-41, kept byte for byte): per row, a length-limited
canonical Huffman code over the 4-bit exponent, sign + mantissa nibbles kept
raw; a record of ``pitch`` bytes = int32 gstart[G+1] | nibble words in
(group, word, lane) order | Huffman words per group in refill order. The
512-byte LUT ((sym << 4) | len) lives outside the record.

``encode`` runs on the host (C++, csrc/codec_host.cpp); ``decode_rows``
expands staging rows on the GPU and ``decode_rows_from_ram`` RAM-tier rows
(csrc/codec.hip).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from vllm_expert_pager import _native as nat

LIMIT = 9
LUT_BYTES = 1 << LIMIT
CHUNK = 512
LANES = 32
GROUP = CHUNK * LANES


def _build(hist) -> tuple[list[int], list[int], list[int]]:
    h = (ctypes.c_int64 * 16)(*[int(x) for x in hist])
    lengths = (ctypes.c_int32 * 16)()
    codes = (ctypes.c_int32 * 16)()
    lut = (ctypes.c_uint8 * LUT_BYTES)()
    nat.call("xp_code_build", h, lengths, codes, lut)
    return list(lengths), list(codes), list(lut)


def code_lengths(hist: list[int], limit: int = LIMIT) -> list[int]:
    """Length-limited Huffman code lengths (codec.py:76-87). Only LIMIT is supported."""
    if limit != LIMIT:
        raise ValueError(f"only limit={LIMIT} is supported")
    return _build(hist)[0]


class Code:
    """Huffman code for the 16 exponent symbols (codec.py:90-114)."""

    def __init__(self, hist: list[int]) -> None:
        self.lengths, self.codes, self.lut = _build(hist)


def pitch_of(n_values: int, ratio: float, align: int) -> int:
    """Fixed record length: ratio times the raw size rounded up to align (codec.py:117-119)."""
    return -(-int(n_values * ratio) // align) * align


def groups(n_bytes: int, chunk: int = CHUNK) -> int:
    """Number of groups in one row (codec.py:292-294)."""
    return n_bytes // (chunk * LANES)


def encode_into(raw: np.ndarray, record: np.ndarray, lut: np.ndarray, chunk: int = CHUNK) -> int:
    """Encode uint8 ``raw`` into the preallocated ``record`` (its length is the pitch) and ``lut``.

    Returns the record's used bytes. Raises ValueError like codec.py:133-166.
    """
    assert raw.dtype == np.uint8 and record.dtype == np.uint8 and lut.dtype == np.uint8
    assert raw.flags.c_contiguous and record.flags.c_contiguous and lut.size == LUT_BYTES
    needed = ctypes.c_int64()
    nat.call("xp_encode_row", raw.ctypes.data, raw.size, chunk, record.ctypes.data, record.size,
             lut.ctypes.data, ctypes.byref(needed))
    return needed.value


def encode_rows(raw: torch.Tensor, pitch: int, chunk: int = CHUNK, records: torch.Tensor | None = None,
                luts: torch.Tensor | None = None, check: bool = True) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Compress the uint8 rows ``raw`` (R, N) on the GPU, one workgroup per row (codec.py:125-193).

    Returns ``(records (R, pitch), luts (R, 512), needed (R,) int64)`` on raw's
    device, byte for byte what ``encode_into`` writes. With ``check`` (it
    synchronises), a row that does not fit the pitch raises ValueError as
    codec.py:160-166 does; otherwise that row's record is left unwritten and
    ``needed`` tells.
    """
    nat.require_device(raw, "raw")
    if raw.dtype != torch.uint8 or raw.dim() != 2 or raw.stride(1) != 1:
        raise ValueError(f"raw must be a (rows, N) uint8 tensor with unit column stride, got {raw.dtype} {tuple(raw.shape)}")
    R, N = raw.shape
    if records is None:
        records = torch.empty((R, pitch), dtype=torch.uint8, device=raw.device)
    if luts is None:
        luts = torch.empty((R, LUT_BYTES), dtype=torch.uint8, device=raw.device)
    for t, name, cols in ((records, "records", pitch), (luts, "luts", LUT_BYTES)):
        nat.require_device(t, name)
        if t.dtype != torch.uint8 or t.dim() != 2 or t.shape[0] != R or t.shape[1] != cols or t.stride(1) != 1:
            raise ValueError(f"{name} must be a ({R}, {cols}) uint8 tensor")
    if records.stride(0) != pitch:
        raise ValueError("records rows must be contiguous at the pitch")
    needed = torch.empty((R,), dtype=torch.int64, device=raw.device)
    nat.call("xp_encode_rows", raw.data_ptr(), R, raw.stride(0), N, chunk, records.data_ptr(), pitch,
             luts.data_ptr(), luts.stride(0), needed.data_ptr(), nat.stream())
    if check and R:
        worst = int(needed.max().item())
        if worst > pitch:
            raise ValueError(
                f"compressed row is {worst} B, pitch is {pitch} B; "
                f"VLLM_EXPERT_PAGER_PITCH must be at least {worst / N:.4f}"
            )
    return records, luts, needed


def encode(raw: torch.Tensor, pitch: int, chunk: int = CHUNK) -> tuple[torch.Tensor, torch.Tensor]:
    """Compress a uint8 row (N,). Returns ``(record of pitch bytes, 512 B LUT)`` on raw's device (codec.py:125-193).

    A row on the GPU is encoded there (encode_rows); a host row by the host encoder.
    """
    if raw.is_cuda and chunk in (16, 32, 64, 128, 256, 512, 1024):
        rec, lut, _ = encode_rows(raw.reshape(1, -1).to(torch.uint8).contiguous(), pitch, chunk)
        return rec[0], lut[0]
    host = raw.reshape(-1).to(torch.uint8).contiguous().cpu().numpy()
    record = np.empty(pitch, np.uint8)
    lut = np.empty(LUT_BYTES, np.uint8)
    encode_into(host, record, lut, chunk)
    return torch.from_numpy(record).to(raw.device), torch.from_numpy(lut).to(raw.device)


def _require_rows(t: torch.Tensor, what: str, i: int) -> None:
    """A 2-D contiguous GPU tensor: the kernels address row r at
    ``r * shape[1] * element_size`` bytes from its start."""
    nat.require_device(t, f"{what}[{i}]")
    if t.dim() != 2 or not t.is_contiguous():
        raise ValueError(f"{what}[{i}] must be a contiguous 2-D tensor of rows, got shape {tuple(t.shape)} "
                         f"strides {t.stride()}")


def decode_rows(
    todo: torch.Tensor,
    dst_row: torch.Tensor,
    cache_row: torch.Tensor,
    staging: list[torch.Tensor],
    dst: list[torch.Tensor],
    lut: torch.Tensor,
    skip: torch.Tensor | None = None,
    chunk: int = CHUNK,
) -> None:
    """Expand ``staging[name][j]`` into ``dst[name][dst_row[todo[j]]]`` (codec.py:297-327).

    ``staging`` is ``(*, pitch)`` uint8, ``dst`` ``(*, N)`` uint8, ``lut`` this
    layer's ``(E, names, 512)``. Experts with ``cache_row[e] >= 0`` and, with
    ``skip``, the experts in that list are skipped.
    """
    for t, what in ((todo, "todo"), (dst_row, "dst_row"), (cache_row, "cache_row"), (lut, "lut")):
        nat.require_device(t, what)
    todo = todo.to(torch.int64).contiguous()
    dst_row = dst_row.to(torch.int64).contiguous()
    cache_row = cache_row.to(torch.int64).contiguous()
    skip_t = None if skip is None else skip.to(torch.int64).contiguous()
    lut = lut.contiguous()
    n = len(dst)
    E = dst_row.shape[0]
    if lut.numel() < E * n * LUT_BYTES:
        raise ValueError(f"lut has {lut.numel()} B, needs {E} x {n} x {LUT_BYTES}")
    if skip_t is not None and skip_t.shape[0] < todo.shape[0]:
        raise ValueError("skip must have at least as many entries as todo")
    if len(staging) != n:
        raise ValueError("staging and dst need one entry per name")
    names = (nat.XpDecodeName * n)()
    for i in range(n):
        s, d = staging[i], dst[i]
        _require_rows(s, "staging", i)
        _require_rows(d, "dst", i)
        names[i] = nat.XpDecodeName(
            s.data_ptr(), s.shape[1] * s.element_size(), s.shape[0],
            d.data_ptr(), d.shape[0], d.shape[1] * d.element_size(),
        )
    nat.call(
        "xp_decode_rows", todo.data_ptr(), todo.shape[0], dst_row.shape[0], dst_row.data_ptr(),
        cache_row.data_ptr(), lut.data_ptr(), names, n, None if skip_t is None else skip_t.data_ptr(),
        chunk, nat.stream(),
    )


def decode_rows_from_ram(
    todo: torch.Tensor,
    dst_row: torch.Tensor,
    cache_row: torch.Tensor,
    src_row: torch.Tensor,
    base: int,
    src: list,
    dst: list[torch.Tensor],
    lut: torch.Tensor,
    scale: list[torch.Tensor],
    scale_dst: list[torch.Tensor],
    skip: torch.Tensor | None = None,
    chunk: int = CHUNK,
) -> None:
    """``decode_rows`` with the records read straight from the RAM tier.

    The record of expert ``e = todo[j]`` is row ``src_row[e] + base`` of
    ``src[name]`` (a ``DeviceRows`` view or pinned tensor of the tier, pitch
    bytes per row), and its scale row ``scale[name][e]`` is copied to
    ``scale_dst[name][dst_row[e]]``; no staging copy is made first. Experts
    with ``cache_row[e] >= 0`` are skipped entirely. The reference decodes a
    staging copy (codec.py:297-327) that a gather fills (gather.py:328-393).
    """
    from vllm_expert_pager.gather import _rows

    for t, what in ((todo, "todo"), (dst_row, "dst_row"), (cache_row, "cache_row"), (src_row, "src_row"),
                    (lut, "lut")):
        nat.require_device(t, what)
    todo = todo.to(torch.int64).contiguous()
    dst_row = dst_row.to(torch.int64).contiguous()
    cache_row = cache_row.to(torch.int64).contiguous()
    src_row = src_row.to(torch.int64).contiguous()
    skip_t = None if skip is None else skip.to(torch.int64).contiguous()
    lut = lut.contiguous()
    n = len(dst)
    E = dst_row.shape[0]
    if len(src) != n or len(scale) != n or len(scale_dst) != n:
        raise ValueError("src, dst, scale and scale_dst need one entry per name")
    if src_row.shape[0] < E:
        raise ValueError(f"src_row has {src_row.shape[0]} entries, fewer than the {E} experts")
    if lut.numel() < E * n * LUT_BYTES:
        raise ValueError(f"lut has {lut.numel()} B, needs {E} x {n} x {LUT_BYTES}")
    if skip_t is not None and skip_t.shape[0] < todo.shape[0]:
        raise ValueError("skip must have at least as many entries as todo")
    names = (nat.XpDecodeName * n)()
    scales = (nat.XpDecodeScale * n)()
    for i in range(n):
        d, c, cd = dst[i], scale[i], scale_dst[i]
        _require_rows(d, "dst", i)
        sp, srows, spitch = _rows(src[i])
        for t, what in ((c, "scale"), (cd, "scale_dst")):
            nat.require_device(t, what)
            if not t.is_contiguous():
                raise ValueError(f"{what}[{i}] must be contiguous")
        row = c[0].numel() * c.element_size() if c.shape[0] else 0
        if cd.shape[0] and cd[0].numel() * cd.element_size() != row:
            raise ValueError(f"scale_dst[{i}] rows are not the size of scale[{i}] rows")
        names[i] = nat.XpDecodeName(sp, spitch, srows, d.data_ptr(), d.shape[0], d.shape[1] * d.element_size())
        scales[i] = nat.XpDecodeScale(c.data_ptr(), cd.data_ptr(), row, c.shape[0], cd.shape[0])
    nat.call(
        "xp_decode_rows_from_ram", todo.data_ptr(), todo.shape[0], E, dst_row.data_ptr(), cache_row.data_ptr(),
        src_row.data_ptr(), int(base), lut.data_ptr(), names, n, scales,
        None if skip_t is None else skip_t.data_ptr(), chunk, nat.stream(),
    )
