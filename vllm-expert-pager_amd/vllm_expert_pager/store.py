"""RAM and SSD tiers of the expert weights (replaces store.py).

The RAM tier is one pinned host allocation per weight name, ``rows = L*R +
working_rows`` rows of ``pitch`` bytes (row ``l*R + s`` = slot s of layer l,
then the shared working rows). The GPU reads it directly over the host link
(``view``, a device-visible address); the host writes it through ``pinned``
(a CPU tensor over the same memory). The SSD tier is a paging file of
fixed-length records (all names' pitches back to back) in [layer][expert]
order; a C++ server thread (csrc/ssd.cpp) answers the GPU's read requests
from a request ring in pinned coherent memory.

Layout, validation and messages follow the reference (store.py:351-599).
"""

from __future__ import annotations

import concurrent.futures
import ctypes
import faulthandler
import logging
import os
import signal
import threading
import time

import numpy as np
import torch

from vllm_expert_pager import _native as nat
from vllm_expert_pager import codec
from vllm_expert_pager.gather import DeviceRows

logger = logging.getLogger(f"vllm.{__name__}")

# O_DIRECT alignment of rows, records and the pinned base (store.py:51-53).
_ALIGN = 4096
# Reader threads of the SSD server. The reference fixes 8 concurrent reads
# (store.py:59-64), sized by hand for its NVMe disk. Here the server starts
# with _READERS_UNSIZED and, once the paging file is complete (sync), probes
# the disk with record-sized O_DIRECT reads of the file from each of
# _READER_DEPTHS threads and restarts with the smallest depth of at least 2
# within 10% of the fastest (see size_readers): disks differ in how much a
# deeper queue helps, and on some every extra read in flight only slows the
# others down. VLLM_EXPERT_PAGER_READ_WORKERS (1..64),
# not a reference setting, fixes the count and skips the probe.
_READERS_UNSIZED = 2
_READER_DEPTHS = (1, 2, 4, 8)


def _read_workers_setting() -> int | None:
    v = os.environ.get("VLLM_EXPERT_PAGER_READ_WORKERS")
    if not v:
        return None
    n = int(v)
    if not 1 <= n <= 64:
        raise ValueError(f"VLLM_EXPERT_PAGER_READ_WORKERS must be in [1, 64], got {n}")
    return n
# Request ring slots (store.py:65-67).
RING = 4


class PinnedBuffer:
    """Page-aligned pinned host memory from hipHostMalloc, visible to the GPU."""

    def __init__(self, nbytes: int, coherent: bool) -> None:
        p = ctypes.c_void_p()
        nat.call("xp_host_alloc", ctypes.byref(p), int(nbytes), 1 if coherent else 0)
        self.ptr = p.value
        self.nbytes = int(nbytes)
        self.coherent = coherent
        self.device_ptr = nat.device_pointer(self.ptr)
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        self._array = np.frombuffer(buf, dtype=np.uint8)

    def tensor(self, dtype: torch.dtype, shape: tuple[int, ...]) -> torch.Tensor:
        """A CPU tensor over the buffer (shares memory; valid while this object lives)."""
        return torch.from_numpy(self._array).view(dtype).view(shape)

    def free(self) -> None:
        if self.ptr:
            self._array = None
            nat.call("xp_host_free", ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


def _coherent_tier(ram_slots: int, num_experts: int) -> bool:
    """Fine-grained (uncached) RAM tier when the host rewrites rows at run time.

    With an SSD tier the server writes RAM rows that the GPU then reads; a
    fine-grained mapping keeps the GPU from reading stale cached lines. With
    every expert in RAM the rows never change after loading, and a
    coarse-grained mapping is allowed. VLLM_EXPERT_PAGER_PINNED overrides
    (coherent | noncoherent).
    """
    mode = os.environ.get("VLLM_EXPERT_PAGER_PINNED", "auto")
    if mode == "coherent":
        return True
    if mode == "noncoherent":
        return False
    if mode != "auto":
        raise ValueError(f"VLLM_EXPERT_PAGER_PINNED must be auto, coherent or noncoherent, got {mode!r}")
    return ram_slots < num_experts


class Store:
    """One per model: the RAM tier's pinned buffers, the paging file and the host server."""

    def __init__(
        self,
        num_layers: int,
        num_experts: int,
        ram_slots: int,
        working_rows: int,
        row_bytes: dict[str, int],
        compress: bool,
        pitch_ratio: float,
        path: str | None,
        device: torch.device,
    ) -> None:
        L, E, R = num_layers, num_experts, ram_slots
        if not 1 <= R <= E:
            raise ValueError(f"VLLM_EXPERT_PAGER_RAM_SLOTS must be in [1, {E}], got {R}")
        if working_rows < 1:
            raise ValueError(f"working_rows must be >= 1, got {working_rows}")
        if R < E and path is None:
            raise ValueError(
                "VLLM_EXPERT_PAGER_SSD_PATH is required when VLLM_EXPERT_PAGER_RAM_SLOTS < num_experts"
            )
        for name, nbytes in row_bytes.items():
            unit = codec.GROUP if compress else _ALIGN
            if nbytes % unit:
                raise ValueError(f"{name}: row of {nbytes} B is not a multiple of {unit}")

        self.num_layers, self.num_experts, self.ram_slots = L, E, R
        self.layers = 0
        self.device = torch.device(device)
        self.compress = compress
        self.names = list(row_bytes)
        self.row_bytes = dict(row_bytes)
        self.pitch = {
            name: codec.pitch_of(nbytes, pitch_ratio, _ALIGN) if compress else nbytes
            for name, nbytes in row_bytes.items()
        }
        self.record_bytes = sum(self.pitch.values())
        self.offset = {}
        pos = 0
        for name in self.names:
            self.offset[name] = pos
            pos += self.pitch[name]
        self.working_base = L * R
        self.rows = L * R + working_rows
        self._handle = None
        self._buffers: list[PinnedBuffer] = []
        coherent = _coherent_tier(R, E)
        logger.info(
            "vllm-expert-pager: RAM tier %d rows x %d B (%s) = %.2f GiB pinned (%s)",
            self.rows, self.record_bytes,
            f"compressed from {sum(row_bytes.values())} B" if compress else "raw",
            self.rows * self.record_bytes / 2**30, "fine-grained" if coherent else "coarse-grained",
        )
        self.pinned: dict[str, torch.Tensor] = {}
        self.view: dict[str, DeviceRows] = {}
        for name, nbytes in self.pitch.items():
            buf = PinnedBuffer(self.rows * nbytes, coherent)
            self._buffers.append(buf)
            host = buf.tensor(torch.int32, (self.rows, nbytes // 4))
            self.pinned[name] = host
            self.view[name] = DeviceRows(host, buf.device_ptr)
        # Per-row Huffman LUTs: lut[l, e, i] for expert e of layer l, name i
        # (store.py:422-429).
        self.lut = torch.zeros(
            (L if compress else 1, E, len(self.names), codec.LUT_BYTES), dtype=torch.uint8, device=self.device
        )

        # req = [re-publishes, give-ups] + RING slots of [seq, layer,
        # expert[B], row[B]] with B the power of two >= E (store.py:434-451).
        self.block = 1 << (E - 1).bit_length()
        self.ring = RING
        self.retry_at, self.giveup_at = 0, 1
        self.slot_words = 2 + 2 * self.block
        self._req_buf = PinnedBuffer(8 * (2 + RING * self.slot_words), True)
        self._done_buf = PinnedBuffer(_ALIGN, True)
        self.req = self._req_buf.tensor(torch.int64, (2 + RING * self.slot_words,))
        self.done = self._done_buf.tensor(torch.int64, (_ALIGN // 8,))[:1]
        self.req.zero_()
        self.done.zero_()
        self.seq = torch.zeros((1,), dtype=torch.int64, device=self.device)
        self.ticket_chunk = torch.zeros((2,), dtype=torch.int64, device=self.device)
        self._ring = nat.XpRing(self._req_buf.device_ptr, self._done_buf.device_ptr, self.seq.data_ptr(),
                                self.block, self.ring)

        self.readers = 0  # SSD server reader threads (set when it starts)
        self.reader_probe: dict | None = None  # disk GB/s by probe depth, from size_readers()
        self.path = path if R < E else None
        self.fd_w = self.fd_r = None
        self.synced: float | None = None  # seconds of the last sync()
        if self.path is not None:
            size = L * E * self.record_bytes
            if os.path.exists(path) and os.path.getsize(path) != size:
                raise FileExistsError(f"{path} exists and is not a paging file of {size} B; remove it first")
            self.fd_w = os.open(path, os.O_WRONLY | os.O_CREAT | os.O_TRUNC, 0o600)
            self.fd_r = os.open(path, os.O_RDONLY | os.O_DIRECT)
            logger.info("vllm-expert-pager: paging file %s (%.1f GiB)", path, size / 2**30)
            self._start_server()
        if threading.current_thread() is threading.main_thread():
            try:
                faulthandler.register(signal.SIGUSR2, all_threads=True)
            except (AttributeError, ValueError, RuntimeError):
                pass

    def ring_struct(self) -> nat.XpRing:
        return self._ring

    def _start_server(self, readers: int | None = None) -> None:
        self.readers = readers or _read_workers_setting() or _READERS_UNSIZED
        n = len(self.names)
        pinned = (ctypes.c_void_p * n)(*(self.pinned[k].data_ptr() for k in self.names))
        pitch = (ctypes.c_long * n)(*(self.pitch[k] for k in self.names))
        self._so = nat.lib()
        self._handle = self._so.ssd_start(
            self.fd_r, ctypes.c_void_p(self.req.data_ptr()), ctypes.c_void_p(self.done.data_ptr()), self.ring,
            self.block, self.num_layers, self.num_experts, self.rows, self.record_bytes, n, pinned, pitch,
            self.readers - 1,
        )
        if not self._handle:
            raise RuntimeError("vllm-expert-pager: cannot start the SSD server")

    def close(self) -> None:
        """Stop the host server threads (they otherwise end with the process)."""
        if getattr(self, "_handle", None):
            self._so.ssd_stop(ctypes.c_void_p(self._handle))
            self._handle = None
        for fd_name in ("fd_w", "fd_r"):
            fd = getattr(self, fd_name, None)
            if fd is not None:
                try:
                    os.close(fd)
                except OSError:
                    pass
                setattr(self, fd_name, None)

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def test_delay(self, seconds: float) -> None:
        """For tests: delay the host between seeing a request and serving it. 0 clears it."""
        self._so.ssd_test_delay(ctypes.c_void_p(self._handle), seconds)

    def _stats(self) -> tuple[int, int, float, int]:
        if not self._handle:
            return 0, 0, 0.0, 0
        fetches, reads, missed = (ctypes.c_long() for _ in range(3))
        io_seconds = ctypes.c_double()
        self._so.ssd_stats(ctypes.c_void_p(self._handle), ctypes.byref(fetches), ctypes.byref(reads),
                           ctypes.byref(io_seconds), ctypes.byref(missed))
        return fetches.value, reads.value, io_seconds.value, missed.value

    def sync(self) -> float:
        """Flush the paging file to the disk and drop it from the page cache;
        returns the seconds it took (0 without a paging file).

        The records are written through the page cache. Until the kernel has
        written them back, the server's O_DIRECT reads share the disk with that
        writeback (and a read of a range with dirty pages waits for it), so a
        loader calls this once after the last layer.
        """
        if self.fd_w is None:
            return 0.0
        t0 = time.perf_counter()
        os.fdatasync(self.fd_w)
        os.posix_fadvise(self.fd_w, 0, 0, os.POSIX_FADV_DONTNEED)
        self.synced = time.perf_counter() - t0
        if _read_workers_setting() is None:
            self.size_readers()
        return self.synced

    def size_readers(self, seconds: float = 0.05) -> dict | None:
        """Probe the paging file with record-sized O_DIRECT reads of random
        records from 1, 2, 4 and 8 threads (two passes in opposite orders,
        each about ``seconds`` long at 3 GB/s, the better kept), and restart
        the server with the smallest depth of at least 2 within 10% of the
        fastest, or 1 when no deeper one is (fewer reads in flight serve a
        decode step's single records sooner; a second reader still pays:
        while one reads, the other's bounce copy is under way, and the
        server's own sweeps moved 6 GB/s at two readers against 3-5.6 at
        one on disks whose probe put the two depths within 10%). Only while
        no request has been made: a new server starts from seq 1. Returns
        the rates (GB/s by depth), or None when nothing was done."""
        if not self._handle or self.fd_r is None:
            return None
        slots = self.req[2:].view(self.ring, self.slot_words)
        if int(self.done[0]) != 0 or bool((slots[:, 0] != 0).any()):
            logger.info("vllm-expert-pager: SSD readers not re-sized: requests were already made")
            return None
        records = self.num_layers * self.num_experts
        rng = np.random.default_rng(records)
        rates: dict[int, float] = {}
        for order in (_READER_DEPTHS, _READER_DEPTHS[::-1]):
            for depth in order:
                count = max(4 * depth, int(3e9 * seconds / self.record_bytes))
                idx = rng.integers(0, records, size=count)
                offs = (ctypes.c_int64 * count)(*(int(i) * self.record_bytes for i in idx))
                sec = ctypes.c_double()
                if self._so.xp_ssd_read_probe(self.fd_r, self.record_bytes, offs, count, depth, 0, ctypes.byref(sec)):
                    logger.warning("vllm-expert-pager: SSD reader probe failed: %s",
                                   self._so.xp_last_error().decode(errors="replace"))
                    return None
                rates[depth] = max(rates.get(depth, 0.0), count * self.record_bytes / sec.value / 1e9)
        best = max(rates.values())
        close = [d for d, r in rates.items() if r >= 0.9 * best]
        deeper = [d for d in close if d >= 2]
        readers = min(deeper) if deeper else 1
        self.reader_probe = {str(d): round(r, 3) for d, r in sorted(rates.items())}
        if readers != self.readers:
            self._so.ssd_stop(ctypes.c_void_p(self._handle))
            self._handle = None
            self._start_server(readers)
        logger.info("vllm-expert-pager: SSD server reads with %d thread(s); disk GB/s by depth %s", self.readers,
                    self.reader_probe)
        return self.reader_probe

    def stats(self) -> tuple[int, int, float, int]:
        """(requests served, experts read, seconds from request to done, requests missed)."""
        return self._stats()

    def phase_stats(self) -> dict:
        """The seconds with a request in flight (``busy_s``), and where the
        server's time went, summed over the records it read: seconds waiting
        in the readers' queue, in preadv and copying out of bounce buffers;
        the records read (one preadv each, ``preads``), the reader threads,
        and whether the rows refused O_DIRECT (``bounce``)."""
        if not self._handle:
            return {}
        b, q, r, c = (ctypes.c_double() for _ in range(4))
        preads = ctypes.c_long()
        readers, bounce = ctypes.c_int(), ctypes.c_int()
        self._so.xp_ssd_phase_stats(ctypes.c_void_p(self._handle), ctypes.byref(b), ctypes.byref(q),
                                    ctypes.byref(r), ctypes.byref(c), ctypes.byref(preads), ctypes.byref(readers),
                                    ctypes.byref(bounce))
        return {"busy_s": b.value, "queue_s": q.value, "read_s": r.value, "copy_s": c.value,
                "preads": preads.value, "readers": readers.value, "bounce": bool(bounce.value)}

    @property
    def fetches(self) -> int:
        """Requests served."""
        return self._stats()[0]

    @property
    def reads(self) -> int:
        """Experts read."""
        return self._stats()[1]

    @property
    def io_seconds(self) -> float:
        """Total time from seeing a request to writing done."""
        return self._stats()[2]

    @property
    def missed(self) -> int:
        """Requests the GPU gave up on before they arrived."""
        return self._stats()[3]

    @property
    def failed(self) -> str | None:
        """Description of a failed read, if any."""
        if not self._handle:
            return None
        err = self._so.ssd_error(ctypes.c_void_p(self._handle))
        return None if err is None else err.decode(errors="replace")

    def layer_lut(self, layer: int) -> torch.Tensor:
        """The LUTs ``(E, names, 512)`` of layer ``layer``."""
        return self.lut[layer if self.compress else 0]

    def add_layer(self) -> int:
        """Hand out a layer number in construction order."""
        if self.layers >= self.num_layers:
            raise RuntimeError(f"more MoE layers than num_hidden_layers={self.num_layers}")
        self.layers += 1
        return self.layers - 1

    def write(self, layer: int, expert: int, name: str, row: torch.Tensor) -> None:
        """Put one expert's row in the paging file and, if expert < R, in RAM-tier slot expert."""
        raw = row.contiguous().view(torch.uint8).reshape(-1)
        if raw.numel() != self.row_bytes[name]:
            raise ValueError(
                f"{name}: expert {expert} of layer {layer} has {raw.numel()} B, expected {self.row_bytes[name]}"
            )
        if self.compress and raw.is_cuda:  # encoded on the GPU, as the reference's torch encode is
            rec, lut, _ = codec.encode_rows(raw.view(1, -1), self.pitch[name])
            self.lut[layer, expert, self.names.index(name)] = lut[0].to(self.device)
            words = rec[0].cpu().numpy()
        elif self.compress:
            record = np.empty(self.pitch[name], np.uint8)
            lut = np.empty(codec.LUT_BYTES, np.uint8)
            codec.encode_into(raw.cpu().numpy(), record, lut)
            self.lut[layer, expert, self.names.index(name)] = torch.from_numpy(lut).to(self.device)
            words = record
        else:
            words = raw.cpu().numpy()
        if expert < self.ram_slots:
            self.pinned[name][layer * self.ram_slots + expert].copy_(torch.from_numpy(words.view(np.int32)))
        if self.fd_w is not None:
            offset = (layer * self.num_experts + expert) * self.record_bytes + self.offset[name]
            os.pwrite(self.fd_w, memoryview(words), offset)

    def write_rows(self, layer: int, name: str, rows: torch.Tensor, threads: int = 16) -> None:
        """Put experts 0..n-1 of ``layer`` at once, as ``write`` would place each of them.

        ``rows`` is ``(n, row_bytes)`` of any 1-byte dtype on any device.
        Compressed tiers encode the rows on the GPU when they are there
        (one launch for all of them), else in a thread pool (the host
        encoder releases the GIL); RAM-tier slots 0..min(n, R)-1 of the layer
        are filled with one copy and each expert's record goes to the paging
        file.
        """
        raw = rows.contiguous().view(torch.uint8)
        if raw.dim() != 2 or raw.shape[1] != self.row_bytes[name] or raw.shape[0] > self.num_experts:
            raise ValueError(f"{name}: rows must be (n <= {self.num_experts}, {self.row_bytes[name]}) bytes")
        n = raw.shape[0]
        r = min(n, self.ram_slots)
        base = layer * self.ram_slots
        if not self.compress and self.fd_w is None:
            self.pinned[name][base : base + r].view(torch.uint8).copy_(raw[:r])
            return
        if self.compress and raw.is_cuda:
            recs, luts, _ = codec.encode_rows(raw, self.pitch[name])
            self.lut[layer, :n, self.names.index(name)] = luts.to(self.device)
            self.pinned[name][base : base + r].view(torch.uint8).copy_(recs[:r])
            if self.fd_w is not None:
                words = recs.cpu().numpy()
                for e in range(n):
                    offset = (layer * self.num_experts + e) * self.record_bytes + self.offset[name]
                    os.pwrite(self.fd_w, memoryview(words[e]), offset)
            return
        host = raw.cpu().numpy()
        if self.compress:
            words = np.zeros((n, self.pitch[name]), np.uint8)
            luts = np.empty((n, codec.LUT_BYTES), np.uint8)

            def encode(e: int) -> None:
                codec.encode_into(host[e], words[e], luts[e])

            with concurrent.futures.ThreadPoolExecutor(max(1, threads)) as pool:
                list(pool.map(encode, range(n)))
            self.lut[layer, :n, self.names.index(name)] = torch.from_numpy(luts).to(self.device)
        else:
            words = host
        self.pinned[name][base : base + r].view(torch.uint8).copy_(torch.from_numpy(words[:r]))
        if self.fd_w is not None:
            for e in range(n):
                offset = (layer * self.num_experts + e) * self.record_bytes + self.offset[name]
                os.pwrite(self.fd_w, memoryview(words[e]), offset)
