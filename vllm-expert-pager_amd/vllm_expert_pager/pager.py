"""Per-layer expert paging: slabs, tables, and the decode and prefill paths.

This is the body of the reference's ``ExpertPagerRoutedExperts`` without the
vLLM class around it (experts.py:86-650): settings, the per-model store and
working slab, the per-layer slot tables and cache slab, the decode sequence
(``forward_modular``, experts.py:380-453), the prefill overflow chunk loop
(``_expert_pager_forward_working``, experts.py:455-577) and the expert run
on a slab with ``expert_map`` (``_expert_pager_run``, experts.py:579-604).
The vLLM hook in ``experts.py`` delegates to it; tests and benchmarks drive
it directly.

Every step is a fixed sequence of device launches chosen from the shapes
alone (``topk_ids.numel() > cache_slots`` selects the overflow path), so
decode steps can be captured in a hipGraph.
"""

from __future__ import annotations

import logging
import os
from dataclasses import dataclass
from typing import Callable

import torch

from vllm_expert_pager import moe, trace
from vllm_expert_pager.acquire import AcquirePair
from vllm_expert_pager.codec import decode_rows_from_ram
from vllm_expert_pager.gather import as_rows, fetch_publish_rows, fetch_wait_rows, gather_rows
from vllm_expert_pager.store import Store
from vllm_expert_pager.table import ExpertTable

logger = logging.getLogger(f"vllm.{__name__}")

# Expert weights referenced through the slab, then their block scales, in
# the order the gather lists take them (experts.py:76, 280-283).
PARAMS = ("w13_weight", "w2_weight")
SCALE_NAME = "weight_scale_inv"
SCALES = tuple(f"{w}_{SCALE_NAME}" for w in ("w13", "w2"))


@dataclass
class Settings:
    """The VLLM_EXPERT_PAGER_* settings (experts.py:41-72)."""

    cache_slots: int = 32
    ram_slots: int | None = None  # None: every expert (RAM only)
    ssd_path: str | None = None
    compress: str = "auto"  # auto | on | off
    pitch_ratio: float = 0.89
    working_rows: int = 64
    log_interval: int = 1000

    @classmethod
    def from_env(cls, environ=None) -> "Settings":
        env = os.environ if environ is None else environ
        ram = env.get("VLLM_EXPERT_PAGER_RAM_SLOTS")
        return cls(
            cache_slots=int(env.get("VLLM_EXPERT_PAGER_CACHE_SLOTS", "32")),
            ram_slots=int(ram) if ram else None,
            ssd_path=env.get("VLLM_EXPERT_PAGER_SSD_PATH"),
            compress=env.get("VLLM_EXPERT_PAGER_COMPRESS", "auto"),
            pitch_ratio=float(env.get("VLLM_EXPERT_PAGER_PITCH", "0.89")),
            working_rows=int(env.get("VLLM_EXPERT_PAGER_WORKING_ROWS", "64")),
            log_interval=int(env.get("VLLM_EXPERT_PAGER_LOG_INTERVAL", "1000")),
        )


def _shapes(hidden: int, intermediate: int) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
    """Per-expert shape and dtype of each staged tensor (w8a8 block fp8)."""
    H, I, B = hidden, intermediate, moe.BLOCK
    return {
        "w13_weight": ((2 * I, H), torch.uint8),
        "w2_weight": ((H, I), torch.uint8),
        SCALES[0]: ((2 * I // B, H // B), torch.float32),
        SCALES[1]: ((H // B, I // B), torch.float32),
    }


class Pager:
    """One per model: the store and the shared working slab.

    Mirrors the module-level ``_store`` and ``_working_slab`` of the
    reference (experts.py:78-83, 114-146, 290-318): layers run one after
    another on one stream, so they share the working rows. Its
    ``_prefill_staging`` has no counterpart: compressed rows are expanded
    straight from the RAM tier.
    """

    def __init__(self, settings: Settings, num_layers: int, num_experts: int, hidden: int, intermediate: int,
                 device: torch.device) -> None:
        s, E = settings, num_experts
        R = s.ram_slots if s.ram_slots else E
        if R < s.cache_slots:
            raise ValueError(
                f"VLLM_EXPERT_PAGER_RAM_SLOTS={R} must be >= VLLM_EXPERT_PAGER_CACHE_SLOTS={s.cache_slots}"
            )
        if s.working_rows < 1:
            raise ValueError(f"VLLM_EXPERT_PAGER_WORKING_ROWS must be >= 1, got {s.working_rows}")
        if s.compress not in ("auto", "on", "off"):
            raise ValueError(f"VLLM_EXPERT_PAGER_COMPRESS must be auto, on or off, got {s.compress!r}")
        if hidden % moe.BLOCK or intermediate % moe.BLOCK:
            raise ValueError(f"hidden={hidden} and intermediate={intermediate} must be multiples of {moe.BLOCK}")
        self.settings = s
        self.num_layers = num_layers
        self.layers_ready = 0
        self.num_experts, self.hidden, self.intermediate = E, hidden, intermediate
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.shapes = _shapes(hidden, intermediate)
        compress = R < E if s.compress == "auto" else s.compress == "on"
        row_bytes = {n: self.shapes[n][0][0] * self.shapes[n][0][1] for n in PARAMS}
        # Two faces of shared working rows: chunk k+1 reads into the face
        # whose copies finished with chunk k-1.
        self.store = Store(num_layers, E, R, 2 * s.working_rows, row_bytes, compress, s.pitch_ratio, s.ssd_path,
                           self.device)
        W = s.working_rows
        self.working_slab = {
            n: torch.empty((W, *shape), dtype=dt, device=self.device) for n, (shape, dt) in self.shapes.items()
        }
        # Compressed prefill chunks gather only their cached experts (the
        # decoder expands the others straight from pinned RAM); the gather
        # takes the tier's pitch from these one-row tensors and never
        # writes them.
        self.pitch_rows = (
            [torch.zeros((1, self.store.pitch[n] // 4), dtype=torch.int32, device=self.device) for n in PARAMS]
            if compress else None
        )

    def close(self) -> None:
        self.store.close()

    def add_layer(self, activation: str = "silu") -> "PagedExperts":
        """A new layer whose experts compute ``activation(gate) * up`` ("silu" or "gelu")."""
        return PagedExperts(self, activation)

    def layer_ready(self) -> None:
        """Count a layer whose weights are in; after the last one, flush the
        paging file (``flush``)."""
        self.layers_ready += 1
        if self.layers_ready == self.num_layers:
            self.flush()

    def flush(self) -> None:
        """Flush the paging file to disk once, so that serving reads do not
        share the disk with the page cache's write-back of the load (not a
        reference step). Runs after the last layer's weights are in, or at
        the first forward when the model has fewer MoE layers than layers."""
        if self.store.path is not None and self.store.synced is None:
            seconds = self.store.sync()
            logger.info("vllm-expert-pager: paging file flushed to disk in %.1f s", seconds)


class PagedExperts:
    """One MoE layer whose expert weights live in the tiers and are staged into slabs."""

    def __init__(self, pager: Pager, activation: str = "silu") -> None:
        moe.activation_code(activation)
        self.pager = pager
        self.activation = activation
        self.store = pager.store
        self.layer = self.store.add_layer()
        self.calls = 0
        self.ready = False

    # ---- loading ----

    def load_expert(self, expert: int, name: str, row: torch.Tensor) -> None:
        """Write one expert's fp8 weight (``w13_weight`` = gate rows then up rows, or ``w2_weight``)."""
        if name not in PARAMS:
            raise ValueError(f"unknown weight {name!r}; expected one of {PARAMS}")
        self.store.write(self.layer, expert, name, row)

    def setup(self, scales: dict[str, torch.Tensor]) -> None:
        """Build the tables, the cache slab and the row views once the weights are in (experts.py:233-376).

        ``scales`` maps ``w13_weight_scale_inv`` / ``w2_weight_scale_inv`` to
        ``(E, ...)`` float32 device tensors; they stay resident and gather
        copies the rows of staged experts next to the weights.
        """
        p, store = self.pager, self.store
        S, W, E, R = p.settings.cache_slots, p.settings.working_rows, p.num_experts, store.ram_slots
        dev = p.device
        for n in SCALES:
            shape, dt = p.shapes[n]
            t = scales[n]
            if tuple(t.shape) != (E, *shape) or t.dtype != dt or t.device != dev:
                raise ValueError(f"{n} must be {dt} {(E, *shape)} on {dev}, got {t.dtype} {tuple(t.shape)}")
        self.scales = {n: scales[n].contiguous() for n in SCALES}
        self.table = ExpertTable(E, S, dev)
        self.ram = ExpertTable(E, R, dev)
        # Warm start: at load time expert e < R was placed in RAM-tier slot e.
        self.ram.slot_of[:R] = self.ram.experts[:R]
        self.ram.expert_in[:R] = self.ram.experts[:R]
        self.acquire = AcquirePair(self.table, self.ram)
        # The expert_map the expert kernels read: int32 at a fixed address.
        # acquire writes it; the overflow path copies each chunk's map in.
        self.expert_map = self.acquire.expert_map
        self.cache_slab = {
            n: torch.empty((S, *shape), dtype=dt, device=dev) for n, (shape, dt) in p.shapes.items()
        }
        order = list(PARAMS) + list(SCALES)
        self.cache_rows = [as_rows(self.cache_slab[n]) for n in order]
        self.working_rows = [as_rows(p.working_slab[n]) for n in order]
        self.scale_rows = [as_rows(self.scales[n]) for n in SCALES]
        self.cache_bytes = [self.cache_slab[n].view(torch.uint8).reshape(S, -1) for n in PARAMS]
        self.working_bytes = [p.working_slab[n].view(torch.uint8).reshape(W, -1) for n in PARAMS]
        self.ready = True
        p.layer_ready()

    # ---- forward ----

    def forward(self, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                shared: Callable[[], object] | None = None) -> torch.Tensor:
        """The routed-expert output ``(T, H)`` bf16 of this layer (experts.py:380-453).

        ``shared``, if given, runs the layer's shared experts. It is called
        once per forward, right before the first expert launch: on the
        decode path before the expert FFN, on the overflow path before
        chunk 0's (experts.py:452, 569-573). Its result is not part of the
        returned routed sum.
        """
        if not self.ready:
            raise RuntimeError(f"layer {self.layer}: setup() has not run")
        store = self.store
        if store.path is not None and store.synced is None:
            self.pager.flush()
        if store.failed is not None:
            raise RuntimeError(f"vllm-expert-pager: SSD read failed\n{store.failed}")
        # The path is chosen from the shape alone, so capture and replay of a
        # graph take the same path.
        if topk_ids.numel() > self.table.num_slots:
            return self._forward_working(x, topk_weights, topk_ids, shared)

        layer, E = self.layer, self.pager.num_experts
        with trace.range(f"expert_pager L{layer} acquire"):
            todo, ssd_todo = self.acquire(topk_ids)
        dst_row, src_row = self.acquire.vram_slot, self.acquire.ram_slot
        cached_row = self.table.no_cache  # everything comes from the RAM tier
        base = layer * store.ram_slots
        lut = store.layer_lut(layer)
        if store.compress:
            # The decoder reads each miss's record straight from the RAM tier
            # (its loads run over the host link while it decodes) and copies
            # the scales, so no gather into staging comes first.
            src = [store.view[n] for n in PARAMS]
            dst = (self.cache_bytes, lut, self.scale_rows, self.cache_rows[2:])
            if store.path is None:
                with trace.range(f"expert_pager L{layer} decode"):
                    decode_rows_from_ram(todo, dst_row, cached_row, src_row, base, src, *dst)
            else:
                # Publish the SSD request, expand the experts that are in RAM
                # while the host reads, then wait and expand the rest. Every
                # listed SSD expert must fit the request slot, or one left
                # out would be expanded from a row the host never wrote.
                if ssd_todo.shape[0] > store.block:
                    raise RuntimeError(f"layer {layer}: {ssd_todo.shape[0]} SSD entries exceed the ring block "
                                       f"{store.block}")
                ticket = store.ticket_chunk[:1]
                fetch_publish_rows(ssd_todo, src_row, base, layer, store, ticket)
                with trace.range(f"expert_pager L{layer} decode"):
                    decode_rows_from_ram(todo, dst_row, cached_row, src_row, base, src, *dst, skip=ssd_todo)
                with trace.range(f"expert_pager L{layer} ssd wait"):
                    fetch_wait_rows(ssd_todo, store, ticket)
                with trace.range(f"expert_pager L{layer} decode ssd rows"):
                    decode_rows_from_ram(ssd_todo, dst_row, cached_row, src_row, base, src, *dst)
        elif store.path is None:
            rows = ([store.view[n] for n in PARAMS], self.cache_rows[:2], self.cache_rows[:2], None,
                    self.scale_rows, self.cache_rows[2:])
            # Every expert is in RAM (R = E): the RAM table always hits, so
            # there is never an SSD read and one copy does it all.
            with trace.range(f"expert_pager L{layer} gather"):
                gather_rows(todo, dst_row, cached_row, src_row, base, *rows)
        else:
            rows = ([store.view[n] for n in PARAMS], self.cache_rows[:2], self.cache_rows[:2], None,
                    self.scale_rows, self.cache_rows[2:])
            # One launch publishes the SSD request and copies the experts
            # that are in RAM while the host reads; then the ones read from SSD.
            with trace.range(f"expert_pager L{layer} gather + ssd wait"):
                gather_rows(todo, dst_row, cached_row, src_row, base, *rows, fetch=(ssd_todo, layer, store))
            with trace.range(f"expert_pager L{layer} gather ssd rows"):
                gather_rows(ssd_todo, dst_row, cached_row, src_row, base, *rows)

        if shared is not None:
            shared()
        with trace.range(f"expert_pager L{layer} experts"):
            if moe.decode_pays(x, topk_ids, self.pager.intermediate):
                slab = self.cache_slab
                out = moe.decode_experts(x, topk_weights, topk_ids, self.expert_map, E, slab[PARAMS[0]],
                                         slab[SCALES[0]], slab[PARAMS[1]], slab[SCALES[1]], self.table.num_slots,
                                         pair_slot=self.acquire.pair_slot, activation=self.activation)
                self._log()
                return out
            xq, xs, routing = moe.quant_route(x, topk_ids, self.expert_map, self.table.num_slots)
            contrib = self._contrib(topk_weights, x)
            self._run(self.cache_slab, xq, xs, topk_weights, topk_ids, contrib, routing)
        self._log()
        return moe.topk_sum(contrib, topk_ids, E)

    def _forward_working(self, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                         shared: Callable[[], object] | None = None) -> torch.Tensor:
        """Prefill (K > S): the experts go through the W-row working slab in chunks (experts.py:455-577).

        The VRAM table is not updated; VRAM hits are copied raw from the cache
        slab. The RAM tier acquires when K <= R and is otherwise seeded with
        the step's most referenced experts. Chunk k: copy the experts that
        need no wait -> publish chunk k+1's SSD read -> wait for chunk k's ->
        copy the experts that were read -> run the experts of chunk k. Every
        pair's contribution is written once; the top-k sum runs once at the
        end, so the result is that of a single run over all experts.
        ``shared`` runs once, before chunk 0's experts.
        """
        p, store = self.pager, self.store
        vram, ram = self.table, self.ram
        E, W = p.num_experts, p.settings.working_rows
        R, layer = store.ram_slots, self.layer

        need = ram.need_mask(topk_ids)
        cached_row = vram.slot_of[:E]
        before = ram.slot_of[:E].clone()
        if topk_ids.numel() <= R:
            ram.acquire(topk_ids)
        else:
            ram.seed(vram, topk_ids, need)
        dst_row, src_row, maps, todo, ssd, late = ram.plan_chunks(
            before, need, cached_row, W, layer * R, store.working_base
        )
        lut = store.layer_lut(layer)
        src = [store.view[n] for n in PARAMS]
        rows = (src, self.cache_rows[:2], self.working_rows[:2], p.pitch_rows, self.scale_rows,
                self.working_rows[2:])
        tickets = store.ticket_chunk

        def copy(part: torch.Tensor) -> None:
            # Cached experts raw from the cache slab; with a compressed tier
            # the others are expanded straight from the RAM tier.
            gather_rows(part, dst_row, cached_row, src_row, 0, *rows, cached_only=store.compress)
            if store.compress:
                decode_rows_from_ram(part, dst_row, cached_row, src_row, 0, src, self.working_bytes, lut,
                                     self.scale_rows, self.working_rows[2:])

        def chunk(t: torch.Tensor, k: int) -> torch.Tensor:
            return t[k * W : (k + 1) * W]

        def ticket(k: int) -> torch.Tensor:
            return tickets[k % 2 : k % 2 + 1]

        xq, xs = moe.quant_tokens(x)
        contrib = self._contrib(topk_weights, x)
        N = maps.shape[0]
        fetch_publish_rows(chunk(ssd, 0), src_row, 0, layer, store, ticket(0))
        for k in range(N):
            with trace.range(f"expert_pager L{layer} chunk {k}"):
                copy(chunk(todo, k))
                if k + 1 < N:
                    fetch_publish_rows(chunk(ssd, k + 1), src_row, 0, layer, store, ticket(k + 1))
                with trace.range(f"expert_pager L{layer} chunk {k} ssd wait"):
                    fetch_wait_rows(chunk(ssd, k), store, ticket(k))
                copy(chunk(late, k))
                self.expert_map.copy_(maps[k])
                if k == 0 and shared is not None:
                    shared()
                self._run(p.working_slab, xq, xs, topk_weights, topk_ids, contrib)
        self._log()
        return moe.topk_sum(contrib, topk_ids, E)

    def _contrib(self, topk_weights: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        # Every pair with a valid expert id is written: acquire maps every
        # needed expert, and plan_chunks maps each needed expert in exactly
        # one chunk. Pairs with an id outside [0, E) are skipped by the top-k
        # sum. So no zero fill is needed (the reference's kernel writes zeros
        # for experts outside a chunk's map, which the sum adds exactly).
        T, topk = topk_weights.shape
        return torch.empty((T * topk, x.shape[1]), dtype=torch.bfloat16, device=x.device)

    def _run(self, slab: dict[str, torch.Tensor], xq: torch.Tensor, xs: torch.Tensor, topk_weights: torch.Tensor,
             topk_ids: torch.Tensor, contrib: torch.Tensor, routing: moe.Routing | None = None) -> None:
        """Run the experts that ``expert_map`` places in ``slab`` (experts.py:579-604)."""
        S = slab[PARAMS[0]].shape[0]
        r = routing if routing is not None else moe.route(topk_ids, self.expert_map, S)
        moe.run_experts(xq, xs, topk_weights, slab[PARAMS[0]], slab[SCALES[0]], slab[PARAMS[1]], slab[SCALES[1]],
                        r, contrib, self.activation)

    # ---- counters ----

    def hit_rates(self) -> tuple[int, int, int, int]:
        """(vram hits, vram misses, ram hits, ram misses); reads the device."""
        vh, vm, rh, rm = torch.stack([self.table.hits, self.table.misses, self.ram.hits, self.ram.misses]).tolist()
        return vh, vm, rh, rm

    def _log(self) -> None:
        """Hit rates every ``log_interval`` eager calls (experts.py:613-649)."""
        self.calls += 1
        n = self.pager.settings.log_interval
        if n <= 0 or self.calls % n or not logger.isEnabledFor(logging.INFO):
            return
        if torch.cuda.is_current_stream_capturing():
            return
        vh, vm, rh, rm = self.hit_rates()
        logger.info(
            "vllm-expert-pager layer %d: vram hit %.1f%% (%d/%d), ram hit %.1f%% (%d/%d)", self.layer,
            100.0 * vh / (vh + vm) if vh + vm else 0.0, vh, vh + vm,
            100.0 * rh / (rh + rm) if rh + rm else 0.0, rh, rh + rm,
        )
        # The SSD tier is shared by every layer, so layer 0 reports it.
        store = self.store
        if self.layer == 0 and store.path is not None:
            fetches, reads, io_seconds, missed = store.stats()
            if fetches:
                logger.info(
                    "vllm-expert-pager ssd: %d fetches, %d reads, %.3f s, %.2f ms/fetch, "
                    "%d re-publishes, %d give-ups, %d missed",
                    fetches, reads, io_seconds, 1e3 * io_seconds / fetches,
                    int(store.req[store.retry_at]), int(store.req[store.giveup_at]), missed,
                )
