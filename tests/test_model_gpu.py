"""The 40-layer model configurations at full size, through the pager on the GPU.

40 MoE layers x 256 experts of w13 (1024 x 2048) + w2 (2048 x 512) fp8 e4m3,
3 MiB per expert, N(0, 0.02) weights quantised with 128 x 128 block scales,
distinct per layer; 32 cache slots (experts.py:380-577):

- decode trace, raw tier (every expert in a raw pinned RAM tier): batch 1,
  top-8 Zipf(1.1) routing over a per-layer permutation with 70% reuse of the
  previous step's set, each step of all 40 layers one hipGraph replay;
- the same trace through the compressed tier (128 RAM slots of rows
  compressed at pitch 0.89, the other experts in a paging file read with
  O_DIRECT by the host server);
- one 2048-token prefill through the compressed tier (16384 ids > 32 slots:
  the RAM tier is seeded and every layer runs through the 64-row working slab
  in chunks), then more decode steps.

Checks, on sampled steps: every layer's output equals a one-shot run of the
same kernels over a slab of all 256 experts, bit for bit; both tables of
every layer equal the oracle's (TableRef fed the same ids); on sampled layers
every cache slot holds its expert's raw weights and scales, and (compressed
tier) every RAM slot holds its expert's record.
"""

from __future__ import annotations

import gc
import shutil
import time

import numpy as np
import pytest
import torch

from oracle.table_ref import TableRef

pytestmark = pytest.mark.gpu

L, E, H, I, K = 40, 256, 2048, 512, 8
S, W = 32, 64
CHECK_EVERY = 25


def log(msg: str) -> None:
    print(f"[model] {msg}", flush=True)


def layer_weights(layer: int, dev):
    """Block-fp8 experts of one layer, generated on the GPU from a per-layer seed."""
    g = torch.Generator(device=dev).manual_seed(5000 + layer)

    def one(n, k):
        q = torch.empty((E, n, k), dtype=torch.uint8, device=dev)
        s = torch.empty((E, n // 128, k // 128), dtype=torch.float32, device=dev)
        for e0 in range(0, E, 32):
            w = torch.randn((32, n, k), generator=g, device=dev) * 0.02
            b = w.view(32, n // 128, 128, k // 128, 128)
            se = (b.abs().amax(dim=(2, 4)) / 448.0).clamp_min(1e-10)
            q[e0 : e0 + 32] = (b / se[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(
                torch.uint8).view(32, n, k)
            s[e0 : e0 + 32] = se
        return q, s

    w13, w13s = one(2 * I, H)
    w2, w2s = one(H, I)
    return w13, w13s, w2, w2s


def zipf_trace(rng, steps: int, s: float = 1.1, reuse: float = 0.7) -> np.ndarray:
    """(steps, L, K) ids: K distinct per step from Zipf(s) over a per-layer
    permutation; with probability `reuse` a layer repeats its last set."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perms = [rng.permutation(E) for _ in range(L)]
    out = np.empty((steps, L, K), np.int64)
    for t in range(steps):
        for layer in range(L):
            if t > 0 and rng.random() < reuse:
                out[t, layer] = out[t - 1, layer]
            else:
                out[t, layer] = perms[layer][rng.choice(E, K, replace=False, p=p)]
    return out


# Table state without the sink elements (slot_of[E], expert_in[S],
# last_used[S]): they absorb the writes of unneeded experts, and which of
# several duplicate writes lands there is unspecified (table.py:96-104).
def table_state(t) -> tuple:
    E, n = t.num_experts, t.num_slots
    return (t.slot_of[:E].cpu().numpy(), t.expert_in[:n].cpu().numpy(), t.last_used[:n].cpu().numpy(),
            int(t.step), int(t.hits), int(t.misses))


def ref_state(t: TableRef) -> tuple:
    E, n = t.num_experts, t.num_slots
    return t.slot_of[:E], t.expert_in[:n], t.last_used[:n], t.step, t.hits, t.misses


def assert_same_table(got: tuple, want: tuple, what: str) -> None:
    names = ("slot_of", "expert_in", "last_used", "step", "hits", "misses")
    for n, a, b in zip(names, got, want):
        assert np.array_equal(np.asarray(a), np.asarray(b)), f"{what}: {n} differs"


class FullModel:
    """A pager over the 40 layers, the same weights kept on the GPU for one-shot
    checks, and the oracle's two tables per layer."""

    def __init__(self, settings, dev):
        from vllm_expert_pager import pager as pg

        t0 = time.time()
        self.dev = dev
        self.pager = pg.Pager(settings, L, E, H, I, dev)
        self.layers, self.weights = [], []
        for layer in range(L):
            w13, w13s, w2, w2s = layer_weights(layer, dev)
            lay = self.pager.add_layer()
            self.pager.store.write_rows(lay.layer, "w13_weight", w13.view(E, -1))
            self.pager.store.write_rows(lay.layer, "w2_weight", w2.view(E, -1))
            lay.setup({pg.SCALES[0]: w13s, pg.SCALES[1]: w2s})
            self.layers.append(lay)
            self.weights.append((w13, w13s, w2, w2s))
        torch.cuda.synchronize()
        self.R = self.pager.store.ram_slots
        self.vref = [TableRef(E, S) for _ in range(L)]
        self.rref = [TableRef(E, self.R) for _ in range(L)]
        for r in self.rref:
            r.warm(self.R)
        log(f"{L} layers loaded in {time.time() - t0:.1f} s (R={self.R}, "
            f"{'compressed' if self.pager.store.compress else 'raw'})")
        self.graph = None

    def close(self) -> None:
        self.graph = None
        self.pager.close()

    # ---- decode ----

    def _step(self) -> None:
        for layer, lay in enumerate(self.layers):
            self.out[layer] = lay.forward(self.x[layer], self.tw[layer], self.ids[layer])

    def first_step(self, ids: np.ndarray, gen: torch.Generator) -> None:
        """Static buffers of a 40-layer decode step, and step `ids` run eagerly."""
        dev = self.dev
        self.x = torch.empty((L, 1, H), dtype=torch.bfloat16, device=dev)
        self.tw = torch.empty((L, 1, K), dtype=torch.float32, device=dev)
        self.ids = torch.empty((L, 1, K), dtype=torch.int64, device=dev)
        self.out = [None] * L
        self._fill(ids, gen)
        self._step()
        self._advance_oracle(ids)

    def capture(self) -> None:
        """One graph of the decode step over the static buffers (recorded, not run)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=side):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()

    def _fill(self, ids: np.ndarray, gen: torch.Generator) -> None:
        self.x.copy_(torch.randn((L, 1, H), generator=gen, device=self.dev))
        self.tw.copy_(torch.softmax(torch.randn((L, 1, K), generator=gen, device=self.dev), dim=2))
        self.ids.copy_(torch.from_numpy(ids).view(L, 1, K))

    def _advance_oracle(self, ids: np.ndarray) -> None:
        for layer in range(L):
            self.vref[layer].acquire(ids[layer], pair_slots=True)
            self.rref[layer].acquire(ids[layer], pair_slots=True)

    def decode(self, ids: np.ndarray, gen: torch.Generator) -> None:
        self._fill(ids, gen)
        self.graph.replay()
        self._advance_oracle(ids)

    # ---- checks ----

    def check_outputs(self, what: str, x=None, tw=None, ids=None, outs=None) -> None:
        from vllm_expert_pager import moe

        torch.cuda.synchronize()
        for layer in range(L):
            xl = self.x[layer] if x is None else x[layer]
            twl = self.tw[layer] if tw is None else tw[layer]
            il = self.ids[layer] if ids is None else ids[layer]
            got = self.out[layer] if outs is None else outs[layer]
            want = moe.fused_moe(xl, twl, il, *self.weights[layer])
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"{what}: layer {layer} output"

    def check_tables(self, what: str) -> None:
        for layer, lay in enumerate(self.layers):
            assert_same_table(table_state(lay.table), ref_state(self.vref[layer]), f"{what} layer {layer} VRAM")
            assert_same_table(table_state(lay.ram), ref_state(self.rref[layer]), f"{what} layer {layer} RAM")

    def check_cache_slab(self, layer: int, what: str) -> None:
        from vllm_expert_pager import pager as pg

        lay, (w13, w13s, w2, w2s) = self.layers[layer], self.weights[layer]
        occupant = lay.table.expert_in[:S]
        used = torch.nonzero(occupant >= 0).view(-1)
        e = occupant[used]
        slab = lay.cache_slab
        for name, ref in (("w13_weight", w13), ("w2_weight", w2), (pg.SCALES[0], w13s), (pg.SCALES[1], w2s)):
            assert torch.equal(slab[name][used], ref[e]), f"{what}: layer {layer} cache slab {name}"

    def check_ram_rows(self, layer: int, what: str) -> None:
        """Every occupied RAM slot of `layer` holds its expert's row (record when compressed)."""
        from vllm_expert_pager import codec

        st = self.pager.store
        lay = self.layers[layer]
        occupant = lay.ram.expert_in[: self.R].cpu()
        used = torch.nonzero(occupant >= 0).view(-1)
        e = occupant[used].to(self.dev)
        for name, w in (("w13_weight", self.weights[layer][0]), ("w2_weight", self.weights[layer][2])):
            rows = st.pinned[name][layer * self.R + used].view(torch.uint8).to(self.dev)
            want = w[e].view(len(e), -1)
            if st.compress:
                want = codec.encode_rows(want, st.pitch[name])[0]
            assert torch.equal(rows, want), f"{what}: layer {layer} RAM rows of {name}"


def run_trace(m: FullModel, steps: int, seed: int, label: str, check_slabs=(0, 17, 39)) -> None:
    gen = torch.Generator(device=m.dev).manual_seed(seed)
    trace = zipf_trace(np.random.default_rng(seed), steps)
    t0 = time.time()
    m.first_step(trace[0], gen)
    m.check_outputs(f"{label} step 0 (eager)")
    m.check_tables(f"{label} step 0 (eager)")
    m.capture()
    for t in range(1, steps):
        m.decode(trace[t], gen)
        if t % CHECK_EVERY == 0 or t == steps - 1:
            m.check_outputs(f"{label} step {t}")
            m.check_tables(f"{label} step {t}")
            for layer in check_slabs:
                m.check_cache_slab(layer, f"{label} step {t}")
            if m.pager.store.compress and t % (4 * CHECK_EVERY) == 0:
                m.check_ram_rows(check_slabs[t // (4 * CHECK_EVERY) % len(check_slabs)], f"{label} step {t}")
    torch.cuda.synchronize()
    vh = sum(r.hits for r in m.vref)
    vm = sum(r.misses for r in m.vref)
    rh = sum(r.hits for r in m.rref)
    rm = sum(r.misses for r in m.rref)
    log(f"{label}: {steps} steps in {time.time() - t0:.1f} s, VRAM hit {vh / (vh + vm):.3f}, "
        f"RAM hit {rh / (rh + rm):.3f}")
    assert m.pager.store.failed is None, m.pager.store.failed


def _release(m: FullModel) -> None:
    m.close()
    del m
    gc.collect()
    torch.cuda.empty_cache()


def test_decode_trace_raw_tier():
    """Config 3: 40 x 256 x 3 MiB, 32 cache slots, every expert in RAM (raw)."""
    from vllm_expert_pager import pager as pg

    settings = pg.Settings(cache_slots=S, ram_slots=None, compress="off", working_rows=W, log_interval=0)
    m = FullModel(settings, torch.device("cuda"))
    try:
        run_trace(m, 300, seed=31, label="raw tier")
    finally:
        _release(m)


@pytest.fixture(scope="module")
def compressed(tmp_path_factory):
    """Configs 4 and 5: 128 compressed RAM slots at pitch 0.89 and a paging file."""
    from vllm_expert_pager import pager as pg

    where = tmp_path_factory.mktemp("paging")
    need = L * E * (1_867_776 + 933_888)
    free = shutil.disk_usage(where).free
    if free < need + (4 << 30):
        pytest.skip(f"the paging file needs {need / 2**30:.1f} GiB; {free / 2**30:.1f} GiB free at {where}")
    settings = pg.Settings(cache_slots=S, ram_slots=128, ssd_path=str(where / "paging.bin"), compress="on",
                           pitch_ratio=0.89, working_rows=W, log_interval=0)
    m = FullModel(settings, torch.device("cuda"))
    assert m.pager.store.record_bytes == 1_867_776 + 933_888
    yield m
    _release(m)


def test_decode_trace_compressed_tier(compressed):
    run_trace(compressed, 200, seed=41, label="compressed tier")
    st = compressed.pager.store
    fetches, reads, _, missed = st.stats()
    log(f"compressed tier: {fetches} requests, {reads} records read, {missed} missed")
    assert reads > 0 and missed == 0
    assert int(st.req[st.giveup_at]) == 0


def test_prefill_2048_tokens_then_decode(compressed):
    """Config 5 on the same model (after the decode trace): all 40 layers of a
    2048-token prompt bit-exact against one-shot runs, the RAM tables equal to
    the oracle's seed, and decode steps after it still exact."""
    m = compressed
    dev = m.dev
    T = 2048
    g = torch.Generator(device=dev).manual_seed(77)
    xs = torch.randn((L, T, H), generator=g, device=dev).to(torch.bfloat16)
    top, ids = torch.randn((L, T, E), generator=g, device=dev).topk(K, dim=2)
    tws = torch.softmax(top, dim=2).float().contiguous()
    ids_np = ids.cpu().numpy()
    st = m.pager.store
    f0, r0 = st.fetches, st.reads
    t0 = time.time()
    outs = [lay.forward(xs[layer], tws[layer], ids[layer]) for layer, lay in enumerate(m.layers)]
    torch.cuda.synchronize()
    log(f"prefill of {T} tokens over {L} layers: {time.time() - t0:.2f} s, {st.fetches - f0} requests, "
        f"{st.reads - r0} records read")
    for layer in range(L):  # the RAM tier is seeded, the VRAM table untouched (table.py:140-171)
        ref = m.rref[layer]
        ref.seed(m.vref[layer], ids_np[layer], ref.need_mask(ids_np[layer]))
    m.check_outputs("prefill", x=xs, tw=tws, ids=ids, outs=outs)
    m.check_tables("after prefill")
    for layer in (0, 39):
        m.check_ram_rows(layer, "after prefill")
    assert st.failed is None, st.failed
    del xs, tws, ids, outs
    gen = torch.Generator(device=dev).manual_seed(43)
    trace = zipf_trace(np.random.default_rng(43), 30)
    start = 0
    if not hasattr(m, "x"):  # run without the decode trace before it: capture here
        m.first_step(trace[0], gen)
        m.capture()
        start = 1
    for t in range(start, 30):
        m.decode(trace[t], gen)
    m.check_outputs("decode after prefill")
    m.check_tables("decode after prefill")
    m.check_cache_slab(5, "decode after prefill")
    assert st.failed is None, st.failed
