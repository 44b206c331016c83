"""The per-layer paging engine end to end on the GPU (pager.py).

Decode steps (K <= cache slots: acquire both tables, gather from the RAM
tier with the SSD request overlapped, expand compressed rows, run the
experts on the cache slab) and prefill overflow (K > cache slots: seed or
acquire the RAM tier, plan the chunks, copy/fetch/expand per chunk, run the
experts of each chunk on the working slab, one top-k sum) must both give
the bits of a one-shot run over a slab holding every expert
(experts.py:380-604). Covers the compressed tier with the paging file,
the raw RAM-only tier, prefill between decode steps, several layers sharing
the working slab, and a decode step captured in a hipGraph.
"""

import logging

import numpy as np
import pytest
import torch

from oracle import moe_ref as M

pytestmark = pytest.mark.gpu

H, I = 256, 128


def _mods():
    from vllm_expert_pager import moe, pager

    return moe, pager


class Model:
    """A pager with L layers of random block-fp8 experts, and the same weights on the GPU."""

    def __init__(self, tmp_path, E, S, R, W, compress, L=1, seed=0, log_interval=0, declared=None):
        moe, pager = _mods()
        settings = pager.Settings(
            cache_slots=S, ram_slots=R, ssd_path=str(tmp_path / "paging.bin") if R < E else None,
            compress="on" if compress else "off", working_rows=W, log_interval=log_interval,
        )
        self.pager = pager.Pager(settings, declared or L, E, H, I, torch.device("cuda"))
        self.E = E
        self.layers, self.weights = [], []
        rng = np.random.default_rng(seed)
        for _ in range(L):
            layer = self.pager.add_layer()
            w13, w13s, w2, w2s = M.random_experts(rng, E, H, I)
            for e in range(E):
                layer.load_expert(e, "w13_weight", torch.from_numpy(w13[e]))
                layer.load_expert(e, "w2_weight", torch.from_numpy(w2[e]))
            dev = [torch.from_numpy(a).cuda() for a in (w13, w13s, w2, w2s)]
            layer.setup({pager.SCALES[0]: dev[1], pager.SCALES[1]: dev[3]})
            self.layers.append(layer)
            self.weights.append(dev)

    def one_shot(self, i, x, tw, ids):
        moe = _mods()[0]
        w13, w13s, w2, w2s = self.weights[i]
        return moe.fused_moe(x, tw, ids, w13, w13s, w2, w2s)

    def close(self):
        self.pager.close()


@pytest.fixture
def model(tmp_path):
    made = []

    def make(*args, **kw):
        m = Model(tmp_path, *args, **kw)
        made.append(m)
        return m

    yield make
    for m in made:
        m.close()


def routing(rng, T, E, topk, zipf=1.1):
    """Top-k ids from a Zipf over a random permutation, softmax weights."""
    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** zipf
    p /= p.sum()
    ids = np.stack([perm[rng.choice(E, topk, replace=False, p=p)] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, topk)).astype(np.float32)
    w = np.exp(w) / np.exp(w).sum(1, keepdims=True)
    x = rng.standard_normal((T, H)).astype(np.float32)
    return (torch.from_numpy(x).to(torch.bfloat16).cuda(), torch.from_numpy(w.astype(np.float32)).cuda(),
            torch.from_numpy(ids).cuda())


def same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("compress, R", [(True, 16), (True, 64), (False, 64)])
def test_decode_steps_match_one_shot(model, compress, R):
    m = model(64, 4, R, 8, compress)
    rng = np.random.default_rng(1)
    layer = m.layers[0]
    for step in range(40):
        x, tw, ids = routing(rng, 1, m.E, 4)
        out = layer.forward(x, tw, ids)
        assert same(out, m.one_shot(0, x, tw, ids)), f"step {step}"
    vh, vm, rh, rm = layer.hit_rates()
    assert vh + vm == 160 and rh + rm == 160 and vh > 0
    assert m.pager.store.failed is None


@pytest.mark.parametrize("compress, R", [(True, 160), (False, 256)])
def test_batched_decode_steps_in_the_fused_step(model, compress, R):
    """2, 4 and 5 tokens x top-8 = 16, 32 and 40 pairs: the fused two-launch
    step, fed the acquire's per-pair slots, equals a one-shot run; the
    compressed case pages through the SSD tier (R < E)."""
    moe = _mods()[0]
    m = model(256, 128, R, 8, compress)
    rng = np.random.default_rng(12)
    layer = m.layers[0]
    for step in range(12):
        T = (2, 4, 5)[step % 3]
        x, tw, ids = routing(rng, T, m.E, 8, zipf=0.8)
        assert moe.decode_pays(x, ids, I)
        out = layer.forward(x, tw, ids)
        assert same(out, m.one_shot(0, x, tw, ids)), f"step {step}"
    vh, vm, rh, rm = layer.hit_rates()
    assert vh > 0 and vm > 0 and (rm > 0) == (R < 256)
    assert m.pager.store.failed is None


@pytest.mark.parametrize("compress, R", [(True, 160), (False, 256)])
def test_batched_decode_steps_beyond_the_fused_step(model, compress, R):
    """12, 9 and 6 tokens x top-8 = 96, 72 and 48 pairs over 128 cache slots:
    still the decode path (pairs <= S), but more pairs than the fused
    two-launch step is used for (96 and 72 are more than it takes, 48 more
    than it pays for), so quantise + route, the expert launches and the top-k
    sum run separately. The compressed case pages through the SSD tier (R < E)."""
    moe = _mods()[0]
    m = model(256, 128, R, 8, compress)
    rng = np.random.default_rng(11)
    layer = m.layers[0]
    for step in range(12):
        T = (9, 12, 6)[step % 3]
        x, tw, ids = routing(rng, T, m.E, 8, zipf=0.8)
        assert ids.numel() <= 128 and not moe.decode_pays(x, ids, I)
        assert moe.decode_fits(x, ids, I) == (T == 6)
        out = layer.forward(x, tw, ids)
        assert same(out, m.one_shot(0, x, tw, ids)), f"step {step}"
    vh, vm, rh, rm = layer.hit_rates()
    assert vh > 0 and vm > 0 and (rm > 0) == (R < 256)
    assert m.pager.store.failed is None


@pytest.mark.parametrize("compress, R", [(True, 16), (True, 64), (False, 64)])
@pytest.mark.parametrize("T", [3, 48])
def test_prefill_overflow_matches_one_shot(model, compress, R, T):
    """T=3 x top-4 = 12 ids: the RAM tier acquires; T=48: 192 ids > R, the RAM tier is seeded."""
    m = model(64, 4, R, 8, compress)
    rng = np.random.default_rng(T)
    layer = m.layers[0]
    for _ in range(3):
        x, tw, ids = routing(rng, T, m.E, 4, zipf=0.3)
        out = layer.forward(x, tw, ids)
        assert same(out, m.one_shot(0, x, tw, ids))
    assert m.pager.store.failed is None


@pytest.mark.parametrize("compress", [True, False])
def test_prefill_with_more_working_rows_than_experts(model, compress):
    """W = 64 working rows over 16 experts: a chunk's SSD listing (64 entries)
    is longer than a ring slot (16 entries, the power of two >= E); its
    experts sit below position 16, and only the slot's worth is published."""
    m = model(16, 4, 8, 64, compress)
    assert m.pager.store.block == 16
    rng = np.random.default_rng(12)
    layer = m.layers[0]
    for T in (3, 10, 1, 10):
        x, tw, ids = routing(rng, T, m.E, 4, zipf=0.3)
        out = layer.forward(x, tw, ids)
        assert same(out, m.one_shot(0, x, tw, ids)), f"T={T}"
    assert m.pager.store.failed is None
    assert m.pager.store.reads > 0


def test_paging_file_flushed_after_the_last_layer(model):
    """Once every layer's weights are in, the pager flushes the paging file
    (so that the server's reads do not wait on the page cache's write-back)
    and the reads that follow still serve the right rows."""
    m = model(64, 4, 16, 8, True, L=2)
    assert m.pager.layers_ready == 2 and m.pager.store.synced is not None
    rng = np.random.default_rng(5)
    for i, layer in enumerate(m.layers):
        x, tw, ids = routing(rng, 12, m.E, 4, zipf=0.3)
        assert same(layer.forward(x, tw, ids), m.one_shot(i, x, tw, ids))
    assert m.pager.store.failed is None


def test_paging_file_flushed_at_the_first_forward(model):
    """A model with fewer MoE layers than layers (dense layers in between)
    never reports its last layer: the flush then comes at the first forward."""
    m = model(64, 4, 16, 8, True, L=1, declared=3)
    assert m.pager.layers_ready == 1 and m.pager.store.synced is None
    rng = np.random.default_rng(6)
    x, tw, ids = routing(rng, 1, m.E, 4)
    assert same(m.layers[0].forward(x, tw, ids), m.one_shot(0, x, tw, ids))
    assert m.pager.store.synced is not None


def test_prefill_between_decode_steps_two_layers(model):
    """Layers share the working slab; decode steps between prefills read the RAM tier."""
    m = model(64, 4, 16, 8, True, L=2)
    rng = np.random.default_rng(7)
    for step in range(12):
        T = 40 if step % 4 == 1 else 1
        for i, layer in enumerate(m.layers):
            x, tw, ids = routing(rng, T, m.E, 4)
            out = layer.forward(x, tw, ids)
            assert same(out, m.one_shot(i, x, tw, ids)), f"step {step} layer {i} T={T}"


def test_decode_step_in_graph(model):
    m = model(64, 4, 16, 8, True)
    layer = m.layers[0]
    rng = np.random.default_rng(3)
    x0, tw0, ids0 = routing(rng, 1, m.E, 4)
    sx, stw, sids = x0.clone(), tw0.clone(), ids0.clone()
    layer.forward(sx, stw, sids)  # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            sout = layer.forward(sx, stw, sids)
    torch.cuda.current_stream().wait_stream(s)
    for step in range(20):
        x, tw, ids = routing(rng, 1, m.E, 4)
        sx.copy_(x)
        stw.copy_(tw)
        sids.copy_(ids)
        g.replay()
        torch.cuda.synchronize()
        assert same(sout, m.one_shot(0, x, tw, ids)), f"replay {step}"
    assert m.pager.store.failed is None


def test_log_and_roctx_ranges(model, caplog, monkeypatch):
    """Every log_interval eager calls a layer logs its hit rates and layer 0 the
    SSD tier's stats (experts.py:613-649); VLLM_EXPERT_PAGER_ROCTX=1 marks the
    steps as roctx ranges."""
    from vllm_expert_pager import trace

    monkeypatch.setenv("VLLM_EXPERT_PAGER_ROCTX", "1")
    monkeypatch.setattr(trace, "_loaded", False)
    monkeypatch.setattr(trace, "_lib", None)
    m = model(64, 4, 16, 8, True, log_interval=5)
    caplog.set_level(logging.INFO, logger="vllm.vllm_expert_pager.pager")
    rng = np.random.default_rng(5)
    layer = m.layers[0]
    for _ in range(10):
        x, tw, ids = routing(rng, 1, m.E, 4, zipf=0.5)
        layer.forward(x, tw, ids)
    x, tw, ids = routing(rng, 40, m.E, 4, zipf=0.5)
    layer.forward(x, tw, ids)  # the prefill path's chunk ranges
    torch.cuda.synchronize()
    msgs = [r.getMessage() for r in caplog.records]
    assert sum("layer 0: vram hit" in t for t in msgs) == 2, msgs
    assert any(t.startswith("vllm-expert-pager ssd:") and "fetches" in t for t in msgs), msgs
    assert trace._lib is not None
