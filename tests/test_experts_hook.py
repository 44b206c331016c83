"""The vLLM-facing hook (experts.py) against a stand-in vLLM (tests/_fake_vllm.py).

CPU: the plugin entry registers the class; expert and tensor parallelism
are refused; settings are validated with the reference's messages
(experts.py:100-130); shared experts and ``apply_router_weight_on_input``
reach the pager as the reference hands them to vLLM (experts.py:380-387,
452, 569-573). GPU: a two-layer model loads its experts through
``weight_loader`` (w1/w3 shards staged into w13), runs the wrapped
``process_weights_after_loading``, and ``forward_modular`` on decode and
prefill shapes gives the bits of a one-shot run over all experts, with the
shared experts called once per forward on their input. Parity of the shared
experts' placement against vLLM itself is unpinned (vLLM is not installed).
"""

import importlib

import numpy as np
import pytest
import torch

import _fake_vllm
from oracle import moe_ref as M

H, I, E = 256, 128, 32


@pytest.fixture
def hook(monkeypatch, tmp_path):
    _fake_vllm.install()
    for k, v in {
        "VLLM_EXPERT_PAGER_CACHE_SLOTS": "4",
        "VLLM_EXPERT_PAGER_RAM_SLOTS": "16",
        "VLLM_EXPERT_PAGER_WORKING_ROWS": "8",
        "VLLM_EXPERT_PAGER_SSD_PATH": str(tmp_path / "paging.bin"),
        "VLLM_EXPERT_PAGER_LOG_INTERVAL": "0",
    }.items():
        monkeypatch.setenv(k, v)
    experts = importlib.import_module("vllm_expert_pager.experts")
    yield experts
    if experts._pager is not None:
        experts._pager.close()
        experts._pager = None
    _fake_vllm.uninstall()


def test_register_adds_the_class(hook):
    from vllm_expert_pager import plugin

    base = _fake_vllm.RoutedExperts
    n = len(base.registered)
    plugin.register()
    assert base.registered[n:] == [hook.ExpertPagerRoutedExperts]


def test_refuses_expert_and_tensor_parallelism(hook):
    with pytest.raises(RuntimeError, match="expert parallelism"):
        hook.ExpertPagerRoutedExperts(E, H, I, use_ep=True, device="cpu")
    with pytest.raises(RuntimeError, match="tensor parallelism"):
        hook.ExpertPagerRoutedExperts(E, H, I, tp_size=2, device="cpu")


class _Act(__import__("enum").Enum):
    SILU = "silu"
    GELU = "gelu"
    GELU_TANH = "gelu_tanh"


@pytest.mark.parametrize(
    "kw, match",
    [
        (dict(activation="gelu_tanh"), "activation 'gelu_tanh'"),
        (dict(activation=_Act.GELU_TANH), "activation 'gelu_tanh'"),
        (dict(config_activation="swigluoai"), "activation 'swigluoai'"),
        (dict(activation="silu", config_activation="gelu"), "different activations"),
    ],
)
def test_refuses_modes_the_kernels_do_not_compute(hook, kw, match):
    """The expert FFN is this package's own (silu or gelu of the gate times
    up, routed weight on the output, routed sum only); anything else vLLM's
    fused MoE would have done for the reference (experts.py:594-600) is
    refused at construction."""
    with pytest.raises(RuntimeError, match=match):
        hook.ExpertPagerRoutedExperts(E, H, I, device="cpu", **kw)
    assert hook._pager is None  # refused before any tier is allocated


@pytest.mark.parametrize("act, name", [("silu", "silu"), ("SiLU", "silu"), (_Act.SILU, "silu"),
                                       ("gelu", "gelu"), ("GELU", "gelu"), (_Act.GELU, "gelu")])
def test_accepts_silu_and_gelu_in_any_spelling(hook, act, name):
    layer = _fake_vllm.RoutedExperts(E, H, I, device="cpu", activation=act)
    assert hook._unsupported_modes(layer) == []
    assert hook._activation(layer) == name


def test_activation_from_the_config_alone(hook):
    layer = _fake_vllm.RoutedExperts(E, H, I, device="cpu", activation=None, config_activation="gelu")
    assert hook._unsupported_modes(layer) == []
    assert hook._activation(layer) == "gelu"
    assert hook._activation(_fake_vllm.RoutedExperts(E, H, I, device="cpu", activation=None)) == "silu"


class _StubPager:
    """Records what forward_modular hands the layer's pager."""

    expert_map = None

    def __init__(self):
        self.calls = []

    def forward(self, x, topk_weights, topk_ids, shared=None):
        self.calls.append((x, topk_weights, topk_ids, shared))
        if shared is not None:
            shared()
        return x


def _stub_layer(**kw):
    layer = _fake_vllm.RoutedExperts(E, H, I, device="cpu", **kw)
    layer._expert_pager = _StubPager()
    return layer


@pytest.mark.parametrize("T", [1, 3, 40])  # decode and overflow shapes alike
@pytest.mark.parametrize("separate_input", [False, True])
def test_shared_experts_reach_the_pager(hook, T, separate_input):
    """The shared experts run once per forward, on ``shared_experts_input``
    when given and on ``x`` otherwise; the routed result is returned alone."""
    layer = _stub_layer()
    shared = _fake_vllm.SharedExperts()
    x = torch.randn((T, H)).to(torch.bfloat16)
    sx = torch.randn((T, H)).to(torch.bfloat16) if separate_input else None
    tw, ids = torch.ones((T, 4)), torch.zeros((T, 4), dtype=torch.int64)
    out = hook.ExpertPagerRoutedExperts.forward_modular(layer, x, tw, ids, shared_experts=shared,
                                                        shared_experts_input=sx)
    assert out is x
    assert len(shared.inputs) == 1 and shared.inputs[0] is (sx if separate_input else x)
    assert len(layer._expert_pager.calls) == 1
    assert layer.expert_map is None
    # Without shared experts the pager gets no callback.
    hook.ExpertPagerRoutedExperts.forward_modular(layer, x, tw, ids)
    assert layer._expert_pager.calls[-1][3] is None and len(shared.inputs) == 1


def test_router_weight_on_input(hook):
    """vLLM's no-EP prepare step for ``apply_router_weight_on_input``: the
    tokens are multiplied by their routed weight rounded to the token dtype,
    the experts add their outputs unweighted, and top-k must be 1."""
    layer = _stub_layer(apply_router_weight_on_input=True)
    x = torch.randn((5, H)).to(torch.bfloat16)
    tw = torch.rand((5, 1))
    ids = torch.zeros((5, 1), dtype=torch.int64)
    hook.ExpertPagerRoutedExperts.forward_modular(layer, x, tw, ids)
    px, ptw, pids, _ = layer._expert_pager.calls[-1]
    want = (x.float() * tw.to(torch.bfloat16).float()).to(torch.bfloat16)
    assert px.dtype == torch.bfloat16 and torch.equal(px.view(torch.int16), want.view(torch.int16))
    assert ptw.dtype == torch.float32 and torch.equal(ptw, torch.ones((5, 1))) and pids is ids
    with pytest.raises(RuntimeError, match="layers.0.*top-k 1, got 2"):
        hook.ExpertPagerRoutedExperts.forward_modular(layer, x, torch.rand((5, 2)), torch.zeros((5, 2)))
    # The mode may also sit on the layer's moe_config.
    layer = _stub_layer()
    layer.moe_config.apply_router_weight_on_input = True
    with pytest.raises(RuntimeError, match="top-k 1"):
        hook.ExpertPagerRoutedExperts.forward_modular(layer, x, torch.rand((5, 2)), torch.zeros((5, 2)))


def test_settings_are_validated(hook):
    hook.SETTINGS.ram_slots = 2
    with pytest.raises(ValueError, match="RAM_SLOTS=2 must be >= VLLM_EXPERT_PAGER_CACHE_SLOTS=4"):
        hook.ExpertPagerRoutedExperts(E, H, I, device="cpu")
    hook.SETTINGS.ram_slots = 16
    hook.SETTINGS.working_rows = 0
    with pytest.raises(ValueError, match="WORKING_ROWS must be >= 1"):
        hook.ExpertPagerRoutedExperts(E, H, I, device="cpu")
    hook.SETTINGS.working_rows = 8
    hook.SETTINGS.compress = "maybe"
    with pytest.raises(ValueError, match="COMPRESS must be auto, on or off"):
        hook.ExpertPagerRoutedExperts(E, H, I, device="cpu")


def test_settings_from_env(hook):
    s = hook.SETTINGS
    assert (s.cache_slots, s.ram_slots, s.working_rows, s.compress, s.pitch_ratio) == (4, 16, 8, "auto", 0.89)


def _load_layer(hook, rng, li, **kw):
    """One hooked layer on the GPU with random block-fp8 experts loaded the
    way vLLM's loader sends them (w3, w2, w1 shards, then scales)."""
    layer = hook.ExpertPagerRoutedExperts(E, H, I, device="cuda", layer_name=f"model.layers.{li}.mlp.experts", **kw)
    w13, w13s, w2, w2s = M.random_experts(rng, E, H, I)
    f8 = lambda a: torch.from_numpy(a).view(torch.float8_e4m3fn)
    for e in rng.permutation(E):
        layer.weight_loader(layer.w13_weight, f8(w13[e, I:]), "w3", "w3", int(e))
        layer.weight_loader(layer.w2_weight, f8(w2[e]), "w2", "w2", int(e))
        layer.weight_loader(layer.w13_weight, f8(w13[e, :I]), "w1", "w1", int(e))
        layer.weight_loader(layer.w13_weight_scale_inv, torch.from_numpy(w13s[e, : I // 128]), "s", "w1", int(e))
        layer.weight_loader(layer.w13_weight_scale_inv, torch.from_numpy(w13s[e, I // 128 :]), "s", "w3", int(e))
        layer.weight_loader(layer.w2_weight_scale_inv, torch.from_numpy(w2s[e]), "s", "w2", int(e))
    assert not layer._expert_pager_stage
    layer.quant_method.process_weights_after_loading(layer)
    assert layer.quant_method.processed == 1 and layer.w13_weight.shape[0] == 1
    return layer, [torch.from_numpy(a).cuda() for a in (w13, w13s, w2, w2s)]


@pytest.mark.gpu
def test_load_and_forward_bit_exact(hook):
    """Decode steps and a 37-token overflow prefill (148 pairs through 8
    working rows, so several chunks), each layer's routed output equal to a
    one-shot run; on every other call shared experts are handed in, and they
    run exactly once per forward on their own input."""
    from vllm_expert_pager import moe

    rng = np.random.default_rng(0)
    layers, weights = zip(*[_load_layer(hook, rng, li) for li in range(_fake_vllm.NUM_LAYERS)])
    shared = _fake_vllm.SharedExperts()
    for step, T in enumerate([1, 1, 37, 1, 2, 1, 37]):
        for li, layer in enumerate(layers):
            x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).cuda()
            ids = torch.from_numpy(np.stack([rng.permutation(E)[:4] for _ in range(T)])).cuda()
            tw = torch.softmax(torch.randn((T, 4), device="cuda"), dim=1)
            use_shared = (step + li) % 2 == 0
            sx = torch.randn((T, H), device="cuda").to(torch.bfloat16) if step % 3 == 2 else None
            n = len(shared.inputs)
            out = layer.forward_modular(x, tw, ids, shared_experts=shared if use_shared else None,
                                        shared_experts_input=sx)
            ref = moe.fused_moe(x, tw, ids, *weights[li])
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step} layer {li} T={T}"
            assert layer.expert_map is None
            assert len(shared.inputs) == n + use_shared, f"step {step} layer {li}: shared experts calls"
            if use_shared:
                want = x if sx is None else sx
                assert shared.inputs[-1] is want and torch.equal(shared.output, want * 2)
    with pytest.raises(RuntimeError, match="monolithic"):
        layers[0].forward_monolithic()


@pytest.mark.gpu
def test_router_weight_on_input_bit_exact(hook):
    """``apply_router_weight_on_input`` at top-k 1, decode and overflow
    shapes: the output equals a one-shot run on the tokens scaled by their
    bf16-rounded routed weight with unit output weights."""
    from vllm_expert_pager import moe

    rng = np.random.default_rng(1)
    layer, weights = _load_layer(hook, rng, 0, apply_router_weight_on_input=True)
    for step, T in enumerate([1, 3, 40, 1]):
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).cuda()
        ids = torch.from_numpy(rng.integers(0, E, (T, 1))).cuda()
        tw = torch.rand((T, 1), device="cuda")
        out = layer.forward_modular(x, tw, ids)
        xin = (x.float() * tw.to(torch.bfloat16).float()).to(torch.bfloat16)
        ref = moe.fused_moe(xin, torch.ones_like(tw), ids, *weights)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step} T={T}"


@pytest.mark.gpu
def test_gelu_layer_bit_exact(hook):
    """A layer whose activation is GELU: decode and overflow shapes equal a
    one-shot GELU run, and differ from the SiLU one (the activation reaches
    the kernels)."""
    from vllm_expert_pager import moe

    rng = np.random.default_rng(2)
    layer, weights = _load_layer(hook, rng, 0, activation="gelu")
    for step, T in enumerate([1, 2, 37, 1]):
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).cuda()
        ids = torch.from_numpy(np.stack([rng.permutation(E)[:4] for _ in range(T)])).cuda()
        tw = torch.softmax(torch.randn((T, 4), device="cuda"), dim=1)
        out = layer.forward_modular(x, tw, ids)
        ref = moe.fused_moe(x, tw, ids, *weights, activation="gelu")
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step} T={T}"
        silu = moe.fused_moe(x, tw, ids, *weights)
        assert not torch.equal(out.view(torch.int16), silu.view(torch.int16)), f"step {step} T={T}"
