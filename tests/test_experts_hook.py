"""The vLLM-facing hook (experts.py) against a stand-in vLLM (tests/_fake_vllm.py).

CPU: the plugin entry registers the class; expert and tensor parallelism
are refused; settings are validated with the reference's messages
(experts.py:100-130). GPU: a two-layer model loads its experts through
``weight_loader`` (w1/w3 shards staged into w13), runs the wrapped
``process_weights_after_loading``, and ``forward_modular`` on decode and
prefill shapes gives the bits of a one-shot run over all experts.
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


@pytest.mark.parametrize(
    "kw, match",
    [
        (dict(activation="gelu"), "activation 'gelu'"),
        (dict(activation=_Act.GELU), "activation 'gelu'"),
        (dict(config_activation="swigluoai"), "activation 'swigluoai'"),
        (dict(apply_router_weight_on_input=True), "apply_router_weight_on_input"),
        (dict(shared_experts=object()), "shared experts"),
    ],
)
def test_refuses_modes_the_kernels_do_not_compute(hook, kw, match):
    """The expert FFN is this package's own (silu(gate) * up, routed weight on
    the output, routed sum only); anything else vLLM's fused MoE would have
    done for the reference (experts.py:594-600) is refused at construction."""
    with pytest.raises(RuntimeError, match=match):
        hook.ExpertPagerRoutedExperts(E, H, I, device="cpu", **kw)
    assert hook._pager is None  # refused before any tier is allocated


def test_accepts_silu_in_any_spelling(hook):
    for act in ("silu", "SiLU", _Act.SILU):
        assert hook._unsupported_modes(_fake_vllm.RoutedExperts(E, H, I, device="cpu", activation=act)) == []


def test_shared_experts_passed_at_forward_are_refused(hook):
    """A layer that hands shared experts to forward_modular is refused rather
    than given the routed output alone (the shared output's contract is
    vLLM's). Checked before any GPU work, so it runs without a GPU."""
    layer = _fake_vllm.RoutedExperts(E, H, I, device="cpu")
    layer.layer_name = "model.layers.3.mlp.experts"
    x = torch.zeros((1, H), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="layers.3.*shared experts"):
        hook.ExpertPagerRoutedExperts.forward_modular(layer, x, torch.ones((1, 4)), torch.zeros((1, 4)),
                                                      shared_experts=lambda t: t)


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


@pytest.mark.gpu
def test_load_and_forward_bit_exact(hook):
    from vllm_expert_pager import moe

    rng = np.random.default_rng(0)
    layers, weights = [], []
    for li in range(_fake_vllm.NUM_LAYERS):
        layer = hook.ExpertPagerRoutedExperts(E, H, I, device="cuda", layer_name=f"model.layers.{li}.mlp.experts")
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
        layers.append(layer)
        weights.append([torch.from_numpy(a).cuda() for a in (w13, w13s, w2, w2s)])

    for step, T in enumerate([1, 1, 37, 1, 2, 1]):
        for li, layer in enumerate(layers):
            x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).cuda()
            ids = torch.from_numpy(np.stack([rng.permutation(E)[:4] for _ in range(T)])).cuda()
            tw = torch.softmax(torch.randn((T, 4), device="cuda"), dim=1)
            out = layer.forward_modular(x, tw, ids)
            ref = moe.fused_moe(x, tw, ids, *weights[li])
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step} layer {li} T={T}"
            assert layer.expert_map is None
    with pytest.raises(RuntimeError, match="monolithic"):
        layers[0].forward_monolithic()
