"""A stand-in for the few vLLM names the plugin touches (vLLM is not installed).

Installs modules ``vllm.config``, ``vllm.logger``,
``vllm.model_executor.layers.fused_moe.oracle.fp8``,
``vllm.model_executor.layers.fused_moe.routed_experts`` and
``...fused_moe.shared_experts`` (a ``SharedExperts`` that records its calls
and keeps its output) into ``sys.modules`` with a ``RoutedExperts`` base that carries the layer's ``activation``,
``apply_router_weight_on_input`` and shared experts (as vLLM's MoE layers
do) and creates block-fp8 expert parameters the way a w8a8 block-quantised
MoE layer does: ``w13_weight (E, 2I, H)``,
``w2_weight (E, H, I)`` float8_e4m3fn, ``w13_weight_scale_inv`` and
``w2_weight_scale_inv`` float32 per 128x128 block. It holds no vLLM code.
"""

from __future__ import annotations

import enum
import logging
import sys
import types
from types import SimpleNamespace

import torch

NUM_LAYERS = 2


class Fp8MoeBackend(enum.Enum):
    TRITON = "triton"
    MARLIN = "marlin"


class _QuantMethod:
    weight_scale_name = "weight_scale_inv"

    def __init__(self, backend=Fp8MoeBackend.TRITON):
        self.fp8_backend = backend
        self.processed = 0

    def process_weights_after_loading(self, layer) -> None:
        self.processed += 1


class SharedExperts(torch.nn.Module):
    """Shared experts as the MoE kernel sees them: called once with their
    input, they keep their output themselves. Records every input."""

    def __init__(self) -> None:
        super().__init__()
        self.inputs: list[torch.Tensor] = []
        self.output: torch.Tensor | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        self.inputs.append(x)
        self.output = x * 2
        return self.output


class RoutedExperts(torch.nn.Module):
    registered: list = []

    def __init__(self, num_experts, hidden_size, intermediate_size, *, use_ep=False, tp_size=1, device="cuda",
                 backend=Fp8MoeBackend.TRITON, layer_name="model.layers.0.mlp.experts", activation="silu",
                 apply_router_weight_on_input=False, shared_experts=None, config_activation=None):
        super().__init__()
        E, H, I = num_experts, hidden_size, intermediate_size
        self.layer_name = layer_name
        self.global_num_experts = E
        self.local_num_experts = E // 2 if use_ep else E
        self.use_ep = use_ep
        self.hidden_size, self.intermediate_size_per_partition = H, I
        self.activation = activation
        self.apply_router_weight_on_input = apply_router_weight_on_input
        self._shared_experts = shared_experts
        self.moe_config = SimpleNamespace(moe_parallel_config=SimpleNamespace(tp_size=tp_size))
        if config_activation is not None:  # newer layouts keep the activation on the config
            self.moe_config.activation = config_activation
        self.quant_method = _QuantMethod(backend)
        fp8 = torch.float8_e4m3fn
        p = lambda shape, dt: torch.nn.Parameter(torch.zeros(shape, dtype=dt, device=device), requires_grad=False)
        self.w13_weight = p((E, 2 * I, H), fp8)
        self.w2_weight = p((E, H, I), fp8)
        self.w13_weight_scale_inv = p((E, 2 * I // 128, H // 128), torch.float32)
        self.w2_weight_scale_inv = p((E, H // 128, I // 128), torch.float32)

    @property
    def expert_map(self):
        return None

    def weight_loader(self, param, loaded_weight, weight_name, shard_id, expert_id, return_success=False):
        if param is self.w13_weight_scale_inv:
            I = self.intermediate_size_per_partition // 128
            half = 0 if shard_id == "w1" else I
            param.data[expert_id, half : half + I].copy_(loaded_weight)
        else:
            param.data[expert_id].copy_(loaded_weight)
        return True if return_success else None

    @classmethod
    def register_oot(cls, sub):
        cls.registered.append(sub)


def install() -> None:
    def mod(name, **attrs):
        m = types.ModuleType(name)
        m.__dict__.update(attrs)
        sys.modules[name] = m
        return m

    config = SimpleNamespace(model_config=SimpleNamespace(hf_text_config=SimpleNamespace(num_hidden_layers=NUM_LAYERS)))
    mod("vllm")
    mod("vllm.config", get_current_vllm_config=lambda: config)
    mod("vllm.logger", init_logger=logging.getLogger)
    for pkg in ("vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.layers.fused_moe",
                "vllm.model_executor.layers.fused_moe.oracle"):
        mod(pkg)
    mod("vllm.model_executor.layers.fused_moe.oracle.fp8", Fp8MoeBackend=Fp8MoeBackend)
    mod("vllm.model_executor.layers.fused_moe.routed_experts", RoutedExperts=RoutedExperts)
    mod("vllm.model_executor.layers.fused_moe.shared_experts", SharedExperts=SharedExperts)


def uninstall() -> None:
    for name in [n for n in sys.modules if n == "vllm" or n.startswith("vllm.")]:
        del sys.modules[name]
    sys.modules.pop("vllm_expert_pager.experts", None)
