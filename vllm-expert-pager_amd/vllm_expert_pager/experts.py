"""vLLM hook: a ``RoutedExperts`` whose expert weights are paged through a slab.

Same surface as the reference's ``ExpertPagerRoutedExperts`` (experts.py:86-653):
the ``vllm.general_plugins`` entry registers it out of tree; construction
replaces the ``(E, ...)`` expert weights by one-row placeholders;
``weight_loader`` sends each expert's fp8 rows to the store (w1 into the
first half of w13, w3 into the second); the quant method's
``process_weights_after_loading`` is wrapped so the slabs and tables are
built right after it; ``forward_modular`` runs the decode or the prefill
overflow path of the layer's ``PagedExperts`` (pager.py). The expert FFN is
this package's own fp8 MFMA kernels (csrc/moe.hip) rather than vLLM's fused
MoE, so no ``moe_sum`` intercept is needed: the top-k sum runs once by
construction. Shared experts handed to ``forward_modular`` run once per
forward, right before the first expert launch (the reference passes them to
the decode run and to chunk 0 of the overflow path, experts.py:452, 569-573),
and the routed sum alone is returned, the shared output staying with the
shared experts object (experts.py:475-477). ``apply_router_weight_on_input``
scales the tokens by their routed weight before the experts and leaves the
outputs unweighted, as vLLM's no-EP prepare step does (top-k must be 1).
The kernels compute ``act(gate) * up`` for act SiLU or (erf) GELU, vLLM's
``silu_and_mul`` and ``gelu_and_mul``; layers that ask for another
activation are refused with ``RuntimeError``. Settings are the
``VLLM_EXPERT_PAGER_*`` environment variables, read at import.

Importing this module requires vLLM; ``plugin.register`` imports it only
after vLLM has loaded.
"""

from __future__ import annotations

import torch
from vllm.config import get_current_vllm_config
from vllm.logger import init_logger
from vllm.model_executor.layers.fused_moe.oracle.fp8 import Fp8MoeBackend
from vllm.model_executor.layers.fused_moe.routed_experts import RoutedExperts

from vllm_expert_pager.moe import ACTIVATIONS
from vllm_expert_pager.pager import PARAMS, SCALES, Pager, PagedExperts, Settings

logger = init_logger(f"vllm.{__name__}")

SETTINGS = Settings.from_env()

# One pager per model: the store and the shared working slab.
_pager: Pager | None = None


def _mode_name(value) -> str:
    """Lower-case name of a mode given as a string or an enum member."""
    if isinstance(value, str):
        return value.lower()
    inner = getattr(value, "value", None)
    if isinstance(inner, str):
        return inner.lower()
    return str(getattr(value, "name", value)).lower()


def _activation(layer) -> str:
    """The layer's expert activation name: its own ``activation``, else its
    ``moe_config``'s, else "silu" (vLLM's default)."""
    for owner in (layer, getattr(layer, "moe_config", None)):
        act = getattr(owner, "activation", None) if owner is not None else None
        if act is not None:
            return _mode_name(act)
    return "silu"


def _unsupported_modes(layer) -> list[str]:
    """What the layer asks of the expert FFN that csrc/moe.hip does not compute.

    The kernels compute ``act(gate) * up`` over w13's gate rows then up rows,
    for the activations in ``moe.ACTIVATIONS``. The reference leaves the
    activation to vLLM's fused MoE (experts.py:594-600), which reads the
    layer's ``activation`` (on the layer or its ``moe_config``). Each
    activation the kernels would get silently wrong is listed here so
    construction can refuse it.
    """
    found = []
    for owner in (layer, getattr(layer, "moe_config", None)):
        if owner is None:
            continue
        act = getattr(owner, "activation", None)
        if act is not None and _mode_name(act) not in ACTIVATIONS:
            found.append(f"activation {_mode_name(act)!r} (the kernels compute {' or '.join(ACTIVATIONS)})")
        if getattr(owner, "is_act_and_mul", True) is False:
            found.append("an activation without the gate/up product")
    names = {_mode_name(getattr(o, "activation")) for o in (layer, getattr(layer, "moe_config", None))
             if o is not None and getattr(o, "activation", None) is not None}
    if len(names) > 1:
        found.append(f"different activations on the layer and its config ({', '.join(sorted(names))})")
    return list(dict.fromkeys(found))


def _router_weight_on_input(layer) -> bool:
    """Whether the layer (or its ``moe_config``) applies the routed weight to
    the expert input instead of the expert output."""
    return any(
        bool(getattr(owner, "apply_router_weight_on_input", False))
        for owner in (layer, getattr(layer, "moe_config", None))
        if owner is not None
    )


class ExpertPagerRoutedExperts(RoutedExperts):
    """``RoutedExperts`` that references expert weights through a slab.

    Uses the cache slab when ``topk_ids`` has no more elements than there are
    cache slots and the working slab otherwise, decided on the shape alone so
    that graph capture and replay take the same path.
    """

    _expert_pager_expert_map: torch.Tensor | None = None

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        if self.use_ep or self.local_num_experts != self.global_num_experts:
            raise RuntimeError(
                f"{self.layer_name}: vllm-expert-pager does not support expert parallelism "
                f"(local={self.local_num_experts}, global={self.global_num_experts})"
            )
        if self.moe_config.moe_parallel_config.tp_size != 1:
            raise RuntimeError(f"{self.layer_name}: vllm-expert-pager does not support tensor parallelism")
        unsupported = _unsupported_modes(self)
        if unsupported:
            raise RuntimeError(
                f"{self.layer_name}: vllm-expert-pager runs its own fp8 expert kernels, which do not "
                f"support {'; '.join(unsupported)}"
            )
        E = self.global_num_experts
        params = {name: getattr(self, name) for name in PARAMS}

        global _pager
        if _pager is None:
            _pager = Pager(
                SETTINGS,
                num_layers=get_current_vllm_config().model_config.hf_text_config.num_hidden_layers,
                num_experts=E,
                hidden=self.hidden_size,
                intermediate=self.intermediate_size_per_partition,
                device=params["w13_weight"].device,
            )
        self._expert_pager: PagedExperts = _pager.add_layer(_activation(self))

        # Compression assumes raw fp8 rows; Marlin repacks them.
        if _pager.store.compress and getattr(self.quant_method, "fp8_backend", None) == Fp8MoeBackend.MARLIN:
            raise RuntimeError(
                f"{self.layer_name}: vllm-expert-pager compresses raw fp8 rows and does not support the "
                "MARLIN backend; set VLLM_EXPERT_PAGER_COMPRESS=off"
            )
        # Free the (E, ...) weights and keep their shape: one row shown E
        # times through a stride-0 expand until setup shrinks it.
        for p in params.values():
            p.data = torch.empty((1, *p.shape[1:]), dtype=p.dtype, device=p.device).expand(p.shape)
        # w13 arrives as separate gate (w1) and up (w3) shards.
        self._expert_pager_stage: dict[int, tuple[torch.Tensor, set[str]]] = {}

        original = self.quant_method.process_weights_after_loading

        def process_weights_after_loading(layer: RoutedExperts) -> None:
            original(layer)
            layer._expert_pager_setup()

        self.quant_method.process_weights_after_loading = process_weights_after_loading

    @property
    def expert_map(self) -> torch.Tensor | None:
        if self._expert_pager_expert_map is not None:
            return self._expert_pager_expert_map
        return super().expert_map

    # ---- loading ----

    def weight_loader(
        self,
        param: torch.nn.Parameter,
        loaded_weight: torch.Tensor,
        weight_name: str,
        shard_id: str,
        expert_id: int,
        return_success: bool = False,
    ) -> bool | None:
        if param is self.w13_weight:
            N, H = self.intermediate_size_per_partition, self.hidden_size
            buf, seen = self._expert_pager_stage.setdefault(
                expert_id, (torch.empty((2 * N, H), dtype=loaded_weight.dtype, device="cpu"), set())
            )
            half = 0 if shard_id == "w1" else N
            buf[half : half + N].copy_(loaded_weight)
            seen.add(shard_id)
            if seen != {"w1", "w3"}:
                return True if return_success else None
            del self._expert_pager_stage[expert_id]
            self._expert_pager.load_expert(expert_id, "w13_weight", buf)
        elif param is self.w2_weight:
            self._expert_pager.load_expert(expert_id, "w2_weight", loaded_weight)
        else:
            return super().weight_loader(param, loaded_weight, weight_name, shard_id, expert_id, return_success)
        return True if return_success else None

    def _expert_pager_setup(self) -> None:
        store = self._expert_pager.store
        for name in PARAMS:
            p = getattr(self, name)
            p.data = p.data[:1].clone()
            if p.data.numel() * p.element_size() != store.row_bytes[name]:
                raise RuntimeError(
                    f"{self.layer_name}: {name} row has {p.data.numel() * p.element_size()} B after "
                    f"process_weights_after_loading, expected {store.row_bytes[name]}"
                )
        scale_name = getattr(self.quant_method, "weight_scale_name", None)
        if scale_name is None:
            raise RuntimeError(
                f"{self.layer_name}: {type(self.quant_method).__name__} has no weight_scale_name; "
                "vllm-expert-pager only knows how to stage block-fp8 scales"
            )
        scales = [getattr(self, f"{w}_{scale_name}").data for w in ("w13", "w2")]
        for s in scales:
            if s.dtype != torch.float32:
                raise RuntimeError(f"{self.layer_name}: expert scales must be float32, got {s.dtype}")
        try:
            self._expert_pager.setup({SCALES[0]: scales[0], SCALES[1]: scales[1]})
        except ValueError as e:
            raise RuntimeError(
                f"{self.layer_name}: vllm-expert-pager needs 128x128 block-quantised fp8 experts ({e})"
            ) from e

    # ---- forward ----

    def forward_modular(
        self,
        x: torch.Tensor,
        topk_weights: torch.Tensor,
        topk_ids: torch.Tensor,
        shared_experts=None,
        shared_experts_input: torch.Tensor | None = None,
    ) -> torch.Tensor:
        # The reference hands shared experts to vLLM's modular kernel with the
        # first expert run of the forward (experts.py:452, 569-573); that run
        # returns the routed output alone and the shared output stays inside
        # the shared experts object (experts.py:475-477). The pager calls this
        # once, right before its first expert launch.
        shared = None
        if shared_experts is not None:
            shared_input = x if shared_experts_input is None else shared_experts_input

            def shared() -> None:
                shared_experts(shared_input)

        if _router_weight_on_input(self):
            # vLLM's prepare step for this mode scales the tokens by their
            # routed weight (rounded to the token dtype) and the experts then
            # add their outputs unweighted; it allows top-k 1 only.
            if topk_ids.shape[1] != 1:
                raise RuntimeError(
                    f"{self.layer_name}: apply_router_weight_on_input needs top-k 1, got {topk_ids.shape[1]}"
                )
            x = x * topk_weights.to(x.dtype)
            topk_weights = torch.ones_like(topk_weights, dtype=torch.float32)
        pager = self._expert_pager
        self._expert_pager_expert_map = pager.expert_map
        try:
            return pager.forward(x, topk_weights, topk_ids, shared)
        finally:
            self._expert_pager_expert_map = None

    def forward_monolithic(self, *args, **kwargs) -> torch.Tensor:
        raise RuntimeError(
            f"{self.layer_name}: vllm-expert-pager only supports modular MoE kernels, but "
            f"{type(self.quant_method).__name__} is monolithic. Expert weights would not be staged."
        )


def register() -> None:
    RoutedExperts.register_oot(ExpertPagerRoutedExperts)
