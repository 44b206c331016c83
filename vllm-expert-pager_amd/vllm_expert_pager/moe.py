"""fp8 expert FFN on the slab and the single top-k combine (csrc/moe.hip).

Stands where the reference calls vLLM's fused fp8 MoE with ``expert_map``
pointing into a slab (``_expert_pager_run``, experts.py:579-604) and where it
intercepts ``moe_sum`` to take the top-k sum once over all chunks
(experts.py:538-556). Weights are w8a8 block-fp8: e4m3 rows with one fp32
scale per 128x128 block, activations quantised per token and 128 columns.

The work of one MoE call is split in four launches so that the overflow path
can quantise once, run the experts chunk by chunk, and combine once:

    xq, xs = quant_tokens(x)
    r = route(topk_ids, expert_map, slots)          # per chunk
    run_experts(xq, xs, topk_weights, slab, r, contrib)   # per chunk
    out = topk_sum(contrib, topk_ids, num_experts)  # once

Each (token, k) pair's contribution depends only on its token and expert,
so the chunked sequence writes the same bits as ``fused_moe`` over all
experts at once.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from vllm_expert_pager import _native as nat

BLOCK = 128  # quantisation group and weight scale block
MAX_SLOTS = 1024  # slots one route call can address

_FP8 = tuple(t for t in (getattr(torch, "float8_e4m3fn", None), torch.uint8) if t is not None)

# Expert activations the kernels compute (act(gate) * up), by vLLM's names.
ACTIVATIONS = {"silu": 0, "gelu": 1}


def activation_code(activation: str) -> int:
    """The kernels' code of an activation name; ValueError for others."""
    code = ACTIVATIONS.get(activation)
    if code is None:
        raise ValueError(f"activation {activation!r}: the expert kernels compute {sorted(ACTIVATIONS)}")
    return code


def _fp8_ptr(t: torch.Tensor, what: str) -> int:
    nat.require_device(t, what)
    if t.dtype not in _FP8 or t.element_size() != 1:
        raise ValueError(f"{what} must be float8_e4m3fn or uint8, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return t.data_ptr()


def _f32(t: torch.Tensor, what: str) -> torch.Tensor:
    nat.require_device(t, what)
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous float32 tensor")
    return t


def quant_tokens(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 ``(T, H)`` -> fp8 ``(T, H)`` as uint8 and fp32 scales ``(T, H/128)``."""
    nat.require_device(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError(f"x must be a 2-D bfloat16 tensor, got {x.dtype} {tuple(x.shape)}")
    x = x.contiguous()
    T, H = x.shape
    xq = torch.empty((T, H), dtype=torch.uint8, device=x.device)
    xs = torch.empty((T, H // BLOCK if H % BLOCK == 0 else 0), dtype=torch.float32, device=x.device)
    nat.call("xp_quant_tokens", x.data_ptr(), T, H, xq.data_ptr(), xs.data_ptr(), nat.stream())
    return xq, xs


@dataclass
class Routing:
    """CSR pair lists per slab slot and the tile list of one route call."""

    slots: int
    offsets: torch.Tensor  # int32 (slots + 1,)
    pairs: torch.Tensor  # int32 (T * topk,)
    tiles: torch.Tensor  # int32 (1 + 2 * bound,)

    @property
    def count(self) -> torch.Tensor:
        """Pairs routed to each slot (device tensor)."""
        return self.offsets[1:] - self.offsets[:-1]


def _shape(topk_ids: torch.Tensor) -> tuple[int, int]:
    """(tokens, top-k) of a routing tensor; a 1-D tensor is one id per token."""
    if topk_ids.dim() == 2:
        return topk_ids.shape[0], topk_ids.shape[1]
    return topk_ids.numel(), 1


def _routing(topk_ids: torch.Tensor, expert_map: torch.Tensor, slots: int, out: Routing | None) -> Routing:
    nat.require_device(expert_map, "expert_map")
    if expert_map.dtype != torch.int32 or not expert_map.is_contiguous():
        raise ValueError("expert_map must be a contiguous int32 tensor")
    if not 1 <= slots <= MAX_SLOTS:
        raise ValueError(f"slots must be in [1, {MAX_SLOTS}], got {slots}")
    T, topk = _shape(topk_ids)
    n = T * topk
    bound = int(nat.lib().xp_moe_max_tiles(n, slots))
    if out is None or out.slots != slots or out.pairs.numel() < n or out.tiles.numel() < 1 + 2 * bound:
        dev = expert_map.device
        out = Routing(
            slots,
            torch.empty((slots + 1,), dtype=torch.int32, device=dev),
            torch.empty((max(n, 1),), dtype=torch.int32, device=dev),
            torch.empty((1 + 2 * max(bound, 1),), dtype=torch.int32, device=dev),
        )
    return out


def route(topk_ids: torch.Tensor, expert_map: torch.Tensor, slots: int, out: Routing | None = None) -> Routing:
    """List the pairs whose expert ``expert_map`` places in a slot ``< slots``."""
    ids, eb = nat.ids_arg(topk_ids)
    out = _routing(topk_ids, expert_map, slots, out)
    T, topk = _shape(topk_ids)
    nat.call(
        "xp_moe_route", nat.ptr(ids), eb, T, topk, expert_map.data_ptr(), expert_map.numel(), slots,
        out.offsets.data_ptr(), out.pairs.data_ptr(), out.tiles.data_ptr(), nat.stream(),
    )
    return out


def quant_route(x: torch.Tensor, topk_ids: torch.Tensor, expert_map: torch.Tensor,
                slots: int) -> tuple[torch.Tensor, torch.Tensor, Routing]:
    """``quant_tokens(x)`` and ``route(topk_ids, expert_map, slots)`` in one launch."""
    nat.require_device(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError(f"x must be a 2-D bfloat16 tensor, got {x.dtype} {tuple(x.shape)}")
    x = x.contiguous()
    T, H = x.shape
    if _shape(topk_ids)[0] != T:
        raise ValueError(f"topk_ids has {_shape(topk_ids)[0]} tokens, x has {T}")
    ids, eb = nat.ids_arg(topk_ids)
    topk = _shape(topk_ids)[1]
    r = _routing(topk_ids, expert_map, slots, None)
    xq = torch.empty((T, H), dtype=torch.uint8, device=x.device)
    xs = torch.empty((T, H // BLOCK if H % BLOCK == 0 else 0), dtype=torch.float32, device=x.device)
    nat.call(
        "xp_moe_quant_route", x.data_ptr(), T, H, xq.data_ptr(), xs.data_ptr(), nat.ptr(ids), eb, topk,
        expert_map.data_ptr(), expert_map.numel(), slots, r.offsets.data_ptr(), r.pairs.data_ptr(),
        r.tiles.data_ptr(), nat.stream(),
    )
    return xq, xs, r


def run_experts(
    xq: torch.Tensor,
    xs: torch.Tensor,
    topk_weights: torch.Tensor,
    w13: torch.Tensor,
    w13_scale: torch.Tensor,
    w2: torch.Tensor,
    w2_scale: torch.Tensor,
    routing: Routing,
    contrib: torch.Tensor,
    activation: str = "silu",
) -> None:
    """Write ``contrib[t*topk + k]`` (bf16, ``(T*topk, H)``) for every routed pair.

    ``w13`` is the slab ``(S, 2I, H)`` (gate rows then up rows), ``w2``
    ``(S, H, I)``, scales ``(S, 2I/128, H/128)`` and ``(S, H/128, I/128)``
    fp32. Rows of pairs that were not routed are left as they are.
    ``activation`` ("silu" or "gelu") is applied to the gate before the
    product with up.
    """
    act = activation_code(activation)
    T, H = xq.shape
    if topk_weights.dim() != 2 or topk_weights.shape[0] != T:
        raise ValueError("topk_weights must be (T, topk)")
    topk = topk_weights.shape[1]
    tw = topk_weights if topk_weights.dtype == torch.float32 else topk_weights.float()
    tw = _f32(tw.contiguous(), "topk_weights")
    S = w13.shape[0]
    if w13.dim() != 3 or w13.shape[2] != H or w13.shape[1] % 2:
        raise ValueError(f"w13 must be (slots, 2I, {H}), got {tuple(w13.shape)}")
    I = w13.shape[1] // 2
    if tuple(w2.shape) != (S, H, I):
        raise ValueError(f"w2 must be {(S, H, I)}, got {tuple(w2.shape)}")
    if H % BLOCK or I % BLOCK:
        raise ValueError(f"H={H} and I={I} must be multiples of {BLOCK}")
    if tuple(w13_scale.shape) != (S, 2 * I // BLOCK, H // BLOCK):
        raise ValueError(f"w13 scale must be {(S, 2 * I // BLOCK, H // BLOCK)}, got {tuple(w13_scale.shape)}")
    if tuple(w2_scale.shape) != (S, H // BLOCK, I // BLOCK):
        raise ValueError(f"w2 scale must be {(S, H // BLOCK, I // BLOCK)}, got {tuple(w2_scale.shape)}")
    if routing.slots > S:
        raise ValueError(f"routing addresses {routing.slots} slots, the slab has {S}")
    if contrib.dtype != torch.bfloat16 or tuple(contrib.shape) != (T * topk, H) or not contrib.is_contiguous():
        raise ValueError(f"contrib must be contiguous bfloat16 {(T * topk, H)}")
    nbytes = int(nat.lib().xp_moe_workspace_bytes(T * topk, I))
    work = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=xq.device)
    nat.call(
        "xp_moe_experts", _fp8_ptr(xq, "xq"), _f32(xs, "xs").data_ptr(), T, topk, tw.data_ptr(), H, I,
        _fp8_ptr(w13, "w13"), _f32(w13_scale, "w13_scale").data_ptr(), _fp8_ptr(w2, "w2"),
        _f32(w2_scale, "w2_scale").data_ptr(), routing.slots, routing.offsets.data_ptr(),
        routing.pairs.data_ptr(), routing.tiles.data_ptr(), work.data_ptr(), nbytes, contrib.data_ptr(), act,
        nat.stream(),
    )


def topk_sum(contrib: torch.Tensor, topk_ids: torch.Tensor, num_experts: int,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """``out[t] = bf16(sum_k fp32(contrib[t*topk + k]))`` over pairs with a valid expert id."""
    ids, eb = nat.ids_arg(topk_ids)
    T, topk = _shape(topk_ids)
    nat.require_device(contrib, "contrib")
    if contrib.dtype != torch.bfloat16 or contrib.dim() != 2 or contrib.shape[0] != T * topk:
        raise ValueError(f"contrib must be bfloat16 ({T * topk}, H)")
    H = contrib.shape[1]
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=contrib.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (T, H) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous bfloat16 {(T, H)}")
    nat.call("xp_moe_topk_sum", contrib.contiguous().data_ptr(), T, topk, H, nat.ptr(ids), eb, num_experts,
             out.data_ptr(), nat.stream())
    return out


DECODE_PAIRS = 64  # a fused decode call's limits: pairs (T * topk), H, topk * I
DECODE_MAX_H = 4096
DECODE_ACT_BYTES = 32768
# Above this many pairs the separate calls are faster than the fused step:
# the down projection of the fused step reads each pair's w2 rows once per
# token, while run_experts reads an expert's rows once for all its tokens.
# Measured with 2048 x 512 experts at top-8: 4 tokens 38 us fused against
# 46 us separate, 5 tokens 48 against 50, 6 tokens 58 against 52, 8 tokens
# 81 against 47.
DECODE_STEP_PAIRS = 40


def decode_fits(x: torch.Tensor, topk_ids: torch.Tensor, intermediate: int) -> bool:
    """Whether ``decode_experts`` accepts this step."""
    T, topk = _shape(topk_ids)
    return (0 < T * topk <= DECODE_PAIRS and x.dim() == 2 and x.shape[1] <= DECODE_MAX_H
            and topk * intermediate <= DECODE_ACT_BYTES)


def decode_pays(x: torch.Tensor, topk_ids: torch.Tensor, intermediate: int) -> bool:
    """Whether a decode step takes ``decode_experts`` (else the separate calls)."""
    T, topk = _shape(topk_ids)
    return T * topk <= DECODE_STEP_PAIRS and decode_fits(x, topk_ids, intermediate)


def decode_experts(
    x: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    expert_map: torch.Tensor,
    num_experts: int,
    w13: torch.Tensor,
    w13_scale: torch.Tensor,
    w2: torch.Tensor,
    w2_scale: torch.Tensor,
    slots: int,
    pair_slot: torch.Tensor | None = None,
    activation: str = "silu",
) -> torch.Tensor:
    """``quant_route`` + ``run_experts`` + ``topk_sum`` of a decode step in two launches, same bits.

    Every pair with a valid expert id should have a slot below ``slots``
    (one without adds nothing, where the separate calls would read a
    contribution never written). ``pair_slot`` (int32, at least T * topk
    entries), when given, holds each pair's slot as ``AcquirePair`` writes
    it, and the routing reads it instead of ``expert_map[topk_ids]``.
    """
    act = activation_code(activation)
    nat.require_device(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError(f"x must be a 2-D bfloat16 tensor, got {x.dtype} {tuple(x.shape)}")
    x = x.contiguous()
    T, H = x.shape
    Tk, topk = _shape(topk_ids)
    if Tk != T or tuple(topk_weights.shape) != (T, topk):
        raise ValueError(f"topk_ids {tuple(topk_ids.shape)} and topk_weights {tuple(topk_weights.shape)} "
                         f"must both be ({T}, topk)")
    nat.require_device(expert_map, "expert_map")
    if expert_map.dtype != torch.int32 or not expert_map.is_contiguous():
        raise ValueError("expert_map must be a contiguous int32 tensor")
    ids, eb = nat.ids_arg(topk_ids)
    if pair_slot is not None:
        nat.require_device(pair_slot, "pair_slot")
        if pair_slot.dtype != torch.int32 or not pair_slot.is_contiguous() or pair_slot.numel() < T * topk:
            raise ValueError(f"pair_slot must be a contiguous int32 tensor of at least {T * topk} entries")
    tw = topk_weights if topk_weights.dtype == torch.float32 else topk_weights.float()
    tw = _f32(tw.contiguous(), "topk_weights")
    S = w13.shape[0]
    I = w13.shape[1] // 2
    nbytes = int(nat.lib().xp_moe_workspace_bytes(T * topk, I))
    work = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=x.device)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=x.device)
    nat.call(
        "xp_moe_decode_experts", x.data_ptr(), T, H, nat.ptr(ids), eb, topk, tw.data_ptr(), expert_map.data_ptr(),
        nat.ptr(pair_slot), num_experts, I, _fp8_ptr(w13, "w13"), _f32(w13_scale, "w13_scale").data_ptr(),
        _fp8_ptr(w2, "w2"), _f32(w2_scale, "w2_scale").data_ptr(), min(slots, S), work.data_ptr(), nbytes,
        out.data_ptr(), act, nat.stream(),
    )
    return out


def fused_moe(
    x: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    w13: torch.Tensor,
    w13_scale: torch.Tensor,
    w2: torch.Tensor,
    w2_scale: torch.Tensor,
    expert_map: torch.Tensor | None = None,
    num_experts: int | None = None,
    activation: str = "silu",
) -> torch.Tensor:
    """One-shot MoE over a slab: quantise, route, experts, combine.

    Without ``expert_map`` the slab holds every expert (slot e = expert e).
    Pairs whose expert has no slot contribute nothing.
    """
    S = w13.shape[0]
    E = num_experts if num_experts is not None else (expert_map.numel() if expert_map is not None else S)
    if expert_map is None:
        expert_map = torch.arange(E, dtype=torch.int32, device=x.device)
    xq, xs = quant_tokens(x)
    r = route(topk_ids, expert_map, min(S, MAX_SLOTS))
    T, topk = topk_weights.shape
    contrib = torch.zeros((T * topk, x.shape[1]), dtype=torch.bfloat16, device=x.device)
    run_experts(xq, xs, topk_weights, w13, w13_scale, w2, w2_scale, r, contrib, activation)
    return topk_sum(contrib, topk_ids, E)
