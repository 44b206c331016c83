"""Oracle of the w8a8 block-fp8 expert FFN and the single top-k combine -- test infrastructure only.

The reference runs vLLM's fused fp8 MoE on the slab (experts.py:579-604)
and takes the top-k sum once over all chunks (experts.py:538-556); vLLM
itself is not part of the reference tree, so this module restates the
published w8a8 block-fp8 MoE of vLLM 0.29.0 (per-token-group activation
quantisation, 128x128 weight scale blocks, SiLU-and-mul, routed-weight
multiply, moe_sum) in numpy/torch on the CPU:

  quant_groups  x -> fp8 per 128 columns: s = max(amax, 1e-10) / 448 (fp32),
                q = rne(clamp(x / s, -448, 448))
  expert_ffn    per (token, k) pair: h = dequant(xq) . dequant(w13)^T,
                gate/up -> bf16, a = bf16(bf16(silu(gate)) * up) (vLLM's
                silu_and_mul returns silu in the activation dtype and then
                multiplies two bf16 values), a -> fp8 per 128 columns,
                y = dequant(aq) . dequant(w2)^T,
                contribution = bf16(y * routed weight)
  topk_sum      bf16(fp32 sum over k ascending of the contributions)

Dot products are taken in float64 over the exactly dequantised values (an
fp8 value times an fp32 scale is exact in float64), so the oracle is the
w8a8 result up to float64 rounding before each bf16/fp8 rounding step; a
GPU kernel that accumulates in fp32 agrees with it to a few bf16 ulps.

Pinning (tests/test_oracle_moe.py): fp8_values against torch's
float8_e4m3fn for all 256 codes; to_fp8 on round-to-nearest-even ties,
subnormals and the clamp; quant_groups on its closed form (the group
maximum maps to +-448); expert_ffn on the one-hot closed form (x = c*e_i
selects column i of w13, a permutation w2 selects activation entries),
which fixes operand orientation and indexing; invariance under relabelling
experts, exact scaling by powers of two of the routed weights, and
independence of tokens; topk_sum against exact integer sums.
"""

from __future__ import annotations

import numpy as np
import torch

BLOCK = 128
FP8_MAX = 448.0
EPS = 1e-10


def fp8_values() -> np.ndarray:
    """float64 value of each e4m3fn code (OCP: bias 7, no infinities, 0x7f/0xff NaN)."""
    out = np.empty(256, np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        e, m = (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            out[code] = np.nan
        elif e == 0:
            out[code] = sign * m * 2.0**-9
        else:
            out[code] = sign * (1 + m / 8) * 2.0 ** (e - 7)
    return out


_FP8 = fp8_values()


def to_fp8(v: np.ndarray) -> np.ndarray:
    """Round float32 values in [-448, 448] to e4m3fn codes, nearest even."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def bf16(v: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest even), returned as float32."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return torch.from_numpy(v).to(torch.bfloat16).float().numpy()


def bf16_bits(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def quant_groups(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float32 (T, H) -> fp8 codes (T, H) and float32 scales (T, H/128)."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    g = x.reshape(T, H // BLOCK, BLOCK)
    amax = np.abs(g).max(axis=2)
    s = (np.maximum(amax, np.float32(EPS)) / np.float32(FP8_MAX)).astype(np.float32)
    q = np.clip(g / s[:, :, None], np.float32(-FP8_MAX), np.float32(FP8_MAX)).astype(np.float32)
    return to_fp8(q).reshape(T, H), s


def dequant_rows(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """(T, H) codes with (T, H/128) scales -> float64."""
    return _FP8[q] * np.repeat(s.astype(np.float64), BLOCK, axis=1)


def dequant_weight(w: np.ndarray, ws: np.ndarray) -> np.ndarray:
    """(N, K) codes with (N/128, K/128) block scales -> float64."""
    return _FP8[w] * np.kron(ws.astype(np.float64), np.ones((BLOCK, BLOCK)))


# Planted mistakes for tests that show a set of inputs tells the rounding
# sequence apart (expert_ffn's `variant`); each changes exactly one step.
VARIANTS = (
    "gate_up_unrounded",   # gate and up kept in fp32 instead of rounded to bf16
    "gate_up_truncated",   # gate and up rounded to bf16 toward zero
    "silu_unrounded",      # silu(gate) kept in fp32 before the product with up
    "act_unrounded",       # silu(gate) * up not rounded to bf16 before quantisation
    "quant_reciprocal",    # activation scale applied as a * (448 / amax) instead of a / (amax / 448)
    "fp8_truncated",       # activations converted to fp8 toward zero
    "weight_after_round",  # routed weight applied to bf16(y) rather than to y
)


def _bf16_toward_zero(v: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(v, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)
    return b.view(np.float32)


def _fp8_toward_zero(v: np.ndarray) -> np.ndarray:
    """fp8 codes of float32 values in [-448, 448], rounded toward zero."""
    v = np.asarray(v, np.float32)
    pos = np.sort(_FP8[:127])  # codes 0x00..0x7e: every finite non-negative value
    mag = np.abs(v).astype(np.float64)
    idx = np.searchsorted(pos, mag, side="right") - 1
    code = np.argsort(_FP8[:127])[idx].astype(np.uint8)
    return np.where(np.signbit(v) & (code != 0), code | 0x80, code).astype(np.uint8)


def _quant_variant(x: np.ndarray, variant: str | None) -> tuple[np.ndarray, np.ndarray]:
    if variant not in ("quant_reciprocal", "fp8_truncated"):
        return quant_groups(x)
    x = np.asarray(x, np.float32)
    T, H = x.shape
    g = x.reshape(T, H // BLOCK, BLOCK)
    amax = np.abs(g).max(axis=2)
    s = (np.maximum(amax, np.float32(EPS)) / np.float32(FP8_MAX)).astype(np.float32)
    if variant == "quant_reciprocal":
        inv = (np.float32(FP8_MAX) / np.maximum(amax, np.float32(EPS))).astype(np.float32)
        q = np.clip(g * inv[:, :, None], -FP8_MAX, FP8_MAX).astype(np.float32)
        return to_fp8(q).reshape(T, H), s
    q = np.clip(g / s[:, :, None], np.float32(-FP8_MAX), np.float32(FP8_MAX)).astype(np.float32)
    return _fp8_toward_zero(q).reshape(T, H), s


def expert_ffn(x: np.ndarray, topk_weights: np.ndarray, topk_ids: np.ndarray, w13: np.ndarray, w13_scale: np.ndarray,
               w2: np.ndarray, w2_scale: np.ndarray, variant: str | None = None) -> np.ndarray:
    """bf16 contributions (T*topk, H) as float32; pairs with an id outside [0, E) are 0.

    x: (T, H) float32 holding bf16 values; w13: (E, 2I, H) fp8 codes (gate
    rows then up rows), w2: (E, H, I); scales (E, 2I/128, H/128) and
    (E, H/128, I/128) float32. `variant` (one of VARIANTS) plants one
    mistake in the rounding sequence, for tests of test inputs only.
    """
    if variant is not None and variant not in VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    x = np.asarray(x, np.float32)
    T, H = x.shape
    ids = np.asarray(topk_ids).reshape(T, -1)
    topk = ids.shape[1]
    tw = np.asarray(topk_weights, np.float32).reshape(T, topk)
    E, I2, _ = w13.shape
    I = I2 // 2
    xq, xs = quant_groups(x)
    xd = dequant_rows(xq, xs)
    out = np.zeros((T * topk, H), np.float32)
    flat = ids.reshape(-1)
    for e in np.unique(flat):
        if e < 0 or e >= E:
            continue
        pairs = np.nonzero(flat == e)[0]
        tok = pairs // topk
        h = (xd[tok] @ dequant_weight(w13[e], w13_scale[e]).T).astype(np.float32)
        if variant == "gate_up_unrounded":
            gate, up = h[:, :I], h[:, I:]
        elif variant == "gate_up_truncated":
            gate, up = _bf16_toward_zero(h[:, :I]), _bf16_toward_zero(h[:, I:])
        else:
            gate, up = bf16(h[:, :I]), bf16(h[:, I:])
        with np.errstate(over="ignore"):
            silu = (gate / (np.float32(1) + np.exp(-gate))).astype(np.float32)
        if variant != "silu_unrounded":
            silu = bf16(silu)
        a = (silu * up).astype(np.float32) if variant == "act_unrounded" else bf16(silu * up)
        aq, as_ = _quant_variant(a, variant)
        y = (dequant_rows(aq, as_) @ dequant_weight(w2[e], w2_scale[e]).T).astype(np.float32)
        w = tw.reshape(-1)[pairs][:, None]
        out[pairs] = bf16(bf16(y) * w) if variant == "weight_after_round" else bf16(y * w)
    return out


def bf16_midpoint_margin(v: np.ndarray) -> np.ndarray:
    """Relative distance of each non-zero float64 value to the nearest point
    halfway between two neighbouring bf16 values (where rounding to bf16
    changes direction)."""
    m, _ = np.frexp(np.abs(np.asarray(v, np.float64)))  # |v| = m * 2^e, m in [0.5, 1)
    k = m * 256.0  # |v| in units of the bf16 spacing at its binade: 8 significant bits
    return np.abs(k - np.floor(k) - 0.5) / k


# Probe gates of exact_inputs are v * c / 4: v the token's column-0 value
# (m * 2^a, m in 1..3), c the weight code (+-1..4). The (m, a) pairs for which
# silu of every such gate is at least PROBE_MARGIN (relative) away from a bf16
# rounding midpoint, so that bf16(silu(g)) does not depend on how an fp32 exp
# and division round (a few fp32 ulps, about 2^-21).
PROBE_MARGIN = 2.0**-14


def _safe_probe_values() -> list[tuple[int, int]]:
    safe = []
    for a in range(-3, 4):
        for m in (1, 2, 3):
            g = np.array([s * m * 2.0**a * c / 4 for s in (1, -1) for c in (1, 2, 3, 4, -1, -2, -3, -4)])
            silu = g / (1 + np.exp(-g))
            if bf16_midpoint_margin(silu).min() >= PROBE_MARGIN:
                safe.append((m, a))
    return safe


def exact_inputs(rng: np.random.Generator, E: int, H: int, I: int, T: int, topk: int):
    """A MoE case on which every sum is exact in fp32 and every SiLU is exact
    or rounds to bf16 unambiguously, while every rounding step of the
    sequence still rounds: the rounding sequence, not summation order,
    decides the output bits.

    - x: per token one or two active 128-column groups, group 0 always
      among them; each has one value of +-448 * 2^a (so the group scale is
      exactly 2^a) and a few of +-1..3 * 2^a; the other groups are zero.
      Column 0 holds +-m * 2^a with (m, a) drawn from _safe_probe_values.
    - w13 gate rows 0-127 (the first activation group) have codes in
      {0, +-1, +-2} over every column and block scale 2^10, so each block
      dot is an integer below 2^11 and every such gate is 0 or at least 104
      in magnitude: silu(g) is g or -0 whatever exp's last bit.
    - w13 gate rows 128-255 (the second activation group, when I >= 256)
      are probes: one code c in {+-1..4} at column 0, block scale 2^-2, so
      the gate is v * c / 4, between 2^-5 and 24 in magnitude, where silu
      is a general value; its bf16 rounding is unambiguous (PROBE_MARGIN),
      and bf16(silu(g)) * up rounds differently from silu(g) * up.
    - Up rows: codes in {0, +-1, +-2, +-3}, scale 2^-4.
    - gate and up then carry up to 11 significant bits (bf16 keeps 8), and
      a = bf16(bf16(silu(gate)) * up) up to 16: the roundings round, ties
      included.
    - w2 rows: one non-zero code in {+-1..+-4} per row, scale 2^-2, in the
      first activation group for even rows and in the second (the probes)
      for odd rows when I >= 256: each dot is a single exact product, the
      activation scale amax/448 is a general float and a / scale a general
      quotient, so the requantisation's division and fp8 rounding are
      exercised.
    - routed weights: softmax over random logits.
    Returns (x float32 holding bf16 values, topk_weights, topk_ids, w13,
    w13_scale, w2, w2_scale) for fused_moe_ref.
    """
    G, GI = H // BLOCK, I // BLOCK
    code = {v: int(to_fp8(np.array([v], np.float32))[0]) for v in (0, 1, 2, 3, 4, -1, -2, -3, -4)}
    probes = GI >= 2

    def codes(values, p, shape):
        pick = rng.choice(len(values), size=shape, p=p)
        return np.vectorize(lambda i: code[values[i]])(pick).astype(np.uint8)

    w13 = np.zeros((E, 2 * I, H), np.uint8)
    w13[:, :BLOCK] = codes([0, 1, -1, 2, -2], [0.8, 0.06, 0.06, 0.04, 0.04], (E, BLOCK, H))
    w13[:, I:] = codes([0, 1, -1, 2, -2, 3, -3], [0.7, 0.08, 0.08, 0.05, 0.05, 0.02, 0.02], (E, I, H))
    w13s = np.ones((E, 2 * GI, G), np.float32)
    w13s[:, 0] = 2.0**10
    w13s[:, GI:] = 2.0**-4
    if probes:
        w13[:, BLOCK : 2 * BLOCK, 0] = codes([1, -1, 2, -2, 3, -3, 4, -4], [0.125] * 8, (E, BLOCK))
        w13s[:, 1, 0] = 2.0**-2
    w2 = np.zeros((E, H, I), np.uint8)
    cols = rng.integers(0, BLOCK, (E, H))
    if probes:
        cols[:, 1::2] += BLOCK
    vals = codes([1, -1, 2, -2, 3, -3, 4, -4], [0.125] * 8, (E, H))
    np.put_along_axis(w2, cols[:, :, None], vals[:, :, None], axis=2)
    w2s = np.full((E, H // BLOCK, GI), 2.0**-2, np.float32)

    safe = _safe_probe_values()
    x = np.zeros((T, H), np.float32)
    for t in range(T):
        extra = rng.choice(np.arange(1, G), size=int(rng.integers(0, 2)), replace=False) if G > 1 else []
        for g in [0, *extra]:
            if g == 0:
                m, a = safe[int(rng.integers(len(safe)))]
                cols_t = rng.choice(np.arange(1, BLOCK), size=3, replace=False)
                x[t, 0] = rng.choice([-1.0, 1.0]) * m * 2.0**a
                x[t, cols_t[0]] = rng.choice([-448.0, 448.0]) * 2.0**a
                x[t, cols_t[1:]] = rng.choice([-3.0, -2.0, -1.0, 1.0, 2.0, 3.0], size=2) * 2.0**a
                continue
            a = int(rng.integers(-3, 4))
            cols_t = rng.choice(BLOCK, size=4, replace=False) + g * BLOCK
            x[t, cols_t[0]] = rng.choice([-448.0, 448.0]) * 2.0**a
            x[t, cols_t[1:]] = rng.choice([-3.0, -2.0, -1.0, 1.0, 2.0, 3.0], size=3) * 2.0**a
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int64)
    logits = rng.standard_normal((T, topk)).astype(np.float32)
    tw = (np.exp(logits) / np.exp(logits).sum(1, keepdims=True)).astype(np.float32)
    return x, tw, ids, w13, w13s, w2, w2s


def topk_sum(contrib: np.ndarray, topk_ids: np.ndarray, num_experts: int) -> np.ndarray:
    """bf16(fp32 sum over k ascending) per token, skipping ids outside [0, E); float32 out."""
    ids = np.asarray(topk_ids)
    T = ids.shape[0]
    ids = ids.reshape(T, -1)
    topk = ids.shape[1]
    c = np.asarray(contrib, np.float32).reshape(T, topk, -1)
    acc = np.zeros((T, c.shape[2]), np.float32)
    for k in range(topk):
        ok = (ids[:, k] >= 0) & (ids[:, k] < num_experts)
        acc = np.where(ok[:, None], acc + c[:, k], acc).astype(np.float32)
    return bf16(acc)


def fused_moe_ref(x, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale, variant=None) -> np.ndarray:
    """The layer output (T, H) as float32 holding bf16 values."""
    contrib = expert_ffn(x, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale, variant)
    return topk_sum(contrib, topk_ids, w13.shape[0])


def random_experts(rng: np.random.Generator, E: int, H: int, I: int, std: float = 0.02):
    """Weights ~ N(0, std) quantised to e4m3 with one amax/448 scale per 128x128 block."""
    def one(n, k):
        w = rng.standard_normal((E, n, k)).astype(np.float32) * np.float32(std)
        b = w.reshape(E, n // BLOCK, BLOCK, k // BLOCK, BLOCK)
        s = (np.abs(b).max(axis=(2, 4)) / np.float32(FP8_MAX)).astype(np.float32)
        s = np.maximum(s, np.float32(EPS))
        q = np.clip(b / s[:, :, None, :, None], -FP8_MAX, FP8_MAX).astype(np.float32)
        return to_fp8(q).reshape(E, n, k), s
    w13, w13s = one(2 * I, H)
    w2, w2s = one(H, I)
    return w13, w13s, w2, w2s
