"""Oracle of the w8a8 block-fp8 expert FFN and the single top-k combine -- test infrastructure only.

The reference runs vLLM's fused fp8 MoE on the slab (experts.py:579-604)
and takes the top-k sum once over all chunks (experts.py:538-556); vLLM
itself is not part of the reference tree, so this module restates the
published w8a8 block-fp8 MoE of vLLM 0.29.0 (per-token-group activation
quantisation, 128x128 weight scale blocks, SiLU-and-mul or GELU-and-mul,
routed-weight multiply, moe_sum) in numpy/torch on the CPU:

  quant_groups  x -> fp8 per 128 columns: s = max(amax, 1e-10) / 448 (fp32),
                q = rne(clamp(x / s, -448, 448))
  expert_ffn    per (token, k) pair: h = dequant(xq) . dequant(w13)^T,
                gate/up -> bf16, a = bf16(bf16(act(gate)) * up) (vLLM's
                silu_and_mul / gelu_and_mul return act in the activation
                dtype and then multiply two bf16 values; act in fp32,
                SiLU g / (1 + exp(-g)), GELU (g * 0.5) * (1 + erf(g * fp32(1/sqrt 2)))),
                a -> fp8 per 128 columns,
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
independence of tokens; topk_sum against exact integer sums; activation
against torch's silu and exact-erf gelu, and GELU's closed forms (odd part
gelu(g) - gelu(-g) = g, saturation to g and -0).
"""

from __future__ import annotations

import numpy as np
import scipy.special
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


ACTIVATIONS = ("silu", "gelu")
_SQRT1_2 = np.float32(0.70710678118654752)


def _ulp_step(v: np.ndarray, k: int) -> np.ndarray:
    """v moved by k float32 ulps (toward +inf for k > 0)."""
    v = np.asarray(v, np.float32)
    to = np.float32(np.inf if k > 0 else -np.inf)
    for _ in range(abs(k)):
        v = np.nextafter(v, to).astype(np.float32)
    return v


def activation(gate: np.ndarray, name: str = "silu", erf_ulps: int = 0) -> np.ndarray:
    """act(gate) in float32 as vLLM's act-and-mul kernels evaluate it, each
    fp32 operation rounded: SiLU g / (1 + exp(-g)); GELU
    (g * 0.5) * (1 + erf(g * fp32(1/sqrt 2))) with erf correctly rounded to
    fp32, or moved by `erf_ulps` ulps (a device erff's error)."""
    g = np.asarray(gate, np.float32)
    if name == "silu":
        with np.errstate(over="ignore"):
            return (g / (np.float32(1) + np.exp(-g))).astype(np.float32)
    if name == "gelu":
        t = (g * _SQRT1_2).astype(np.float32)
        e = scipy.special.erf(t.astype(np.float64)).astype(np.float32)
        if erf_ulps:
            e = _ulp_step(e, erf_ulps)
        return ((g * np.float32(0.5)) * (np.float32(1) + e)).astype(np.float32)
    raise ValueError(f"unknown activation {name!r}")


# Planted mistakes for tests that show a set of inputs tells the rounding
# sequence apart (expert_ffn's `variant`); each changes exactly one step.
VARIANTS = (
    "gate_up_unrounded",   # gate and up kept in fp32 instead of rounded to bf16
    "gate_up_truncated",   # gate and up rounded to bf16 toward zero
    "silu_unrounded",      # act(gate) kept in fp32 before the product with up
    "act_unrounded",       # bf16(act(gate)) * up not rounded to bf16 before quantisation
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
               w2: np.ndarray, w2_scale: np.ndarray, variant: str | None = None,
               act: str = "silu") -> np.ndarray:
    """bf16 contributions (T*topk, H) as float32; pairs with an id outside [0, E) are 0.

    x: (T, H) float32 holding bf16 values; w13: (E, 2I, H) fp8 codes (gate
    rows then up rows), w2: (E, H, I); scales (E, 2I/128, H/128) and
    (E, H/128, I/128) float32; `act` one of ACTIVATIONS. `variant` (one of
    VARIANTS) plants one mistake in the rounding sequence, for tests of test
    inputs only.
    """
    if variant is not None and variant not in VARIANTS:
        raise ValueError(f"unknown variant {variant!r}")
    if act not in ACTIVATIONS:
        raise ValueError(f"unknown activation {act!r}")
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
        g = activation(gate, act)
        if variant != "silu_unrounded":
            g = bf16(g)
        a = (g * up).astype(np.float32) if variant == "act_unrounded" else bf16(g * up)
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
# the activation of every such gate rounds to bf16 the same whichever way a
# device's fp32 transcendental rounds: for SiLU, silu(g) at least PROBE_MARGIN
# (relative) away from a bf16 rounding midpoint (an fp32 exp and division are
# off by a few fp32 ulps, about 2^-21); for GELU, the fp32 evaluation rounds
# to the same bf16 bits with erf moved by up to ERF_ULPS fp32 ulps (1 + erf
# cancels for negative gates, so the margin is taken through erf itself).
PROBE_MARGIN = 2.0**-14
ERF_ULPS = 4


def _probe_gates(m: int, a: int) -> np.ndarray:
    return np.array([s * m * 2.0**a * c / 4 for s in (1, -1) for c in (1, 2, 3, 4, -1, -2, -3, -4)], np.float32)


def probe_is_safe(g: np.ndarray, act: str) -> bool:
    """Whether bf16(act(g)) is fixed for every gate in g (see PROBE_MARGIN)."""
    if act == "silu":
        g64 = np.asarray(g, np.float64)
        return bool(bf16_midpoint_margin(g64 / (1 + np.exp(-g64))).min() >= PROBE_MARGIN)
    bits = [bf16_bits(activation(g, act, k)) for k in range(-ERF_ULPS, ERF_ULPS + 1)]
    return all(np.array_equal(b, bits[0]) for b in bits)


def _safe_probe_values(act: str = "silu") -> list[tuple[int, int]]:
    return [(m, a) for a in range(-3, 4) for m in (1, 2, 3) if probe_is_safe(_probe_gates(m, a), act)]


def exact_inputs(rng: np.random.Generator, E: int, H: int, I: int, T: int, topk: int, act: str = "silu"):
    """A MoE case on which every sum is exact in fp32 and every activation
    (`act`) is exact or rounds to bf16 unambiguously, while every rounding
    step of the sequence still rounds: the rounding sequence, not summation
    order, decides the output bits.

    - x: per token one or two active 128-column groups, group 0 always
      among them; each has one value of +-448 * 2^a (so the group scale is
      exactly 2^a) and a few of +-1..3 * 2^a; the other groups are zero.
      Column 0 holds +-m * 2^a with (m, a) drawn from _safe_probe_values(act).
    - w13 gate rows 0-127 (the first activation group) have codes in
      {0, +-1, +-2} over every column and block scale 2^10, so each block
      dot is an integer below 2^11 and every such gate is 0 or at least 104
      in magnitude: silu(g) is g or -0 whatever exp's last bit, and gelu(g)
      g or -0 (erf(+-73.5) is +-1 in fp32, which every erff returns).
    - w13 gate rows 128-255 (the second activation group, when I >= 256)
      are probes: one code c in {+-1..4} at column 0, block scale 2^-2, so
      the gate is v * c / 4, between 2^-5 and 24 in magnitude, where the
      activation is a general value; its bf16 rounding is unambiguous
      (probe_is_safe), and bf16(act(g)) * up rounds differently from
      act(g) * up.
    - Up rows: codes in {0, +-1, +-2, +-3}, scale 2^-4.
    - gate and up then carry up to 11 significant bits (bf16 keeps 8), and
      a = bf16(bf16(act(gate)) * up) up to 16: the roundings round, ties
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

    safe = _safe_probe_values(act)
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


def fused_moe_ref(x, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale, variant=None, act="silu") -> np.ndarray:
    """The layer output (T, H) as float32 holding bf16 values."""
    contrib = expert_ffn(x, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale, variant, act)
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
