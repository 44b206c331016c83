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
                gate/up -> bf16, a = bf16(silu(gate) * up), a -> fp8 per 128
                columns, y = dequant(aq) . dequant(w2)^T,
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


def expert_ffn(x: np.ndarray, topk_weights: np.ndarray, topk_ids: np.ndarray, w13: np.ndarray, w13_scale: np.ndarray,
               w2: np.ndarray, w2_scale: np.ndarray) -> np.ndarray:
    """bf16 contributions (T*topk, H) as float32; pairs with an id outside [0, E) are 0.

    x: (T, H) float32 holding bf16 values; w13: (E, 2I, H) fp8 codes (gate
    rows then up rows), w2: (E, H, I); scales (E, 2I/128, H/128) and
    (E, H/128, I/128) float32.
    """
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
        gate, up = bf16(h[:, :I]), bf16(h[:, I:])
        with np.errstate(over="ignore"):
            silu = (gate / (np.float32(1) + np.exp(-gate))).astype(np.float32)
        a = bf16(silu * up)
        aq, as_ = quant_groups(a)
        y = (dequant_rows(aq, as_) @ dequant_weight(w2[e], w2_scale[e]).T).astype(np.float32)
        out[pairs] = bf16(y * tw.reshape(-1)[pairs][:, None])
    return out


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


def fused_moe_ref(x, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale) -> np.ndarray:
    """The layer output (T, H) as float32 holding bf16 values."""
    contrib = expert_ffn(x, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale)
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
