"""Pins of the MoE oracle (oracle/moe_ref.py) on the CPU.

vLLM's fused fp8 MoE is not part of the reference tree and no reference
test exercises it, so the oracle is pinned by what the format and the
mathematics fix: the e4m3fn code table, round-to-nearest-even, closed forms
of the quantisation and of a one-hot token, invariances, exact sums, and
the activations against torch and their closed forms.
"""

import numpy as np
import pytest
import torch

from oracle import moe_ref as M


def test_fp8_table_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    ours = M.fp8_values()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0**-9 and ours[0x08] == 2.0**-6


@pytest.mark.parametrize(
    "value, code",
    [
        (1.0625, 0x38),  # tie between 1.0 (even) and 1.125 -> 1.0
        (1.1875, 0x3A),  # tie between 1.125 and 1.25 (even) -> 1.25
        (448.0, 0x7E),
        (-448.0, 0xFE),
        (2.0**-9, 0x01),
        (2.0**-10, 0x00),  # half the smallest subnormal: tie to even 0
        (3 * 2.0**-10, 0x02),  # tie between 1 and 2 subnormal units -> 2
        (0.0, 0x00),
    ],
)
def test_to_fp8_rounding(value, code):
    assert int(M.to_fp8(np.array([value], np.float32))[0]) == code


def test_quant_groups_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    x[1, :128] = 0.0
    q, s = M.quant_groups(x)
    assert s.shape == (3, 2)
    vals = M.fp8_values()[q]
    for t in range(3):
        for g in range(2):
            blk = x[t, 128 * g : 128 * (g + 1)]
            amax = np.float32(np.abs(blk).max())
            if amax == 0:
                assert s[t, g] == np.float32(1e-10) / np.float32(448) and not q[t, 128 * g : 128 * (g + 1)].any()
                continue
            assert s[t, g] == amax / np.float32(448)
            i = int(np.abs(blk).argmax())
            assert abs(vals[t, 128 * g + i]) == 448.0
            # every value is within half an fp8 step of x / s
            err = np.abs(vals[t, 128 * g : 128 * (g + 1)] - blk / s[t, g])
            assert (err <= np.maximum(np.abs(blk / s[t, g]) / 16, 2.0**-10) + 1e-6).all()


def _experts(E=3, H=256, I=128, seed=1):
    return M.random_experts(np.random.default_rng(seed), E, H, I)


def _ulp(v: np.ndarray) -> np.ndarray:
    v = np.abs(np.asarray(v, np.float32))
    return np.nextafter(v, np.float32(np.inf)) - v


def _gates() -> np.ndarray:
    rng = np.random.default_rng(9)
    g = np.concatenate([rng.standard_normal(20000) * 4, rng.uniform(-30, 30, 20000), [0.0, 1.0, -1.0, 104.0, -104.0]])
    return g.astype(np.float32)


def test_silu_against_torch_and_closed_forms():
    g = _gates()
    ours = M.activation(g, "silu")
    ref = torch.nn.functional.silu(torch.from_numpy(g).double()).numpy()
    # three fp32 roundings and exp's own error: 3 ulps; far below zero
    # exp(-g) overflows fp32 and silu(g) is -0 where its float64 value is a
    # subnormal: an absolute 2^-126
    assert (np.abs(ours - ref) <= 3 * _ulp(ref) + 2.0**-126).all()
    assert M.activation(np.float32([0.0]), "silu")[0] == 0.0
    assert M.activation(np.float32([104.0]), "silu")[0] == 104.0
    assert M.activation(np.float32([-104.0]), "silu").view(np.uint32)[0] == 0x80000000  # -0
    assert abs(M.activation(np.float32([1.0]), "silu")[0] - 0.7310585786300049) <= 6e-8


def test_gelu_against_torch_and_closed_forms():
    """GELU is g * Phi(g): against torch's exact-erf gelu in float64, to the
    bound the fp32 evaluation allows (1 + erf cancels for negative g, so the
    error is absolute, |g| * 2^-23, plus two ulps of the result); its odd
    part gelu(g) - gelu(-g) = g; Phi(1) = 0.8413447460685429; saturation to g
    and -0 far out."""
    g = _gates()
    ours = M.activation(g, "gelu")
    ref = torch.nn.functional.gelu(torch.from_numpy(g).double(), approximate="none").numpy()
    assert (np.abs(ours - ref) <= np.abs(g) * 2.0**-23 + 2 * _ulp(ref) + 2.0**-126).all()
    # torch's own fp32 gelu (its vectorised erf is a few fp32 ulps off)
    ref32 = torch.nn.functional.gelu(torch.from_numpy(g), approximate="none").numpy()
    assert (np.abs(ours - ref32) <= np.abs(g) * 2.0**-20 + 4 * _ulp(ref) + 2.0**-126).all()
    odd = M.activation(g, "gelu").astype(np.float64) - M.activation(-g, "gelu").astype(np.float64)
    assert (np.abs(odd - g) <= np.abs(g) * 2.0**-22).all()
    assert abs(M.activation(np.float32([1.0]), "gelu")[0] - 0.8413447460685429) <= 6e-8
    assert M.activation(np.float32([0.0]), "gelu").view(np.uint32)[0] == 0
    assert M.activation(np.float32([104.0]), "gelu")[0] == 104.0
    assert M.activation(np.float32([-104.0]), "gelu").view(np.uint32)[0] == 0x80000000  # -0
    with pytest.raises(ValueError, match="unknown activation"):
        M.activation(g, "relu")


@pytest.mark.parametrize("act", M.ACTIVATIONS)
def test_expert_ffn_one_hot_closed_form(act):
    """x = c * e_i makes h column i of w13; w2 = a permutation picks activation entries."""
    E, H, I, c, i = 2, 256, 128, 1.5, 37
    w13, w13s, _, _ = _experts(E, H, I)
    # w2[e][h][n] = 1.0 at n = (h + 5e) % I, scale 1
    w2 = np.zeros((E, H, I), np.uint8)
    for e in range(E):
        w2[e, np.arange(H), (np.arange(H) + 5 * e) % I] = 0x38
    w2s = np.ones((E, H // 128, I // 128), np.float32)
    x = np.zeros((2, H), np.float32)
    x[:, i] = c
    ids = np.array([[0], [1]])
    tw = np.array([[0.5], [2.0]], np.float32)
    got = M.expert_ffn(x, tw, ids, w13, w13s, w2, w2s, act=act)
    v = M.fp8_values()
    for t, e in enumerate((0, 1)):
        col = v[w13[e][:, i]] * np.repeat(w13s[e][:, i // 128], 128)  # dequantised column i
        h = (c * col).astype(np.float32)
        gate, up = M.bf16(h[:I]), M.bf16(h[I:])
        a = M.bf16(M.bf16(M.activation(gate, act)) * up)
        aq, as_ = M.quant_groups(a[None, :])
        ad = v[aq[0]] * np.repeat(as_[0].astype(np.float64), 128)
        y = ad[(np.arange(H) + 5 * e) % I].astype(np.float32)
        assert np.array_equal(got[t], M.bf16(y * tw[t, 0]))


def test_expert_ffn_invariances():
    rng = np.random.default_rng(2)
    E, H, I, T, K = 4, 256, 128, 5, 2
    w13, w13s, w2, w2s = _experts(E, H, I, seed=3)
    x = M.bf16(rng.standard_normal((T, H)).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    tw = rng.random((T, K)).astype(np.float32)
    base = M.fused_moe_ref(x, tw, ids, w13, w13s, w2, w2s)
    # relabel the experts
    perm = rng.permutation(E)
    inv = np.argsort(perm)
    relabelled = M.fused_moe_ref(x, tw, perm[ids], w13[inv], w13s[inv], w2[inv], w2s[inv])
    assert np.array_equal(base, relabelled)
    # routed weights times a power of two scale the output exactly
    assert np.array_equal(M.fused_moe_ref(x, 4 * tw, ids, w13, w13s, w2, w2s), 4 * base)
    # a token's output does not depend on the other tokens
    sub = M.fused_moe_ref(x[2:4], tw[2:4], ids[2:4], w13, w13s, w2, w2s)
    assert np.array_equal(sub, base[2:4])
    # an id outside [0, E) contributes nothing
    ids2 = ids.copy()
    ids2[0, 1] = -1
    c = M.expert_ffn(x, tw, ids2, w13, w13s, w2, w2s)
    assert not c[1].any()


def test_topk_sum_exact_and_skips_invalid():
    T, K, H = 3, 4, 8
    c = np.arange(T * K * H, dtype=np.float32).reshape(T * K, H) % 7 - 3
    ids = np.array([[0, 1, 2, 3], [1, -1, 2, 9], [3, 3, 0, 1]])
    got = M.topk_sum(c, ids, 4)
    cc = c.reshape(T, K, H)
    ok = ((ids >= 0) & (ids < 4))[:, :, None]
    assert np.array_equal(got, (cc * ok).sum(axis=1))


# (experts, tokens, top-k, seed) of the exact-input cases, shared with the GPU
# test: 150 tokens x top-4 over 64 experts is a prefill-sized call (the wide
# GEMM kernels), 8 x top-8 over 8 experts a decode-sized one (the narrow ones).
EXACT_CASES = [(64, 150, 4, 0), (8, 8, 8, 108)]


@pytest.mark.parametrize("act", M.ACTIVATIONS)
@pytest.mark.parametrize("E, T, topk, seed", EXACT_CASES)
def test_exact_inputs_tell_every_rounding_step_apart(E, T, topk, seed, act):
    """On exact_inputs every sum is exact and every activation is exact or
    rounds to bf16 unambiguously, so the output is decided by the rounding
    sequence alone; each planted mistake in that sequence (M.VARIANTS)
    changes it, and so does the other activation. A GPU kernel that equals
    the oracle bit for bit on these inputs (tests/test_moe_gpu.py) therefore
    rounds gate and up to bf16 to nearest even, rounds act(gate) to bf16 and
    then bf16(act(gate)) * up to bf16, divides by amax / 448, converts to fp8
    to nearest even and weights y before its one bf16 rounding."""
    rng = np.random.default_rng(seed)
    case = M.exact_inputs(rng, E, 512, 256, T, topk, act)
    ref = M.fused_moe_ref(*case, act=act)
    assert np.isfinite(ref).all() and (ref != 0).mean() > 0.1
    for v in M.VARIANTS:
        assert not np.array_equal(M.fused_moe_ref(*case, variant=v, act=act), ref), v
    other = [a for a in M.ACTIVATIONS if a != act][0]
    assert not np.array_equal(M.fused_moe_ref(*case, act=other), ref)


@pytest.mark.parametrize("act", M.ACTIVATIONS)
def test_exact_inputs_keep_their_promises(act):
    """Group scales of x are powers of two; every gate of the first 128 rows
    is 0 or of magnitude >= 104 (exp(-|g|) below half an fp32 ulp of 1,
    exp(|g|) beyond fp32, erf(g / sqrt 2) = +-1 in fp32); every probe gate
    (rows 128-255) is non-zero with bf16(act(g)) fixed however the device's
    exp or erf rounds its last bits (M.probe_is_safe); every block dot is an
    integer below 2^11 (exact in any fp32 accumulation)."""
    rng = np.random.default_rng(5)
    x, tw, ids, w13, w13s, w2, w2s = M.exact_inputs(rng, 8, 512, 256, 64, 4, act)
    xq, xs = M.quant_groups(x)
    live = xs > 1e-9
    assert np.all(np.log2(xs[live]) == np.round(np.log2(xs[live])))
    fp8 = M.fp8_values()
    xv = fp8[xq].reshape(64, 4, 128)
    for e in range(8):
        w = fp8[w13[e]].reshape(512, 4, 128)
        dots = np.einsum("tgk,ngk->tng", xv, w)
        assert np.all(dots == np.round(dots)) and np.abs(dots).max() < 2**11
        gate = (M.dequant_rows(xq, xs) @ M.dequant_weight(w13[e], w13s[e]).T)[:, :256]
        nz = gate[:, :128][gate[:, :128] != 0]
        assert nz.size and np.abs(nz).min() >= 104
        probe = gate[:, 128:]
        assert (probe != 0).all() and np.abs(probe).min() >= 2.0**-5 and np.abs(probe).max() <= 24
        assert M.probe_is_safe(probe.astype(np.float32).ravel(), act)
    assert ((w2 != 0).sum(axis=2) == 1).all()
