"""CPU checks of the codec oracle (oracle/codec_ref.py) and of the host encoder of libxp.

The oracle is pinned by the reference encoder's golden records, by the
round trip through the reference's sequential decoder rule, and by the Kraft
equality of the code lengths. The product's C++ encoder (host code, no GPU
needed) is checked byte for byte against the same golden records.
"""

import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import codec_ref

CHUNK = 64
N = 2 * CHUNK * codec_ref.LANES

EXP_P = [0.0] * 4 + [0.001, 0.002, 0.004, 0.008, 0.016, 0.032, 0.064, 0.125, 0.228, 0.315, 0.188, 0.015]


def rows(seed, n=N, p=EXP_P):
    rng = np.random.default_rng(seed)
    p = np.asarray(p, np.float64)
    exp = rng.choice(16, size=n, p=p / p.sum()).astype(np.uint8)
    sm = rng.integers(0, 256, size=n, dtype=np.uint8) & 0x87
    return sm | (exp << 3)


DISTS = {
    "realistic": lambda: rows(0),
    "uniform": lambda: rows(1, p=[1.0] * 16),
    "geometric": lambda: rows(2, p=[2.0**k for k in range(16)]),
    "constant": lambda: np.full(N, 13 << 3, np.uint8),
}


def golden():
    return np.load(os.path.join(GOLDEN, "codec_vectors.npz"), allow_pickle=False)


def test_oracle_encode_matches_reference_records():
    g = golden()
    for name in g["cases"]:
        rec, lut = codec_ref.encode(g[f"{name}_raw"], int(g[f"{name}_pitch"]), int(g[f"{name}_chunk"]))
        np.testing.assert_array_equal(rec, g[f"{name}_record"], err_msg=str(name))
        np.testing.assert_array_equal(lut, g[f"{name}_lut"], err_msg=str(name))


def test_oracle_code_matches_reference():
    g = golden()
    for h, lengths, codes, lut in zip(g["hists"], g["lengths"], g["codes"], g["luts"]):
        assert codec_ref.code_lengths(h.tolist()) == lengths.tolist()
        c = codec_ref.Code(h.tolist())
        assert c.codes == codes.tolist() and c.lut == lut.tolist()


@pytest.mark.parametrize("dist", sorted(DISTS))
def test_round_trip_through_sequential_decoder(dist):
    raw = DISTS[dist]()
    rec, lut = codec_ref.encode(raw, codec_ref.pitch_of(N, 1.25, 4096), CHUNK)
    assert codec_ref.decode_ref(rec.tobytes(), lut.tobytes(), N, CHUNK) == raw.tolist()
    np.testing.assert_array_equal(codec_ref.decode_fast(rec, lut, N, CHUNK)[0], raw)


def test_golden_records_decode_to_their_rows():
    g = golden()
    for name in g["cases"]:
        raw, chunk = g[f"{name}_raw"], int(g[f"{name}_chunk"])
        out = codec_ref.decode_fast(g[f"{name}_record"], g[f"{name}_lut"], raw.size, chunk)[0]
        np.testing.assert_array_equal(out, raw, err_msg=str(name))


def test_code_lengths_are_limited_and_complete():
    for hist in ([2**k for k in range(16)], [1] * 16, [0] * 16, [5] + [0] * 15):
        lengths = codec_ref.code_lengths(hist)
        assert max(lengths) <= codec_ref.LIMIT
        assert sum(2.0**-n for n in lengths) == 1.0


def test_oracle_errors():
    with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
        codec_ref.encode(rows(3), N // 4, CHUNK)
    with pytest.raises(ValueError, match="not a multiple"):
        codec_ref.encode(rows(3, n=N + 8), 8 * N, CHUNK)


def test_decoder_detects_a_planted_mistake():
    """A record with one Huffman word changed no longer decodes to its row."""
    raw = DISTS["realistic"]()
    rec, lut = codec_ref.encode(raw, codec_ref.pitch_of(N, 1.25, 4096), CHUNK)
    bad = rec.copy()
    head = 4 * (N // (CHUNK * 32) + 1) + N // 2
    bad[head + 8] ^= 0x5A
    assert not np.array_equal(codec_ref.decode_fast(bad, lut, N, CHUNK)[0], raw)


# ---- the product's host encoder (C++ in libxp.so; CPU code) ----

def _native_codec():
    from vllm_expert_pager import _native, codec

    try:
        _native.lib()
    except ImportError as e:
        pytest.fail(f"libxp.so must be built for the CPU suite: {e}")
    return codec


def test_host_encoder_matches_reference_records():
    codec = _native_codec()
    g = golden()
    for name in g["cases"]:
        raw, pitch, chunk = g[f"{name}_raw"], int(g[f"{name}_pitch"]), int(g[f"{name}_chunk"])
        rec = np.empty(pitch, np.uint8)
        lut = np.empty(512, np.uint8)
        used = codec.encode_into(np.ascontiguousarray(raw), rec, lut, chunk)
        np.testing.assert_array_equal(rec, g[f"{name}_record"], err_msg=str(name))
        np.testing.assert_array_equal(lut, g[f"{name}_lut"], err_msg=str(name))
        assert used <= pitch


def test_host_code_matches_reference():
    codec = _native_codec()
    g = golden()
    for h, lengths, codes, lut in zip(g["hists"], g["lengths"], g["codes"], g["luts"]):
        c = codec.Code(h.tolist())
        assert c.lengths == lengths.tolist() and c.codes == codes.tolist() and c.lut == lut.tolist()


@pytest.mark.parametrize("dist", sorted(DISTS))
def test_host_encoder_matches_oracle(dist):
    codec = _native_codec()
    raw = DISTS[dist]()
    pitch = codec_ref.pitch_of(N, 1.25, 4096)
    want_rec, want_lut = codec_ref.encode(raw, pitch, CHUNK)
    rec, lut = np.empty(pitch, np.uint8), np.empty(512, np.uint8)
    codec.encode_into(raw, rec, lut, CHUNK)
    np.testing.assert_array_equal(rec, want_rec)
    np.testing.assert_array_equal(lut, want_lut)


def test_host_encoder_errors():
    codec = _native_codec()
    raw = rows(3)
    with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
        codec.encode_into(raw, np.empty(N // 4, np.uint8), np.empty(512, np.uint8), CHUNK)
    r2 = rows(3, n=N + 8)
    with pytest.raises(ValueError, match="not a multiple"):
        codec.encode_into(r2, np.empty(8 * N, np.uint8), np.empty(512, np.uint8), CHUNK)


def test_host_code_matches_oracle_on_random_histograms():
    """The native code construction (lengths by merging, length limiting,
    canonical codes, LUT) against the oracle's on 400 random histograms:
    ties of equal counts, zero counts, skewed ones that need the length
    limit, and near-uniform ones."""
    codec = _native_codec()
    rng = np.random.default_rng(41)
    for i in range(400):
        kind = i % 4
        if kind == 0:  # many ties
            h = rng.integers(0, 4, 16) * 1000
        elif kind == 1:  # geometric: lengths beyond the limit before limiting
            h = (2.0 ** rng.permutation(16) * rng.integers(1, 4)).astype(np.int64)
        elif kind == 2:  # sparse, with zeros
            h = rng.integers(0, 10**6, 16) * (rng.random(16) < 0.4)
        else:
            h = rng.integers(10**5, 2 * 10**5, 16)
        c = codec.Code([int(x) for x in h])
        r = codec_ref.Code([int(x) for x in h])
        assert c.lengths == list(r.lengths) and c.codes == list(r.codes) and c.lut == list(r.lut), h.tolist()
        assert max(c.lengths) <= 9
