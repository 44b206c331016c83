"""GPU encoder parity: records and LUTs byte-equal to the host encoder and to
the reference encoder's golden vectors, for the reference's distributions,
both chunk sizes, full-size expert rows (then decoded back), and the pitch
error of codec.py:160-166."""

import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import codec_ref
from test_codec_gpu import EXP_P, decode_one, fp8_expert, rows

pytestmark = pytest.mark.gpu


def _codec():
    from vllm_expert_pager import codec

    return codec


def _host(codec, raw, pitch, chunk):
    rec = np.empty(pitch, np.uint8)
    lut = np.empty(512, np.uint8)
    needed = codec.encode_into(raw, rec, lut, chunk)
    return rec, lut, needed


def test_golden_records():
    codec = _codec()
    g = np.load(os.path.join(GOLDEN, "codec_vectors.npz"), allow_pickle=False)
    for name in g["cases"]:
        raw = g[f"{name}_raw"]
        want_rec, want_lut = g[f"{name}_record"], g[f"{name}_lut"]
        chunk = int(g[f"{name}_chunk"])
        rec, lut, _ = codec.encode_rows(torch.from_numpy(raw.reshape(1, -1)).cuda(), want_rec.size, chunk)
        np.testing.assert_array_equal(rec[0].cpu().numpy(), want_rec, err_msg=str(name))
        np.testing.assert_array_equal(lut[0].cpu().numpy(), want_lut, err_msg=str(name))


def _dist(dist, n, seed):
    return {
        "realistic": lambda: rows(seed, n),
        "uniform": lambda: rows(seed + 1, n, [1.0] * 16),
        "geometric": lambda: rows(seed + 2, n, [2.0**k for k in range(16)]),
        "constant": lambda: np.full(n, 13 << 3, np.uint8),
        "long_codes": lambda: np.concatenate([np.full(n // 2, 13 << 3, np.uint8), rows(seed + 5, n // 2, [1.0] * 16)]),
        "one_symbol_rare": lambda: np.where(np.arange(n) % 997 == 0, 2 << 3, 13 << 3).astype(np.uint8),
    }[dist]()


@pytest.mark.parametrize("dist", ["realistic", "uniform", "geometric", "constant", "long_codes", "one_symbol_rare"])
@pytest.mark.parametrize("chunk", [64, 512])
def test_matches_host_encoder(dist, chunk):
    _matches_host_encoder(dist, chunk, 6)


# The groups of a row are encoded 8 per workgroup: 9 and 17 groups leave a
# last workgroup with one group (a spare upper half-wave), 11 one with three.
@pytest.mark.parametrize("groups", [1, 9, 11, 17])
def test_matches_host_encoder_group_counts(groups):
    _matches_host_encoder("realistic", 64, groups)


def _matches_host_encoder(dist, chunk, groups):
    codec = _codec()
    n = groups * chunk * 32
    raws = np.stack([_dist(dist, n, 10 * k) for k in range(3)])
    pitch = codec_ref.pitch_of(n, 1.6, 4096)
    rec, lut, needed = codec.encode_rows(torch.from_numpy(raws).cuda(), pitch, chunk)
    rec, lut, needed = rec.cpu().numpy(), lut.cpu().numpy(), needed.cpu().numpy()
    for k in range(3):
        hrec, hlut, hneeded = _host(codec, raws[k], pitch, chunk)
        assert needed[k] == hneeded
        np.testing.assert_array_equal(lut[k], hlut)
        np.testing.assert_array_equal(rec[k], hrec)
        ref_rec, ref_lut = codec_ref.encode(raws[k], pitch, chunk)
        np.testing.assert_array_equal(rec[k], ref_rec)
        np.testing.assert_array_equal(lut[k], ref_lut)


def test_full_size_expert_rows():
    """w13 (2 MiB) and w2 (1 MiB) rows of two synthetic experts at pitch 0.89,
    equal to the host encoder and decoded back on the GPU."""
    codec = _codec()
    for shape in ((1024, 2048), (2048, 512)):
        n = shape[0] * shape[1]
        raws = np.stack([fp8_expert(40 + k, shape) for k in range(2)])
        pitch = codec_ref.pitch_of(n, 0.89, 4096)
        rec, lut, _ = codec.encode_rows(torch.from_numpy(raws).cuda(), pitch)
        rec, lut = rec.cpu().numpy(), lut.cpu().numpy()
        for k in range(2):
            hrec, hlut, _ = _host(codec, raws[k], pitch, 512)
            np.testing.assert_array_equal(lut[k], hlut)
            np.testing.assert_array_equal(rec[k], hrec)
            np.testing.assert_array_equal(decode_one(codec, rec[k], lut[k], n, 512), raws[k])


def test_rows_that_do_not_fit_the_pitch():
    codec = _codec()
    n = 4 * 512 * 32
    raws = np.stack([rows(1, n, [1.0] * 16), rows(2, n, EXP_P)])  # about 1.0 and 0.84 of the row
    pitch = codec_ref.pitch_of(n, 0.9, 4096)
    with pytest.raises(ValueError, match="VLLM_EXPERT_PAGER_PITCH must be at least"):
        codec.encode_rows(torch.from_numpy(raws).cuda(), pitch)
    rec, lut, needed = codec.encode_rows(torch.from_numpy(raws).cuda(), pitch, check=False)
    needed = needed.cpu().numpy()
    host_needed = [_host(codec, raws[k], codec_ref.pitch_of(n, 1.6, 4096), 512)[2] for k in range(2)]
    assert list(needed) == host_needed
    assert needed[0] > pitch >= needed[1]
    hrec, hlut, _ = _host(codec, raws[1], pitch, 512)
    np.testing.assert_array_equal(rec[1].cpu().numpy(), hrec)


def test_encode_of_a_gpu_row():
    codec = _codec()
    raw = rows(7, 2 * 512 * 32)
    pitch = codec_ref.pitch_of(raw.size, 1.25, 4096)
    rec, lut = codec.encode(torch.from_numpy(raw).cuda(), pitch)
    assert rec.is_cuda and lut.is_cuda
    hrec, hlut, _ = _host(codec, raw, pitch, 512)
    np.testing.assert_array_equal(rec.cpu().numpy(), hrec)
    np.testing.assert_array_equal(lut.cpu().numpy(), hlut)
