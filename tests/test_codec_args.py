"""Argument checks of the decode launchers, on the CPU (no kernel is launched).

``decode_rows`` and ``decode_rows_from_ram`` write row r of ``dst[i]`` at
``r * shape[1] * element_size`` bytes from the tensor's start, so every
``dst`` (and staging) tensor must be a contiguous 2-D GPU tensor; anything
else is refused with ``ValueError`` before the launch.
"""

import pytest
import torch

from vllm_expert_pager import codec


def _args(dst):
    E = 4
    idx = torch.zeros((E,), dtype=torch.int64)
    lut = torch.zeros((E, 1, codec.LUT_BYTES), dtype=torch.uint8)
    return idx, lut, [dst]


def test_cpu_dst_is_refused():
    idx, lut, dst = _args(torch.zeros((2, 64), dtype=torch.uint8))
    staging = [torch.zeros((2, 64), dtype=torch.uint8)]
    with pytest.raises(ValueError, match="must be a GPU tensor"):
        codec.decode_rows(idx, idx, idx, staging, dst, lut)
    with pytest.raises(ValueError, match="must be a GPU tensor"):
        codec.decode_rows_from_ram(idx, idx, idx, idx, 0, staging, dst, lut, [idx], [idx])


@pytest.mark.parametrize("bad", ["strided", "1d"])
def test_dst_rows_must_be_contiguous_2d(monkeypatch, bad):
    # Stand in for the device check so the row check is reached on the CPU.
    monkeypatch.setattr(codec.nat, "require_device", lambda t, what: None)
    whole = torch.zeros((2, 128), dtype=torch.uint8)
    d = whole[:, :64] if bad == "strided" else whole.reshape(-1)
    idx, lut, dst = _args(d)
    staging = [torch.zeros((2, 64), dtype=torch.uint8)]
    with pytest.raises(ValueError, match=r"dst\[0\] must be a contiguous 2-D tensor"):
        codec.decode_rows(idx, idx, idx, staging, dst, lut)
    scale = [torch.zeros((4, 2), dtype=torch.float32)]
    with pytest.raises(ValueError, match=r"dst\[0\] must be a contiguous 2-D tensor"):
        codec.decode_rows_from_ram(idx, idx, idx, idx, 0, staging, dst, lut, scale, scale)
