"""xp_moe_experts_noalloc: the expert FFN with the library's own workspace.

Called through the C ABI and compared bit for bit with xp_moe_experts (the
caller-provided workspace) on the same routing, twice in a row on one device
with the second call smaller than the first: a prefill-sized call (the wide
GEMM kernels) then a decode-sized one (the narrow kernels), which leaves the
first call's contents in the shared array. A call whose workspace would not
fit is refused with XP_E_LIMIT before anything is launched. The static
array sits in a code object of its own, so a process that never calls the
no-alloc entry point does not give up its 32 MiB.
"""

import ctypes
import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import moe_ref as M

pytestmark = pytest.mark.gpu


def _nat():
    from vllm_expert_pager import _native, moe

    return _native, moe


def _inputs(rng, E, H, I, T, topk):
    w13, w13s, w2, w2s = (torch.from_numpy(a).cuda() for a in M.random_experts(rng, E, H, I))
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).cuda()
    ids = torch.from_numpy(np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int64)).cuda()
    tw = torch.softmax(torch.from_numpy(rng.standard_normal((T, topk)).astype(np.float32)), 1).cuda()
    return x, tw, ids, w13, w13s, w2, w2s


def _run(entry, x, tw, ids, w13, w13s, w2, w2s, act=0):
    """One expert call through the C ABI (activation code `act`); returns the
    (T*topk, H) bf16 contributions."""
    nat, moe = _nat()
    E, T, topk, H, I = w13.shape[0], ids.shape[0], ids.shape[1], x.shape[1], w2.shape[2]
    xq, xs = moe.quant_tokens(x)
    r = moe.route(ids, torch.arange(E, dtype=torch.int32, device="cuda"), E)
    out = torch.full((T * topk, H), -1, dtype=torch.int16, device="cuda")
    head = (xq.data_ptr(), xs.data_ptr(), T, topk, tw.data_ptr(), H, I, w13.data_ptr(), w13s.data_ptr(),
            w2.data_ptr(), w2s.data_ptr(), E, r.offsets.data_ptr(), r.pairs.data_ptr(), r.tiles.data_ptr())
    if entry == "xp_moe_experts":
        nbytes = int(nat.lib().xp_moe_workspace_bytes(T * topk, I))
        work = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
        rc = nat.lib().xp_moe_experts(*head, work.data_ptr(), nbytes, out.data_ptr(), act, nat.stream())
    else:
        rc = nat.lib().xp_moe_experts_noalloc(*head, out.data_ptr(), act, nat.stream())
    assert rc == 0, nat.lib().xp_last_error()
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("act", [0, 1], ids=["silu", "gelu"])
def test_noalloc_matches_the_workspace_entry_point_twice(act):
    nat, _ = _nat()
    rng = np.random.default_rng(act)
    E, H, I = 32, 2048, 512
    # 600 tokens x top-8 = 4800 pairs (wide kernels, 8.1 MB of workspace),
    # then 3 tokens (narrow kernels) over the array the first call filled.
    for T in (600, 3):
        case = _inputs(rng, E, H, I, T, 8)
        need = int(nat.lib().xp_moe_workspace_bytes(T * 8, I))
        assert need <= 32 << 20
        want = _run("xp_moe_experts", *case, act=act)
        got = _run("xp_moe_experts_noalloc", *case, act=act)
        assert torch.equal(got, want), f"T={T}"
        assert int((want == -1).sum()) == 0  # every pair was written


def test_noalloc_refuses_a_workspace_above_its_limit():
    nat, moe = _nat()
    lib = nat.lib()
    T, topk, H, I, E = 8192, 8, 2048, 512, 16
    assert int(lib.xp_moe_workspace_bytes(T * topk, I)) > 32 << 20
    dummy = torch.zeros((16,), dtype=torch.uint8, device="cuda")
    p = dummy.data_ptr()
    rc = lib.xp_moe_experts_noalloc(p, p, T, topk, p, H, I, p, p, p, p, E, p, p, p, p, 0, nat.stream())
    assert rc == nat.XP_E_LIMIT
    assert b"above the library's" in lib.xp_last_error()
    rc = lib.xp_moe_experts_noalloc(p, p, 1, topk, p, H, I, p, p, p, p, E, p, p, p, p, 7, nat.stream())
    assert rc == nat.XP_E_ARG and b"unknown activation 7" in lib.xp_last_error()
    torch.cuda.synchronize()


_MEMORY_PROBE = """
import json, sys
sys.path[:0] = sys.argv[1:]
import numpy as np, torch
torch.zeros(1, device="cuda"); torch.cuda.synchronize()
from test_zz_no_alloc import _inputs, _run

def snap():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0], torch.cuda.memory_reserved()

case = _inputs(np.random.default_rng(0), 32, 2048, 512, 3, 8)
s0 = snap(); _run("xp_moe_experts", *case); s1 = snap()
_run("xp_moe_experts_noalloc", *case); s2 = snap()
outside = lambda a, b: ((a[0] - b[0]) - (b[1] - a[1])) / 2**20
print(json.dumps({"first_experts_mib": outside(s0, s1), "first_noalloc_mib": outside(s1, s2)}))
"""


def test_noalloc_array_is_reserved_only_when_called():
    """In a fresh process, device memory taken outside torch's allocator:
    the first xp_moe_experts launch loads the expert kernels without the
    32 MiB array; the first xp_moe_experts_noalloc call then reserves it."""
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [root, os.path.join(root, "vllm-expert-pager_amd"), here]
    r = subprocess.run([sys.executable, "-c", _MEMORY_PROBE, *paths], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    got = json.loads(r.stdout.strip().splitlines()[-1])
    assert got["first_experts_mib"] < 16, got
    assert got["first_noalloc_mib"] >= 32, got
