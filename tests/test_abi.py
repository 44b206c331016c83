"""The C ABI library loads and exports every function include/xp.h declares (CPU, no GPU calls)."""

import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "xp.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_entry_points():
    names = declared()
    for must in ("xp_acquire_pair", "xp_gather_rows", "xp_decode_rows", "xp_moe_experts", "xp_moe_topk_sum",
                 "ssd_start", "ssd_stop", "xp_encode_row"):
        assert must in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    from vllm_expert_pager import _native

    lib = _native.lib()
    raw = ctypes.CDLL(lib._name)
    missing = [n for n in declared() if not hasattr(raw, n)]
    assert not missing, f"libxp.so lacks {missing}"
    raw.xp_version.restype = ctypes.c_char_p
    assert raw.xp_version().decode().startswith("libxp")


def test_every_symbol_has_a_python_signature():
    from vllm_expert_pager import _native

    sig = set(_native._SIGNATURES)
    ssd = {"ssd_start", "ssd_stop", "ssd_stats", "ssd_error", "ssd_test_delay"}
    missing = [n for n in declared() if n not in sig and n not in ssd]
    assert not missing, f"no ctypes signature for {missing}"


def test_roctx_ranges_are_free_when_off(monkeypatch):
    from vllm_expert_pager import trace

    monkeypatch.delenv("VLLM_EXPERT_PAGER_ROCTX", raising=False)
    monkeypatch.setattr(trace, "_loaded", False)
    monkeypatch.setattr(trace, "_lib", None)
    with trace.range("x"):
        pass
    assert trace._lib is None
