"""The C ABI library loads and exports every function include/xp.h declares, and the ctypes
structures of the bindings have the header's layout (CPU, no GPU calls)."""

import ctypes
import os
import re
import shutil
import subprocess

import pytest

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


def declarations() -> dict[str, list[str]]:
    """Each declared function's parameter list (type text of each parameter)."""
    text = open(os.path.join(ROOT, "include", "xp.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*\b([a-z_][a-z0-9_]*)\s*\(([^;{]*?)\)\s*;",
                         text, flags=re.M | re.S):
        params = [" ".join(p.split()) for p in m.group(2).split(",")]
        out[m.group(1)] = [] if params == ["void"] or params == [""] else params
    return out


def _kind(param: str) -> str:
    """'ptr', 'i32' or 'i64' for a C parameter declaration."""
    if "*" in param:
        return "ptr"
    if re.search(r"\b(int64_t|long|size_t)\b", param):
        return "i64"
    if re.search(r"\b(int|int32_t)\b", param):
        return "i32"
    if re.search(r"\bdouble\b", param):
        return "f64"
    raise AssertionError(f"unexpected parameter type {param!r}")


def test_python_signatures_match_the_header():
    """Every ctypes signature has the header's arity and, position by
    position, its pointer / 32-bit / 64-bit integer kinds (a missing or
    extra argument shifts every later one)."""
    from vllm_expert_pager import _native as nat

    ctype_kind = {ctypes.c_void_p: "ptr", ctypes.c_char_p: "ptr", ctypes.c_int: "i32", ctypes.c_int64: "i64",
                  ctypes.c_long: "i64", ctypes.c_double: "f64"}
    decl = declarations()
    assert len(decl) >= 30
    bad = []
    for name, (_, args) in nat._SIGNATURES.items():
        assert name in decl, f"{name} is not declared in include/xp.h"
        want = [_kind(p) for p in decl[name]]
        got = [ctype_kind[a] for a in args]
        if want != got:
            bad.append(f"{name}: header {want}, ctypes {got}")
    assert not bad, "\n".join(bad)


def test_roctx_ranges_are_free_when_off(monkeypatch):
    from vllm_expert_pager import trace

    monkeypatch.delenv("VLLM_EXPERT_PAGER_ROCTX", raising=False)
    monkeypatch.setattr(trace, "_loaded", False)
    monkeypatch.setattr(trace, "_lib", None)
    with trace.range("x"):
        pass
    assert trace._lib is None


def test_struct_layouts_match_the_header(tmp_path):
    """Every struct the bindings pass by pointer has, in ctypes, the size and
    field offsets a C compiler gives it from include/xp.h."""
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    from vllm_expert_pager import _native

    structs = {"xp_table": _native.XpTable, "xp_gather_name": _native.XpGatherName, "xp_ring": _native.XpRing,
               "xp_decode_name": _native.XpDecodeName, "xp_decode_scale": _native.XpDecodeScale}
    header = open(os.path.join(ROOT, "include", "xp.h")).read()
    assert set(re.findall(r"typedef struct (xp_[a-z_]+) \{", header)) == set(structs), "a struct without a check"
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "xp.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src, exe = tmp_path / "layout.c", tmp_path / "layout"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                               check=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert int(got[f"{cname}.{field}"]) == getattr(cls, field).offset, f"{cname}.{field}"
