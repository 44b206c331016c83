"""Recipe: compile the reference's SSD server into oracle/_ref/ (test infrastructure).

The reference's only native code is the C server held as the string
literal ``_C_SOURCE`` in src/vllm_expert_pager/store.py:68-309, which its
native.py:19-41 writes to a file and compiles with ``cc -O3 -fPIC -shared
-pthread`` on first use. This recipe reads that literal from the reference
tree as text (the module is parsed, never imported or run), pipes it into
gcc on stdin and writes only the shared library ``oracle/_ref/libssd_ref.so``.
No reference source is stored in this repository.

The library exports the same ``ssd_*`` C ABI as libxp.so, so the CPU
protocol tests run unchanged against both servers.

    python -m oracle.build_ref [REFERENCE_ROOT]
"""

from __future__ import annotations

import ast
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REF_OUT = os.path.join(HERE, "_ref")
SSD_REF_LIB = os.path.join(REF_OUT, "libssd_ref.so")
DEFAULT_REFERENCE = "/root/reference"
STORE = os.path.join("src", "vllm_expert_pager", "store.py")


def _server_source(reference: str) -> str:
    with open(os.path.join(reference, STORE), encoding="utf-8") as f:
        tree = ast.parse(f.read())
    for node in tree.body:
        if (isinstance(node, ast.Assign) and len(node.targets) == 1
                and isinstance(node.targets[0], ast.Name) and node.targets[0].id == "_C_SOURCE"
                and isinstance(node.value, ast.Constant) and isinstance(node.value.value, str)):
            return node.value.value
    raise RuntimeError(f"no _C_SOURCE string literal in {STORE}")


def build_ssd_ref(reference: str = DEFAULT_REFERENCE, out: str = SSD_REF_LIB) -> str | None:
    """Build the reference server; returns the library path, or None without a reference tree."""
    if not os.path.isfile(os.path.join(reference, STORE)):
        return None
    src = _server_source(reference)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    # The reference's flags (native.py:19) minus -march=native, so the build
    # does not depend on the host it was made on.
    cmd = [os.environ.get("CC", "gcc"), "-x", "c", "-O3", "-funroll-loops", "-fPIC", "-shared", "-pthread",
           "-", "-o", tmp, "-lm"]
    subprocess.run(cmd, input=src.encode(), check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build_ssd_ref(sys.argv[1] if len(sys.argv) > 1 else DEFAULT_REFERENCE)
    print(path or "no reference tree: nothing built")
