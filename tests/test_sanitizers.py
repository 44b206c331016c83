"""The host code of libxp and the oracle's C decoder under the sanitizers.

The SSD request server (ssd.cpp) runs the CPU server tests under
ThreadSanitizer; the server, the host encoder (codec_host.cpp) and the
oracle's C decoder (codec_ref.c) run the CPU codec and server tests under
AddressSanitizer with UndefinedBehaviorSanitizer. Each sanitizer build is a
host-only library (no HIP), loaded by a child pytest through
VLLM_EXPERT_PAGER_LIBRARY / XP_ORACLE_LIBRARY with the sanitizer runtime
preloaded into the interpreter. Python and numpy are not instrumented, so
ThreadSanitizer checks the server's own threads against each other (the
worker pool, the poller, the stop path), not the test thread that plays the
GPU side of the ring.
"""

import importlib.util
import os
import shutil
import subprocess
import sys

import pytest

from oracle import codec_ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "vllm-expert-pager_amd", "csrc")


def _runtime(name):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not installed")
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip(f"{name} is not installed")
    return path


def _build_module():
    spec = importlib.util.spec_from_file_location("xp_build", os.path.join(CSRC, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _run(env_extra, tests):
    env = dict(os.environ)
    env.update(env_extra)
    # -s: a report ends the child at once, and would be lost inside pytest's
    # capture of the failing test.
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-s", "-p", "no:cacheprovider", *tests],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0 and "Sanitizer" not in r.stderr, (
        f"status {r.returncode}\n{r.stderr[-8000:]}\n{r.stdout[-3000:]}")
    return r.stdout


def _loaded(env_extra, runtime):
    """The child interpreter really maps the sanitizer runtime."""
    env = dict(os.environ)
    env.update(env_extra)
    code = "print(open('/proc/self/maps').read().count(%r) > 0)" % os.path.basename(runtime)
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    return out.stdout.strip() == "True"


def test_ssd_server_under_thread_sanitizer(tmp_path):
    tsan = _runtime("libtsan.so")
    lib = _build_module().build_host_sanitized("thread", str(tmp_path / "lib"))
    env = {
        "VLLM_EXPERT_PAGER_LIBRARY": lib,
        "LD_PRELOAD": tsan,
        "TSAN_OPTIONS": "halt_on_error=1 ignore_noninstrumented_modules=1",
        "XP_SSD_TEST_OWN_ONLY": "1",
    }
    assert _loaded(env, tsan)
    out = _run(env, ["tests/test_ssd_cpu.py"])
    assert "passed" in out


def test_host_codec_server_and_oracle_under_address_sanitizer(tmp_path):
    asan = _runtime("libasan.so")
    lib = _build_module().build_host_sanitized("address", str(tmp_path / "lib"))
    oracle = codec_ref.build_lib(str(tmp_path / "liboracle.so"), sanitize=True)
    env = {
        "VLLM_EXPERT_PAGER_LIBRARY": lib,
        "XP_ORACLE_LIBRARY": oracle,
        "LD_PRELOAD": asan,
        # The interpreter's own allocations outlive the run by design.
        "ASAN_OPTIONS": "detect_leaks=0",
        "UBSAN_OPTIONS": "halt_on_error=1 print_stacktrace=1",
        "XP_SSD_TEST_OWN_ONLY": "1",
    }
    assert _loaded(env, asan)
    out = _run(env, ["tests/test_oracle_codec.py", "tests/test_ssd_cpu.py"])
    assert "passed" in out
