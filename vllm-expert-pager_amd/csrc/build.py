"""Build libxp.so (gfx950 HIP kernels + host C++) next to the Python package.

Usage: python build.py [--jobs N] [--verbose]

GPU sources (*.hip) are compiled with hipcc for gfx950 only; host sources
(*.cpp) with g++ (hipcc for the one that calls the HIP runtime). Objects go
to csrc/_build/, the library to vllm_expert_pager/libxp.so.
"""

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "vllm_expert_pager")
OUT = os.path.join(PKG, "libxp.so")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")

# Packed FP32 VALU forms are turned off for every GPU translation unit.
GPU_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs, so the block-scale FMAs read them directly
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-pthread"]

GPU_SOURCES = ["table.hip", "gather.hip", "codec.hip", "encode.hip", "moe.hip", "scratch.hip"]
HIP_HOST_SOURCES = ["host.cpp", "codec_host.cpp"]  # HIP runtime API or headers
HOST_SOURCES = ["error.cpp", "ssd.cpp", "ssd_probe.cpp", "table_host.cpp"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning
    # is expected and dropped.
    err = "\n".join(
        line for line in r.stderr.splitlines() if "packed-fp32-ops" not in line
    ).strip()
    if r.returncode:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err and verbose:
        print(err, file=sys.stderr)


def build(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cmds = []
    objs = []
    for src in GPU_SOURCES:
        if not os.path.exists(os.path.join(HERE, src)):
            continue
        obj = os.path.join(BUILD, src + ".o")
        cmds.append([HIPCC, *GPU_FLAGS, "-c", os.path.join(HERE, src), "-o", obj])
        objs.append(obj)
    for src in HIP_HOST_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        cmds.append(
            [HIPCC, "-O3", "-std=c++17", "-fPIC", "-Wall", "-x", "c++",
             "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", "-c",
             os.path.join(HERE, src), "-o", obj]
        )
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        cmds.append(["g++", *HOST_FLAGS, "-c", os.path.join(HERE, src), "-o", obj])
        objs.append(obj)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = OUT + f".tmp{os.getpid()}"
    _run(
        [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
         "-pthread", f"-L{ROCM}/lib", "-lamdhip64"],
        verbose,
    )
    os.replace(tmp, OUT)
    return OUT


def build_host_sanitized(kind: str, out_dir: str, verbose: bool = False) -> str:
    """The host-only part of libxp (host encoder, code construction, SSD
    server: no HIP) built with a sanitizer (``address`` -- with
    UndefinedBehaviorSanitizer -- or ``thread``) into out_dir/libxp.so, for
    the CPU tests to load through VLLM_EXPERT_PAGER_LIBRARY with the
    sanitizer's runtime preloaded. GPU entry points are absent from it."""
    flags = {"address": ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"],
             "thread": ["-fsanitize=thread"]}[kind]
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libxp.so")
    srcs = [os.path.join(HERE, s) for s in ("error.cpp", "codec_host.cpp", "ssd.cpp", "ssd_probe.cpp")]
    # code_build.h marks its functions __host__ __device__: the HIP headers
    # define those away for a host compiler.
    _run(["g++", "-O1", "-g", "-fno-omit-frame-pointer", "-std=c++17", "-fPIC", "-shared", "-pthread", *flags,
          f"-I{ROCM}/include", "-D__HIP_PLATFORM_AMD__", *srcs, "-o", out], verbose)
    return out


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    p.add_argument("--verbose", action="store_true")
    p.add_argument("--sanitize", choices=["address", "thread"],
                   help="build only the host part, with this sanitizer, into csrc/_build/san-<kind>/")
    a = p.parse_args()
    if a.sanitize:
        print(build_host_sanitized(a.sanitize, os.path.join(BUILD, f"san-{a.sanitize}"), a.verbose))
        return
    print(build(a.jobs, a.verbose))


if __name__ == "__main__":
    main()
