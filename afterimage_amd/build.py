"""Build libafterimage_decode.so in-tree for gfx950.

The device code is compiled by hipcc; the shared object is linked against the
HIP runtime that ships inside the installed PyTorch, so that a Python process
which has imported torch holds a single HIP runtime and torch's streams and
device pointers are valid in this library's launches.

Run as ``python -m afterimage_amd.build``; ``__graft_entry__.build()`` calls
:func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB_NAME = "libafterimage_decode.so"
LIB_PATH = PKG / LIB_NAME

ARCH = "gfx950"
# hipcc-only flags. Packed FP32 instructions are switched off for all device
# code (the host pass warns that it does not know the feature; harmless).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-pthread"]


def _torch_lib_dir() -> Path:
    import torch  # noqa: F401  (only to locate its lib directory)

    return Path(torch.__file__).resolve().parent / "lib"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the decoder needs ROCm's hipcc to build")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("build step failed:\n  %s\n%s%s"
                           % (" ".join(cmd), proc.stdout, proc.stderr))


def build(verbose: bool = False) -> Path:
    """Compile the HIP kernels and host code and link the shared library."""
    BUILD_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    inc = ["-I", str(INCLUDE), "-I", str(CSRC)]
    dev_obj = BUILD_DIR / "aimg_decode.o"
    host_obj = BUILD_DIR / "aimg_host.o"
    cpu_obj = BUILD_DIR / "aimg_cpu.o"
    steps = [
        [hipcc, "-c", *HIP_FLAGS, *inc, str(CSRC / "aimg_decode.hip"), "-o", str(dev_obj)],
        ["g++", "-c", *HOST_FLAGS, *inc, str(CSRC / "aimg_host.cpp"), "-o", str(host_obj)],
        ["g++", "-c", *HOST_FLAGS, *inc, str(CSRC / "aimg_cpu.cpp"), "-o", str(cpu_obj)],
    ]
    torch_lib = _torch_lib_dir()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    steps.append(["g++", "-shared", "-pthread", "-o", str(tmp), str(dev_obj), str(host_obj),
                  str(cpu_obj), f"-L{torch_lib}", "-l:libamdhip64.so", "-Wl,--no-undefined"])
    for cmd in steps:
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
