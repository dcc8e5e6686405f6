"""Build the package's native libraries in-tree.

    python -m sigcomp_amd.build

* libsigcomp_hip.so (gfx950, hipcc): the GPU codec, C ABI in
  include/sigcomp_hip.h; loaded with ctypes after torch so that both share
  torch's HIP runtime.
* libsigcomp_host.so (g++): the host stages either side of it (signal split /
  reassembly, SIG2 chunk framing), C ABI in include/sigcomp_host.h.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libsigcomp_hip.so"
SOURCES = [CSRC / "sc_kernels.hip"]
HOST_LIB = PKG / "libsigcomp_host.so"
HOST_SOURCES = [CSRC / "sc_host.cpp"]
HOST_FLAGS = ["-O3", "-march=x86-64-v3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra",
              f"-I{REPO / 'include'}"]
HEADERS = [CSRC / "sc_device.h", REPO / "include" / "sigcomp_hip.h"]
ARCH = os.environ.get("SIGCOMP_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{REPO / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (Path(cand).exists() or cand == "hipcc"):
            return cand
    raise RuntimeError("hipcc not found")


def build_host(verbose: bool = False) -> Path:
    tmp = HOST_LIB.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), *HOST_FLAGS, *map(str, HOST_SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("g++ failed for libsigcomp_host.so")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build(verbose: bool = False, extra_flags=()) -> Path:
    build_host(verbose)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra_flags, *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed for libsigcomp_hip.so")
    os.replace(tmp, LIB)
    return LIB


def device_asm(out_path: Path) -> Path:
    """Write the gfx950 assembly of the library (for resource / ISA checks)."""
    cmd = [hipcc(), *[f for f in HIPCC_FLAGS if f not in ("-shared", "-fPIC")],
           "--cuda-device-only", "-S", *map(str, SOURCES), "-o", str(out_path)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out_path


if __name__ == "__main__":
    print(build(verbose=True))
