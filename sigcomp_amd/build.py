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
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libsigcomp_hip.so"
# Translation units of libsigcomp_hip.so as (source, defines): the large MLP
# kernels are split over several units so that they compile in parallel.
UNITS = [(CSRC / "sc_kernels.hip", ()), (CSRC / "sc_comp.hip", ()), (CSRC / "sc_gen.hip", ()),
         (CSRC / "sc_dec_split.hip", ()),
         (CSRC / "sc_ctx.hip", ("SC_CTX_MODE=0",)), (CSRC / "sc_ctx.hip", ("SC_CTX_MODE=1",)),
         *[(CSRC / "sc_dec.hip", (f"SC_DEC_RT={rt}",)) for rt in range(1, 6)]]
SOURCES = sorted({src for src, _ in UNITS})
HOST_LIB = PKG / "libsigcomp_host.so"
HOST_SOURCES = [CSRC / "sc_host.cpp"]
HOST_FLAGS = ["-O3", "-march=x86-64-v3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra",
              f"-I{REPO / 'include'}"]
HEADERS = [CSRC / "sc_device.h", CSRC / "sc_pipe.h", CSRC / "sc_kernels.h", CSRC / "sc_gen.h",
           REPO / "include" / "sigcomp_hip.h"]
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


def _unit_obj(tmp: Path, i: int, src: Path, defines) -> Path:
    return tmp / f"{i:02d}_{src.stem}{''.join('_' + d.split('=')[-1] for d in defines)}.o"


def build(verbose: bool = False, extra_flags=()) -> Path:
    """Compile every translation unit (in parallel) and link the library."""
    build_host(verbose)
    with tempfile.TemporaryDirectory(prefix="sc_build_") as td:
        tmp = Path(td)
        compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
        cmds = []
        for i, (src, defines) in enumerate(UNITS):
            obj = _unit_obj(tmp, i, src, defines)
            cmds.append([hipcc(), *compile_flags, *extra_flags, *[f"-D{d}" for d in defines], "-c", str(src),
                         "-o", str(obj)])
        jobs = max(1, min(len(cmds), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            results = list(pool.map(lambda c: (c, subprocess.run(c, capture_output=True, text=True)), cmds))
        for cmd, res in results:
            if verbose:
                print(" ".join(cmd), flush=True)
            if res.returncode != 0:
                sys.stderr.write(res.stdout + res.stderr)
                raise RuntimeError(f"hipcc failed for {cmd[-3]}")
        out = LIB.with_suffix(".so.tmp")
        link = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *extra_flags,
                *[str(_unit_obj(tmp, i, s, d)) for i, (s, d) in enumerate(UNITS)], "-o", str(out)]
        res = subprocess.run(link, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError("hipcc link failed for libsigcomp_hip.so")
        os.replace(out, LIB)
    return LIB


def device_asm(out_path: Path) -> Path:
    """Write the gfx950 assembly of every translation unit of the library,
    concatenated (for resource / ISA checks)."""
    flags = [f for f in HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    with tempfile.TemporaryDirectory(prefix="sc_asm_") as td:
        tmp = Path(td)
        cmds = [[hipcc(), *flags, *[f"-D{d}" for d in defines], "--cuda-device-only", "-S", str(src), "-o",
                 str(_unit_obj(tmp, i, src, defines).with_suffix(".s"))] for i, (src, defines) in enumerate(UNITS)]
        with ThreadPoolExecutor(max_workers=max(1, min(len(cmds), os.cpu_count() or 1, 16))) as pool:
            for res in pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds):
                if res.returncode != 0:
                    raise RuntimeError(res.stderr)
        out_path.write_text("".join(Path(c[-1]).read_text() for c in cmds))
    return out_path


if __name__ == "__main__":
    print(build(verbose=True))
