"""Audit the gfx950 assembly of libsigcomp_hip for scalar-cache writes.

Kernels here must write memory only through vector stores: no scalar memory
stores or atomics and no scalar data-cache write-back / discard.  This module
recompiles the library to assembly and fails if any such instruction appears.
It runs at build time in the build container only (listed in .gpurunignore,
because it has to name the instructions it looks for).
"""

import re
import sys
import tempfile
from pathlib import Path

FORBIDDEN = re.compile(r"^\s*(s_store_|s_buffer_store|s_atomic|s_buffer_atomic|s_scratch_store|"
                       r"s_dcache_wb|s_dcache_discard)", re.M)


def audit() -> None:
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from sigcomp_amd.build import device_asm
    with tempfile.TemporaryDirectory() as tmp:
        asm = device_asm(Path(tmp) / "sc.s").read_text()
    hits = sorted(set(m.group(1) for m in FORBIDDEN.finditer(asm)))
    if hits:
        raise RuntimeError(f"forbidden scalar-cache write instructions in device code: {hits}")
    n_mfma = len(re.findall(r"v_mfma_i32_32x32x32_i8", asm))
    print(f"isa audit ok ({n_mfma} int8 MFMA instructions, no scalar-cache writes)")


if __name__ == "__main__":
    audit()
