"""The C-ABI library loads and exports every entry point include/sigcomp_hip.h
declares (no compute calls: this runs without a GPU)."""

import ctypes
import re

import pytest

from conftest import REPO

HEADER = REPO / "include" / "sigcomp_hip.h"
LIB = REPO / "sigcomp_amd" / "libsigcomp_hip.so"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(sc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("sc_model_create", "sc_compress_chunks", "sc_decompress_chunks",
                 "sc_mlp_forward", "sc_encode_step", "sc_decode_step"):
        assert must in names


@pytest.mark.skipif(not LIB.exists(), reason="libsigcomp_hip.so not built")
def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (same HIP runtime as the product loader)
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    lib.sc_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.sc_version()


@pytest.mark.skipif(not LIB.exists(), reason="libsigcomp_hip.so not built")
def test_python_binding_matches_header():
    from sigcomp_amd import _hip
    assert sorted(_hip.EXPORTED) == declared_functions()
    _hip.lib()
