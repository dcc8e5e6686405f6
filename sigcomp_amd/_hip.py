"""ctypes binding of libsigcomp_hip.so (C ABI: include/sigcomp_hip.h).

torch is imported first so that the library's libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded (same soname): device
pointers and streams are then shared with torch.  There is no fallback: if
the library is missing or no GPU is present, these calls raise.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "libsigcomp_hip.so"

SC_OK = 0
SC_ERR_ARG = 1
SC_ERR_HIP = 2
SC_ERR_UNSUPPORTED = 3
SC_STATUS_OK = 0
SC_STATUS_CAPACITY = 1
SC_STATUS_INVALID_STREAM = 2
SC_STATUS_BAD_TOKEN = 3
SC_STATUS_SYNC_TIMEOUT = 4

EXPORTED = (
    "sc_last_error", "sc_version", "sc_model_create", "sc_model_destroy", "sc_model_lut",
    "sc_model_core",
    "sc_mlp_forward", "sc_mlp_forward_cdf", "sc_logits_to_cdf", "sc_encode_step",
    "sc_encode_seal", "sc_decode_step", "sc_compress_workspace_bytes", "sc_compress_chunks",
    "sc_decompress_workspace_bytes", "sc_decompress_chunks", "sc_decompress_chunks_opts",
    "sc_decompress_chunks_static",
    "sc_gather_words", "sc_mfma_burn_i8",
)

# sc_decompress_chunks_opts options
SC_DEC_OPT_NO_SPLIT = 1

# chunks per sc_decompress_chunks_static call (SC_STATIC_DEC_MAX_CHUNKS)
STATIC_DEC_MAX_CHUNKS = 65536


class LayerDesc(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int32), ("k", ctypes.c_int32),
                ("weight", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("m0", ctypes.c_void_p), ("shift", ctypes.c_void_p),
                ("relu", ctypes.c_int32)]


class EncoderState(ctypes.Structure):
    _fields_ = [("lower", ctypes.c_void_p), ("range", ctypes.c_void_p),
                ("inverted", ctypes.c_void_p), ("first", ctypes.c_void_p),
                ("write_pos", ctypes.c_void_p), ("status", ctypes.c_void_p)]


class DecoderState(ctypes.Structure):
    _fields_ = [("lower", ctypes.c_void_p), ("range", ctypes.c_void_p),
                ("point", ctypes.c_void_p), ("read_pos", ctypes.c_void_p),
                ("end_pos", ctypes.c_void_p), ("status", ctypes.c_void_p)]


class HipError(RuntimeError):
    pass


_LIB = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


def lib():
    """Load the library (raises if it was not built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise HipError(f"{LIB_PATH} is missing; build it with `python -m sigcomp_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        L.sc_last_error.restype = ctypes.c_char_p
        L.sc_version.restype = ctypes.c_char_p
        L.sc_model_create.argtypes = [_P, _I32, _I32, _I32, ctypes.POINTER(LayerDesc), _I32, _P,
                                      _I32, ctypes.POINTER(_P)]
        L.sc_model_destroy.argtypes = [_P]
        L.sc_model_lut.argtypes = [_P]
        L.sc_model_lut.restype = _P
        L.sc_model_core.argtypes = [_P]
        L.sc_mlp_forward.argtypes = [_P, _P, _I64, _P, _P, _P]
        L.sc_mlp_forward_cdf.argtypes = [_P, _P, _I64, _P, _P, _P]
        L.sc_logits_to_cdf.argtypes = [_P, _I64, _P, _P, _P]
        L.sc_encode_step.argtypes = [_P, _P, _P, _P, _I64, _I64, ctypes.POINTER(EncoderState), _P,
                                     _I64, _P]
        L.sc_encode_seal.argtypes = [_I64, ctypes.POINTER(EncoderState), _P, _I64, _P]
        L.sc_decode_step.argtypes = [_P, _P, _P, _I64, _I64, ctypes.POINTER(DecoderState), _P, _P,
                                     _P]
        L.sc_compress_workspace_bytes.argtypes = [_I64, _I64]
        L.sc_compress_workspace_bytes.restype = _I64
        L.sc_compress_chunks.argtypes = [_P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64,
                                         _P]
        L.sc_decompress_workspace_bytes.argtypes = [_I64]
        L.sc_decompress_workspace_bytes.restype = _I64
        L.sc_decompress_chunks.argtypes = [_P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P]
        L.sc_decompress_chunks_opts.argtypes = [_P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _I32, _P]
        L.sc_decompress_chunks_static.argtypes = [_P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P]
        L.sc_gather_words.argtypes = [_P, _P, _P, _I64, _P, _P, _P]
        L.sc_mfma_burn_i8.argtypes = [_P, _I32, _I32, _P, _P]
        for name in EXPORTED:
            fn = getattr(L, name)
            if fn.restype is None or fn.restype is ctypes.c_int:
                if name not in ("sc_model_lut", "sc_compress_workspace_bytes",
                                "sc_decompress_workspace_bytes"):
                    fn.restype = ctypes.c_int
        _LIB = L
    return _LIB


def check(rc: int) -> None:
    if rc != SC_OK:
        raise HipError(lib().sc_last_error().decode(errors="replace") or f"sigcomp HIP error {rc}")


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return t.data_ptr() if t is not None else 0
