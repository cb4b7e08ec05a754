"""ctypes binding of libtans_amd.so (the C ABI in include/tans_amd.h).

The library is built in-tree by ``tans-vectoradd_amd/build.py``.  There is no
fallback: importing the package without the built library raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtans_amd.so")

# every symbol include/tans_amd.h declares
EXPORTS = (
    "tans_last_error",
    "tans_split_fp8",
    "tans_build_decode_table",
    "tans_encode_begin",
    "tans_encode_finish",
    "tans_encode_free",
    "tans_encode_packed_begin",
    "tans_fp8_memcpy",
    "tans_fp8_vecadd_raw",
    "tans_stream_probe",
    "tans_build_decode_table_device",
    "tans_fp8_vecadd_fused",
    "tans_decode",
    "tans_fp8_gemm_fused",
    "tans_fp8_gemm_fused_noalloc",
    "tans_fp8_gemm_raw",
    "tans_build_encode_table",
    "tans_gpu_encode_workspace",
    "tans_gpu_encode_begin",
    "tans_gpu_encode_finish",
    "tans_gpu_encode_packed_begin",
    "tans_gpu_encode_packed_finish",
)

TANS_LANES = 64
TANS_TILE = 16
TANS_GEMM_MAX_BATCH = 8
TANS_GEMM_MAX_SEG_COLS = 1024
TANS_PAIR_LOG2L = 12
TANS_NIBBLE_LOG2L = 11
TANS_PACKED_MAX_N = 64     # the packed layout's longest lane (pair alphabet)

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"rans_vectoradd: native library not built ({LIB_PATH} missing); "
        "run `python tans-vectoradd_amd/build.py` or __graft_entry__.build()")

lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32

lib.tans_last_error.restype = ctypes.c_char_p
lib.tans_last_error.argtypes = []
for _name, _args in {
    "tans_split_fp8": [_P, _I64, _I64, _I32, _P, _P],
    "tans_build_decode_table": [_P, _P, _I32, _I32, _P],
    "tans_encode_begin": [_P, _I64, _I64, _P, _I32, _P, _I32, ctypes.POINTER(_P),
                          ctypes.POINTER(_I64), ctypes.POINTER(_I64)],
    "tans_encode_packed_begin": [_P, _I64, _I64, _P, _I32, _P, _I32, ctypes.POINTER(_P),
                                 ctypes.POINTER(_I64), ctypes.POINTER(_I64)],
    "tans_encode_finish": [_P, _P, _P, _P],
    "tans_fp8_memcpy": [_P, _P, _I64, _P],
    "tans_fp8_vecadd_raw": [_P, _P, _P, _I64, _P],
    "tans_stream_probe": [_I32, _I32, _P, _P, _P, _I64, _P, _P],
    "tans_build_decode_table_device": [_P, _P, _I32, _I32, _P, _P, _P],
    "tans_fp8_vecadd_fused": [_P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I32,
                              _I64, _I64, _P, _P],
    "tans_decode": [_P, _I64, _P, _P, _P, _P, _I32, _I64, _I64, _P, _P],
    "tans_fp8_gemm_fused": [_P, _I64, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P, _I64,
                            ctypes.c_float, _P, _I64, _P, _P],
    "tans_fp8_gemm_fused_noalloc": [_P, _I64, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P,
                                    _I64, ctypes.c_float, _P, _P],
    "tans_fp8_gemm_raw": [_P, _I64, _I64, _P, _I64, ctypes.c_float, _P, _P],
    "tans_build_encode_table": [_P, _P, _I32, _I32, _P, _P],
    "tans_gpu_encode_workspace": [_I64, _I64, _I32, ctypes.POINTER(_I64)],
    "tans_gpu_encode_begin": [_P, _I64, _I64, _P, _P, _I32, _P, _I64, _P, _P, _P, _P, _P],
    "tans_gpu_encode_finish": [_I64, _I64, _I32, _P, _P, _P, _I64, _P],
    "tans_gpu_encode_packed_begin": [_P, _I64, _I64, _P, _P, _I32, _P, _I64, _P, _P, _P, _P],
    "tans_gpu_encode_packed_finish": [_I64, _I64, _I32, _P, _P, _P, _I64, _P],
}.items():
    getattr(lib, _name).restype = ctypes.c_int
    getattr(lib, _name).argtypes = _args
lib.tans_encode_free.restype = None
lib.tans_encode_free.argtypes = [_P]


def check(rc: int, what: str) -> None:
    """Raise RuntimeError (the reference's TORCH_CHECK behaviour) on failure."""
    if rc != 0:
        msg = lib.tans_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
