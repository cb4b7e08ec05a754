"""MI355X (gfx950) fused tANS FP8 decode: drop-in for the reference's
``rans_vectoradd`` package (rans_vectoradd/__init__.py:1-18)."""
from rans_vectoradd._C import (
    fp8_gemm_fused_tans,
    fp8_gemm_raw,
    fp8_memcpy,
    fp8_vecadd_fused_tans,
    fp8_vecadd_raw,
    gpu_tans_decode,
)
from rans_vectoradd.data import QWEN3_14B_FP8_EXP, random_fp8_bytes
from . import tans_codec

__all__ = [
    "QWEN3_14B_FP8_EXP",
    "fp8_gemm_fused_tans",
    "fp8_gemm_raw",
    "fp8_memcpy",
    "fp8_vecadd_fused_tans",
    "fp8_vecadd_raw",
    "gpu_tans_decode",
    "random_fp8_bytes",
    "tans_codec",
]
