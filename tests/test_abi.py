"""The C ABI boundary, CPU only: the library loads, exports every function
include/tans_amd.h declares, and rejects bad arguments before any GPU work
(the reference's TORCH_CHECKs, csrc/vecadd.cu:269-337, become TANS_EINVAL
here and RuntimeError in the Python layer)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tans_amd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+[\s\*]+(tans_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function():
    from rans_vectoradd import _lib
    names = header_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(_lib.lib, n), n
    assert sorted(_lib.EXPORTS) == names


def _rc(fn, *args):
    return fn(*args)


def test_gpu_entry_points_validate_before_launch():
    from rans_vectoradd._lib import lib
    P = ctypes.c_void_p
    dummy = P(16)
    assert lib.tans_fp8_vecadd_raw(dummy, dummy, dummy, 17, None) == -1
    assert b"multiple of 16" in lib.tans_last_error()
    assert lib.tans_fp8_memcpy(dummy, dummy, -16, None) == -1
    assert lib.tans_fp8_vecadd_raw(None, dummy, dummy, 16, None) == -1
    # zero-length work is a no-op that succeeds without touching the device
    assert lib.tans_fp8_vecadd_raw(dummy, dummy, dummy, 0, None) == 0
    assert lib.tans_fp8_vecadd_fused(dummy, 1024, dummy, dummy, dummy, dummy, 1024, dummy, dummy,
                                     dummy, dummy, 10, 64, 16, dummy, None) == -1
    assert b"log2L" in lib.tans_last_error()
    assert lib.tans_fp8_vecadd_fused(dummy, 1024, dummy, dummy, dummy, dummy, 1024, dummy, dummy,
                                     dummy, dummy, 12, 64, 24, dummy, None) == -1
    assert lib.tans_fp8_vecadd_fused(dummy, 1022, dummy, dummy, dummy, dummy, 1024, dummy, dummy,
                                     dummy, dummy, 12, 64, 16, dummy, None) == -1
    assert lib.tans_decode(dummy, 1024, dummy, dummy, dummy, dummy, 12, 64, 3, dummy, None) == -1
    assert lib.tans_decode(dummy, 1024, dummy, dummy, dummy, dummy, 12, 0, 16, dummy, None) == 0
    assert lib.tans_build_decode_table_device(dummy, dummy, 16, 12, dummy, None) == -1


def test_python_api_rejects_cpu_and_mismatched_tensors():
    import rans_vectoradd as R
    a = torch.zeros(32, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="CUDA"):
        R.fp8_vecadd_raw(a, a)
    with pytest.raises(RuntimeError, match="CUDA"):
        R.fp8_memcpy(a)
    t = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(RuntimeError):
        R.gpu_tans_decode(a, t, t, a, a, t, t, 16)
    with pytest.raises(RuntimeError):
        R.fp8_vecadd_fused_tans(a, t, t, a, a, a, t, t, a, a, t, 16)


def test_host_table_builder_rejects_inconsistent_input():
    from rans_vectoradd import tans_codec as T
    f = T.symbol_freqs((1.0,) * 16, "nibble")
    sp = T.build_spread(f)
    with pytest.raises(RuntimeError):
        T.build_decode_table(sp[:1024], f)          # wrong table size
    bad = sp.copy()
    bad[3] = 40
    with pytest.raises(RuntimeError):
        T.build_decode_table(bad, f)                # symbol out of range
