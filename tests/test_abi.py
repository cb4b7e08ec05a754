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
    assert lib.tans_build_decode_table_device(dummy, dummy, 16, 12, dummy, None, None) == -1
    assert lib.tans_stream_probe(3, 1, dummy, dummy, dummy, 16, dummy, None) == -1
    assert b"mode" in lib.tans_last_error()
    assert lib.tans_stream_probe(2, 1, dummy, None, dummy, 16, None, None) == -1
    assert lib.tans_stream_probe(0, 1, dummy, None, None, 16, None, None) == -1    # no sink
    assert lib.tans_stream_probe(1, 0, None, None, dummy, 24, None, None) == -1
    assert lib.tans_stream_probe(1, 0, None, None, None, 0, None, None) == 0


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


def test_nibble_tables_need_frequencies_of_two():
    """2^11-state tables are decoded three steps per 32-bit window, so every
    present symbol needs f >= 2 (nb <= 10): the host table builders and the
    CPU encoder reject a frequency of 1; symbol_freqs floors it."""
    import numpy as np
    from rans_vectoradd import _C, tans_codec as T
    f = np.full(16, 128, dtype=np.int32)
    f[0], f[1] = 1, 255                             # sums to 2048, one symbol at 1
    sp = T.build_spread(f)
    with pytest.raises(RuntimeError, match=">= 2"):
        T.build_decode_table(sp, f)
    sym = torch.zeros((64, 16), dtype=torch.uint8)
    with pytest.raises(RuntimeError, match=">= 2"):
        _C.tans_encode_interleaved(sym, torch.from_numpy(f), torch.from_numpy(sp))
    hist = np.full(16, 1000.0)
    hist[0] = 0.1                                    # far below 1/2048: quantized to 1
    g = T.symbol_freqs(hist, "nibble")
    assert g.sum() == 2048 and g.min() >= 2


def test_gemm_and_gpu_encode_entry_points_validate_before_launch():
    """The decode-GEMM, raw GEMM and GPU encoder entry points reject bad
    shapes and sizes with TANS_EINVAL before touching the device."""
    from rans_vectoradd._lib import lib
    P = ctypes.c_void_p
    d = P(256)
    f = ctypes.c_float(1.0)
    # gemm_fused(comp, bytes, off, st, sm, tbl, log2L, R, C, S, Nc, x, B, scale, ws, ws_bytes, y, stream)
    ok = (d, 1024, d, d, d, d, 12, 128, 100, 2, 64, d, 1, f, d, 1 << 20, d, None)
    bad = [
        dict(i=6, v=10),            # log2L
        dict(i=12, v=9),            # batch > 8
        dict(i=12, v=0),            # batch < 1
        dict(i=10, v=48),           # segment width not a multiple of 32
        dict(i=10, v=1056),         # segment width above 1024
        dict(i=14, v=P(260)),       # workspace not 16-byte aligned
        dict(i=9, v=1),             # S * Nc < C
        dict(i=9, v=3),             # (S - 1) * Nc >= C
        dict(i=15, v=16),           # workspace too small
        dict(i=1, v=1022),          # compressed size not a multiple of 4
    ]
    for case in bad:
        args = list(ok)
        args[case["i"]] = case["v"]
        assert lib.tans_fp8_gemm_fused(*args) == -1, case
    assert lib.tans_fp8_gemm_raw(d, 128, 100, d, 1, f, d, None) == -1     # C % 16
    assert lib.tans_fp8_gemm_raw(d, 128, 96, d, 9, f, d, None) == -1      # batch
    ws = ctypes.c_int64()
    assert lib.tans_gpu_encode_workspace(64, 15, 12, ctypes.byref(ws)) == -1
    assert lib.tans_gpu_encode_workspace(64, 16, 10, ctypes.byref(ws)) == -1
    assert lib.tans_gpu_encode_workspace(64, 16, 12, ctypes.byref(ws)) == 0 and ws.value > 0
    assert lib.tans_gpu_encode_begin(d, 64, 16, d, d, 12, d, 16, d, d, d, d, None) == -1
    assert b"workspace" in lib.tans_last_error()
    assert lib.tans_gpu_encode_finish(64, 16, 12, d, d, d, 100, None) == -1


def test_host_encode_table_matches_its_definition():
    """enc_tab[s] = f_s | start_s << 16 and enc_next[start_s + rank] = L +
    slot of the rank-th occurrence of s in slot order."""
    import numpy as np
    from rans_vectoradd import data as D, tans_codec as T
    from rans_vectoradd._lib import lib
    f = T.symbol_freqs(D.QWEN3_14B_FP8_EXP, "nibble")
    sp = T.build_spread(f)
    tab = np.empty(16, dtype=np.uint32)
    nxt = np.empty(2048, dtype=np.uint16)
    assert lib.tans_build_encode_table(sp.ctypes.data, f.ctypes.data, 16, 11, tab.ctypes.data,
                                       nxt.ctypes.data) == 0
    start = np.concatenate([[0], np.cumsum(f)[:-1]])
    assert np.array_equal(tab & 0xFFFF, f) and np.array_equal(tab >> 16, start)
    for s in range(16):
        slots = np.nonzero(sp == s)[0]
        assert np.array_equal(nxt[start[s]:start[s] + f[s]], 2048 + slots)
    bad = sp.copy()
    bad[0] = 99
    assert lib.tans_build_encode_table(bad.ctypes.data, f.ctypes.data, 16, 11, tab.ctypes.data,
                                       nxt.ctypes.data) != 0


def test_misaligned_buffers_are_rejected_before_launch():
    from rans_vectoradd._lib import lib
    P = ctypes.c_void_p
    d, m = P(4096), P(4097 + 1)          # 16-byte aligned, 2 mod 16
    assert lib.tans_fp8_vecadd_raw(m, d, d, 16, None) == -1
    assert b"aligned" in lib.tans_last_error()
    assert lib.tans_fp8_memcpy(d, m, 16, None) == -1
    assert lib.tans_fp8_vecadd_fused(m, 1024, d, d, d, d, 1024, d, d, d, d, 12, 64, 16, d, None) == -1
    assert lib.tans_decode(m, 1024, d, d, d, d, 12, 64, 16, d, None) == -1
    f = ctypes.c_float(1.0)
    assert lib.tans_fp8_gemm_raw(d, 128, 96, m, 1, f, d, None) == -1
