"""Python face of the CPU oracle.  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker (or the timed CPU baseline).
The shipped package never imports it.

Pure-numpy restatements of the reference's Python table builders:

* ``quantize_freqs``      rans_vectoradd/tans_codec.py:30-46
* ``build_spread``        rans_vectoradd/tans_codec.py:49-60
* ``ref_decode_table``    rans_vectoradd/tans_codec.py:63-87
                          (= csrc/tans_decode.cu:23-59, the C++ twin)
* ``split_fp8`` / ``pair_symbols`` / sm packing
                          rans_vectoradd/tans_codec.py:109-124

plus ctypes bindings of ``oracle.c`` (FP8 add, reference-format codec, and the
wave64-layout checker), and of ``_ref/libref_codec.so`` where it is built: the
reference's own CPU encoder (csrc/tans_codec.cpp), compiled unmodified from the
reference tree (``make -C oracle ref``), the checker of ``ref_encode``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

REF_L = 4096
REF_BLOCK = 128


def build() -> None:
    """Compile oracle.c (gcc) into oracle/liboracle.so."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        _lib.ora_fp8_to_double.restype = ctypes.c_double
        _lib.ora_fp8_to_double.argtypes = [ctypes.c_uint8]
        _lib.ora_fp8_add.restype = ctypes.c_uint8
        _lib.ora_fp8_add.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
        _lib.ora_fp8_add_lut.argtypes = [P]
        _lib.ora_vecadd_lut.argtypes = [P, P, P, P, I64]
        _lib.ora_ref_encode_count.restype = I64
        _lib.ora_ref_encode_count.argtypes = [P, I64, I64, P, I, P, P]
        _lib.ora_ref_encode_write.restype = I
        _lib.ora_ref_encode_write.argtypes = [P, I64, I64, P, I, P, P, P, P, P, P]
        _lib.ora_ref_decode.restype = I
        _lib.ora_ref_decode.argtypes = [P, P, P, P, P, P, I64, I64, P]
        _lib.ora_set_threads.restype = None
        _lib.ora_set_threads.argtypes = [I]
        _lib.ora_ref_decode_add.restype = I
        _lib.ora_ref_decode_add.argtypes = [P] * 12 + [I64, I64, P]
        _lib.ora_w64_decode.restype = I
        _lib.ora_w64_decode.argtypes = [P, P, P, P, P, P, I, I, I, I64, I64, P]
        _lib.ora_packed_decode.restype = I
        _lib.ora_packed_decode.argtypes = [P, P, P, P, P, I64, I64, P]
    return _lib


REF_LIB_PATH = os.path.join(_HERE, "_ref", "libref_codec.so")
_ref_lib = None


def build_ref(ref_csrc: str = "/root/reference/csrc") -> bool:
    """Compile the reference's csrc/tans_codec.cpp with ref_harness.cpp into
    _ref/libref_codec.so when the reference tree is present; True if built."""
    if not os.path.exists(os.path.join(ref_csrc, "tans_codec.cpp")):
        return False
    subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REF={ref_csrc}"], check=True)
    return True


def ref_lib():
    """The compiled reference encoder, or None where it is not built."""
    global _ref_lib
    if _ref_lib is None and os.path.exists(REF_LIB_PATH):
        import torch  # noqa: F401  (loads libtorch's libraries the encoder links)
        lib_ = ctypes.CDLL(REF_LIB_PATH)
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        lib_.ref_encode.restype = P
        lib_.ref_encode.argtypes = [P, I64, I64, P, I64, P, I64, ctypes.POINTER(I64),
                                    ctypes.POINTER(I64)]
        lib_.ref_encode_copy.restype = None
        lib_.ref_encode_copy.argtypes = [P, P, P, P, P]
        lib_.ref_encode_free.restype = None
        lib_.ref_encode_free.argtypes = [P]
        lib_.ref_last_error.restype = ctypes.c_char_p
        lib_.ref_last_error.argtypes = []
        _ref_lib = lib_
    return _ref_lib


def reference_encode(symbols: np.ndarray, freqs, spread):
    """The reference's tans_encode_interleaved (csrc/tans_codec.cpp:69-196)
    itself -> (compressed u8, states u16[K], offsets i32, partial u8[K]);
    raises RuntimeError with the reference's message where it rejects the
    input."""
    lib_ = ref_lib()
    if lib_ is None:
        raise RuntimeError(f"{REF_LIB_PATH} is not built")
    symbols = np.ascontiguousarray(symbols, dtype=np.uint8)
    freqs = np.ascontiguousarray(freqs, dtype=np.int32)
    spread = np.ascontiguousarray(spread, dtype=np.int32)
    K, N = symbols.shape
    nb, no = ctypes.c_int64(), ctypes.c_int64()
    h = lib_.ref_encode(_p(symbols), K, N, _p(freqs), freqs.size, _p(spread), spread.size,
                        ctypes.byref(nb), ctypes.byref(no))
    if not h:
        raise RuntimeError(lib_.ref_last_error().decode(errors="replace"))
    try:
        comp = np.empty(nb.value, np.uint8)
        states = np.empty(K, np.uint16)
        offsets = np.empty(no.value, np.int32)
        partial = np.empty(K, np.uint8)
        lib_.ref_encode_copy(h, _p(comp), _p(states), _p(offsets), _p(partial))
    finally:
        lib_.ref_encode_free(h)
    return comp, states, offsets, partial


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


# --------------------------------------------------------------------------
# FP8 add
# --------------------------------------------------------------------------

def fp8_to_float64(b: np.ndarray) -> np.ndarray:
    """OCP E4M3FN bytes -> float64 (NaN for 0x7F/0xFF)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = b >> 7
    e = (b >> 3) & 0xF
    m = b & 7
    v = np.where(e == 0, np.ldexp(m.astype(np.float64), -9),
                 np.ldexp((8 + m).astype(np.float64), (e - 10).astype(np.int64)))
    v = np.where(s == 1, -v, v)
    return np.where((e == 15) & (m == 7), np.nan, v)


def add_lut() -> np.ndarray:
    """[256, 256] uint8: lut[a, b] = fp8(float(a) + float(b)), RNE, satfinite.
    Restates csrc/vecadd.cu:27-35 from the OCP spec; NaN -> 0x7F (unpinned)."""
    out = np.empty(65536, dtype=np.uint8)
    lib().ora_fp8_add_lut(_p(out))
    return out.reshape(256, 256)


def nan_mask_lut() -> np.ndarray:
    """[256, 256] bool: True where either operand is an E4M3FN NaN."""
    nan = (np.arange(256) & 0x7F) == 0x7F
    return nan[:, None] | nan[None, :]


def vecadd(lut: np.ndarray, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint8).ravel()
    b = np.ascontiguousarray(b, dtype=np.uint8).ravel()
    out = np.empty_like(a)
    lut = np.ascontiguousarray(lut, dtype=np.uint8)
    lib().ora_vecadd_lut(_p(lut), _p(a), _p(b), _p(out), a.size)
    return out


# --------------------------------------------------------------------------
# Table builders (numpy restatements)
# --------------------------------------------------------------------------

def quantize_freqs(probs, target: int) -> np.ndarray:
    """rans_vectoradd/tans_codec.py:30-46: round, floor 1 for p>0, then a
    greedy +-1 fix-up by largest error (first index wins ties)."""
    probs = np.asarray(probs, dtype=np.float64)
    f = np.maximum(np.round(probs * target).astype(np.int64), 1)
    f[probs == 0] = 0
    diff = int(target - f.sum())
    for _ in range(max(diff, 0)):
        err = probs * target - f
        err[probs == 0] = -np.inf
        f[int(np.argmax(err))] += 1
    for _ in range(max(-diff, 0)):
        err = f - probs * target
        err[(probs > 0) & (f <= 1)] = -np.inf
        f[int(np.argmax(err))] -= 1
    assert f.sum() == target
    return f.astype(np.int32)


def sigma(L: int) -> int:
    """Hash-walk stride, rans_vectoradd/tans_codec.py:26."""
    return (L >> 1) + (L >> 3) + 3


def build_spread(freqs, L: int) -> np.ndarray:
    """rans_vectoradd/tans_codec.py:49-60 (symbols in ascending order, each
    placed f_s times at stride SIGMA modulo L)."""
    freqs = np.asarray(freqs, dtype=np.int64)
    assert freqs.sum() == L
    spread = np.full(L, -1, dtype=np.int32)
    cur, st = 0, sigma(L)
    for s in range(len(freqs)):
        for _ in range(int(freqs[s])):
            assert spread[cur] == -1
            spread[cur] = s
            cur = (cur + st) % L
    assert (spread >= 0).all()
    return spread


def slot_table(spread, freqs, L: int):
    """Per slot: (symbol, nb, base) with x_prev = f_s + rank, nb = doublings
    of x_prev until >= L, base = x_prev << nb (tans_codec.py:73-86)."""
    spread = np.asarray(spread, dtype=np.int64)
    freqs = np.asarray(freqs, dtype=np.int64)
    counts = np.zeros(len(freqs), dtype=np.int64)
    sym = np.empty(L, np.int64)
    nb = np.empty(L, np.int64)
    base = np.empty(L, np.int64)
    for slot in range(L):
        s = int(spread[slot])
        xp = int(freqs[s] + counts[s])
        counts[s] += 1
        n = 0
        while (xp << n) < L:
            n += 1
        sym[slot], nb[slot], base[slot] = s, n, xp << n
    return sym, nb, base


def ref_decode_table(spread, freqs) -> np.ndarray:
    """Reference-format packed table: sym | nb<<8 | base<<16 (uint32[4096])."""
    sym, nb, base = slot_table(spread, freqs, REF_L)
    return ((sym & 0xFF) | ((nb & 0xF) << 8) | ((base & 0xFFFF) << 16)).astype(np.uint32)


# --------------------------------------------------------------------------
# Nibble split and reference-format sm packing (tans_codec.py:109-124)
# --------------------------------------------------------------------------

def split_fp8(fp8: np.ndarray):
    fp8 = np.asarray(fp8, dtype=np.uint8)
    exp = (fp8 >> 3) & 0xF
    sm = ((fp8 >> 4) & 0x8) | (fp8 & 0x7)
    return exp, sm


def pair_symbols(fp8: np.ndarray) -> np.ndarray:
    K, N = fp8.shape
    exp, _ = split_fp8(fp8)
    e = exp.reshape(K, N // 2, 2)
    return np.ascontiguousarray((e[..., 0] * 16 + e[..., 1]).astype(np.uint8))


def ref_sm(fp8: np.ndarray, tile: int) -> np.ndarray:
    K, N = fp8.shape
    _, sm = split_fp8(fp8)
    p = sm.reshape(K, N // 2, 2)
    packed = (p[..., 0] | (p[..., 1] << 4)).astype(np.uint8)
    if tile > 0:
        nt = (N // 2) // tile
        return np.ascontiguousarray(packed.reshape(K, nt, tile).transpose(1, 0, 2))
    return np.ascontiguousarray(packed.T)


# --------------------------------------------------------------------------
# Reference-format codec (oracle.c section 2)
# --------------------------------------------------------------------------

def ref_encode(symbols: np.ndarray, freqs, spread):
    """csrc/tans_codec.cpp:69-196 -> (compressed u8, states u16[K],
    offsets i32[ceil(K/128)+1], partial u8[K])."""
    symbols = np.ascontiguousarray(symbols, dtype=np.uint8)
    freqs = np.ascontiguousarray(freqs, dtype=np.int32)
    spread = np.ascontiguousarray(spread, dtype=np.int32)
    K, N = symbols.shape
    slabs = np.empty(K, np.int32)
    total = lib().ora_ref_encode_count(_p(symbols), K, N, _p(freqs), freqs.size,
                                       _p(spread), _p(slabs))
    if total < 0:
        raise ValueError(f"reference-format encode failed ({total})")
    comp = np.empty(total, np.uint8)
    states = np.empty(K, np.uint16)
    offsets = np.empty((K + REF_BLOCK - 1) // REF_BLOCK + 1, np.int32)
    partial = np.empty(K, np.uint8)
    rc = lib().ora_ref_encode_write(_p(symbols), K, N, _p(freqs), freqs.size, _p(spread),
                                    _p(slabs), _p(comp), _p(states), _p(offsets), _p(partial))
    if rc:
        raise ValueError(f"reference-format encode failed ({rc})")
    return comp, states, offsets, partial


def ref_decode(comp, offsets, states, partial, sm_kn, table, K: int, N: int) -> np.ndarray:
    """csrc/tans_decode.cu:125-155: output [N, K]."""
    out = np.empty((N, K), np.uint8)
    args = [np.ascontiguousarray(a) for a in (comp, offsets, states, partial, sm_kn, table)]
    lib().ora_ref_decode(*[_p(a) for a in args], K, N, _p(out))
    return out


def set_threads(n: int) -> None:
    """Threads of the oracle's OpenMP loops."""
    lib().ora_set_threads(int(n))


def ref_decode_add(a_enc, b_enc, table, lut, K: int, N: int) -> np.ndarray:
    """csrc/vecadd.cu:156-243: a_enc/b_enc = (comp, offsets, states, partial,
    sm_tiled); returns the tiled output [N/16, K, 16] flattened."""
    out = np.empty(K * N, np.uint8)
    arrs = [np.ascontiguousarray(x) for x in (*a_enc, *b_enc, table, lut)]
    lib().ora_ref_decode_add(*[_p(a) for a in arrs], K, N, _p(out))
    return out


# --------------------------------------------------------------------------
# wave64-layout checker (oracle.c section 3)
# --------------------------------------------------------------------------

def w64_decode(comp, offsets, states, sm, spread, freqs, log2L: int, sps: int,
               K: int, N: int) -> np.ndarray:
    """Decode the product's wave64 lane layout on the CPU; returns [K, N].
    Raises on any layout inconsistency."""
    out = np.empty((K, N), np.uint8)
    arrs = [np.ascontiguousarray(a) for a in (comp, offsets, states, sm)]
    sp = np.ascontiguousarray(spread, dtype=np.int32)
    fr = np.ascontiguousarray(freqs, dtype=np.int32)
    rc = lib().ora_w64_decode(*[_p(a) for a in arrs], _p(sp), _p(fr), fr.size,
                              log2L, sps, K, N, _p(out))
    if rc:
        raise ValueError(f"wave64 layout check failed ({rc})")
    return out


# --------------------------------------------------------------------------
# packed-layout checker (oracle.c section 4)
# --------------------------------------------------------------------------

def packed_decode(comp, offsets, sm, spread, freqs, K: int, N: int) -> np.ndarray:
    """Decode the product's packed layout of short streams (pair alphabet)
    on the CPU; returns [K, N].  Raises on any layout inconsistency."""
    out = np.empty((K, N), np.uint8)
    arrs = [np.ascontiguousarray(a) for a in (comp, offsets, sm)]
    sp = np.ascontiguousarray(spread, dtype=np.int32)
    fr = np.ascontiguousarray(freqs, dtype=np.int32)
    rc = lib().ora_packed_decode(*[_p(a) for a in arrs], _p(sp), _p(fr), K, N, _p(out))
    if rc:
        raise ValueError(f"packed layout check failed ({rc})")
    return out


def layout_decode(enc, K: int, N: int, log2L: int = 12, sps: int = 2) -> np.ndarray:
    """Decode an encode() 7-tuple of either layout (states empty: packed)."""
    comp, states, offsets, _partial, sm, freqs, spread = (
        t.numpy() if hasattr(t, "numpy") else t for t in enc)
    if K and states.size == 0:
        return packed_decode(comp, offsets, sm, spread, freqs, K, N)
    return w64_decode(comp, offsets, states, sm, spread, freqs, log2L, sps, K, N)
