"""Drop-in for the reference's pybind11 module ``rans_vectoradd._C``
(csrc/fp8_memcpy.cu:66-78): the same five functions, positional arguments
and return shapes, implemented over the C ABI of libtans_amd.so.

Differences from the reference, all inside the tensors the encoder returns:

* ``offsets`` are int64 word offsets of each 64-lane group's stream (the
  reference: int32 byte offsets of 128-stream blocks);
* ``partial_cnts`` is empty: the layout has no partial slabs; it is accepted
  and ignored by the decoders, as any tensor would be;
* ``decode_tbl`` holds 2 int32 words per state (build_decode_table);
* the sign/mantissa tensor uses the 16-element tile layout of
  include/tans_amd.h for both the fused and the standalone decoder.

Validation mirrors the reference's TORCH_CHECKs and raises RuntimeError.
Kernels run on the current torch stream of the inputs' device.
"""
from __future__ import annotations

import contextlib
import ctypes

import torch

from ._lib import (TANS_GEMM_MAX_BATCH, TANS_LANES, TANS_NIBBLE_LOG2L, TANS_PACKED_MAX_N,
                   TANS_PAIR_LOG2L, TANS_TILE, check, lib)

__all__ = [
    "tans_encode_interleaved",
    "gpu_tans_decode",
    "fp8_memcpy",
    "fp8_vecadd_raw",
    "fp8_vecadd_fused_tans",
    "fp8_gemm_fused_tans",
    "fp8_gemm_raw",
]


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _on(device: torch.device):
    """Make `device` current for the launch (a no-op when it already is)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_dev(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    if not (t.is_cuda and t.dtype == dtype and t.is_contiguous()):
        _require(t.is_cuda, f"{name} must be CUDA")
        _require(t.dtype == dtype, f"{name} must be {dtype}")
        _require(t.is_contiguous(), f"{name} must be contiguous")


def _check_cpu(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    _require(t.device.type == "cpu", f"{name} must be a CPU tensor")
    _require(t.dtype == dtype, f"{name} must be {dtype}")
    _require(t.is_contiguous(), f"{name} must be contiguous")


def log2_states(n: int) -> int:
    """log2 of a table size, checking it is a supported alphabet's."""
    _require(n in (1 << TANS_PAIR_LOG2L, 1 << TANS_NIBBLE_LOG2L),
             f"table size must be 2^{TANS_PAIR_LOG2L} (pair) or 2^{TANS_NIBBLE_LOG2L} "
             f"(nibble); got {n}")
    return n.bit_length() - 1


def tans_encode_interleaved(symbols: torch.Tensor, freqs: torch.Tensor,
                            spread: torch.Tensor, *, packed: bool = False):
    """CPU tANS encoder -> wave64 lane layout.  (csrc/tans_codec.cpp:69-196)

    symbols [K, S] uint8 (one symbol per decode step), freqs int32 summing to
    L = spread.numel(), spread [L] int32.  Returns (compressed uint8,
    states uint16 [K], offsets int64 [ceil(K/64)+1], partial uint8 [0]).
    ``packed`` (a keyword the reference does not have) writes the packed
    layout of short streams instead (2^12-state tables, S <= 32): the
    initial states go into the streams and ``states`` comes back empty."""
    _require(symbols.dim() == 2, "symbols must be [K, N]")
    _check_cpu("symbols", symbols, torch.uint8)
    _check_cpu("freqs", freqs, torch.int32)
    _check_cpu("spread", spread, torch.int32)
    L = spread.numel()
    _require(L > 0 and (L & (L - 1)) == 0 and L <= 4096, "spread size must be a power of two <= 4096")
    K, S = symbols.shape
    handle = ctypes.c_void_p()
    comp_bytes = ctypes.c_int64()
    n_off = ctypes.c_int64()
    begin = lib.tans_encode_packed_begin if packed else lib.tans_encode_begin
    check(begin(_ptr(symbols), K, S, _ptr(freqs), freqs.numel(), _ptr(spread),
                L.bit_length() - 1, ctypes.byref(handle), ctypes.byref(comp_bytes),
                ctypes.byref(n_off)),
          "tans_encode_interleaved")
    try:
        comp = torch.empty(comp_bytes.value, dtype=torch.uint8)
        states = torch.empty(0 if packed else K, dtype=torch.uint16)
        offsets = torch.empty(n_off.value, dtype=torch.int64)
    except BaseException:
        lib.tans_encode_free(handle)
        raise
    check(lib.tans_encode_finish(handle, _ptr(comp), _ptr(states), _ptr(offsets)),
          "tans_encode_interleaved")
    return comp, states, offsets, torch.empty(0, dtype=torch.uint8)


def _groups(K: int) -> int:
    return (K + TANS_LANES - 1) // TANS_LANES


def _sm_bytes(K: int, N: int) -> int:
    return ((N + TANS_TILE - 1) // TANS_TILE) * K * 8


def _lanes(states: torch.Tensor, sm: torch.Tensor, N: int) -> int:
    """K, the lanes of an encoding: states.numel(), or for the packed
    layout (no state array) the sign/mantissa size over 8 bytes per tile."""
    if states.numel() or N <= 0:
        return states.numel()
    per_lane = ((N + TANS_TILE - 1) // TANS_TILE) * 8
    _require(sm.numel() % per_lane == 0, "sign/mantissa tensor has the wrong tiled size")
    return sm.numel() // per_lane


def _check_packed(packed: bool, N: int, log2L: int, K: int) -> None:
    if packed and K:
        _require(log2L == TANS_PAIR_LOG2L and N <= TANS_PACKED_MAX_N,
                 f"an encoding without states (the packed layout) needs the pair table "
                 f"and at most {TANS_PACKED_MAX_N} elements per stream")


# (spread, freqs) pairs whose device table build reported no inconsistency:
# id pair -> (weak references, data pointers and version counters).  A pair
# is read back (one host synchronisation) only the first time it is seen and
# after it changes in place.
_VALID_TABLES: dict = {}
_VALID_TABLES_MAX = 64


def _table_key(spread: torch.Tensor, freqs: torch.Tensor):
    return (spread.data_ptr(), spread._version, freqs.data_ptr(), freqs._version)


def _table_known_valid(spread: torch.Tensor, freqs: torch.Tensor) -> bool:
    hit = _VALID_TABLES.get((id(spread), id(freqs)))
    if hit is None:
        return False
    ws, wf, key = hit
    return ws() is spread and wf() is freqs and key == _table_key(spread, freqs)


def _remember_valid_table(spread: torch.Tensor, freqs: torch.Tensor) -> None:
    import weakref
    if len(_VALID_TABLES) >= _VALID_TABLES_MAX:
        _VALID_TABLES.clear()
    _VALID_TABLES[(id(spread), id(freqs))] = (weakref.ref(spread), weakref.ref(freqs),
                                              _table_key(spread, freqs))


def gpu_tans_decode(compressed: torch.Tensor, offsets: torch.Tensor, states: torch.Tensor,
                    partial_cnts: torch.Tensor, sign_mantissa: torch.Tensor,
                    spread: torch.Tensor, freqs: torch.Tensor,
                    n_fp8_per_stream: int) -> torch.Tensor:
    """Standalone decode -> uint8 [n_fp8_per_stream, K].  (csrc/tans_decode.cu:159-210)

    The decode table is built on the device from spread/freqs, without the
    reference's host round trip.  Like the reference's TORCH_CHECKs in its
    table build (csrc/tans_decode.cu:38,50), an inconsistent spread/freqs
    pair raises RuntimeError: the device build's status is read back the
    first time a pair is used (and after it changes in place); later calls
    with the same tensors, and calls under graph capture, do not wait on
    the device."""
    _check_dev("compressed", compressed, torch.uint8)
    _check_dev("offsets", offsets, torch.int64)
    _check_dev("states", states, torch.uint16)
    _check_dev("sign_mantissa", sign_mantissa, torch.uint8)
    _check_dev("spread", spread, torch.int32)
    _check_dev("freqs", freqs, torch.int32)
    N = int(n_fp8_per_stream)
    _require(N >= 0 and N % 2 == 0, "n_fp8_per_stream must be even")
    K = _lanes(states, sign_mantissa, N)
    _require(offsets.numel() == _groups(K) + 1, "offsets must have n_groups + 1 entries")
    _require(sign_mantissa.numel() == _sm_bytes(K, N), "sign_mantissa has the wrong shape")
    log2L = log2_states(spread.numel())
    _check_packed(states.numel() == 0, N, log2L, K)
    nsym = freqs.numel()
    _require((nsym, log2L) in ((256, TANS_PAIR_LOG2L), (16, TANS_NIBBLE_LOG2L)),
             "freqs must hold 256 pair or 16 nibble frequencies matching the spread size")
    dev = compressed.device
    for t in (offsets, states, sign_mantissa, spread, freqs):
        _require(t.device == dev, "all tensors must be on one device")
    out = torch.empty((N, K), dtype=torch.uint8, device=dev)
    if K == 0 or N == 0:
        return out
    with _on(dev):
        table = torch.empty(2 << log2L, dtype=torch.int32, device=dev)
        verify = (not _table_known_valid(spread, freqs)
                  and not torch.cuda.is_current_stream_capturing())
        status = torch.zeros(1, dtype=torch.int32, device=dev) if verify else None
        stream = _stream(dev)
        check(lib.tans_build_decode_table_device(_ptr(spread), _ptr(freqs), nsym, log2L,
                                                 _ptr(table),
                                                 _ptr(status) if verify else None, stream),
              "gpu_tans_decode")
        if verify:
            rc = int(status.item())
            _require(rc == 0, "gpu_tans_decode: spread and freqs do not form a valid decode "
                              "table (frequencies must sum to the spread size, match the "
                              "spread's symbol counts, and be >= 2 for every present symbol "
                              "of a 2^11-state table)")
            _remember_valid_table(spread, freqs)
        check(lib.tans_decode(_ptr(compressed), compressed.numel(), _ptr(offsets), _ptr(states),
                              _ptr(sign_mantissa), _ptr(table), log2L, K, N, _ptr(out), stream),
              "gpu_tans_decode")
    return out


def fp8_memcpy(A: torch.Tensor) -> torch.Tensor:
    """C[i] = A[i] through 16-byte streaming loads.  (csrc/fp8_memcpy.cu:45-64)"""
    _check_dev("A", A, torch.uint8)
    _require(A.numel() % 16 == 0, "A length must be a multiple of 16")
    C = torch.empty_like(A)
    with _on(A.device):
        check(lib.tans_fp8_memcpy(_ptr(A), _ptr(C), A.numel(), _stream(A.device)), "fp8_memcpy")
    return C


def fp8_vecadd_raw(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """C[i] = fp8(float(A[i]) + float(B[i])), RNE, saturating.  (csrc/vecadd.cu:268-288)"""
    _check_dev("A", A, torch.uint8)
    _check_dev("B", B, torch.uint8)
    _require(A.numel() == B.numel(), "A and B must have the same length")
    _require(A.numel() % 16 == 0, "A/B length must be a multiple of 16")
    _require(A.device == B.device, "A and B must be on the same device")
    C = torch.empty_like(A)
    with _on(A.device):
        check(lib.tans_fp8_vecadd_raw(_ptr(A), _ptr(B), _ptr(C), A.numel(), _stream(A.device)),
              "fp8_vecadd_raw")
    return C


_PROBE_MODES = {"read": 0, "write": 1, "stream21": 2}


def stream_probe(mode: str, A: torch.Tensor | None = None, B: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, nontemporal: bool = True) -> torch.Tensor | None:
    """Bandwidth probe at fp8_vecadd_raw's launch shape, no arithmetic
    (no reference counterpart; its fp8_memcpy is the one ceiling it
    measures).  "read": reads A; "write": writes `out`; "stream21": writes
    out = A ^ B.  Returns `out` (allocated like A when not given) or None
    for "read"."""
    _require(mode in _PROBE_MODES, f"mode must be one of {sorted(_PROBE_MODES)}")
    m = _PROBE_MODES[mode]
    if m != 1:
        _check_dev("A", A, torch.uint8)
    if m == 2:
        _check_dev("B", B, torch.uint8)
        _require(A.numel() == B.numel() and A.device == B.device, "A and B must match")
    if m != 0:
        if out is None:
            _require(A is not None, "write needs `out` or A to size it")
            out = torch.empty_like(A)
        _check_dev("out", out, torch.uint8)
    ref = A if A is not None else out
    n = ref.numel()
    _require(n % 16 == 0, "length must be a multiple of 16")
    with _on(ref.device):
        sink = torch.empty(1, dtype=torch.int32, device=ref.device) if m == 0 else None
        check(lib.tans_stream_probe(m, int(bool(nontemporal)), _ptr(A) if m != 1 else None,
                                    _ptr(B) if m == 2 else None,
                                    _ptr(out) if m != 0 else None, n,
                                    _ptr(sink) if m == 0 else None, _stream(ref.device)),
              "stream_probe")
    return out if m != 0 else None


def fp8_vecadd_fused_tans(a_comp: torch.Tensor, a_offsets: torch.Tensor, a_states: torch.Tensor,
                          a_partial: torch.Tensor, a_sm: torch.Tensor,
                          b_comp: torch.Tensor, b_offsets: torch.Tensor, b_states: torch.Tensor,
                          b_partial: torch.Tensor, b_sm: torch.Tensor,
                          decode_tbl: torch.Tensor, n_fp8_per_stream: int) -> torch.Tensor:
    """Fused tANS decode of A and B + FP8 add -> tiled uint8 [N/16 * K * 16].
    (csrc/vecadd.cu:290-393)"""
    for name, t in (("a_comp", a_comp), ("a_sm", a_sm), ("b_comp", b_comp), ("b_sm", b_sm)):
        _check_dev(name, t, torch.uint8)
    _check_dev("a_offsets", a_offsets, torch.int64)
    _check_dev("b_offsets", b_offsets, torch.int64)
    _check_dev("a_states", a_states, torch.uint16)
    _check_dev("b_states", b_states, torch.uint16)
    _check_dev("decode_tbl", decode_tbl, torch.int32)
    N = int(n_fp8_per_stream)
    _require(N >= 0 and N % 16 == 0, "n_fp8_per_stream must be divisible by 16")
    K = _lanes(a_states, a_sm, N)
    _require((a_states.numel() == 0) == (b_states.numel() == 0),
             "A and B must share a layout (both with states, or both packed)")
    _require(_lanes(b_states, b_sm, N) == K, "A/B stream counts must match")
    _require(a_offsets.numel() == _groups(K) + 1 and b_offsets.numel() == _groups(K) + 1,
             "offset tensors must have n_groups + 1 entries")
    _require(a_sm.numel() == _sm_bytes(K, N) and b_sm.numel() == _sm_bytes(K, N),
             "sign/mantissa tensors have the wrong tiled size")
    _require(decode_tbl.numel() % 2 == 0, "decode_tbl must hold 2 words per state")
    log2L = log2_states(decode_tbl.numel() // 2)
    _check_packed(a_states.numel() == 0, N, log2L, K)
    dev = a_comp.device
    for t in (a_offsets, a_states, a_sm, b_comp, b_offsets, b_states, b_sm, decode_tbl):
        _require(t.device == dev, "all tensors must be on one device")
    out = torch.empty(K * N, dtype=torch.uint8, device=dev)
    if K == 0 or N == 0:
        return out
    with _on(dev):
        check(lib.tans_fp8_vecadd_fused(_ptr(a_comp), a_comp.numel(), _ptr(a_offsets),
                                        _ptr(a_states), _ptr(a_sm), _ptr(b_comp), b_comp.numel(),
                                        _ptr(b_offsets), _ptr(b_states), _ptr(b_sm),
                                        _ptr(decode_tbl), log2L, K, N, _ptr(out), _stream(dev)),
              "fp8_vecadd_fused_tans")
    return out


def _batch_view(x: torch.Tensor, C: int):
    """x bf16 [C] or [B, C] -> (x2d [B, C], B, squeeze)."""
    _check_dev("x", x, torch.bfloat16)
    _require(x.dim() in (1, 2) and x.shape[-1] == C, f"x must be [C] or [B, C] with C = {C}")
    x2 = x.view(1, C) if x.dim() == 1 else x
    B = x2.shape[0]
    _require(1 <= B <= TANS_GEMM_MAX_BATCH, f"batch must be 1..{TANS_GEMM_MAX_BATCH}")
    return x2, B, x.dim() == 1


def fp8_gemm_fused_tans(m, decode_tbl: torch.Tensor, x: torch.Tensor,
                        scale: float = 1.0) -> torch.Tensor:
    """y = scale * (W @ x^T) as bf16, W decoded from its tANS encoding inside
    the kernel.  No counterpart in the reference (its configs 3-4).

    m: a TansMatrix from tans_codec.encode_matrix, its tensors on the GPU;
    decode_tbl: build_decode_table of its spread/freqs (on the GPU);
    x: bf16 [C] or [B, C] (B <= 8).  Returns bf16 [R] or [B, R]; fp32
    accumulation, segment sums added in a fixed order."""
    R, C, S, Nc = m.rows, m.cols, m.segments, m.seg_cols
    for name in ("comp", "sm"):
        _check_dev(name, getattr(m, name), torch.uint8)
    _check_dev("offsets", m.offsets, torch.int64)
    _check_dev("states", m.states, torch.uint16)
    _check_dev("decode_tbl", decode_tbl, torch.int32)
    x2, B, squeeze = _batch_view(x, C)
    Rp = (R + TANS_LANES - 1) // TANS_LANES * TANS_LANES
    K = S * Rp * 4                  # lanes: S segments x Rp / 16 groups x 64
    _require(Nc % 32 == 0, "segment width must be a multiple of 32")
    _require(m.states.numel() == K, "states do not match the matrix shape")
    _require(m.offsets.numel() == _groups(K) + 1, "offsets do not match the matrix shape")
    _require(m.sm.numel() == _sm_bytes(K, Nc // 4),
             "sign/mantissa tiles do not match the matrix shape")
    n_states = {"pair": 1 << TANS_PAIR_LOG2L, "nibble": 1 << TANS_NIBBLE_LOG2L}.get(m.alphabet)
    _require(n_states is not None and decode_tbl.numel() == 2 * n_states,
             f"decode_tbl must hold 2 words per state of the matrix's {m.alphabet} alphabet")
    log2L = log2_states(n_states)
    dev = m.comp.device
    for t in (m.offsets, m.states, m.sm, decode_tbl, x2):
        _require(t.device == dev, "all tensors must be on one device")
    y = torch.empty((B, R), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        ws = torch.empty(S * B * Rp, dtype=torch.float32, device=dev)
        check(lib.tans_fp8_gemm_fused(_ptr(m.comp), m.comp.numel(), _ptr(m.offsets),
                                      _ptr(m.states), _ptr(m.sm), _ptr(decode_tbl), log2L, R, C,
                                      S, Nc, _ptr(x2), B, float(scale), _ptr(ws), ws.numel() * 4,
                                      _ptr(y), _stream(dev)), "fp8_gemm_fused_tans")
    return y.view(R) if squeeze else y


def fp8_gemm_raw(W: torch.Tensor, x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """The same product from uncompressed FP8 bytes W [R, C] (C % 16 == 0)."""
    _check_dev("W", W, torch.uint8)
    _require(W.dim() == 2 and W.shape[1] % 16 == 0, "W must be [R, C] with C % 16 == 0")
    R, C = W.shape
    x2, B, squeeze = _batch_view(x, C)
    _require(x2.device == W.device, "W and x must be on one device")
    y = torch.empty((B, R), dtype=torch.bfloat16, device=W.device)
    with _on(W.device):
        check(lib.tans_fp8_gemm_raw(_ptr(W), R, C, _ptr(x2), B, float(scale), _ptr(y),
                                    _stream(W.device)), "fp8_gemm_raw")
    return y.view(R) if squeeze else y
