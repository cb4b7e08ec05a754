"""tANS table construction and FP8 stream preparation (drop-in for the
reference's rans_vectoradd/tans_codec.py).

The exponent nibble e = (b >> 3) & 15 of each FP8 E4M3FN byte is tANS-coded;
the sign and mantissa bits pass through as packed nibbles.  Two alphabets:

* ``"pair"`` (default, as the reference): one symbol e0*16+e1 per two
  elements, L = 2^12 states, pair probabilities = outer product of the
  nibble marginals (reference tans_codec.py:123-130).
* ``"nibble"``: one symbol per element, 16 symbols, L = 2^11 states.

The encoded layout (wave64 lane groups, one shared word stream per group,
16-element sign/mantissa tiles) is described in include/tans_amd.h.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import torch

from . import _C
from ._lib import (TANS_GEMM_MAX_SEG_COLS, TANS_LANES, TANS_NIBBLE_LOG2L, TANS_PACKED_MAX_N,
                   TANS_PAIR_LOG2L, check, lib)

PAIR_L = 1 << TANS_PAIR_LOG2L
NIBBLE_L = 1 << TANS_NIBBLE_LOG2L
L = PAIR_L
M = L
BLOCK_STREAMS = TANS_LANES   # lanes per group (reference: 128 streams per block)

ALPHABETS = {"pair": (256, PAIR_L, 2), "nibble": (16, NIBBLE_L, 1)}


def sigma_for(n_states: int) -> int:
    """Hash-walk stride (n/2 + n/8 + 3), odd for n >= 8 so the walk visits
    every slot (reference tans_codec.py:26)."""
    return (n_states >> 1) + (n_states >> 3) + 3


SIGMA = sigma_for(L)


def quantize_freqs(probs, target: int = M) -> np.ndarray:
    """Scale probabilities to integer frequencies summing to ``target``.

    Same rule as the reference (tans_codec.py:30-46): round to nearest, give
    every p > 0 at least 1 and every p == 0 exactly 0, then move one unit at
    a time to (or from) the symbol whose rounding error is largest, lowest
    index first on ties.  The result is a drop-in for the reference's.

    One deliberate difference: when the total is over target and every
    shrinkable symbol is already under-served, the reference's argmax can
    pick a zero-probability symbol (its error is 0) and return frequency -1,
    which no spread can hold; that happens for the pair alphabet whenever an
    exponent never occurs.  Zero-probability symbols are never shrunk here,
    so the results agree wherever the reference's are valid."""
    p = np.asarray(probs, dtype=np.float64).reshape(-1)
    scaled = p * target
    f = np.where(p > 0, np.maximum(np.rint(scaled), 1.0), 0.0).astype(np.int64)
    short = int(target - f.sum())
    while short > 0:                       # under target: grow most under-served
        gain = np.where(p > 0, scaled - f, -np.inf)
        f[int(np.argmax(gain))] += 1
        short -= 1
    while short < 0:                       # over target: shrink most over-served
        excess = np.where((p == 0) | (f <= 1), -np.inf, f - scaled)
        f[int(np.argmax(excess))] -= 1
        short += 1
    if int(f.sum()) != target:
        raise ValueError("quantize_freqs: probabilities cannot fill the target")
    return f.astype(np.int32)


def build_spread(freqs, n_states: int | None = None) -> np.ndarray:
    """Slot -> symbol map: symbols in ascending order each take f_s slots
    along the walk slot_k = k * SIGMA mod L (reference tans_codec.py:49-60).
    ``n_states`` defaults to sum(freqs)."""
    f = np.asarray(freqs, dtype=np.int64).reshape(-1)
    n = int(f.sum()) if n_states is None else int(n_states)
    if int(f.sum()) != n or n & (n - 1):
        raise ValueError("build_spread: freqs must sum to a power of two")
    step = sigma_for(n)
    symbols = np.repeat(np.arange(f.size, dtype=np.int32), f)
    slots = (np.arange(n, dtype=np.int64) * step) % n
    spread = np.full(n, -1, dtype=np.int32)
    spread[slots] = symbols
    if (spread < 0).any():
        raise ValueError("build_spread: walk does not cover every slot")
    return spread


def build_decode_table(spread, freqs) -> torch.Tensor:
    """Decode table for the GPU kernels: int32 [2 * L], two words per state
    (layout in include/tans_amd.h).  Alphabet from len(freqs): 256 -> pair
    (L must be 4096), 16 -> nibble (L must be 2048)."""
    sp = np.ascontiguousarray(np.asarray(spread, dtype=np.int32).reshape(-1))
    fr = np.ascontiguousarray(np.asarray(freqs, dtype=np.int32).reshape(-1))
    n = sp.size
    out = torch.empty(2 * n, dtype=torch.int32)
    check(lib.tans_build_decode_table(ctypes.c_void_p(sp.ctypes.data),
                                      ctypes.c_void_p(fr.ctypes.data), fr.size,
                                      max(n.bit_length() - 1, 0),
                                      ctypes.c_void_p(out.data_ptr())),
          "build_decode_table")
    return out


def split_fp8(fp8_bytes: torch.Tensor, alphabet: str = "pair"):
    """FP8 bytes [K, N] -> (symbols [K, N/2] or [K, N] uint8, packed
    sign/mantissa tiles uint8 [ceil(N/16), K, 8])."""
    nsym, _, sps = ALPHABETS[alphabet]
    x = fp8_bytes.contiguous()
    K, N = x.shape
    S = N // sps
    symbols = torch.empty((K, S), dtype=torch.uint8)
    sm = torch.empty(((N + 15) // 16, K, 8), dtype=torch.uint8)
    check(lib.tans_split_fp8(ctypes.c_void_p(x.data_ptr()), K, N, sps,
                             ctypes.c_void_p(symbols.data_ptr()), ctypes.c_void_p(sm.data_ptr())),
          "split_fp8")
    return symbols, sm


# Every present symbol of a 2^11-state (nibble) table needs a frequency of
# at least 2: then no step reads more than 10 bits, and the decoders read
# three steps from one 32-bit window (the refill schedule of
# csrc/schedule.h).
NIBBLE_MIN_FREQ = 2


def floor_freqs(freqs, fmin: int) -> np.ndarray:
    """Raise every present symbol's frequency to at least ``fmin``, taking
    the units from the largest frequencies (one at a time, the largest
    first, lowest index on ties); the total is unchanged."""
    f = np.asarray(freqs, dtype=np.int64).reshape(-1).copy()
    low = (f > 0) & (f < fmin)
    need = int((fmin - f[low]).sum())
    f[low] = fmin
    for _ in range(need):
        i = int(np.argmax(f))
        if f[i] <= fmin:
            raise ValueError("floor_freqs: too many symbols for the table size")
        f[i] -= 1
    return f.astype(np.int32)


def symbol_freqs(exp_freqs, alphabet: str = "pair") -> np.ndarray:
    """Quantised symbol frequencies from a 16-entry exponent histogram
    (the nibble alphabet's floored at NIBBLE_MIN_FREQ)."""
    nsym, n_states, _ = ALPHABETS[alphabet]
    # normalised in float32, as the reference does (tans_codec.py:126-128),
    # so the quantised frequencies match its pair_freqs
    p = np.asarray(exp_freqs, dtype=np.float32).reshape(-1)
    if p.size != 16 or not p.sum() > 0 or (p < 0).any():
        raise ValueError("exp_freqs must be 16 non-negative weights")
    p = p / p.sum()
    if nsym == 256:
        p = (p[:, None] * p[None, :]).reshape(-1)
        return quantize_freqs(p, target=n_states)
    return floor_freqs(quantize_freqs(p, target=n_states), NIBBLE_MIN_FREQ)


def _check_tile(tile: int, N: int) -> None:
    """The reference's condition on encode's tile (tans_codec.py:115-120):
    0, or a positive tile dividing the N / 2 sign/mantissa pairs."""
    if not isinstance(tile, (int, np.integer)) or tile < 0 or (tile > 0 and (N // 2) % tile):
        raise ValueError(f"tile must be 0 or divide N / 2 = {N // 2}; got {tile}")


LAYOUTS = ("auto", "words", "packed")


def packed_layout(N: int, alphabet: str, layout: str = "auto") -> bool:
    """Whether encode() writes the packed layout of short streams for lanes
    of N elements: "packed" asks for it (pair alphabet, 2 <= N <= 64),
    "words" for the refill-schedule layout, and "auto" takes the packed
    one wherever it applies."""
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {LAYOUTS}")
    fits = alphabet == "pair" and 2 <= N <= TANS_PACKED_MAX_N
    if layout == "packed" and not fits:
        raise ValueError(f"the packed layout needs the pair alphabet and 2 <= N <= "
                         f"{TANS_PACKED_MAX_N}")
    return fits and layout != "words"


def encode(fp8_bytes: torch.Tensor, exp_freqs, tile: int = 0, *, alphabet: str = "pair",
           layout: str = "auto"):
    """tANS-encode FP8 bytes [K, N] (K lanes of N elements, N even).

    Returns the reference's 7-tuple: (compressed uint8, states uint16 [K],
    offsets int64 [ceil(K/64)+1], partial uint8 [0], sm uint8 tiles,
    freqs int32, spread int32).  ``tile`` is accepted as the reference
    accepts it (rans_vectoradd/tans_codec.py:115-120: 0, or any tile that
    divides N / 2; otherwise it raises), but the sign/mantissa layout here
    is always the 16-element tiles that both decoders read.  ``layout``
    (packed_layout): lanes of at most 64 elements with the pair alphabet
    are written in the packed layout by default, whose states live in the
    streams (``states`` is then empty); the decoders tell the layouts apart
    by that."""
    if not (isinstance(fp8_bytes, torch.Tensor) and fp8_bytes.dim() == 2
            and fp8_bytes.dtype == torch.uint8):
        raise ValueError("fp8_bytes must be a 2-D uint8 tensor [K, N]")
    if alphabet not in ALPHABETS:
        raise ValueError(f"alphabet must be one of {sorted(ALPHABETS)}")
    K, N = fp8_bytes.shape
    if N % 2:
        raise ValueError("N must be even")
    _check_tile(tile, N)
    packed = packed_layout(N, alphabet, layout)
    if isinstance(exp_freqs, torch.Tensor):
        exp_freqs = exp_freqs.detach().cpu().float().numpy()
    freqs = symbol_freqs(exp_freqs, alphabet)
    spread = build_spread(freqs)
    symbols, sm = split_fp8(fp8_bytes.cpu(), alphabet)
    freqs_t = torch.from_numpy(freqs)
    spread_t = torch.from_numpy(spread)
    comp, states, offsets, partial = _C.tans_encode_interleaved(symbols, freqs_t, spread_t,
                                                                packed=packed)
    return comp, states, offsets, partial, sm, freqs_t, spread_t


def untile(out_flat: torch.Tensor, K: int, N: int) -> torch.Tensor:
    """Tiled fused-vecadd output [N/16, K, 16] -> row-major [K, N]
    (the helper of the reference's test_vecadd_tans.py:20-27)."""
    return out_flat.view(N // 16, K, 16).permute(1, 0, 2).reshape(K, N).contiguous()


def compressed_bytes(comp, states, offsets, partial, sm) -> int:
    """Bytes a decoder reads for one tensor, counted as the reference's bench
    does (bench_vecadd.py:75-78): payload + sign/mantissa + metadata."""
    return (comp.numel() + sm.numel() + states.numel() * 2 + offsets.numel()
            * offsets.element_size() + partial.numel())


# ---------------------------------------------------------------------------
# Weight matrices for the fused decode-GEMM (no counterpart in the reference)
# ---------------------------------------------------------------------------

GEMM_GROUP_ROWS = 16          # rows of a lane group of the GEMM layout
GEMM_BLOCK_ROW_GROUPS = 32    # row groups per workgroup of the GEMM kernel
GEMM_COL_UNIT = 32            # segment widths are multiples of this
GEMM_MIN_SEG_COLS = 256       # default segments are at least this wide (64 elements per lane)
GEMM_TARGET_BLOCKS = 256      # workgroups that fill MI355X once (one per CU)


@dataclasses.dataclass
class TansMatrix:
    """A tANS-coded FP8 matrix W [rows, cols] in the layout the fused GEMM
    reads (see encode_matrix).  The tensors are the encode() 7-tuple of the
    slab view; ``to`` moves them to a device."""
    comp: torch.Tensor
    states: torch.Tensor
    offsets: torch.Tensor
    partial: torch.Tensor
    sm: torch.Tensor
    freqs: torch.Tensor
    spread: torch.Tensor
    rows: int
    cols: int
    segments: int
    seg_cols: int
    alphabet: str

    def to(self, device) -> "TansMatrix":
        moved = {f.name: getattr(self, f.name).to(device)
                 for f in dataclasses.fields(self) if isinstance(getattr(self, f.name), torch.Tensor)}
        return dataclasses.replace(self, **moved)

    def decode_table(self) -> torch.Tensor:
        return build_decode_table(self.spread.cpu().numpy(), self.freqs.cpu().numpy())

    def compressed_bytes(self) -> int:
        return compressed_bytes(self.comp, self.states, self.offsets, self.partial, self.sm)


def gemm_segments(rows: int, cols: int) -> int:
    """Default column-segment count: the most segments whose workgroups
    (segments x workgroups per segment) still run in one round, one per CU,
    so each workgroup's share (and the call's time) is as short as it gets,
    but segments of at least GEMM_MIN_SEG_COLS columns (shorter lane
    streams cost more in per-lane state than they save); at least enough
    segments for the 1024-column limit."""
    rp = -(-rows // TANS_LANES) * TANS_LANES
    blocks_per_seg = -(-(rp // GEMM_GROUP_ROWS) // GEMM_BLOCK_ROW_GROUPS)
    s = min(max(1, GEMM_TARGET_BLOCKS // blocks_per_seg), max(1, cols // GEMM_MIN_SEG_COLS))
    return max(s, -(-cols // TANS_GEMM_MAX_SEG_COLS))


def gemm_slab(w: torch.Tensor, S: int, Nc: int) -> torch.Tensor:
    """The lane streams of a padded matrix w [Rp, S * Nc]: [S * Rp * 4,
    Nc / 4], lanes ordered (segment, 16-row group, q, r).  Lane (q, r) of a
    group holds row r of the group and, of each 64-column block of the
    segment, columns 16 q .. 16 q + 15; of a last block of 32 columns,
    columns 8 q .. 8 q + 7."""
    Rp = w.shape[0]
    G = Rp // GEMM_GROUP_ROWS
    T, half = divmod(Nc, 64)
    v = w.reshape(G, GEMM_GROUP_ROWS, S, Nc)
    full = v[..., :64 * T].reshape(G, GEMM_GROUP_ROWS, S, T, 4, 16)
    full = full.permute(2, 0, 4, 1, 3, 5).reshape(S, G, 4, GEMM_GROUP_ROWS, 16 * T)
    parts = [full]
    if half:
        tail = v[..., 64 * T:].reshape(G, GEMM_GROUP_ROWS, S, 4, 8)
        parts.append(tail.permute(2, 0, 3, 1, 4))
    return torch.cat(parts, dim=-1).reshape(S * G * 4 * GEMM_GROUP_ROWS, Nc // 4).contiguous()


def encode_matrix(w_fp8: torch.Tensor, exp_freqs, *, segments: int | None = None,
                  alphabet: str = "pair") -> TansMatrix:
    """tANS-encode an FP8 matrix [R, C] for fp8_gemm_fused_tans.

    Rows are padded to Rp (a multiple of 64) and columns to S * Nc, Nc a
    multiple of 32 and at most 1024; segment s holds columns
    [s Nc, (s + 1) Nc).  The lane streams gemm_slab() cuts from it are
    encoded with encode(): a 64-lane group is 16 rows of one segment, each
    lane holding a quarter of every 64-column block of its row (the A
    operand of the kernel's 16x16x32 matrix-core products).  Padding bytes
    hold the most frequent exponent (a finite value with a nonzero
    frequency); the kernel multiplies them by zero.  A GPU tensor is laid
    out and encoded on its GPU (encode_gpu: the same bytes), and the
    result's tensors stay there; a CPU tensor is encoded on the CPU."""
    if not (isinstance(w_fp8, torch.Tensor) and w_fp8.dim() == 2 and w_fp8.dtype == torch.uint8):
        raise ValueError("w_fp8 must be a 2-D uint8 tensor [R, C]")
    R, C = w_fp8.shape
    if R == 0 or C == 0:
        raise ValueError("empty matrix")
    S = segments if segments is not None else gemm_segments(R, C)
    if S < 1:
        raise ValueError("segments must be >= 1")
    Nc = -(-C // (S * GEMM_COL_UNIT)) * GEMM_COL_UNIT
    if Nc > TANS_GEMM_MAX_SEG_COLS:
        raise ValueError(f"segments of {Nc} columns exceed {TANS_GEMM_MAX_SEG_COLS}; use more segments")
    S = -(-C // Nc)                       # (S - 1) * Nc < C <= S * Nc
    Rp = -(-R // TANS_LANES) * TANS_LANES
    if isinstance(exp_freqs, torch.Tensor):
        exp_freqs = exp_freqs.detach().cpu().double().numpy()
    pad = int(np.argmax(np.asarray(exp_freqs, dtype=np.float64))) << 3
    w = w_fp8
    if Rp != R or S * Nc != C:
        wp = torch.full((Rp, S * Nc), pad, dtype=torch.uint8, device=w.device)
        wp[:R, :C] = w
        w = wp
    slab = gemm_slab(w, S, Nc)
    # the GEMM kernel reads the refill-schedule layout
    if slab.is_cuda:
        enc = encode_gpu(slab, exp_freqs, alphabet=alphabet, layout="words")
    else:
        enc = encode(slab, exp_freqs, alphabet=alphabet, layout="words")
    comp, states, offsets, partial, sm, freqs, spread = enc
    return TansMatrix(comp, states, offsets, partial, sm, freqs, spread, rows=R, cols=C,
                      segments=S, seg_cols=Nc, alphabet=alphabet)


# ---------------------------------------------------------------------------
# GPU encoder (the same bytes as encode(), from FP8 bytes on the device)
# ---------------------------------------------------------------------------

_ENC_TABLES: dict = {}
_ENC_TABLES_MAX = 16


def _encode_tables(exp_freqs, alphabet: str, dev: torch.device):
    """(freqs, spread, enc_tab on dev, enc_next on dev) for a histogram.  The
    quantization costs about a millisecond of host time, so the tables of the
    last few (histogram, alphabet, device) keys are kept; the numpy arrays
    are read-only so a caller cannot change a cached entry."""
    h = np.ascontiguousarray(np.asarray(exp_freqs, dtype=np.float64))
    key = (alphabet, h.shape, h.tobytes(), str(dev))
    hit = _ENC_TABLES.get(key)
    if hit is not None:
        return hit
    nsym, L, _ = ALPHABETS[alphabet]
    log2L = L.bit_length() - 1
    freqs = symbol_freqs(h, alphabet)
    spread = build_spread(freqs)
    enc_tab = np.empty(nsym, dtype=np.uint32)
    enc_next = np.empty(L, dtype=np.uint16)
    check(lib.tans_build_encode_table(ctypes.c_void_p(spread.ctypes.data),
                                      ctypes.c_void_p(freqs.ctypes.data), nsym, log2L,
                                      ctypes.c_void_p(enc_tab.ctypes.data),
                                      ctypes.c_void_p(enc_next.ctypes.data)),
          "encode_gpu")
    freqs.setflags(write=False)
    spread.setflags(write=False)
    with torch.cuda.device(dev):
        tab_d = torch.from_numpy(enc_tab.view(np.int32)).to(dev)
        next_d = torch.from_numpy(enc_next.view(np.int16)).to(dev)
    if len(_ENC_TABLES) >= _ENC_TABLES_MAX:
        _ENC_TABLES.pop(next(iter(_ENC_TABLES)))
    _ENC_TABLES[key] = (freqs, spread, tab_d, next_d)
    return _ENC_TABLES[key]


def encode_gpu(fp8_bytes: torch.Tensor, exp_freqs, tile: int = 0, *, alphabet: str = "pair",
               layout: str = "auto"):
    """encode() on the GPU: FP8 bytes [K, N] (uint8, on a GPU, N even) ->
    the 7-tuple of encode() with the same arguments, byte for byte, as
    device tensors (freqs and spread included, ready for gpu_tans_decode).
    ``layout`` as in encode(): the packed layout of short streams by
    default where it applies (pair alphabet, N <= 64; states empty).  Reads the stream length
    back from the device once (the size of the compressed tensor)."""
    if not (isinstance(fp8_bytes, torch.Tensor) and fp8_bytes.dim() == 2
            and fp8_bytes.dtype == torch.uint8):
        raise ValueError("fp8_bytes must be a 2-D uint8 tensor [K, N]")
    if not fp8_bytes.is_cuda:
        raise ValueError("encode_gpu needs a GPU tensor; use encode() for CPU tensors")
    if alphabet not in ALPHABETS:
        raise ValueError(f"alphabet must be one of {sorted(ALPHABETS)}")
    K, N = fp8_bytes.shape
    if N % 2:
        raise ValueError("N must be even")
    _check_tile(tile, N)
    packed = packed_layout(N, alphabet, layout)
    if isinstance(exp_freqs, torch.Tensor):
        exp_freqs = exp_freqs.detach().cpu().float().numpy()
    nsym, L, _ = ALPHABETS[alphabet]
    log2L = L.bit_length() - 1
    dev = fp8_bytes.device
    freqs, spread, tab_d, next_d = _encode_tables(exp_freqs, alphabet, dev)
    x = fp8_bytes.contiguous()
    if x.data_ptr() % 16:            # the kernels read 4- and 16-byte words
        x = x.clone()
    G = -(-K // TANS_LANES)
    with torch.cuda.device(dev):
        ws_bytes = ctypes.c_int64()
        check(lib.tans_gpu_encode_workspace(K, N, log2L, ctypes.byref(ws_bytes)), "encode_gpu")
        ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=dev)
        offsets = torch.empty(G + 1, dtype=torch.int64, device=dev)
        states = torch.empty(0 if packed else K, dtype=torch.uint16, device=dev)
        sm = torch.empty(((N + 15) // 16, K, 8), dtype=torch.uint8, device=dev)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        if packed and K:
            check(lib.tans_gpu_encode_packed_begin(
                x.data_ptr(), K, N, tab_d.data_ptr(), next_d.data_ptr(), log2L, ws.data_ptr(),
                ws.numel(), offsets.data_ptr(), sm.data_ptr(), status.data_ptr(), stream),
                "encode_gpu")
        else:
            check(lib.tans_gpu_encode_begin(
                x.data_ptr(), K, N, tab_d.data_ptr(), next_d.data_ptr(), log2L, ws.data_ptr(),
                ws.numel(), offsets.data_ptr(), states.data_ptr(), sm.data_ptr(),
                status.data_ptr(), stream), "encode_gpu")
        total, bad = (int(v) for v in torch.stack([offsets[G], status[0].to(torch.int64)]).tolist())
        if bad:
            raise RuntimeError("encode_gpu: data holds a symbol whose frequency is 0")
        comp = torch.empty((total + 256) * 4, dtype=torch.uint8, device=dev)
        finish = lib.tans_gpu_encode_packed_finish if packed and K else lib.tans_gpu_encode_finish
        check(finish(K, N, log2L, ws.data_ptr(), offsets.data_ptr(), comp.data_ptr(),
                     comp.numel(), stream), "encode_gpu")
    partial = torch.empty(0, dtype=torch.uint8, device=dev)
    return (comp, states, offsets, partial, sm, torch.from_numpy(freqs.copy()).to(dev),
            torch.from_numpy(spread.copy()).to(dev))


@dataclasses.dataclass
class TansTensor:
    """A tANS-coded FP8 tensor in the lane layout: K lanes of N elements,
    the encode() 7-tuple plus its shape and alphabet (what a caller keeps to
    decode or add it later; stored by rans_vectoradd.container)."""
    comp: torch.Tensor
    states: torch.Tensor
    offsets: torch.Tensor
    partial: torch.Tensor
    sm: torch.Tensor
    freqs: torch.Tensor
    spread: torch.Tensor
    K: int
    N: int
    alphabet: str

    @classmethod
    def from_tuple(cls, enc, K: int, N: int, alphabet: str = "pair") -> "TansTensor":
        return cls(*enc, K=K, N=N, alphabet=alphabet)

    def as_tuple(self):
        return (self.comp, self.states, self.offsets, self.partial, self.sm, self.freqs,
                self.spread)

    def to(self, device) -> "TansTensor":
        moved = {f.name: getattr(self, f.name).to(device)
                 for f in dataclasses.fields(self) if isinstance(getattr(self, f.name), torch.Tensor)}
        return dataclasses.replace(self, **moved)

    def decode_table(self) -> torch.Tensor:
        return build_decode_table(self.spread.cpu().numpy(), self.freqs.cpu().numpy())

    def compressed_bytes(self) -> int:
        return compressed_bytes(self.comp, self.states, self.offsets, self.partial, self.sm)
