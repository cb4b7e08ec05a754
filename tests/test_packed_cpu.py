"""The packed layout of short streams (pair alphabet, at most 64 elements
per lane; include/tans_amd.h), CPU only: the product encoder's output
decoded by the oracle's independent checker (oracle.c section 4), its
header and size bounds, what it costs on config-1 data against the
refill-schedule layout, and that the checker catches a planted mistake."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


@pytest.fixture(scope="module")
def T():
    from rans_vectoradd import tans_codec
    return tans_codec


def _hdr(N):
    return 1 if N // 2 <= 8 else 2


def _streams(enc):
    comp, _st, off = enc[0].numpy(), enc[1], enc[2].numpy()
    return [comp[4 * off[g]:4 * off[g + 1]] for g in range(len(off) - 1)]


def _lane_bits(T, fp8, hist):
    """Bits of each lane: 12 for the state plus the nb of every step, from
    the oracle's own encoder tables (x walks back from L as in
    csrc/tans_codec.cpp:22-60)."""
    f = T.symbol_freqs(hist, "pair")
    sp = T.build_spread(f)
    L = 4096
    nxt = {}
    cnt = np.zeros(256, np.int64)
    for slot in range(L):
        s = int(sp[slot])
        nxt[(s, int(f[s]) + int(cnt[s]))] = L + slot
        cnt[s] += 1
    sym = O.pair_symbols(fp8.numpy())
    bits = np.zeros(sym.shape[0], np.int64)
    for k in range(sym.shape[0]):
        x, n = L, 12
        for s in sym[k, ::-1]:
            fs = int(f[s])
            nb = 0
            while (x >> nb) >= 2 * fs:
                nb += 1
            n += nb
            x = nxt[(int(s), x >> nb)]
        bits[k] = n
    return bits


@pytest.mark.parametrize("K,N", [(64, 16), (65, 2), (130, 46), (1, 64), (127, 18), (200, 32)])
def test_header_counts_and_padding(T, K, N):
    """Each group's header holds its lane pairs' bit counts (the lanes' own
    bit totals, recomputed here from the tables), lanes past K count 0,
    streams are 16-byte multiples and the stream ends with zero bits."""
    from rans_vectoradd import data as D
    torch.manual_seed(K + N)
    fp8 = D.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    hist = torch.tensor(D.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    enc = T.encode(fp8, hist)
    assert enc[1].numel() == 0 and enc[3].numel() == 0
    bits = np.zeros(((K + 63) // 64) * 64, np.int64)
    bits[:K] = _lane_bits(T, fp8, hist.numpy())
    hb = _hdr(N)
    for g, st in enumerate(_streams(enc)):
        assert st.size % 16 == 0
        cnt = st[:32 * hb].view(np.uint8 if hb == 1 else np.uint16).astype(np.int64)
        pair = bits[64 * g:64 * g + 64].reshape(32, 2).sum(1)
        assert np.array_equal(cnt, pair), g
        used = 32 * hb * 8 + int(cnt.sum())
        assert st.size * 8 - used < 128
        area = np.unpackbits(st, bitorder="little")
        assert not area[used:].any()
    assert np.array_equal(O.layout_decode(enc, K, N), fp8.numpy())


@pytest.mark.parametrize("N", [2, 16, 18, 64])
def test_longest_streams_fit_the_bound(T, N):
    """Every step at nb = 12 (data of the rarest pair symbol, frequency 1):
    a group's stream is exactly max_stream_bytes, the size the decoders'
    LDS region is built for (3232 bytes at 64 elements per lane)."""
    from rans_vectoradd import data as D
    exp = np.array(D.QWEN3_14B_FP8_EXP, np.float64)
    f = T.symbol_freqs(exp, "pair")
    rare = int(np.argmin(np.where(f > 0, f, 1 << 30)))
    assert f[rare] == 1
    e0, e1 = rare >> 4, rare & 15
    K = 128
    fp8 = torch.empty((K, N), dtype=torch.uint8)
    g = torch.Generator().manual_seed(N)
    sm = torch.randint(0, 256, (K, N), dtype=torch.uint8, generator=g) & 0x87
    fp8[:, 0::2] = sm[:, 0::2] | (e0 << 3)
    fp8[:, 1::2] = sm[:, 1::2] | (e1 << 3)
    enc = T.encode(fp8, exp)
    S = N // 2
    hdr = 32 * _hdr(N)
    bound = (hdr + (64 * (12 + 12 * S) + 7) // 8 + 15) // 16 * 16
    assert all(st.size == bound for st in _streams(enc))
    if N == 64:
        assert bound == 3232
    assert np.array_equal(O.layout_decode(enc, K, N), fp8.numpy())


def test_config1_short_stream_sizes(T):
    """Config-1 data (N(0, 0.02) scaled to 448, its own histogram): 1Ki and
    4Ki-element streams (16 and 64 elements per lane) cost at most 7.8 and
    7.0 bits per FP8 byte in the packed layout, against 9.18 and 7.31 in
    the refill-schedule layout, and decode back exactly."""
    from rans_vectoradd import data as D
    n = 1 << 20
    q, _ = D.gaussian_fp8_bytes(n, seed=0)
    hist = D.exp_histogram(q)
    got = {}
    for N in (16, 64):
        x = q.reshape(n // N, N)
        for layout in ("words", "packed"):
            enc = T.encode(x, hist, layout=layout)
            got[N, layout] = T.compressed_bytes(*enc[:5]) * 8 / n
            assert np.array_equal(O.layout_decode(enc, n // N, N), x.numpy())
    assert got[16, "packed"] <= 7.8 and got[64, "packed"] <= 7.0, got
    assert got[16, "words"] > 9.0 and got[64, "words"] > 7.2, got


def test_layout_choice(T):
    assert T.packed_layout(16, "pair") and T.packed_layout(64, "pair")
    assert not T.packed_layout(66, "pair") and not T.packed_layout(16, "nibble")
    assert not T.packed_layout(16, "pair", "words")
    with pytest.raises(ValueError):
        T.packed_layout(80, "pair", "packed")
    with pytest.raises(ValueError):
        T.packed_layout(16, "nibble", "packed")
    with pytest.raises(ValueError):
        T.packed_layout(16, "pair", "slabs")
    x = torch.zeros((4, 80), dtype=torch.uint8)
    with pytest.raises(ValueError):
        T.encode(x, np.ones(16), layout="packed")


def test_packed_encoder_rejects_what_it_cannot_write(T):
    from rans_vectoradd import _C
    syms = torch.zeros((4, 33), dtype=torch.uint8)           # 33 steps: 66 elements
    f = torch.from_numpy(T.symbol_freqs(np.ones(16), "pair"))
    sp = torch.from_numpy(T.build_spread(f.numpy()))
    with pytest.raises(RuntimeError, match="1..32 steps"):
        _C.tans_encode_interleaved(syms, f, sp, packed=True)
    fn = torch.from_numpy(T.symbol_freqs(np.ones(16), "nibble"))
    spn = torch.from_numpy(T.build_spread(fn.numpy()))
    with pytest.raises(RuntimeError, match="2\\^12-state"):
        _C.tans_encode_interleaved(syms[:, :8].contiguous(), fn, spn, packed=True)


def test_checker_catches_planted_mistakes(T):
    """The oracle's checker, handed a stream with one thing wrong, rejects
    it or decodes different bytes: a count moved between two pairs, a bit
    of the area flipped, a padding bit set, the two lanes of a pair
    swapped."""
    from rans_vectoradd import data as D
    K, N = 128, 32
    torch.manual_seed(7)
    fp8 = D.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    enc = T.encode(fp8, np.array(D.QWEN3_14B_FP8_EXP))
    want = fp8.numpy()
    assert np.array_equal(O.layout_decode(enc, K, N), want)
    comp0 = enc[0].numpy().copy()

    def check(comp):
        e = (torch.from_numpy(comp),) + tuple(enc[1:])
        try:
            return not np.array_equal(O.layout_decode(e, K, N), want)
        except ValueError:
            return True

    c = comp0.copy()                       # count of pair 0 +1, pair 1 -1 (u16 header)
    h = c[:64].view(np.uint16)
    h[0] += 1
    h[1] -= 1
    assert check(c)
    c = comp0.copy()                       # one bit of the area flipped
    c[64 + 5] ^= 0x10
    assert check(c)
    c = comp0.copy()                       # a padding bit set
    end = 4 * int(enc[2][1])
    used = 64 * 8 + int(comp0[:64].view(np.uint16).astype(np.int64).sum())
    assert used < end * 8
    c[end - 1] |= 0x80
    assert check(c)
    c = comp0.copy()                       # lanes 0 and 1 swapped (area reversed)
    n0 = int(comp0[:64].view(np.uint16)[0])
    bits = np.unpackbits(c[64:end], bitorder="little")
    bits[:n0] = bits[:n0][::-1].copy()
    c[64:end] = np.packbits(bits, bitorder="little")
    assert check(c)
