"""Pins for the CPU oracle (oracle/), CPU only.

Every oracle function is checked against something it does not share code
with: the golden vectors written from the reference's own Python
(tests/golden/reference_vectors.npz), torch's independent E4M3FN cast, hand
computed known answers from the OCP FP8 rules, closed forms and tANS
invariants, and brute-force round trips on tiny inputs.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                            "reference_vectors.npz"))
NAN = (np.arange(256) & 0x7F) == 0x7F


# --------------------------------------------------------------------------
# FP8 E4M3FN decode and RNE-saturating add (reference csrc/vecadd.cu:27-35)
# --------------------------------------------------------------------------

def test_fp8_decode_matches_torch():
    b = np.arange(256, dtype=np.uint8)
    ours = O.fp8_to_float64(b)
    theirs = torch.from_numpy(b).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    ok = ~np.isnan(ours)
    assert np.array_equal(ours[ok], theirs[ok])
    assert np.array_equal(np.isnan(ours), NAN)


def test_add_lut_matches_torch_clamped_cast():
    """lut[a, b] == e4m3fn(clamp(float(a) + float(b), -448, 448)).  The sum of
    two E4M3 values is exact in float32, so torch's float -> e4m3fn cast (its
    own RNE code) gives the single correctly rounded result once clamped."""
    lut = O.add_lut()
    v = torch.from_numpy(np.arange(256, dtype=np.uint8)).view(torch.float8_e4m3fn).float()
    s = (v[:, None] + v[None, :]).clamp(-448.0, 448.0)
    ref = s.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    finite = ~(NAN[:, None] | NAN[None, :])
    assert np.array_equal(lut[finite], ref[finite])
    # NaN operands give the canonical NaN byte (not pinned by the reference)
    assert (lut[~finite] == 0x7F).all()


@pytest.mark.parametrize("a,b,want", [
    (0x38, 0x38, 0x40),   # 1 + 1 = 2
    (0x7E, 0x7E, 0x7E),   # 448 + 448 saturates to 448
    (0xFE, 0xFE, 0xFE),   # -448 - 448 saturates to -448
    (0x77, 0x77, 0x7E),   # 240 + 240 = 480 > 448: saturates (480 is not finite)
    (0x7E, 0x08, 0x7E),   # 448 + 2^-6 rounds back to 448
    (0x7E, 0xFE, 0x00),   # 448 - 448 = +0
    (0x80, 0x00, 0x00),   # -0 + +0 = +0
    (0x80, 0x80, 0x80),   # -0 + -0 = -0
    (0x01, 0x01, 0x02),   # subnormals: 2^-9 + 2^-9 = 2^-8
    (0x07, 0x01, 0x08),   # 7 * 2^-9 + 2^-9 = 2^-6, the smallest normal
    (0x38, 0x18, 0x38),   # 1 + 1/16 = 1.0625: tie between 1 and 1.125, to even (1)
    (0x39, 0x18, 0x3A),   # 1.125 + 1/16 = 1.1875: tie, to even (1.25)
    (0x7D, 0x58, 0x7E),   # 416 + 16 = 432: tie between 416 and 448, to even (448)
    (0x38, 0x01, 0x38),   # 1 + 2^-9 rounds to 1
])
def test_add_known_answers(a, b, want):
    assert O.lib().ora_fp8_add(a, b) == want
    assert O.lib().ora_fp8_add(b, a) == want


def test_add_is_commutative_and_sign_symmetric():
    lut = O.add_lut()
    assert np.array_equal(lut, lut.T)
    neg = np.arange(256) ^ 0x80
    finite = ~(NAN[:, None] | NAN[None, :])
    flipped = lut[neg][:, neg] ^ 0x80
    # -(a + b) == (-a) + (-b), except that +0 stays +0 under negation
    zero = (lut == 0x00) | (lut == 0x80)
    assert np.array_equal(flipped[finite & ~zero], lut[finite & ~zero])


# --------------------------------------------------------------------------
# Table construction (reference rans_vectoradd/tans_codec.py:24-87)
# --------------------------------------------------------------------------

def test_quantize_freqs_matches_reference_golden():
    assert np.array_equal(O.quantize_freqs(GOLDEN["qf_pair_qwen_in"], 4096),
                          GOLDEN["qf_pair_qwen_out"])
    for i in range(7):
        got = O.quantize_freqs(GOLDEN[f"qf_case{i}_in"], int(GOLDEN[f"qf_case{i}_target"][0]))
        assert np.array_equal(got, GOLDEN[f"qf_case{i}_out"]), f"case {i}"


def test_sigma_is_odd_so_the_walk_covers_every_slot():
    for log2L in range(4, 13):   # L >= 16: L/2 + L/8 is even, so SIGMA is odd
        L = 1 << log2L
        assert O.sigma(L) % 2 == 1
        assert len({(k * O.sigma(L)) % L for k in range(L)}) == L


@pytest.mark.parametrize("L,nsym,seed", [(4096, 256, 0), (2048, 16, 1), (64, 5, 2), (16, 16, 3)])
def test_build_spread_closed_form(L, nsym, seed):
    """The k-th placement (symbols in ascending order) lands on k*SIGMA mod L."""
    rng = np.random.default_rng(seed)
    p = rng.random(nsym) ** 3
    p /= p.sum()
    f = O.quantize_freqs(p, L)
    sp = O.build_spread(f, L)
    order = np.repeat(np.arange(nsym), f)
    slots = (np.arange(L) * O.sigma(L)) % L
    closed = np.empty(L, np.int64)
    closed[slots] = order
    assert np.array_equal(sp, closed)
    assert np.array_equal(np.bincount(sp, minlength=nsym), f)


@pytest.mark.parametrize("L,nsym", [(4096, 256), (2048, 16), (256, 7)])
def test_slot_table_invariants(L, nsym):
    rng = np.random.default_rng(L)
    p = rng.random(nsym) ** 2
    p /= p.sum()
    f = O.quantize_freqs(p, L)
    sp = O.build_spread(f, L)
    sym, nb, base = O.slot_table(sp, f, L)
    assert (base >= L).all() and (base < 2 * L).all()
    assert ((base + (1 << nb) - 1) < 2 * L).all()
    for s in range(nsym):
        m = sym == s
        xp = base[m] >> nb[m]
        # the slots of s cover x_prev in [f_s, 2 f_s) once each, in slot order
        assert np.array_equal(xp, np.arange(f[s], 2 * f[s]))
        assert ((base[m] >> nb[m]) << nb[m] == base[m]).all()


def _tiny_tans_roundtrip(f, msg):
    """Brute-force tANS on a tiny table: encode with the textbook
    construction (state x in [L, 2L), emit low bits until x < 2 f_s, jump to
    the rank-th slot of s), decode with the oracle's slot table."""
    L = int(np.sum(f))
    sp = O.build_spread(f, L)
    sym, nb, base = O.slot_table(sp, f, L)
    enc = {}
    rank = np.zeros(len(f), np.int64)
    for slot in range(L):
        s = int(sp[slot])
        enc[(s, int(f[s] + rank[s]))] = L + slot
        rank[s] += 1
    x, bits = L, []
    for s in reversed(msg):
        chunk = []
        while x >= 2 * f[s]:
            chunk.append(x & 1)
            x >>= 1
        bits.append(chunk[::-1])          # read back most significant first
        x = enc[(s, x)]
    stream = [b for chunk in reversed(bits) for b in chunk]
    out, pos = [], 0
    for _ in msg:
        slot = x - L
        k = int(nb[slot])
        v = 0
        for _ in range(k):
            v = (v << 1) | stream[pos]
            pos += 1
        out.append(int(sym[slot]))
        x = int(base[slot]) + v
    assert x == L and pos == len(stream)
    return out


@pytest.mark.parametrize("f", [[15, 1], [3, 1, 12], [5, 2, 1, 8], [1] * 16, [40, 3, 1, 20]])
def test_slot_table_decodes_textbook_tans(f):
    rng = np.random.default_rng(len(f))
    f = np.array(f)
    for n in (1, 2, 7, 40):
        msg = [int(s) for s in rng.choice(len(f), size=n, p=f / f.sum())]
        assert _tiny_tans_roundtrip(f, msg) == msg


def test_ref_decode_table_packing():
    f = O.quantize_freqs(GOLDEN["qf_pair_qwen_in"], 4096)
    sp = O.build_spread(f, 4096)
    t = O.ref_decode_table(sp, f)
    sym, nb, base = O.slot_table(sp, f, 4096)
    assert np.array_equal(t & 0xFF, sym)
    assert np.array_equal((t >> 8) & 0xF, nb)
    assert np.array_equal(t >> 16, base)


# --------------------------------------------------------------------------
# Generators (reference rans_vectoradd/data.py:41-69)
# --------------------------------------------------------------------------

def test_random_fp8_bytes_matches_reference_golden():
    from rans_vectoradd import data as D
    torch.manual_seed(42)
    assert np.array_equal(D.random_fp8_bytes(128 * 128, device="cpu").numpy(),
                          GOLDEN["rand_seed42_n16384"])
    torch.manual_seed(0)
    assert np.array_equal(D.random_fp8_bytes(4096, device="cpu").numpy(), GOLDEN["rand_seed0_a_n4096"])
    assert np.array_equal(D.random_fp8_bytes(4096, device="cpu").numpy(), GOLDEN["rand_seed0_b_n4096"])
    g = torch.Generator().manual_seed(7)
    got = D.random_fp8_bytes(2048, exp_probs=tuple([1.0] * 16), device="cpu", generator=g)
    assert np.array_equal(got.numpy(), GOLDEN["rand_gen7_flat_n2048"])


def test_gaussian_generator_is_rne_of_scaled_samples():
    """Config 0 input: N(0, 0.02) scaled so |max| -> 448, RNE-cast.  Checked
    against the oracle's own double -> E4M3 rounding."""
    from rans_vectoradd import data as D
    n = 1 << 16
    q, inv_scale = D.gaussian_fp8_bytes(n, seed=3)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(n, generator=g) * 0.02).double()
    scale = 448.0 / float(x.abs().max())
    lib = O.lib()
    import ctypes
    lib.ora_double_to_fp8_rne_sat.restype = ctypes.c_uint8
    lib.ora_double_to_fp8_rne_sat.argtypes = [ctypes.c_double]
    xs = (x.float() * torch.tensor(scale, dtype=torch.float32)).double().numpy()
    want = np.array([lib.ora_double_to_fp8_rne_sat(float(v)) for v in xs[:4096]], np.uint8)
    assert np.array_equal(q.numpy()[:4096], want)
    assert ((q.numpy() & 0x7F) == 0x7E).any()            # |max| maps to 448
    assert not NAN[q.numpy()].any()
    assert abs(inv_scale * 448.0 - float(x.abs().max())) < 1e-9


# --------------------------------------------------------------------------
# Reference-format codec restatement (csrc/tans_codec.cpp, tans_decode.cu,
# vecadd.cu): round trips and agreement with the add table
# --------------------------------------------------------------------------

def _ref_setup(K, N, seed):
    from rans_vectoradd import data as D
    torch.manual_seed(seed)
    fp8 = D.random_fp8_bytes(K * N, device="cpu").reshape(K, N).numpy()
    p = np.asarray(D.QWEN3_14B_FP8_EXP, dtype=np.float32)
    p = p / p.sum()
    f = O.quantize_freqs((p[:, None] * p[None, :]).reshape(-1), 4096)
    sp = O.build_spread(f, 4096)
    return fp8, f, sp


@pytest.mark.parametrize("K,N", [(128, 128), (1000, 64), (129, 16), (3, 256)])
def test_ref_codec_roundtrip(K, N):
    fp8, f, sp = _ref_setup(K, N, 42)
    comp, states, offsets, partial = O.ref_encode(O.pair_symbols(fp8), f, sp)
    assert offsets[0] == 0 and offsets[-1] == comp.size
    assert ((states >= 4096) & (states < 8192)).all()
    out = O.ref_decode(comp, offsets, states, partial, O.ref_sm(fp8, 0), O.ref_decode_table(sp, f), K, N)
    assert np.array_equal(out.T, fp8)


def test_ref_decode_add_matches_lut():
    K, N = 300, 128
    a, f, sp = _ref_setup(K, N, 0)
    b, _, _ = _ref_setup(K, N, 1)
    lut = O.add_lut()
    ea = O.ref_encode(O.pair_symbols(a), f, sp)
    eb = O.ref_encode(O.pair_symbols(b), f, sp)
    tiled = O.ref_decode_add((ea[0], ea[2], ea[1], ea[3], O.ref_sm(a, 8)),
                             (eb[0], eb[2], eb[1], eb[3], O.ref_sm(b, 8)),
                             O.ref_decode_table(sp, f), lut, K, N)
    got = tiled.reshape(N // 16, K, 16).transpose(1, 0, 2).reshape(K, N)
    assert np.array_equal(got, O.vecadd(lut, a, b).reshape(K, N))


def test_ref_encoder_rejects_missing_symbol():
    fp8, f, sp = _ref_setup(4, 32, 5)
    syms = O.pair_symbols(fp8)
    f2 = f.copy()
    s = int(syms[0, 0])
    donor = int(np.argmax(f2))
    f2[donor] += f2[s]
    f2[s] = 0
    with pytest.raises(ValueError):
        O.ref_encode(syms, f2, O.build_spread(f2, 4096))
