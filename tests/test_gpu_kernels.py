"""GPU parity tests: every kernel through the C ABI, checked bit for bit
against the CPU oracle (oracle/) on seeded inputs.

Mirrors the reference's own scripts: test_gpu_decode_tans.py (round trip,
cases :69-74, seed 42) and test_vecadd_tans.py (fused == raw, cases :76-80,
seed 0), adding the absolute check of every add against the oracle's
RNE-satfinite table and both alphabets."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ALPHABETS = ["pair", "nibble"]
# alphabet[:layout] for the tests with lanes of at most 64 elements, where
# "pair" means the packed layout and "pair:words" the refill-schedule one
CODECS = ["pair", "pair:words", "nibble"]


def _codec(codec):
    """encode() keywords of a CODECS entry."""
    alphabet, _, layout = codec.partition(":")
    return dict(alphabet=alphabet, layout=layout or "auto")


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


def test_add_all_pairs_vs_oracle(R, lut):
    _say("case: fp8_vecadd_raw over all 65536 byte pairs")
    a = torch.arange(256, dtype=torch.uint8).repeat_interleave(256)
    b = torch.arange(256, dtype=torch.uint8).repeat(256)
    out = R.fp8_vecadd_raw(a.cuda(), b.cuda()).cpu().numpy().reshape(256, 256)
    nan = O.nan_mask_lut()
    bad = (out != lut) & ~nan
    assert not bad.any(), f"{bad.sum()} mismatches, first {np.argwhere(bad)[:5].tolist()}"
    # NaN operands must give a NaN byte (the encoding is not pinned)
    assert ((out[nan] & 0x7F) == 0x7F).all()


def test_memcpy(R):
    _say("case: fp8_memcpy 1 MiB + 16 B")
    x = torch.randint(0, 256, ((1 << 20) + 16,), dtype=torch.uint8, device="cuda")
    assert torch.equal(R.fp8_memcpy(x), x)


@pytest.mark.parametrize("nontemporal", [True, False])
def test_stream_probes(R, nontemporal):
    """The bandwidth probes move the bytes they claim: 2:1 writes a ^ b,
    write-only writes its index pattern, read-only runs without error."""
    from rans_vectoradd import _C as C
    n = (1 << 20) + 16
    _say(f"case: stream_probe n={n} nt={nontemporal}")
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    b = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    assert torch.equal(C.stream_probe("stream21", a, b, nontemporal=nontemporal), a ^ b)
    w = C.stream_probe("write", out=torch.zeros_like(a), nontemporal=nontemporal)
    i = torch.arange(n // 16, dtype=torch.int64, device="cuda")
    words = torch.stack([i, i ^ 0x55555555, i ^ 0xAAAAAAAA, i ^ 0xFFFFFFFF], dim=1)
    assert torch.equal(w.view(torch.int32).view(-1, 4).long() & 0xFFFFFFFF, words)
    assert C.stream_probe("read", a, nontemporal=nontemporal) is None
    torch.cuda.synchronize()


def test_raw_ragged_sizes(R, lut):
    for n in (16, 4096 + 16, 1 << 16):
        _say(f"case: fp8_vecadd_raw n={n}")
        g = torch.Generator().manual_seed(n)
        a = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g)
        b = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g)
        out = R.fp8_vecadd_raw(a.cuda(), b.cuda()).cpu().numpy()
        ref = O.vecadd(lut, a.numpy(), b.numpy())
        ok = (out == ref) | O.nan_mask_lut()[a.numpy(), b.numpy()]
        assert ok.all()


@pytest.mark.parametrize("alphabet", ALPHABETS)
def test_table_device_matches_host(R, alphabet):
    from rans_vectoradd import _C, tans_codec as T
    _say(f"case: device table == host table ({alphabet})")
    freqs = T.symbol_freqs(R.QWEN3_14B_FP8_EXP, alphabet)
    spread = T.build_spread(freqs)
    host = T.build_decode_table(spread, freqs)
    dev = torch.empty_like(host).cuda()
    sp = torch.from_numpy(spread).cuda()
    fr = torch.from_numpy(freqs).cuda()
    from rans_vectoradd._lib import check, lib
    import ctypes
    check(lib.tans_build_decode_table_device(ctypes.c_void_p(sp.data_ptr()),
                                             ctypes.c_void_p(fr.data_ptr()), fr.numel(),
                                             spread.size.bit_length() - 1,
                                             ctypes.c_void_p(dev.data_ptr()), None, None),
          "table")
    torch.cuda.synchronize()
    assert torch.equal(dev.cpu(), host)


@pytest.mark.parametrize("alphabet", ALPHABETS)
def test_table_device_any_spread(R, alphabet):
    """Device table for a spread that is not the hash walk: the symbol
    multiset of the frequencies in a random slot order."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: device table, shuffled spread ({alphabet})")
    nsym, L = (256, 4096) if alphabet == "pair" else (16, 2048)
    rng = np.random.default_rng(11)
    f = T.symbol_freqs(R.QWEN3_14B_FP8_EXP, alphabet)
    sp = rng.permutation(np.repeat(np.arange(nsym, dtype=np.int32), f)).astype(np.int32)
    host = T.build_decode_table(sp, f)
    dev = torch.empty(2 * L, dtype=torch.int32, device="cuda")
    from rans_vectoradd._lib import lib
    stream = torch.cuda.current_stream().cuda_stream
    sp_d = torch.from_numpy(sp).cuda()
    f_d = torch.from_numpy(f).cuda()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert lib.tans_build_decode_table_device(sp_d.data_ptr(), f_d.data_ptr(), nsym,
                                              L.bit_length() - 1, dev.data_ptr(),
                                              status.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(dev.cpu(), host)
    assert status.item() == 0


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("K,N", [(128, 128), (1024, 128), (10000, 128), (100000, 128),
                                 (64, 2), (65, 18), (200, 130), (3, 1000),
                                 (130, 30), (192, 64), (66, 80), (1, 16), (4096, 14),
                                 (2064, 48)])
def test_decode_roundtrip(R, alphabet, K, N):
    """The reference's cases (test_gpu_decode_tans.py:69-74) plus ragged
    ones: partial last groups of 1, 2, 3, 8, 16, 32 lanes, a wave holding one
    complete group and no second one (K = 192), and last tiles of 2, 8, 14
    elements.  Complete waves store whole lines when K % 16 == 0 (rows 16-byte
    aligned but not line-aligned at K = 10000 and 2064) and single words
    otherwise (K = 200, 130)."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: gpu_tans_decode K={K} N={N} {alphabet}")
    exp_freqs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    torch.manual_seed(42)
    fp8 = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    comp, st, off, part, sm, fr, sp = T.encode(fp8, exp_freqs, **_codec(alphabet))
    dec = R.gpu_tans_decode(comp.cuda(), off.cuda(), st.cuda(), part.cuda(), sm.cuda(),
                            sp.cuda(), fr.cuda(), N)
    got = dec.cpu().t().contiguous()
    assert torch.equal(got, fp8), f"{(got != fp8).sum().item()} mismatched bytes"


@pytest.mark.parametrize("alphabet,N", [("pair", 20), ("pair", 36), ("pair", 18),
                                         ("pair", 52), ("nibble", 18), ("nibble", 34),
                                         ("nibble", 66)])
@pytest.mark.parametrize("K", [4096, 1000])
def test_decode_last_tile_of_one_segment(R, alphabet, N, K):
    """Streams whose last tile holds a single refill segment (pair: N % 16 =
    2 or 4, nibble: N % 16 = 2, with N > 16), so the final refill check
    follows the last segment of the tile before.  Uniformly random bytes
    coded with the Qwen3 exponent table (which does not match them): many
    lanes hold between the final check's threshold and 32 bits there, so a
    decoder that gave them a word would shift the ranks of the lanes that
    need one.  Decode returns the input."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: gpu_tans_decode one-segment last tile K={K} N={N} {alphabet}")
    g = torch.Generator().manual_seed(N * 7 + K)
    fp8 = torch.randint(0, 256, (K, N), dtype=torch.uint8, generator=g)
    exp_freqs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    comp, st, off, part, sm, fr, sp = [x.cuda() for x in T.encode(fp8, exp_freqs,
                                                                  alphabet=alphabet,
                                                                  layout="words")]
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    got = dec.cpu().t().contiguous()
    assert torch.equal(got, fp8), f"{(got != fp8).sum().item()} mismatched bytes"


def _invalid_tables(exp_probs, alphabet):
    """(name, spread, freqs) triples the host builder rejects with
    TANS_ETABLE."""
    from rans_vectoradd import tans_codec as T
    f = T.symbol_freqs(exp_probs, alphabet).astype(np.int32)
    sp = T.build_spread(f).astype(np.int32)
    out = []
    if alphabet == "nibble":
        # the rarest present symbol at frequency 1, the surplus on the most
        # frequent one (the sum stays L)
        g = f.copy()
        i = int(np.argmax(g))
        j = int(np.argmin(np.where(g > 0, g, 1 << 30)))
        g[i] += g[j] - 1
        g[j] = 1
        out.append(("a present symbol at frequency 1", T.build_spread(g).astype(np.int32), g))
    bad_sum = f.copy()
    bad_sum[int(np.argmax(f))] += 1
    out.append(("frequencies not summing to L", sp, bad_sum))
    bad_sp = sp.copy()
    bad_sp[5] = len(f) + 3
    out.append(("a spread symbol outside the alphabet", bad_sp, f))
    moved = sp.copy()
    k = int(np.argmax(sp != sp[0]))
    moved[k] = sp[0]              # one slot more for sp[0], one fewer for sp[k]
    out.append(("slot counts differing from the frequencies", moved, f))
    return out


@pytest.mark.parametrize("alphabet", ALPHABETS)
def test_table_device_rejects_what_the_host_rejects(R, alphabet):
    """The device table build reports TANS_ETABLE through its status word
    for each input the host builder rejects, and gpu_tans_decode raises
    RuntimeError for it (the reference's TORCH_CHECKs in its table build,
    csrc/tans_decode.cu:38,50); a valid pair keeps decoding after an
    invalid one."""
    from rans_vectoradd import tans_codec as T
    from rans_vectoradd._lib import lib
    L = 4096 if alphabet == "pair" else 2048
    stream = torch.cuda.current_stream().cuda_stream
    K, N = 256, 32
    fp8 = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    exp_probs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    comp, st, off, part, sm, fr, sp = [x.cuda() for x in T.encode(fp8, exp_probs,
                                                                  alphabet=alphabet)]
    for name, bsp, bfr in _invalid_tables(R.QWEN3_14B_FP8_EXP, alphabet):
        _say(f"case: invalid table ({alphabet}): {name}")
        assert lib.tans_build_decode_table(bsp.ctypes.data, bfr.ctypes.data, len(bfr),
                                           L.bit_length() - 1,
                                           np.zeros(2 * L, np.uint32).ctypes.data) == -4
        sp_d = torch.from_numpy(bsp).cuda()
        f_d = torch.from_numpy(bfr).cuda()
        tbl = torch.empty(2 * L, dtype=torch.int32, device="cuda")
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        assert lib.tans_build_decode_table_device(sp_d.data_ptr(), f_d.data_ptr(), len(bfr),
                                                  L.bit_length() - 1, tbl.data_ptr(),
                                                  status.data_ptr(), stream) == 0
        assert status.item() == -4, name
        with pytest.raises(RuntimeError, match="valid decode table"):
            R.gpu_tans_decode(comp, off, st, part, sm, sp_d, f_d, N)
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    assert torch.equal(dec.cpu().t().contiguous(), fp8)
    # an in-place change of a validated pair is checked again
    fr_bad = fr.clone()
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr_bad, N)
    fr_bad[int(torch.argmax(fr_bad))] += 1
    with pytest.raises(RuntimeError, match="valid decode table"):
        R.gpu_tans_decode(comp, off, st, part, sm, sp, fr_bad, N)


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("K,N", [(1024, 128), (10000, 256), (1024, 1024), (64, 16), (70, 32),
                                 (4160, 64), (130, 80), (1, 16), (5, 64), (127, 32)])
def test_vecadd_fused_vs_raw_and_oracle(R, lut, alphabet, K, N):
    """Streams of 1 tile (N = 16: one or two ring segments loaded at a
    group's start), of up to 4 tiles with pairs and 2 with nibbles (the whole
    stream loaded at the start) and longer ones (stage fetches), each with
    a partial last group where K % 64 != 0."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: fp8_vecadd_fused_tans K={K} N={N} {alphabet}")
    exp_freqs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    torch.manual_seed(0)
    fa = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    fb = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    ca, sa, oa, pa, sma, pf, sp = T.encode(fa, exp_freqs, tile=8, **_codec(alphabet))
    cb, sb, ob, pb, smb, _, _ = T.encode(fb, exp_freqs, tile=8, **_codec(alphabet))
    tbl = T.build_decode_table(sp.numpy(), pf.numpy())
    args = [t.cuda() for t in (ca, oa, sa, pa, sma, cb, ob, sb, pb, smb, tbl)]
    raw = R.fp8_vecadd_raw(fa.flatten().cuda(), fb.flatten().cuda()).cpu().reshape(K, N)
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N)
    assert torch.equal(fused, raw), f"{(fused != raw).sum().item()} bytes differ from raw"
    ref = O.vecadd(lut, fa.numpy(), fb.numpy()).reshape(K, N)
    ok = (fused.numpy() == ref) | O.nan_mask_lut()[fa.numpy(), fb.numpy()]
    assert ok.all()


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("K,N", [(600001, 18), (1048617, 16)])
def test_decode_several_group_pairs_per_wave(R, alphabet, K, N):
    """Columns of one or two tiles run one workgroup per CU (8192 group
    pairs per round on MI355X) and each wave loops over its pairs: here
    most waves decode two or more pairs, the last group partial (K % 64 =
    1 and 41) and, at N = 18, a last tile of 2 elements."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: gpu_tans_decode K={K} N={N} {alphabet} (several group pairs per wave)")
    assert (K + 63) // 64 > 2 * 4096
    exp_freqs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    torch.manual_seed(K)
    fp8 = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    comp, st, off, part, sm, fr, sp = T.encode(fp8, exp_freqs, **_codec(alphabet))
    dec = R.gpu_tans_decode(comp.cuda(), off.cuda(), st.cuda(), part.cuda(), sm.cuda(),
                            sp.cuda(), fr.cuda(), N)
    got = dec.cpu().t().contiguous()
    assert torch.equal(got, fp8), f"{(got != fp8).sum().item()} mismatched bytes"


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("K,N", [(300037, 16), (270000, 48)])
def test_vecadd_fused_several_groups_per_wave(R, lut, alphabet, K, N):
    """The fused kernel runs at most one workgroup per CU (4096 waves on
    MI355X) and each wave loops over groups w, w + 4096, ...  With K/64 >
    4096 groups most waves decode two or more groups in turn, the last one
    partial (K % 64 = 5 and 48), with last tiles of 16 elements (one tile
    per lane) and 48."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: fp8_vecadd_fused_tans K={K} N={N} {alphabet} (several groups per wave)")
    assert (K + 63) // 64 > 4096
    exp_freqs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    torch.manual_seed(K + N)
    fa = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    fb = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    ca, sa, oa, pa, sma, pf, sp = T.encode(fa, exp_freqs, **_codec(alphabet))
    cb, sb, ob, pb, smb, _, _ = T.encode(fb, exp_freqs, **_codec(alphabet))
    tbl = T.build_decode_table(sp.numpy(), pf.numpy())
    args = [t.cuda() for t in (ca, oa, sa, pa, sma, cb, ob, sb, pb, smb, tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N)
    ref = O.vecadd(lut, fa.numpy(), fb.numpy()).reshape(K, N)
    ok = (fused.numpy() == ref) | O.nan_mask_lut()[fa.numpy(), fb.numpy()]
    assert ok.all(), f"{(~ok).sum()} bytes differ from the oracle"


@pytest.mark.parametrize("alphabet", ALPHABETS)
@pytest.mark.parametrize("dist", ["gaussian", "laplace"])
def test_decode_config2_data_2p24(R, alphabet, dist):
    """Config-2 data (N(0, 0.02) and Laplace(0, 0.015), scaled to 448, the
    data's own table) at 2^24 elements, 1024 per lane: bit-exact round trip."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: gpu_tans_decode {dist} 2^24 {alphabet}")
    n, N = 1 << 24, 1024
    K = n // N
    gen = D.gaussian_fp8_bytes if dist == "gaussian" else D.laplace_fp8_bytes
    q, _ = gen(n, seed=5)
    hist = D.exp_histogram(q)
    assert (hist > 0).sum() >= 12           # a real spread of exponents
    e = T.encode(q.reshape(K, N), hist, alphabet=alphabet)
    comp, st, off, part, sm, fr, sp = [x.cuda() for x in e]
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    assert torch.equal(dec.cpu(), q.reshape(K, N).t())


@pytest.mark.parametrize("alphabet", ALPHABETS)
def test_vecadd_gaussian_2p24(R, lut, alphabet):
    """Config-1 inputs (N(0,0.02) scaled to 448, data's own histogram) at
    2^24 elements per vector, 1024 elements per lane."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: fused vecadd gaussian 2^24 {alphabet}")
    n, N = 1 << 24, 1024
    K = n // N
    qa, _ = D.gaussian_fp8_bytes(n, seed=1)
    qb, _ = D.gaussian_fp8_bytes(n, seed=2)
    hist = D.exp_histogram(torch.cat([qa, qb]))
    ea = T.encode(qa.reshape(K, N), hist, tile=8, alphabet=alphabet)
    eb = T.encode(qb.reshape(K, N), hist, tile=8, alphabet=alphabet)
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy())
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    args = [x.cuda() for x in (*[ea[i] for i in order], *[eb[i] for i in order], tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N).numpy()
    ref = O.vecadd(lut, qa.numpy(), qb.numpy()).reshape(K, N)
    assert np.array_equal(fused, ref)


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("N", [64, 256])
def test_vecadd_gaussian_short_streams(R, lut, alphabet, N):
    """Config-1 sweep points below the headline: 64 and 256 elements per
    lane (4Ki- and 16Ki-element streams of 64 lanes), N(0, 0.02) data at
    2^24 elements per vector, against the oracle's add table."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: fused vecadd gaussian 2^24, {N} per lane, {alphabet}")
    n = 1 << 24
    K = n // N
    qa, _ = D.gaussian_fp8_bytes(n, seed=11)
    qb, _ = D.gaussian_fp8_bytes(n, seed=12)
    hist = D.exp_histogram(torch.cat([qa, qb]))
    ea = T.encode(qa.reshape(K, N), hist, tile=8, **_codec(alphabet))
    eb = T.encode(qb.reshape(K, N), hist, tile=8, **_codec(alphabet))
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy())
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    args = [x.cuda() for x in (*[ea[i] for i in order], *[eb[i] for i in order], tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N).numpy()
    ref = O.vecadd(lut, qa.numpy(), qb.numpy()).reshape(K, N)
    assert np.array_equal(fused, ref)


def _few_exponent_bytes(K, N, exps, seed):
    """FP8 bytes whose exponent field takes only the values in `exps`
    (random sign and mantissa, never a NaN)."""
    g = torch.Generator().manual_seed(seed)
    e = torch.tensor(exps, dtype=torch.int64)[torch.randint(0, len(exps), (K, N), generator=g)]
    sm = torch.randint(0, 16, (K, N), generator=g)
    m = sm & 7
    m = torch.where(e == 15, torch.clamp(m, max=6), m)
    return (((sm >> 3) << 7) | (e << 3) | m).to(torch.uint8)


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("exps_a,exps_b", [((7,), (7,)), ((15,), (15,)), ((0,), (9,)),
                                           ((7, 8), (7, 8)), ((3,), (3, 12))])
def test_few_exponents_zero_bit_steps(R, lut, alphabet, exps_a, exps_b):
    """Tensors with one or two exponent values.  A one-exponent table gives
    the single symbol the whole state space (f = L), so every step reads 0
    bits and each lane's stream is one zero word (the reference guards
    nb = 0 at csrc/vecadd.cu:128).  Decode returns the input, the fused add
    equals the oracle's table, and the GPU encoder writes the CPU encoder's
    bytes."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: exponents {exps_a} + {exps_b} ({alphabet})")
    K, N = 200, 48
    fa = _few_exponent_bytes(K, N, exps_a, seed=1)
    fb = _few_exponent_bytes(K, N, exps_b, seed=2)
    hist = np.bincount(((torch.cat([fa, fb]).numpy() >> 3) & 15).ravel(), minlength=16)
    ea = T.encode(fa, hist, tile=8, **_codec(alphabet))
    eb = T.encode(fb, hist, tile=8, **_codec(alphabet))
    if len(set(exps_a) | set(exps_b)) == 1:
        tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy()).view(-1, 2)
        assert ((tbl[:, 0] & 0x1F) == 0).all()          # every entry reads 0 bits
    for f, e in ((fa, ea), (fb, eb)):
        comp, st, off, part, sm, fr, sp = [x.cuda() for x in e]
        dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
        assert torch.equal(dec.cpu().t().contiguous(), f)
        g = T.encode_gpu(f.cuda(), hist, tile=8, **_codec(alphabet))
        for i in (0, 1, 2, 4, 5, 6):
            assert torch.equal(g[i].cpu(), e[i]), f"GPU encoder output {i} differs"
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy())
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    args = [x.cuda() for x in (*[ea[i] for i in order], *[eb[i] for i in order], tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N).numpy()
    assert np.array_equal(fused, O.vecadd(lut, fa.numpy(), fb.numpy()).reshape(K, N))


@pytest.mark.parametrize("alphabet", ALPHABETS)
def test_streams_consumed_near_the_feed_limit(R, lut, alphabet):
    """Uniformly random bytes coded with a table built for a steep exponent
    histogram (p_e proportional to 2^-e): most symbols cost 8-12 bits, so
    lanes take a stream word at most refill checks and each wave's feed
    writes segments into its ring close to the stage in which they are
    first read.  Decode returns the input; the fused add equals the raw add
    and the oracle's table."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: fast-consumption streams {alphabet}")
    K, N = 4096, 256
    g = torch.Generator().manual_seed(7)
    fa = torch.randint(0, 256, (K, N), dtype=torch.uint8, generator=g)
    fb = torch.randint(0, 256, (K, N), dtype=torch.uint8, generator=g)
    steep = torch.tensor([2.0 ** -e for e in range(16)], dtype=torch.float64)
    ea = T.encode(fa, steep, tile=8, alphabet=alphabet)
    eb = T.encode(fb, steep, tile=8, alphabet=alphabet)
    assert T.compressed_bytes(*ea[:5]) * 8 / (K * N) > 9.0   # the streams are expensive
    comp, st, off, part, sm, fr, sp = [x.cuda() for x in ea]
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    assert torch.equal(dec.cpu().t().contiguous(), fa)
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy())
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    args = [x.cuda() for x in (*[ea[i] for i in order], *[eb[i] for i in order], tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N)
    raw = R.fp8_vecadd_raw(fa.flatten().cuda(), fb.flatten().cuda()).cpu().reshape(K, N)
    assert torch.equal(fused, raw)
    ref = O.vecadd(lut, fa.numpy(), fb.numpy()).reshape(K, N)
    ok = (fused.numpy() == ref) | O.nan_mask_lut()[fa.numpy(), fb.numpy()]
    assert ok.all()


@pytest.mark.parametrize("alphabet", CODECS)
@pytest.mark.parametrize("N", [16, 32, 48, 64, 80])
def test_longest_short_streams(R, lut, alphabet, N):
    """Streams at the most words a lane can take: every exponent 15, coded
    with a table for p_e proportional to 2^-e, so each step reads the most
    bits the table allows (12 with pairs, 10 with nibbles).  Up to 4 tiles
    (pairs) or 2 (nibbles) the kernels load such streams whole at a group's
    start; past that they fetch by stage.  Decode returns the input and the
    fused add equals the raw add and the oracle's table."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: longest streams N={N} {alphabet}")
    K = 461   # 7 full groups and one of 13 lanes
    g = torch.Generator().manual_seed(N)
    sm = torch.randint(0, 16, (2, K, N), dtype=torch.uint8, generator=g)
    sm = torch.where((sm & 7) == 7, sm - 1, sm)          # mantissa 7 with exponent 15 is NaN
    fa, fb = ((sm & 8) << 4) | (15 << 3) | (sm & 7)
    steep = torch.tensor([2.0 ** -e for e in range(16)], dtype=torch.float64)
    ea = T.encode(fa, steep, tile=8, **_codec(alphabet))
    eb = T.encode(fb, steep, tile=8, **_codec(alphabet))
    comp, st, off, part, smp, fr, sp = [x.cuda() for x in ea]
    dec = R.gpu_tans_decode(comp, off, st, part, smp, sp, fr, N)
    assert torch.equal(dec.cpu().t().contiguous(), fa)
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy())
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    args = [x.cuda() for x in (*[ea[i] for i in order], *[eb[i] for i in order], tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N)
    raw = R.fp8_vecadd_raw(fa.flatten().cuda(), fb.flatten().cuda()).cpu().reshape(K, N)
    assert torch.equal(fused, raw)
    assert np.array_equal(fused.numpy(), O.vecadd(lut, fa.numpy(), fb.numpy()).reshape(K, N))


@pytest.mark.parametrize("alphabet", ALPHABETS)
def test_decoders_replay_in_a_hip_graph(R, alphabet):
    """The fused add and the standalone decode (with its device table build)
    captured in one HIP graph: every replay, with eager launches and host
    synchronisations between replays, gives the eager results."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: fused add + decode in a HIP graph, {alphabet}")
    K, N = 2048, 128
    exp_freqs = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    torch.manual_seed(3)
    fa = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    fb = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    ea = [x.cuda() for x in T.encode(fa, exp_freqs, tile=8, alphabet=alphabet)]
    eb = [x.cuda() for x in T.encode(fb, exp_freqs, tile=8, alphabet=alphabet)]
    tbl = T.build_decode_table(ea[6].cpu().numpy(), ea[5].cpu().numpy()).cuda()
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    fused_args = [*[ea[i] for i in order], *[eb[i] for i in order], tbl, N]
    dec_args = [ea[0], ea[2], ea[1], ea[3], ea[4], ea[6], ea[5], N]

    def step():
        return R.fp8_vecadd_fused_tans(*fused_args), R.gpu_tans_decode(*dec_args)

    eager_sum, eager_dec = step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up off the default stream before capture
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        g_sum, g_dec = step()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_sum, eager_sum), f"replay {i}: fused add differs"
        assert torch.equal(g_dec, eager_dec), f"replay {i}: decode differs"
        step()                      # eager work between replays
        torch.cuda.synchronize()
    assert torch.equal(eager_dec.cpu().t().contiguous(), fa)
