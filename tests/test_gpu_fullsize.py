"""Parity at the benchmark configurations' full sizes, through properties that
do not depend on size:

* config 1 (2^29 elements per vector): the fused tANS add equals the raw add
  on every element, and the raw add equals the oracle's add table (RNE,
  satfinite) on every element, so the fused output is pinned to the oracle;
  the headline encoding stays within 7 bits per FP8 byte, and the packed
  layout's 1Ki / 4Ki streams within 7.8 / 7.0;
* config 2 (2^30 elements): the standalone decode returns its input, for
  both tables (Gaussian and Laplace data) and both alphabets;
* the GPU encoder's bytes at 2^29 elements equal the CPU encoder's.

Inputs are generated on the GPU (seeded torch generators) and encoded with
encode_gpu, which the smaller tests pin byte for byte to the CPU encoder.
Each case prints its name before it touches the GPU."""
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

VEC_ELEMS = 1 << 29      # config 1: elements per vector
DEC_ELEMS = 1 << 30      # config 2: elements decoded per call
CHUNK = 1 << 26          # elements per oracle-table lookup on the GPU


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


@pytest.fixture(scope="module")
def vectors(R):
    """Config-1 inputs a, b (N(0, 0.02) scaled to 448, seeds 1 and 2), their
    joint exponent histogram, and the raw add checked against the oracle."""
    from rans_vectoradd import data as D
    _say("case: config-1 inputs, raw add vs the oracle table (2^29)")
    qa, _ = D.gaussian_fp8_bytes(VEC_ELEMS, seed=1, device="cuda")
    qb, _ = D.gaussian_fp8_bytes(VEC_ELEMS, seed=2, device="cuda")
    hist = D.exp_histogram(torch.cat([qa, qb])).cpu()
    raw = R.fp8_vecadd_raw(qa, qb)
    lut = torch.from_numpy(O.add_lut().reshape(-1)).cuda()
    nan = torch.from_numpy(O.nan_mask_lut().reshape(-1)).cuda()
    for s in range(0, VEC_ELEMS, CHUNK):
        idx = qa[s:s + CHUNK].long() * 256 + qb[s:s + CHUNK].long()
        ok = (raw[s:s + CHUNK] == lut[idx]) | nan[idx]
        assert bool(ok.all()), f"raw add differs from the oracle in elements [{s}, {s + CHUNK})"
    del lut, nan
    return qa, qb, hist, raw


@pytest.mark.parametrize("alphabet,lane", [("pair", 1024), ("pair", 16), ("nibble", 1024)])
def test_vecadd_config1_full_size(R, vectors, alphabet, lane):
    """64Ki-element streams (1024 per lane) and 1Ki-element streams (16 per
    lane): fused == raw on all 2^29 elements."""
    from rans_vectoradd import tans_codec as T
    qa, qb, hist, raw = vectors
    _say(f"case: fused vecadd 2^29 {alphabet} {lane} per lane")
    K = VEC_ELEMS // lane
    ea = T.encode_gpu(qa.reshape(K, lane), hist, tile=8, alphabet=alphabet)
    eb = T.encode_gpu(qb.reshape(K, lane), hist, tile=8, alphabet=alphabet)
    tbl = T.build_decode_table(ea[6].cpu().numpy(), ea[5].cpu().numpy()).cuda()
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    out = R.fp8_vecadd_fused_tans(*[ea[i] for i in order], *[eb[i] for i in order], tbl, lane)
    fused = out.view(lane // 16, K, 16).permute(1, 0, 2).reshape(-1)
    assert torch.equal(fused, raw)
    if alphabet == "pair" and lane == 1024:
        bits = 8 * (T.compressed_bytes(*ea[:5]) + T.compressed_bytes(*eb[:5])) / (2 * VEC_ELEMS)
        assert bits <= 7.0, f"{bits:.3f} bits per FP8 byte"


@pytest.mark.parametrize("lane,max_bits", [(16, 7.8), (64, 7.0)])
def test_vecadd_config1_full_size_packed(R, vectors, lane, max_bits):
    """1Ki- and 4Ki-element streams (16 and 64 per lane) in the packed
    layout, encoded on the CPU: fused == raw on all 2^29 elements, at most
    7.8 and 7.0 bits per FP8 byte."""
    from rans_vectoradd import tans_codec as T
    qa, qb, hist, raw = vectors
    _say(f"case: fused vecadd 2^29 pair {lane} per lane, packed layout")
    K = VEC_ELEMS // lane
    ea = T.encode(qa.cpu().reshape(K, lane), hist.numpy())
    eb = T.encode(qb.cpu().reshape(K, lane), hist.numpy())
    assert ea[1].numel() == 0 and eb[1].numel() == 0
    bits = 8 * (T.compressed_bytes(*ea[:5]) + T.compressed_bytes(*eb[:5])) / (2 * VEC_ELEMS)
    assert bits <= max_bits, f"{bits:.3f} bits per FP8 byte"
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy()).cuda()
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    a = [ea[i].cuda() for i in order]
    b = [eb[i].cuda() for i in order]
    del ea, eb
    out = R.fp8_vecadd_fused_tans(*a, *b, tbl, lane)
    fused = out.view(lane // 16, K, 16).permute(1, 0, 2).reshape(-1)
    assert torch.equal(fused, raw)


@pytest.mark.parametrize("alphabet", ["pair", "nibble"])
@pytest.mark.parametrize("dist", ["gaussian", "laplace"])
def test_decode_config2_full_size(R, alphabet, dist):
    """2^30 elements, 1024 per lane, the data's own table: the decoder's
    [N, K] output is the input, transposed."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: gpu_tans_decode 2^30 {dist} {alphabet}")
    lane = 1024
    K = DEC_ELEMS // lane
    gen = D.gaussian_fp8_bytes if dist == "gaussian" else D.laplace_fp8_bytes
    q, _ = gen(DEC_ELEMS, seed=3, device="cuda")
    hist = D.exp_histogram(q).cpu()
    comp, st, off, part, sm, fr, sp = T.encode_gpu(q.reshape(K, lane), hist, alphabet=alphabet)
    out = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, lane)
    assert torch.equal(out, q.view(K, lane).t())


def test_gpu_encoder_matches_cpu_full_size(R, vectors):
    """The GPU encoder's output for config 1's vector a equals the CPU
    encoder's, tensor for tensor."""
    from rans_vectoradd import tans_codec as T
    qa, _, hist, _ = vectors
    _say("case: encode_gpu vs encode, 2^29 pair")
    lane = 1024
    K = VEC_ELEMS // lane
    gpu = T.encode_gpu(qa.reshape(K, lane), hist, tile=8)
    cpu = T.encode(qa.cpu().reshape(K, lane), hist.numpy(), tile=8)
    names = ("comp", "states", "offsets", "partial", "sm", "freqs", "spread")
    for name, c, g in zip(names, cpu, gpu):
        assert torch.equal(c, g.cpu()), f"{name} differs"
