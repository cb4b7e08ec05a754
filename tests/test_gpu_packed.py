"""The packed layout of short streams on the GPU (pair alphabet, at most 64
elements per lane; include/tans_amd.h): argument checks through the Python
API and the C ABI, mixed layouts, a HIP graph replay, and packed against
refill-schedule encodings of the same data.  Shapes, tables and stream
lengths are swept by test_gpu_kernels.py and test_gpu_random_shapes.py,
whose "pair" cases at N <= 64 take this layout."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ORDER = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


def _pair(R, K, N, seed, layout="auto"):
    from rans_vectoradd import tans_codec as T
    exp = torch.tensor(R.QWEN3_14B_FP8_EXP, dtype=torch.float64)
    torch.manual_seed(seed)
    fa = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    fb = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    ea = [x.cuda() for x in T.encode(fa, exp, layout=layout)]
    eb = [x.cuda() for x in T.encode(fb, exp, layout=layout)]
    tbl = T.build_decode_table(ea[6].cpu().numpy(), ea[5].cpu().numpy()).cuda()
    return fa, fb, ea, eb, tbl


@pytest.mark.parametrize("N", [16, 32, 48, 64])
def test_packed_and_words_agree(R, lut, N):
    """The same data through both layouts: the fused add and the decoder
    give the same bytes, which are the raw add's and the input."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: packed vs words K=1000 N={N}")
    K = 1000
    fa, fb, pa, pb, tbl = _pair(R, K, N, seed=N)
    _, _, wa, wb, _ = _pair(R, K, N, seed=N, layout="words")
    assert pa[1].numel() == 0 and wa[1].numel() == K
    fp = R.fp8_vecadd_fused_tans(*[pa[i] for i in ORDER], *[pb[i] for i in ORDER], tbl, N)
    fw = R.fp8_vecadd_fused_tans(*[wa[i] for i in ORDER], *[wb[i] for i in ORDER], tbl, N)
    assert torch.equal(fp, fw)
    raw = R.fp8_vecadd_raw(fa.flatten().cuda(), fb.flatten().cuda()).cpu().reshape(K, N)
    assert torch.equal(T.untile(fp.cpu(), K, N), raw)
    for e, f in ((pa, fa), (wa, fa)):
        dec = R.gpu_tans_decode(e[0], e[2], e[1], e[3], e[4], e[6], e[5], N)
        assert torch.equal(dec.cpu().t().contiguous(), f)


def test_packed_argument_checks(R):
    """An encoding without states is the packed layout: mixing it with one
    that has states, using it past 64 elements per lane or with the nibble
    table raises (Python) or returns TANS_EINVAL (C ABI)."""
    from rans_vectoradd import tans_codec as T
    from rans_vectoradd._lib import lib
    _say("case: packed-layout argument checks")
    K, N = 128, 32
    fa, fb, pa, pb, tbl = _pair(R, K, N, seed=1)
    _, _, wa, wb, _ = _pair(R, K, N, seed=1, layout="words")
    with pytest.raises(RuntimeError, match="share a layout"):
        R.fp8_vecadd_fused_tans(*[pa[i] for i in ORDER], *[wb[i] for i in ORDER], tbl, N)
    stream = torch.cuda.current_stream().cuda_stream
    out = torch.empty(K * 80, dtype=torch.uint8, device="cuda")
    sm80 = torch.zeros(5 * K * 8, dtype=torch.uint8, device="cuda")
    # N = 80 with no states
    rc = lib.tans_fp8_vecadd_fused(pa[0].data_ptr(), pa[0].numel(), pa[2].data_ptr(), None,
                                   sm80.data_ptr(), pb[0].data_ptr(), pb[0].numel(),
                                   pb[2].data_ptr(), None, sm80.data_ptr(), tbl.data_ptr(), 12,
                                   K, 80, out.data_ptr(), stream)
    assert rc == -1
    rc = lib.tans_decode(pa[0].data_ptr(), pa[0].numel(), pa[2].data_ptr(), None,
                         sm80.data_ptr(), tbl.data_ptr(), 12, K, 80, out.data_ptr(), stream)
    assert rc == -1
    # one side without states
    rc = lib.tans_fp8_vecadd_fused(pa[0].data_ptr(), pa[0].numel(), pa[2].data_ptr(), None,
                                   pa[4].data_ptr(), wb[0].data_ptr(), wb[0].numel(),
                                   wb[2].data_ptr(), wb[1].data_ptr(), wb[4].data_ptr(),
                                   tbl.data_ptr(), 12, K, N, out.data_ptr(), stream)
    assert rc == -1
    # the nibble table
    ntbl = torch.zeros(2 * 2048, dtype=torch.int32, device="cuda")
    rc = lib.tans_decode(pa[0].data_ptr(), pa[0].numel(), pa[2].data_ptr(), None,
                         pa[4].data_ptr(), ntbl.data_ptr(), 11, K, N, out.data_ptr(), stream)
    assert rc == -1
    torch.cuda.synchronize()
    # the same calls with valid arguments work afterwards
    dec = R.gpu_tans_decode(pa[0], pa[2], pa[1], pa[3], pa[4], pa[6], pa[5], N)
    assert torch.equal(dec.cpu().t().contiguous(), fa)


def test_packed_replay_in_a_hip_graph(R):
    """Packed fused add and decode captured in one HIP graph: every replay,
    with eager work and host synchronisations between, gives the eager
    results."""
    _say("case: packed fused add + decode in a HIP graph")
    K, N = 4100, 48
    fa, fb, ea, eb, tbl = _pair(R, K, N, seed=3)
    fused_args = [*[ea[i] for i in ORDER], *[eb[i] for i in ORDER], tbl, N]
    dec_args = [ea[0], ea[2], ea[1], ea[3], ea[4], ea[6], ea[5], N]

    def step():
        return R.fp8_vecadd_fused_tans(*fused_args), R.gpu_tans_decode(*dec_args)

    eager_sum, eager_dec = step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
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
        step()
        torch.cuda.synchronize()
    assert torch.equal(eager_dec.cpu().t().contiguous(), fa)


@pytest.mark.parametrize("N", [16, 64])
def test_packed_config1_data_2p24(R, lut, N):
    """Config-1 data (N(0, 0.02) scaled to 448, own histogram) at 2^24
    elements per vector in the packed layout: several groups per wave
    (2^24 / 16 / 64 = 16384 groups at 16 per lane), fused == the oracle's
    add table, decode == input, and the sizes of the 1Ki / 4Ki sweep
    points."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: packed config-1 data 2^24, {N} per lane")
    n = 1 << 24
    K = n // N
    qa, _ = D.gaussian_fp8_bytes(n, seed=21)
    qb, _ = D.gaussian_fp8_bytes(n, seed=22)
    hist = D.exp_histogram(torch.cat([qa, qb]))
    ea = T.encode(qa.reshape(K, N), hist)
    eb = T.encode(qb.reshape(K, N), hist)
    bits = 8 * (T.compressed_bytes(*ea[:5]) + T.compressed_bytes(*eb[:5])) / (2 * n)
    assert bits <= (7.8 if N == 16 else 7.0), bits
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy()).cuda()
    a = [x.cuda() for x in ea]
    b = [x.cuda() for x in eb]
    fused = T.untile(R.fp8_vecadd_fused_tans(*[a[i] for i in ORDER], *[b[i] for i in ORDER],
                                             tbl, N).cpu(), K, N).numpy()
    assert np.array_equal(fused, O.vecadd(lut, qa.numpy(), qb.numpy()).reshape(K, N))
    dec = R.gpu_tans_decode(a[0], a[2], a[1], a[3], a[4], a[6], a[5], N)
    assert torch.equal(dec.cpu(), qa.reshape(K, N).t())
