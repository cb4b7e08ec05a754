"""GPU encoder (tans_codec.encode_gpu) against the CPU encoder, byte for byte:
compressed words, offsets, states and sign/mantissa tiles, at the reference's
test shapes (test_gpu_decode_tans.py:69-74, seed 42, Qwen3 histogram) and
ragged ones, then GPU encode -> GPU decode round trips on config data."""
import pytest
import torch

pytestmark = pytest.mark.gpu

ALPHABETS = ["pair", "nibble"]


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


def _compare(T, fp8, hist, alphabet, layout="auto"):
    cpu = T.encode(fp8, hist, alphabet=alphabet, layout=layout)
    gpu = T.encode_gpu(fp8.cuda(), hist, alphabet=alphabet, layout=layout)
    names = ("comp", "states", "offsets", "partial", "sm", "freqs", "spread")
    for name, c, g in zip(names, cpu, gpu):
        assert g.is_cuda, name
        assert torch.equal(c, g.cpu()), f"{name} differs"
    return gpu


SHAPES = [(128, 128), (1024, 128), (10000, 128), (100000, 128), (64, 2), (65, 18), (200, 130),
          (3, 1000), (1, 16), (127, 4096), (130, 30), (4096, 14), (300, 208), (70, 48),
          (2000, 20), (2000, 36), (1000, 34)]
# every shape with both alphabets; pair shapes of N <= 64 once more in the
# refill-schedule layout ("auto" gives them the packed one)
CASES = ([(a, K, N, "auto") for a in ALPHABETS for K, N in SHAPES]
         + [("pair", K, N, "words") for K, N in SHAPES if N <= 64])


@pytest.mark.parametrize("alphabet,K,N,layout", CASES)
def test_gpu_encode_matches_cpu(R, alphabet, K, N, layout):
    """N % 16 == 0 takes the backward pass that reads rows in 128-byte blocks
    (whole blocks at N = 128, 4096; a partial last block at 208, 48, 16) and
    writes the sign/mantissa tiles itself; the other widths read one step's
    bytes at a time and leave the tiles to enc_sm_kernel.  K % 64 != 0 and
    K < 64 give groups with lanes out of range; N = 2 (pair) is one step.
    N = 18, 20, 34, 36 end in a tile of one refill segment (18, 34 with both
    alphabets, 20, 36 with pairs), where the check before it is the plain
    one.  With the pair alphabet and N <= 64, layout "auto" is the packed
    layout of short streams (its own place pass)."""
    from rans_vectoradd import tans_codec as T
    _say(f"case: encode_gpu K={K} N={N} {alphabet} {layout}")
    torch.manual_seed(42)
    fp8 = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
    _compare(T, fp8, torch.tensor(R.QWEN3_14B_FP8_EXP), alphabet, layout)


@pytest.mark.parametrize("alphabet", ALPHABETS)
@pytest.mark.parametrize("dist", ["gaussian", "laplace"])
def test_gpu_encode_config_data_roundtrip(R, alphabet, dist):
    """2^24 config data (own histogram, 1024 per lane): GPU encode == CPU
    encode, and GPU decode of the GPU encoding == the input."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: encode_gpu {dist} 2^24 {alphabet}")
    n, N = 1 << 24, 1024
    gen = D.gaussian_fp8_bytes if dist == "gaussian" else D.laplace_fp8_bytes
    q, _ = gen(n, seed=9)
    fp8 = q.reshape(n // N, N)
    comp, st, off, part, sm, fr, sp = _compare(T, fp8, D.exp_histogram(q), alphabet)
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    assert torch.equal(dec.cpu(), fp8.t())


@pytest.mark.parametrize("N", [16, 64, 30])
def test_gpu_encode_packed_config_data(R, N):
    """Config-1 data (own histogram) in the packed layout of short streams,
    2^22 elements at 16, 64 and 30 elements per lane (several rounds of the
    place pass' workgroups; a ragged last tile at 30): GPU encode == CPU
    encode, and the GPU decode of it == the input."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: encode_gpu packed 2^22, {N} per lane")
    K = (1 << 22) // N
    q, _ = D.gaussian_fp8_bytes(K * N, seed=N)
    fp8 = q.reshape(K, N)
    comp, st, off, part, sm, fr, sp = _compare(T, fp8, D.exp_histogram(q), "pair")
    assert st.numel() == 0
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    assert torch.equal(dec.cpu(), fp8.t())


def test_gpu_encode_edge_cases(R):
    from rans_vectoradd import tans_codec as T
    exp = torch.tensor(R.QWEN3_14B_FP8_EXP)
    comp, st, off, part, sm, fr, sp = T.encode_gpu(torch.zeros((0, 16), dtype=torch.uint8).cuda(), exp)
    assert st.numel() == 0 and off.cpu().tolist() == [0] and comp.numel() == 1024
    assert int(comp.sum()) == 0
    # a symbol whose frequency is 0 is reported, as by the CPU encoder
    hist = torch.zeros(16)
    hist[7] = 1.0
    fp8 = torch.full((64, 32), 7 << 3, dtype=torch.uint8)
    fp8[5, 3] = 9 << 3
    with pytest.raises(RuntimeError, match="frequency is 0"):
        T.encode_gpu(fp8.cuda(), hist, alphabet="nibble")
    # a misaligned view (row offset of 2 bytes) encodes like a fresh copy
    torch.manual_seed(5)
    big = R.random_fp8_bytes(65 * 34, device="cpu").reshape(65, 34)
    view = big.cuda().reshape(-1)[2:2 + 64 * 34].reshape(64, 34)
    assert view.data_ptr() % 16 != 0
    a = T.encode_gpu(view, exp)
    b = T.encode(view.cpu().contiguous(), exp)
    assert torch.equal(a[0].cpu(), b[0]) and torch.equal(a[4].cpu(), b[4])
    with pytest.raises(ValueError):
        T.encode_gpu(torch.zeros((4, 16), dtype=torch.uint8), exp)       # CPU tensor
    with pytest.raises(ValueError):
        T.encode_gpu(torch.zeros((4, 15), dtype=torch.uint8).cuda(), exp)


@pytest.mark.parametrize("alphabet", ["pair", "nibble"])
@pytest.mark.parametrize("rows,cols,segments", [(17408, 5120, None), (5120, 17408, None),
                                                (100, 70, None), (130, 1000, 3), (1, 32, None)])
def test_encode_matrix_on_gpu_equals_cpu(R, alphabet, rows, cols, segments):
    """encode_matrix of a GPU tensor (padding, lane layout and encoder on the
    GPU) gives the CPU encoder's bytes, at config 3/4's shapes and ragged
    ones."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: encode_matrix on GPU {rows}x{cols} S={segments} {alphabet}")
    q, _ = D.gaussian_fp8_bytes(rows * cols, seed=rows + cols)
    w = q.reshape(rows, cols)
    hist = D.exp_histogram(q)
    a = T.encode_matrix(w.cuda(), hist, segments=segments, alphabet=alphabet)
    b = T.encode_matrix(w, hist, segments=segments, alphabet=alphabet)
    assert a.comp.is_cuda and (a.segments, a.seg_cols) == (b.segments, b.seg_cols)
    for part in ("comp", "states", "offsets", "sm", "freqs", "spread"):
        assert torch.equal(getattr(a, part).cpu(), getattr(b, part)), part


def test_checkpoint_container_on_gpu(R, tmp_path):
    """A checkpoint encoded with the GPU encoder into a container, loaded on
    the GPU: the lane tensor decodes to its bytes and the matrix gives the
    same product as the raw FP8 kernel."""
    import os
    from safetensors.torch import save_file
    from rans_vectoradd import container, data as D, ingest
    _say("case: checkpoint -> container -> GPU")
    w, scale = D.gaussian_fp8_bytes(1024 * 512, seed=21)
    v, _ = D.laplace_fp8_bytes(1 << 16, seed=22)
    src = os.path.join(tmp_path, "ckpt.safetensors")
    dst = os.path.join(tmp_path, "ckpt.tans.safetensors")
    save_file({"w": w.reshape(1024, 512).view(torch.float8_e4m3fn),
               "v": v.view(torch.float8_e4m3fn)}, src)
    ingest.encode_checkpoint(src, dst, device="cuda")
    got = container.load(dst, device="cuda")
    vec = got["v"]
    dec = R.gpu_tans_decode(vec.comp, vec.offsets, vec.states, vec.partial, vec.sm, vec.spread,
                            vec.freqs, vec.N)
    assert torch.equal(dec.t().reshape(-1).cpu(), v)
    m = got["w"]
    x = torch.randn(3, 512, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    y = R.fp8_gemm_fused_tans(m, m.decode_table().cuda(), x, scale).float()
    y_raw = R.fp8_gemm_raw(w.reshape(1024, 512).cuda(), x, scale).float()
    assert bool(((y - y_raw).abs() <= 2.0 ** -7 * y_raw.abs() + 1e-6).all())
