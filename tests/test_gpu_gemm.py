"""GPU tests of the fused decode + skinny GEMM (no
reference counterpart): y = scale * (W @ x^T) with W tANS-coded, checked
against a float64 product of the same FP8 weights and bf16 activations
(tolerance 1e-2 relative: |y - y_ref| <= 1e-2 |y_ref| + 1e-3 max|y_ref|
per element, which also bounds max|y - y_ref| / max|y_ref| by 1.1e-2), and
against the uncompressed FP8 kernel."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL, FLOOR = 1e-2, 1e-3


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


def _weights(rows, cols, seed, dist="gaussian"):
    from rans_vectoradd import data as D
    gen = D.gaussian_fp8_bytes if dist == "gaussian" else D.laplace_fp8_bytes
    q, scale = gen(rows * cols, seed=seed)
    return q.reshape(rows, cols), scale


def _x(B, cols, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, cols, generator=g).to(torch.bfloat16)


def _reference(w_u8, x_bf16, scale):
    w = w_u8.view(torch.float8_e4m3fn).to(torch.float64)
    return scale * (x_bf16.to(torch.float64) @ w.t())


def _check(y, ref):
    y = y.cpu().to(torch.float64)
    err = (y - ref).abs()
    bound = REL * ref.abs() + FLOOR * ref.abs().max()
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}, max|ref| {ref.abs().max().item():.3e}"
    assert err.max().item() <= 1.1e-2 * ref.abs().max().item()


def _fused(R, m, x, scale):
    from rans_vectoradd import tans_codec as T
    md = m.to("cuda")
    tbl = m.decode_table().cuda()
    return R.fp8_gemm_fused_tans(md, tbl, x.cuda(), scale)


@pytest.mark.parametrize("alphabet", ["pair", "nibble"])
@pytest.mark.parametrize("rows,cols,B,segments", [(2176, 1280, 1, None), (2176, 1280, 3, None),
                                                  (2176, 1280, 8, None), (100, 70, 2, None),
                                                  (130, 1000, 5, 3), (64, 512, 4, 1),
                                                  (5, 18, 7, None)])
def test_gemm_fused_vs_float64(R, alphabet, rows, cols, B, segments):
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: fp8_gemm_fused_tans {rows}x{cols} B={B} S={segments} {alphabet}")
    w, scale = _weights(rows, cols, seed=rows + cols)
    x = _x(B, cols, seed=B)
    m = T.encode_matrix(w, D.exp_histogram(w), segments=segments, alphabet=alphabet)
    y = _fused(R, m, x, scale)
    assert y.shape == (B, rows) and y.dtype == torch.bfloat16
    _check(y, _reference(w, x, scale))


@pytest.mark.parametrize("alphabet", ["pair", "nibble"])
@pytest.mark.parametrize("rows,cols,B,segments", [(48, 96, 8, 1), (200, 544, 6, 2),
                                                  (64, 2048, 2, None), (1, 32, 1, None),
                                                  (130, 1000, 7, 1)])
def test_gemm_fused_half_tiles_and_odd_shapes(R, alphabet, rows, cols, B, segments):
    """Segment widths ending in a half tile (96, 288, 1000 -> 1024 columns of
    which the last 24 are padding), a single row, one segment of 1024
    columns, and batches 1-8 on the matrix cores."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: fp8_gemm_fused_tans {rows}x{cols} B={B} S={segments} {alphabet}")
    w, scale = _weights(rows, cols, seed=rows * 7 + cols)
    x = _x(B, cols, seed=B + 100)
    m = T.encode_matrix(w, D.exp_histogram(w), segments=segments, alphabet=alphabet)
    y = _fused(R, m, x, scale)
    _check(y, _reference(w, x, scale))


def test_gemm_fused_vector_input_and_determinism(R):
    from rans_vectoradd import data as D, tans_codec as T
    _say("case: fp8_gemm_fused_tans vector x, repeated calls")
    w, scale = _weights(640, 960, seed=3)
    x = _x(1, 960, seed=4)[0]
    m = T.encode_matrix(w, D.exp_histogram(w))
    md, tbl = m.to("cuda"), m.decode_table().cuda()
    y1 = R.fp8_gemm_fused_tans(md, tbl, x.cuda(), scale)
    y2 = R.fp8_gemm_fused_tans(md, tbl, x.cuda(), scale)
    assert y1.shape == (640,)
    assert torch.equal(y1, y2)
    _check(y1.view(1, -1), _reference(w, x.view(1, -1), scale))


@pytest.mark.parametrize("rows,cols,B", [(2176, 1280, 1), (2176, 1280, 8), (100, 64, 3),
                                         (5120, 17408 // 4, 2), (5, 16, 2), (33, 48, 8),
                                         (17, 80, 5), (40, 1040, 4), (7, 1040, 1),
                                         (37, 5136, 1), (9, 10256, 1), (70, 12000, 1),
                                         (17408, 5120, 8), (1001, 8176, 3), (403, 4112, 8),
                                         (40003, 2048, 6), (6, 8192, 2), (130, 8208, 8),
                                         (37, 9008, 1), (257, 4096, 7), (64, 256, 4)])
def test_gemm_raw_vs_float64(R, rows, cols, B):
    """The raw kernels: x held in registers for rows of up to 8192 columns
    at every B (one 256-column chunk per wave up to 16 chunks, then two:
    4112 columns give 9 waves, the last with one chunk in range; 8176 a
    partial last chunk); longer rows row-streaming at B = 1 and with x
    loaded per chunk from B = 2 (8208 columns here, 17408 in the config-4
    tests).  Rows not a multiple of 4 or of the row groups in flight, more
    workgroups than CUs (40003 rows), widths not a multiple of 256.  At
    B = 1 rows of more than 8192 columns are split over 2 waves, of 10240 or
    more over 4 (uneven splits at 9008, 10256 and 12000 columns)."""
    _say(f"case: fp8_gemm_raw {rows}x{cols} B={B}")
    w, scale = _weights(rows, cols, seed=7)
    x = _x(B, cols, seed=8)
    y = R.fp8_gemm_raw(w.cuda(), x.cuda(), scale)
    _check(y, _reference(w, x, scale))


@pytest.mark.parametrize("B", [3, 8])
@pytest.mark.parametrize("rows,cols,split", [(131077, 16400, 130944), (262147, 8192, 262016)])
def test_gemm_raw_several_launches(R, B, rows, cols, split):
    """A W above 2^31 bytes: the raw kernels' launchers split the rows into
    launches that each address less than 2^31 bytes (131077 x 16400, x
    loaded per chunk: 130944 rows, then 133; 262147 x 8192, x in registers:
    262016 rows, then 131).  Rows at the start, around the split and at the
    end are checked against float64."""
    _say(f"case: fp8_gemm_raw {rows}x{cols} B={B} (two launches)")
    g = torch.Generator(device="cuda").manual_seed(B)
    w = torch.randint(0, 256, (rows, cols), dtype=torch.uint8, device="cuda", generator=g)
    w = torch.where((w & 0x7F) == 0x7F, torch.zeros_like(w), w)     # no NaN bytes
    x = _x(B, cols, seed=B + 5).cuda()
    y = R.fp8_gemm_raw(w, x, 0.5)
    for lo, hi in ((0, 64), (split - 100, split + 100), (rows - 64, rows)):
        ref = _reference(w[lo:hi].cpu(), x.cpu(), 0.5)
        _check(y[:, lo:hi], ref)
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [1, 8])
def test_gemm_config3_shape_fused_vs_raw(R, B):
    """Config 3's W_up shape (17408 x 5120) and config 4's mismatched-table
    case (a table from a Laplace histogram): both match float64, and the
    fused and raw kernels agree to a bf16 rounding step."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: gemm 17408x5120 B={B}")
    w, scale = _weights(17408, 5120, seed=11)
    x = _x(B, 5120, seed=12)
    ref = _reference(w, x, scale)
    raw = R.fp8_gemm_raw(w.cuda(), x.cuda(), scale)
    _check(raw, ref)
    lap, _ = D.laplace_fp8_bytes(1 << 20, seed=13)
    for hist in (D.exp_histogram(w), D.exp_histogram(lap)):
        m = T.encode_matrix(w, hist)
        y = _fused(R, m, x, scale)
        _check(y, ref)
        d = (y.float() - raw.float()).abs()
        assert bool((d <= 2.0 ** -7 * raw.float().abs() + 1e-6).all())


@pytest.mark.parametrize("B", [1, 2, 4, 8])
@pytest.mark.parametrize("table", ["matched", "laplace"])
def test_gemm_config4_down_shape(R, B, table):
    """Config 4's W_down shape (5120 x 17408: 25 segments of 704 columns,
    the last one ragged) at the batch sizes the bench times, with the
    matrix's own table and with a mismatched (Laplace) one."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: gemm 5120x17408 B={B} {table} table")
    w, scale = _weights(5120, 17408, seed=21)
    x = _x(B, 17408, seed=22 + B)
    if table == "matched":
        hist = D.exp_histogram(w)
    else:
        hist = D.exp_histogram(D.laplace_fp8_bytes(1 << 20, seed=23)[0])
    m = T.encode_matrix(w, hist)
    assert (m.segments, m.seg_cols) == (25, 704) and m.cols % m.seg_cols != 0
    _check(_fused(R, m, x, scale), _reference(w, x, scale))


@pytest.mark.parametrize("B", [2, 4])
def test_gemm_config4_up_shape_batches(R, B):
    """W_up (17408 x 5120: 7 segments of 736 columns, each lane's stream
    ending in a half tile) at the batch sizes between 1 and 8."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: gemm 17408x5120 B={B}")
    w, scale = _weights(17408, 5120, seed=31)
    x = _x(B, 5120, seed=32 + B)
    m = T.encode_matrix(w, D.exp_histogram(w))
    assert (m.segments, m.seg_cols) == (7, 736)
    _check(_fused(R, m, x, scale), _reference(w, x, scale))


def test_gemm_config4_layer_pair_chained(R):
    """One config-4 layer as the bench runs it: y1 = W_up x (bf16), then
    y2 = W_down y1, against the float64 chain (the intermediate rounded to
    bf16 as the kernel's output is)."""
    from rans_vectoradd import data as D, tans_codec as T
    _say("case: gemm layer pair up -> down, B=4")
    wu, su = _weights(17408, 5120, seed=41)
    wd, sd = _weights(5120, 17408, seed=42, dist="laplace")
    x = _x(4, 5120, seed=43)
    mu = T.encode_matrix(wu, D.exp_histogram(wu))
    md = T.encode_matrix(wd, D.exp_histogram(wd))
    y1 = _fused(R, mu, x, su)
    y2 = R.fp8_gemm_fused_tans(md.to("cuda"), md.decode_table().cuda(), y1, sd)
    ref1 = _reference(wu, x, su)
    _check(y1, ref1)
    ref2 = _reference(wd, ref1.to(torch.bfloat16), sd)
    _check(y2, ref2)


@pytest.mark.parametrize("B", [1, 8])
def test_gemm_config4_four_layer_chain(R, B):
    """Two config-4 layers in a row (W_up, W_down, W_up, W_down), the first
    layer's matrices coded with their own tables and the second layer's
    with a table from Laplace data (the bench's mismatched half), each
    product fed the previous one's bf16 output.  Every stage is checked
    against the float64 chain, whose intermediates are rounded to bf16 as
    the kernel's outputs are."""
    from rans_vectoradd import data as D, tans_codec as T
    _say(f"case: gemm four-layer chain B={B}")
    lap_hist = D.exp_histogram(D.laplace_fp8_bytes(1 << 20, seed=59)[0])
    shapes = [(17408, 5120), (5120, 17408), (17408, 5120), (5120, 17408)]
    x = _x(B, 5120, seed=60 + B)
    y, ref = x.cuda(), x.to(torch.float64)
    for i, (rows, cols) in enumerate(shapes):
        w, scale = _weights(rows, cols, seed=61 + i, dist="gaussian" if i % 2 == 0 else "laplace")
        hist = D.exp_histogram(w) if i < 2 else lap_hist
        m = T.encode_matrix(w, hist)
        y = R.fp8_gemm_fused_tans(m.to("cuda"), m.decode_table().cuda(), y, scale)
        assert y.shape == (B, rows)
        ref = _reference(w, ref.to(torch.bfloat16), scale)
        _check(y, ref)


def test_gemm_argument_errors(R):
    from rans_vectoradd import data as D, tans_codec as T
    w, scale = _weights(64, 32, seed=1)
    m = T.encode_matrix(w, D.exp_histogram(w))
    md, tbl = m.to("cuda"), m.decode_table().cuda()
    with pytest.raises(RuntimeError):
        R.fp8_gemm_fused_tans(md, tbl, _x(9, 32, 0).cuda(), scale)       # batch > 8
    with pytest.raises(RuntimeError):
        R.fp8_gemm_fused_tans(md, tbl, _x(1, 31, 0).cuda(), scale)       # wrong width
    with pytest.raises(RuntimeError):
        R.fp8_gemm_fused_tans(md, tbl, _x(1, 32, 0).float().cuda(), scale)   # not bf16
    with pytest.raises(RuntimeError, match="alphabet"):
        nib = T.encode_matrix(w, D.exp_histogram(w), alphabet="nibble").decode_table().cuda()
        R.fp8_gemm_fused_tans(md, nib, _x(1, 32, 0).cuda(), scale)       # table of the other alphabet
    with pytest.raises(RuntimeError):
        R.fp8_gemm_raw(torch.zeros(4, 24, dtype=torch.uint8).cuda(), _x(1, 24, 0).cuda())
