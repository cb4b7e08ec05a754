"""The GEMM entry point that allocates nothing (tans_fp8_gemm_fused_noalloc,
no counterpart in the reference): through the C ABI, its output equals the
workspace entry point's (tans_fp8_gemm_fused, here via fp8_gemm_fused_tans)
bit for bit, on two calls in a row, the second smaller than the first; and
products whose partial sums exceed its 16 MiB device array are refused
before any GPU work."""
import ctypes

import pytest
import torch


def _say(msg):
    print(msg, flush=True)


def _call_noalloc(lib, m, tbl, x, scale):
    from rans_vectoradd._C import log2_states
    B = x.shape[0]
    y = torch.empty((B, m.rows), dtype=torch.bfloat16, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.tans_fp8_gemm_fused_noalloc(m.comp.data_ptr(), m.comp.numel(), m.offsets.data_ptr(),
                                         m.states.data_ptr(), m.sm.data_ptr(), tbl.data_ptr(),
                                         log2_states(tbl.numel() // 2), m.rows, m.cols,
                                         m.segments, m.seg_cols, x.data_ptr(), B,
                                         ctypes.c_float(scale), y.data_ptr(), stream)
    assert rc == 0, lib.tans_last_error()
    return y


def test_noalloc_rejects_products_beyond_its_scratch():
    from rans_vectoradd._lib import lib
    d = ctypes.c_void_p(256)
    # 80 segments of 64 columns x 8 rows x 17408 outputs of fp32 partial sums: 42.5 MiB
    rc = lib.tans_fp8_gemm_fused_noalloc(d, 1024, d, d, d, d, 12, 17408, 5120, 80, 64, d, 8,
                                         ctypes.c_float(1.0), d, None)
    assert rc == -1 and b"16 MiB" in lib.tans_last_error()


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point_twice():
    import rans_vectoradd as R
    from rans_vectoradd import data as D, tans_codec as T
    from rans_vectoradd._lib import lib
    assert torch.cuda.is_available()
    cases = [(17408, 5120, 8, "pair", 51), (2176, 1280, 3, "nibble", 52)]
    for rows, cols, B, alphabet, seed in cases:   # the second call is the smaller one
        _say(f"case: gemm_fused_noalloc {rows}x{cols} B={B} {alphabet}")
        q, scale = D.gaussian_fp8_bytes(rows * cols, seed=seed)
        w = q.reshape(rows, cols)
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(B, cols, generator=g).to(torch.bfloat16).cuda()
        m = T.encode_matrix(w, D.exp_histogram(w), alphabet=alphabet).to("cuda")
        tbl = m.decode_table().cuda()
        ref = R.fp8_gemm_fused_tans(m, tbl, x, scale)
        got = _call_noalloc(lib, m, tbl, x, scale)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"{(got != ref).sum().item()} outputs differ"
