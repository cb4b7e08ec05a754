"""Tensors past the 32-bit limits, at sizes a 288 GB MI355X holds:

* the raw add at 2^36 + 2^20 bytes per vector (64 GiB and a little more):
  one launch counts its work items in 32 bits, so the add runs as three
  launches (2^31 vectors, 2^31 vectors, 2^16 vectors); every output byte is
  checked against the oracle's add table (RNE, satfinite);
* the fused tANS add and the standalone decode at 2^34 elements per tensor:
  every compressed stream set, sign/mantissa array and output is larger
  than 4 GiB, so stream offsets, tile rows and output rows need 64-bit
  addresses; fused == raw and decode == input on every element.

Each case frees what it holds and skips when the GPU lacks the free memory
it needs.  Each case prints its name before it touches the GPU."""
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

GiB = 1 << 30
RAW_BYTES = (1 << 36) + (1 << 20)     # per vector: 3 launches of the streaming kernel
BIG_ELEMS = 1 << 34                   # per tensor for the tANS cases
CHUNK = 1 << 28                       # elements per checking step


def _say(msg):
    print(msg, flush=True)


def _need(nbytes):
    torch.cuda.empty_cache()
    free, _ = torch.cuda.mem_get_info()
    if free < nbytes:
        pytest.skip(f"needs {nbytes / GiB:.0f} GiB of free GPU memory, {free / GiB:.0f} GiB free")


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


def test_raw_add_past_one_launch(R):
    """64 GiB + 1 MiB per vector of random bytes (every byte pair, NaN
    included): raw add == the oracle's table on every element."""
    _say("case: fp8_vecadd_raw at 2^36 + 2^20 bytes per vector")
    _need(3 * RAW_BYTES + 8 * GiB)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    a = torch.empty(RAW_BYTES, dtype=torch.uint8, device="cuda").random_(0, 256, generator=g)
    b = torch.empty(RAW_BYTES, dtype=torch.uint8, device="cuda").random_(0, 256, generator=g)
    c = R.fp8_vecadd_raw(a, b)
    lut = torch.from_numpy(O.add_lut().reshape(-1)).cuda()
    nan = torch.from_numpy(O.nan_mask_lut().reshape(-1)).cuda()
    for s in range(0, RAW_BYTES, CHUNK):
        idx = a[s:s + CHUNK].long() * 256 + b[s:s + CHUNK].long()
        ok = (c[s:s + CHUNK] == lut[idx]) | nan[idx]
        assert bool(ok.all()), f"raw add differs from the oracle in bytes [{s}, {s + CHUNK})"
        del idx, ok
    del a, b, c


@pytest.fixture(scope="module")
def big(R):
    """Two 2^34-element tensors (N(0, 0.02) scaled to 448 per 2^30 block,
    seeds 20.. and 40..), their joint exponent histogram, and both encoded
    on the GPU with 1024 elements per lane (pair alphabet)."""
    from rans_vectoradd import data as D, tans_codec as T
    _say("case: 2^34-element inputs, GPU encoder")
    _need(130 * GiB)
    blk = 1 << 30
    qs = []
    for seed0 in (20, 40):
        q = torch.empty(BIG_ELEMS, dtype=torch.uint8, device="cuda")
        for i, s in enumerate(range(0, BIG_ELEMS, blk)):
            q[s:s + blk] = D.gaussian_fp8_bytes(blk, seed=seed0 + i, device="cuda")[0]
        qs.append(q)
    hist = torch.zeros(16, dtype=torch.float64)
    for q in qs:
        for s in range(0, BIG_ELEMS, blk):
            hist += D.exp_histogram(q[s:s + blk]).cpu()
    lane = 1024
    K = BIG_ELEMS // lane
    encs = [T.encode_gpu(q.view(K, lane), hist, tile=8) for q in qs]
    # the sizes that make this case: streams and tiles past 4 GiB
    assert all(e[0].numel() > 4 * GiB and e[4].numel() > 4 * GiB for e in encs)
    tbl = T.build_decode_table(encs[0][6].cpu().numpy(), encs[0][5].cpu().numpy()).cuda()
    yield qs, encs, tbl, K, lane
    del qs, encs, tbl
    torch.cuda.empty_cache()


def test_fused_add_past_4gib(R, big):
    """fused == raw on all 2^34 elements (output in tile-major order)."""
    qs, encs, tbl, K, lane = big
    _say("case: fp8_vecadd_fused_tans at 2^34 elements per vector")
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    out = R.fp8_vecadd_fused_tans(*[encs[0][i] for i in order], *[encs[1][i] for i in order],
                                  tbl, lane)
    raw = R.fp8_vecadd_raw(qs[0], qs[1]).view(K, lane)
    tiles = out.view(lane // 16, K, 16)
    for t in range(lane // 16):
        assert torch.equal(tiles[t], raw[:, 16 * t:16 * t + 16]), f"tile {t} differs"
    del out, raw, tiles


def test_decode_past_4gib(R, big):
    """decode == input on all 2^34 elements ([N, K] output)."""
    qs, encs, tbl, K, lane = big
    _say("case: gpu_tans_decode at 2^34 elements")
    comp, st, off, part, sm, fr, sp = encs[0]
    out = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, lane)
    src = qs[0].view(K, lane)
    for s in range(0, lane, 64):
        assert torch.equal(out[s:s + 64], src[:, s:s + 64].t()), f"rows [{s}, {s + 64}) differ"
    del out
