"""Seeded sweep over shapes and tables for the fused add and the decoder:
lane counts with and without a partial last group, stream lengths that
take each kernel variant (one tile, streams loaded whole, streams fetched
by stage; ragged last tiles for the decoder), both alphabets, and tables
that match the data, do not (uniform bytes under the Qwen3 histogram) or
make every step long (a steep histogram).  The fused add is checked
against the raw add and the oracle's table, the decoder against the input.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

STEEP = [2.0 ** -e for e in range(16)]


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        # "pair" takes the packed layout up to 4 tiles, "pair:words" the other
        alphabet = ("pair", "nibble", "pair:words")[i % 3]
        K = int(rng.choice([1, 13, 64, 65, 127, 200, 640, 1000, 4095]))
        tiles = int(rng.choice([1, 2, 3, 4, 5, 9]))
        table = ("data", "qwen", "steep")[int(rng.integers(3))]
        out.append((alphabet, K, tiles, table, int(rng.integers(1 << 30))))
    return out


def _bytes(K, N, table, seed, R):
    g = torch.Generator().manual_seed(seed)
    if table == "data":
        fp8 = R.random_fp8_bytes(K * N, device="cpu").reshape(K, N)
        hist = np.bincount(((fp8.numpy() >> 3) & 15).ravel(), minlength=16).astype(np.float64)
        return fp8, torch.tensor(hist / hist.sum())
    fp8 = torch.randint(0, 256, (K, N), dtype=torch.uint8, generator=g)
    probs = R.QWEN3_14B_FP8_EXP if table == "qwen" else STEEP
    return fp8, torch.tensor(probs, dtype=torch.float64)


def _codec(codec):
    """encode() keywords of an alphabet[:layout] case."""
    alphabet, _, layout = codec.partition(":")
    return dict(alphabet=alphabet, layout=layout or "auto")


@pytest.fixture(scope="module")
def R():
    import rans_vectoradd
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return rans_vectoradd


@pytest.mark.parametrize("alphabet,K,tiles,table,seed", _cases(24, 11))
def test_fused_random_shape(R, lut, alphabet, K, tiles, table, seed):
    from rans_vectoradd import tans_codec as T
    N = 16 * tiles
    print(f"case: fused K={K} N={N} {alphabet} table={table} seed={seed}", flush=True)
    torch.manual_seed(seed)
    fa, probs = _bytes(K, N, table, seed, R)
    fb, _ = _bytes(K, N, table, seed + 1, R)
    if table == "data":
        hist = np.bincount(((torch.cat([fa, fb]).numpy() >> 3) & 15).ravel(), minlength=16)
        probs = torch.tensor(hist / hist.sum(), dtype=torch.float64)
    ea = T.encode(fa, probs, tile=8, **_codec(alphabet))
    eb = T.encode(fb, probs, tile=8, **_codec(alphabet))
    tbl = T.build_decode_table(ea[6].numpy(), ea[5].numpy())
    order = (0, 2, 1, 3, 4)   # comp, offsets, states, partial, sm
    args = [x.cuda() for x in (*[ea[i] for i in order], *[eb[i] for i in order], tbl)]
    fused = T.untile(R.fp8_vecadd_fused_tans(*args, N).cpu(), K, N)
    raw = R.fp8_vecadd_raw(fa.flatten().cuda(), fb.flatten().cuda()).cpu().reshape(K, N)
    assert torch.equal(fused, raw), f"{(fused != raw).sum().item()} bytes differ from raw"
    ref = O.vecadd(lut, fa.numpy(), fb.numpy()).reshape(K, N)
    ok = (fused.numpy() == ref) | O.nan_mask_lut()[fa.numpy(), fb.numpy()]
    assert ok.all()


@pytest.mark.parametrize("alphabet,K,tiles,table,seed", _cases(24, 12))
def test_decode_random_shape(R, alphabet, K, tiles, table, seed):
    from rans_vectoradd import tans_codec as T
    N = 16 * tiles - 2 * (seed % 8)   # ragged last tiles of 2..16 elements
    print(f"case: decode K={K} N={N} {alphabet} table={table} seed={seed}", flush=True)
    torch.manual_seed(seed)
    fp8, probs = _bytes(K, N, table, seed, R)
    enc = [x.cuda() for x in T.encode(fp8, probs, **_codec(alphabet))]
    comp, st, off, part, sm, fr, sp = enc
    dec = R.gpu_tans_decode(comp, off, st, part, sm, sp, fr, N)
    got = dec.cpu().t().contiguous()
    assert torch.equal(got, fp8), f"{(got != fp8).sum().item()} mismatched bytes"
