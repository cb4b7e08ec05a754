"""The oracle's restatement of the reference's CPU encoder (oracle.c,
``O.ref_encode``) against the reference's own encoder, tans_encode_interleaved
(csrc/tans_codec.cpp:69-196), compiled unmodified from the reference tree into
oracle/_ref/ (``make -C oracle ref``, run by ``__graft_entry__.build()`` where
the reference is present).  Byte for byte on every output: compressed bytes,
final states, block offsets and partial-slab counts.  Skipped where the
compiled reference is absent."""
import os

import numpy as np
import pytest

from oracle import oracle as O

# Only the path is checked at collection: the library is loaded by the tests
# that run, so a process that deselects them (the GPU suite) never maps it.
pytestmark = pytest.mark.skipif(not os.path.exists(O.REF_LIB_PATH),
                                reason="oracle/_ref/libref_codec.so not built "
                                       "(needs the reference tree and torch's headers)")


def _pair_setup(K, N, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, scale, (K, N))
    x *= 448.0 / np.abs(x).max()
    import torch
    fp8 = torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    exps = (fp8 >> 3) & 0xF
    p = np.bincount(exps.ravel(), minlength=16).astype(np.float64) + 1e-6
    p = p / p.sum()
    f = O.quantize_freqs((p[:, None] * p[None, :]).reshape(-1), 4096)
    return O.pair_symbols(fp8), f, O.build_spread(f, 4096)


def _same(a, b):
    for name, x, y in zip(("compressed", "states", "offsets", "partial"), a, b):
        assert x.dtype == y.dtype, name
        assert np.array_equal(x, y), f"{name} differs"


@pytest.mark.parametrize("K,N,seed", [(128, 128, 0), (300, 64, 1), (129, 16, 2), (3, 256, 3),
                                      (1, 2, 4), (257, 6, 5), (64, 1024, 6)])
def test_oracle_encoder_equals_reference(K, N, seed):
    sym, f, sp = _pair_setup(K, N, seed)
    _same(O.ref_encode(sym, f, sp), O.reference_encode(sym, f, sp))


def test_oracle_encoder_equals_reference_skewed_and_flat():
    """A near-single-symbol table (one symbol holds almost every state, so
    its steps emit 0 bits) and a flat 256-symbol table."""
    rng = np.random.default_rng(7)
    f = np.full(256, 1, np.int32)
    f[37] = 4096 - 255
    sp = O.build_spread(f, 4096)
    sym = np.full((200, 48), 37, np.uint8)
    sym[rng.random(sym.shape) < 0.01] = 5
    _same(O.ref_encode(sym, f, sp), O.reference_encode(sym, f, sp))
    f = np.full(256, 16, np.int32)
    sp = O.build_spread(f, 4096)
    sym = rng.integers(0, 256, (130, 40), dtype=np.uint8)
    _same(O.ref_encode(sym, f, sp), O.reference_encode(sym, f, sp))


def test_oracle_encoder_equals_reference_small_alphabet():
    """A 16-symbol alphabet at L = 4096 (the reference encoder takes any
    alphabet whose frequencies sum to L)."""
    rng = np.random.default_rng(8)
    p = rng.random(16) + 0.05
    f = O.quantize_freqs(p / p.sum(), 4096)
    sp = O.build_spread(f, 4096)
    sym = rng.choice(16, size=(150, 80), p=p / p.sum()).astype(np.uint8)
    _same(O.ref_encode(sym, f, sp), O.reference_encode(sym, f, sp))


def test_reference_rejects_a_short_spread():
    """The harness passes the reference's TORCH_CHECK failures on as errors
    (csrc/tans_codec.cpp:80, spread.numel() == L)."""
    sym, f, sp = _pair_setup(4, 32, 9)
    with pytest.raises(RuntimeError):
        O.reference_encode(sym, f, sp[:2048])
