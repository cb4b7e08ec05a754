"""The on-disk container and checkpoint ingestion (CPU): safetensors round
trips, histograms against numpy, and encoded entries decoded back to the
original bytes by the oracle's independent decoder."""
import json
import os

import numpy as np
import pytest
import torch

from gemm_layout import matrix_from_lanes
from oracle import oracle as O

LOG2L = {"pair": (12, 2), "nibble": (11, 1)}


def _decode_lanes(e):
    log2L, sps = LOG2L[e.alphabet]
    return O.layout_decode(e.as_tuple(), e.K, e.N, log2L, sps)


def _decode_matrix(m):
    log2L, sps = LOG2L[m.alphabet]
    Rp = -(-m.rows // 64) * 64
    dec = O.w64_decode(m.comp.numpy(), m.offsets.numpy(), m.states.numpy(), m.sm.numpy(),
                       m.spread.numpy(), m.freqs.numpy(), log2L, sps, m.segments * Rp * 4,
                       m.seg_cols // 4)
    return matrix_from_lanes(dec, m.segments, Rp, m.seg_cols, m.rows, m.cols)


def test_container_roundtrip(tmp_path):
    from rans_vectoradd import container, data as D, tans_codec as T
    q, _ = D.gaussian_fp8_bytes(64 * 96, seed=4)
    lanes = T.TansTensor.from_tuple(T.encode(q.reshape(64, 96), D.exp_histogram(q)), 64, 96, "pair")
    w, _ = D.laplace_fp8_bytes(100 * 70, seed=5)
    mat = T.encode_matrix(w.reshape(100, 70), D.exp_histogram(w), alphabet="nibble")
    scale = torch.tensor([0.125], dtype=torch.float32)
    path = os.path.join(tmp_path, "c.safetensors")
    container.save(path, {"a": lanes, "w": mat, "w_scale": scale}, metadata={"note": "x"})
    got = container.load(path)
    assert set(got) == {"a", "w", "w_scale"}
    assert container.metadata(path) == {"note": "x"}
    for name, ref in (("a", lanes), ("w", mat)):
        for part in ("comp", "states", "offsets", "sm", "freqs", "spread"):
            assert torch.equal(getattr(got[name], part), getattr(ref, part)), (name, part)
    assert (got["a"].K, got["a"].N, got["a"].alphabet) == (64, 96, "pair")
    assert (got["w"].rows, got["w"].cols, got["w"].segments, got["w"].seg_cols) == \
        (mat.rows, mat.cols, mat.segments, mat.seg_cols)
    assert torch.equal(got["w_scale"], scale)
    assert np.array_equal(_decode_lanes(got["a"]), q.reshape(64, 96).numpy())
    assert np.array_equal(_decode_matrix(got["w"]), w.reshape(100, 70).numpy())


def test_container_rejects_plain_names_that_shadow_encoded_parts(tmp_path):
    """A plain tensor named '<entry>.<part>' would overwrite that part of an
    encoded entry on save; save refuses it.  Other dotted names are fine."""
    from rans_vectoradd import container, data as D, tans_codec as T
    q, _ = D.gaussian_fp8_bytes(64 * 32, seed=2)
    lanes = T.TansTensor.from_tuple(T.encode(q.reshape(64, 32), D.exp_histogram(q)), 64, 32, "pair")
    path = os.path.join(tmp_path, "c.safetensors")
    with pytest.raises(ValueError, match="overwrite"):
        container.save(path, {"w": lanes, "w.comp": torch.zeros(5, dtype=torch.int32)})
    container.save(path, {"w": lanes, "w.bias": torch.ones(3), "v.comp": torch.ones(2)})
    got = container.load(path)
    assert torch.equal(got["w"].comp, lanes.comp)
    assert torch.equal(got["w.bias"], torch.ones(3)) and torch.equal(got["v.comp"], torch.ones(2))


def test_container_rejects_other_files(tmp_path):
    from safetensors.torch import save_file
    from rans_vectoradd import container
    path = os.path.join(tmp_path, "plain.safetensors")
    save_file({"x": torch.zeros(2)}, path)
    with pytest.raises(ValueError):
        container.load(path)
    with pytest.raises(ValueError):
        container.save(path, {"x": torch.zeros(2)}, metadata={"tans_format": "y"})
    # a file of an older layout version (other stream schedule and matrix lanes)
    old = os.path.join(tmp_path, "v1.safetensors")
    save_file({"x": torch.zeros(2)}, old, metadata={"tans_format": "tans-wave64-v1"})
    with pytest.raises(ValueError, match="re-encode"):
        container.load(old)


def test_container_reads_v2_pair_entries_only(tmp_path):
    """v2 containers differ from v3 only in the nibble alphabet's refill
    schedule: their pair entries load (at lengths the v4 change leaves
    alone), a nibble entry is refused."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    from rans_vectoradd import container, data as D, tans_codec as T
    q, _ = D.gaussian_fp8_bytes(64 * 32, seed=3)
    for alphabet, ok in (("pair", True), ("nibble", False)):
        t = T.TansTensor.from_tuple(T.encode(q.reshape(64, 32), D.exp_histogram(q),
                                             alphabet=alphabet, layout="words"),
                                    64, 32, alphabet)
        path = os.path.join(tmp_path, f"{alphabet}.safetensors")
        container.save(path, {"w": t})
        with safe_open(path, framework="pt") as f:
            meta, tensors = f.metadata(), {k: f.get_tensor(k) for k in f.keys()}
        meta["tans_format"] = "tans-wave64-v2"
        v2 = os.path.join(tmp_path, f"{alphabet}_v2.safetensors")
        save_file(tensors, v2, metadata=meta)
        if ok:
            assert torch.equal(container.load(v2)["w"].comp, t.comp)
        else:
            with pytest.raises(ValueError, match="re-encode"):
                container.load(v2)


def test_container_reads_v3_unless_the_last_tile_rule_changed(tmp_path):
    """v3 containers differ from v4 only for entries of lanes whose last
    16-element tile holds one refill segment (N > 16 and N % 16 in 1..4 with
    pairs, 1..3 with nibbles): such entries are refused, the others load; a v2
    pair entry at such a length is refused too."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    from rans_vectoradd import container, data as D, tans_codec as T
    cases = [("pair", 32, True), ("pair", 20, False), ("pair", 18, False), ("pair", 22, True),
             ("pair", 4, True), ("nibble", 34, False), ("nibble", 36, True)]
    for alphabet, N, ok in cases:
        q, _ = D.gaussian_fp8_bytes(64 * N, seed=N)
        t = T.TansTensor.from_tuple(T.encode(q.reshape(64, N), D.exp_histogram(q),
                                             alphabet=alphabet, layout="words"),
                                    64, N, alphabet)
        path = os.path.join(tmp_path, f"{alphabet}{N}.safetensors")
        container.save(path, {"w": t})
        with safe_open(path, framework="pt") as f:
            meta, tensors = f.metadata(), {k: f.get_tensor(k) for k in f.keys()}
        assert meta["tans_format"] == "tans-wave64-v5"
        olds = ("tans-wave64-v4", "tans-wave64-v3", "tans-wave64-v2")
        for old in olds if alphabet == "pair" else olds[:2]:
            meta["tans_format"] = old
            prev = os.path.join(tmp_path, f"{alphabet}{N}_{old[-2:]}.safetensors")
            save_file(tensors, prev, metadata=meta)
            if ok or old.endswith("v4"):
                assert torch.equal(container.load(prev)["w"].comp, t.comp)
            else:
                with pytest.raises(ValueError, match="one refill segment"):
                    container.load(prev)


@pytest.mark.parametrize("N", [16, 46, 64])
def test_container_packed_entry_roundtrip(tmp_path, N):
    """Entries of short lanes in the packed layout (no states: the part is
    stored empty) load back unchanged and decode to the input."""
    from rans_vectoradd import container, data as D, tans_codec as T
    q, _ = D.gaussian_fp8_bytes(130 * N, seed=N)
    t = T.TansTensor.from_tuple(T.encode(q.reshape(130, N), D.exp_histogram(q)), 130, N, "pair")
    assert t.states.numel() == 0
    path = os.path.join(tmp_path, "p.safetensors")
    container.save(path, {"p": t})
    got = container.load(path)["p"]
    for part in ("comp", "states", "offsets", "sm", "freqs", "spread"):
        assert torch.equal(getattr(got, part), getattr(t, part)), part
    assert np.array_equal(_decode_lanes(got), q.reshape(130, N).numpy())


def _checkpoint(path):
    from safetensors.torch import save_file
    from rans_vectoradd import data as D
    w1, s1 = D.gaussian_fp8_bytes(192 * 160, seed=11)
    w2, s2 = D.laplace_fp8_bytes(4096, seed=12)
    tensors = {
        "layer0_up": w1.reshape(192, 160).view(torch.float8_e4m3fn),
        "layer0_up_scale": torch.tensor([s1], dtype=torch.float32),
        "layer0_vec": w2.view(torch.float8_e4m3fn),
        "layer0_bias": torch.randn(160, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16),
    }
    save_file(tensors, path)
    return tensors


def test_scan_histograms_match_numpy(tmp_path):
    from rans_vectoradd import ingest
    src = os.path.join(tmp_path, "ckpt.safetensors")
    t = _checkpoint(src)
    hists = ingest.scan(src)
    assert set(hists) == {"layer0_up", "layer0_vec"}
    for name, h in hists.items():
        b = t[name].view(torch.uint8).numpy().reshape(-1)
        assert np.array_equal(h, np.bincount((b >> 3) & 15, minlength=16).astype(np.float64))
    slabs = ingest.scan(src, per="slab", rows_per_slab=64)["layer0_up"]
    assert slabs.shape == (3, 16)
    assert np.array_equal(slabs.sum(axis=0), hists["layer0_up"])
    b = t["layer0_up"].view(torch.uint8).numpy()[64:128].reshape(-1)
    assert np.array_equal(slabs[1], np.bincount((b >> 3) & 15, minlength=16))
    agg = ingest.aggregate(hists)
    assert abs(agg.sum() - 1.0) < 1e-12
    assert np.allclose(agg, (hists["layer0_up"] + hists["layer0_vec"]) /
                       (hists["layer0_up"].sum() + hists["layer0_vec"].sum()))


@pytest.mark.parametrize("table", ["tensor", "global"])
def test_encode_checkpoint_decodes_back(tmp_path, table):
    from rans_vectoradd import container, ingest
    src = os.path.join(tmp_path, "ckpt.safetensors")
    dst = os.path.join(tmp_path, "ckpt.tans.safetensors")
    t = _checkpoint(src)
    report = ingest.encode_checkpoint(src, dst, table=table, lane_elems=256)
    assert report["layer0_up"]["kind"] == "matrix" and report["layer0_vec"]["kind"] == "lanes"
    for r in report.values():
        assert 4.0 < r["bits_per_byte"] < 12.0   # tiny tensors: per-lane states dominate
    got = container.load(dst)
    up = got["layer0_up"]
    assert np.array_equal(_decode_matrix(up), t["layer0_up"].view(torch.uint8).numpy())
    vec = got["layer0_vec"]
    assert (vec.K, vec.N) == (16, 256)
    assert np.array_equal(_decode_lanes(vec).reshape(-1), t["layer0_vec"].view(torch.uint8).numpy())
    assert torch.equal(got["layer0_bias"], t["layer0_bias"])
    assert torch.equal(got["layer0_up_scale"], t["layer0_up_scale"])
    shapes = json.loads(container.metadata(dst)["shapes"])
    assert shapes["layer0_up"] == {"shape": [192, 160], "dtype": "float8_e4m3fn"}
    if table == "global":   # one table for both tensors
        assert torch.equal(up.freqs, vec.freqs)
