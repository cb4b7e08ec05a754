"""Write the golden vectors under tests/golden/ (run in the build container,
where /root/reference exists; the GPU box never runs this).

Only the two reference functions that no closed form or invariant pins are
run here, each loaded by file path from the reference checkout:

* ``random_fp8_bytes`` (rans_vectoradd/data.py:41-69): the exact bytes a
  seed yields depend on torch's RNG call order.
* ``quantize_freqs`` (rans_vectoradd/tans_codec.py:30-46): the greedy fix-up
  breaks ties by index.

Everything else (spread, decode table, codec, add) is pinned by closed forms,
invariants and round trips in tests/test_oracle.py.

    python tests/golden/make_golden.py [/root/reference]
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(path: str, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main(ref: str) -> None:
    data = _load(os.path.join(ref, "rans_vectoradd", "data.py"), "ref_data")
    codec = _load(os.path.join(ref, "rans_vectoradd", "tans_codec.py"), "ref_codec")

    out = {}
    # random_fp8_bytes under the seeds and call orders of the reference tests
    torch.manual_seed(42)   # test_gpu_decode_tans.py:20-21 (K*N = 128*128)
    out["rand_seed42_n16384"] = data.random_fp8_bytes(128 * 128, device="cpu").numpy()
    torch.manual_seed(0)    # test_vecadd_tans.py:32-34: two draws back to back
    out["rand_seed0_a_n4096"] = data.random_fp8_bytes(4096, device="cpu").numpy()
    out["rand_seed0_b_n4096"] = data.random_fp8_bytes(4096, device="cpu").numpy()
    g = torch.Generator().manual_seed(7)
    out["rand_gen7_flat_n2048"] = data.random_fp8_bytes(
        2048, exp_probs=tuple([1.0] * 16), device="cpu", generator=g).numpy()

    # quantize_freqs: the pair table of the reference's encode() for the
    # Qwen3 histogram (float32 normalisation as tans_codec.py:126-129) ...
    p = torch.tensor(data.QWEN3_14B_FP8_EXP, dtype=torch.float64).float().numpy()
    p = p / p.sum()
    pair = (p[:, None] * p[None, :]).flatten()
    out["qf_pair_qwen_in"] = pair.astype(np.float64)
    out["qf_pair_qwen_out"] = codec.quantize_freqs(pair, target=4096)
    # ... and vectors that exercise both fix-up directions, zeros and ties
    rng = np.random.default_rng(1234)
    cases = []
    for target, n in ((4096, 256), (2048, 16), (2048, 16), (64, 16), (4096, 40)):
        v = rng.random(n) ** 4
        v[rng.random(n) < 0.2] = 0.0
        v /= v.sum()
        cases.append((v, target))
    tie = np.full(16, 1.0 / 16)
    cases.append((tie, 100))            # 16 equal shares of 100: ties
    many_small = np.full(300, 1e-6)
    many_small[0] = 1.0
    many_small /= many_small.sum()
    cases.append((many_small, 4096))    # floor-to-1 overshoot: down fix-up
    for i, (v, target) in enumerate(cases):
        out[f"qf_case{i}_in"] = v
        out[f"qf_case{i}_target"] = np.array([target])
        out[f"qf_case{i}_out"] = codec.quantize_freqs(v, target=target)

    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
