"""FP8 E4M3FN test-data generators.

``random_fp8_bytes`` and ``QWEN3_14B_FP8_EXP`` are the reference's
(rans_vectoradd/data.py:21-69): exponent drawn from a fixed histogram, sign
and mantissa uniform.  Its torch RNG calls are made in the same order, so a
given seed yields the reference's bytes.

``gaussian_fp8_bytes`` / ``laplace_fp8_bytes`` make the benchmark inputs:
N(0, std) or Laplace(0, b) samples scaled per tensor so |max| maps to 448,
then round-to-nearest cast to E4M3FN.
"""
from __future__ import annotations

import torch

# Aggregate exponent histogram of the FP8 linear weights of Qwen3-14B-FP8
# (reference data.py:21-38; entropy 2.787 bits).
QWEN3_14B_FP8_EXP: tuple[float, ...] = (
    0.0005, 0.0005, 0.0009, 0.0018, 0.0034, 0.0062, 0.0104, 0.0167,
    0.0283, 0.0480, 0.0838, 0.1502, 0.2417, 0.2715, 0.1273, 0.0088,
)

E4M3_MAX = 448.0


def random_fp8_bytes(n: int, *, exp_probs: tuple[float, ...] = QWEN3_14B_FP8_EXP,
                     device: str | torch.device = "cuda",
                     generator: torch.Generator | None = None) -> torch.Tensor:
    """n FP8 bytes: exponent ~ exp_probs (inverse-CDF of one uniform draw per
    element, clamped to 15), sign+mantissa nibble uniform over 16 values."""
    w = torch.tensor(exp_probs, dtype=torch.float32, device=device)
    cdf = torch.cumsum(w / w.sum(), dim=0)
    u = torch.rand(n, device=device, generator=generator)
    exp = torch.searchsorted(cdf, u).clamp_max_(15).to(torch.uint8)
    nib = torch.randint(0, 16, (n,), dtype=torch.uint8, device=device, generator=generator)
    return ((nib & 8) << 4) | (exp << 3) | (nib & 7)


def _scale_to_fp8(x: torch.Tensor) -> tuple[torch.Tensor, float]:
    amax = float(x.abs().max())
    scale = E4M3_MAX / amax if amax > 0 else 1.0
    q = (x * scale).clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), 1.0 / scale


def gaussian_fp8_bytes(n: int, *, std: float = 0.02, seed: int = 0,
                       device: str | torch.device = "cpu") -> tuple[torch.Tensor, float]:
    """n bytes of N(0, std) scaled so |max| -> 448, RNE-cast to E4M3FN.
    Returns (uint8 bytes, dequant scale = absmax / 448)."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(n, generator=g, device=device) * std
    return _scale_to_fp8(x)


def laplace_fp8_bytes(n: int, *, b: float = 0.015, seed: int = 0,
                      device: str | torch.device = "cpu") -> tuple[torch.Tensor, float]:
    """n bytes of Laplace(0, b) (inverse CDF), scaled and cast as above.

    torch.rand can return exactly 0, i.e. u = -0.5, where the inverse CDF
    is infinite (about 64 times in 2^30 draws), and one infinity would
    scale every other value to zero; 2|u| is therefore capped at 1 - 2^-24,
    the largest float32 below 1, which bounds |x| by 24 ln2 b."""
    g = torch.Generator(device=device).manual_seed(seed)
    u = torch.rand(n, generator=g, device=device) - 0.5
    a = (2.0 * u.abs()).clamp_max_(1.0 - 2.0 ** -24)
    x = -b * torch.sign(u) * torch.log1p(-a)
    return _scale_to_fp8(x)


def exp_histogram(fp8: torch.Tensor) -> torch.Tensor:
    """Counts of the 16 exponent-nibble values (float64 [16])."""
    e = ((fp8.reshape(-1) >> 3) & 0xF).to(torch.int64)
    return torch.bincount(e, minlength=16).to(torch.float64)
