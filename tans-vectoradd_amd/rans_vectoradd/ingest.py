"""Exponent histograms of real FP8 weights, and checkpoint encoding.

The reference's QWEN3_14B_FP8_EXP histogram (rans_vectoradd/data.py:11-20)
was produced by an offline scan of Qwen3-14B-FP8 (an ``analyze_fp8.py`` that
the repository does not ship).  This module restores that capability for any
safetensors checkpoint: per-tensor (or per-row-slab) exponent histograms of
its FP8 E4M3FN tensors, their aggregate, and ``encode_checkpoint``, which
writes every FP8 tensor tANS-coded into a container (rans_vectoradd.container)
with a table built from its own histogram (or from the aggregate).
"""
from __future__ import annotations

import json

import numpy as np
import torch

from . import container
from .tans_codec import TansTensor, encode, encode_gpu, encode_matrix

FP8_DTYPES = (torch.float8_e4m3fn,)


def _fp8_bytes(t: torch.Tensor) -> torch.Tensor:
    if t.dtype in FP8_DTYPES:
        return t.view(torch.uint8)
    if t.dtype == torch.uint8:
        return t
    raise TypeError(f"not an FP8 E4M3FN tensor: {t.dtype}")


def exponent_histogram(t: torch.Tensor) -> np.ndarray:
    """Counts of the 16 exponent-nibble values of an FP8 tensor (any device)."""
    b = _fp8_bytes(t).reshape(-1)
    e = ((b >> 3) & 0xF).to(torch.int64)
    return torch.bincount(e, minlength=16).cpu().numpy().astype(np.float64)


def slab_histograms(w: torch.Tensor, rows_per_slab: int = 64) -> np.ndarray:
    """Exponent histograms of consecutive row slabs of a 2-D FP8 tensor:
    float64 [ceil(rows / rows_per_slab), 16]."""
    b = _fp8_bytes(w)
    if b.dim() != 2:
        raise ValueError("slab_histograms needs a 2-D tensor")
    R = b.shape[0]
    n = -(-R // rows_per_slab)
    e = ((b >> 3) & 0xF).to(torch.int64)
    slab = (torch.arange(R, device=b.device) // rows_per_slab).unsqueeze(1)
    idx = (slab * 16 + e).reshape(-1)
    return torch.bincount(idx, minlength=n * 16).cpu().numpy().astype(np.float64).reshape(n, 16)


def scan(path: str, *, per: str = "tensor", rows_per_slab: int = 64) -> dict:
    """Histograms of the FP8 tensors of a safetensors file: name -> [16]
    (per="tensor") or [slabs, 16] (per="slab", 2-D tensors only; others get
    one row).  Tensors are read one at a time."""
    from safetensors import safe_open

    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        for name in f.keys():
            sl = f.get_slice(name)
            if sl.get_dtype() not in ("F8_E4M3",):
                continue
            t = f.get_tensor(name)
            if per == "slab" and t.dim() == 2:
                out[name] = slab_histograms(t, rows_per_slab)
            elif per in ("tensor", "slab"):
                h = exponent_histogram(t)
                out[name] = h if per == "tensor" else h[None, :]
            else:
                raise ValueError("per must be 'tensor' or 'slab'")
    return out


def aggregate(hists: dict) -> np.ndarray:
    """The normalised sum of histograms (a table source like
    QWEN3_14B_FP8_EXP)."""
    tot = sum(np.asarray(h, dtype=np.float64).reshape(-1, 16).sum(axis=0) for h in hists.values())
    s = float(np.sum(tot))
    if s <= 0:
        raise ValueError("no FP8 elements")
    return tot / s


def _lane_shape(numel: int, lane_elems: int):
    """(K, N) for the lane layout of a flat tensor, or None if it has no even
    factorisation with N <= lane_elems."""
    if numel % lane_elems == 0:
        return numel // lane_elems, lane_elems
    for n in range(min(lane_elems, numel) // 2 * 2, 1, -2):
        if numel % n == 0:
            return numel // n, n
    return None


def encode_checkpoint(src: str, dst: str, *, alphabet: str = "pair", table: str = "tensor",
                      matrices: bool = True, lane_elems: int = 1024, device="cpu") -> dict:
    """Encode every FP8 tensor of the safetensors file ``src`` into the
    container ``dst``.

    2-D tensors become TansMatrix entries (the layout of
    fp8_gemm_fused_tans) when ``matrices``; other FP8 tensors become
    TansTensor entries of lane_elems elements per lane.  ``table``: "tensor"
    builds each table from the tensor's own histogram, "global" from the
    aggregate of all FP8 tensors.  Non-FP8 tensors are copied unchanged.
    ``device`` "cuda" encodes with the GPU encoder (matrices and lanes).
    Returns name -> {"kind", "shape", "bits_per_byte"}; the original shape
    and dtype of each encoded entry are kept in the metadata key
    ``shapes``."""
    from safetensors import safe_open

    if table not in ("tensor", "global"):
        raise ValueError("table must be 'tensor' or 'global'")
    hists = scan(src)
    glob = aggregate(hists) if table == "global" and hists else None
    entries, report, shapes = {}, {}, {}
    with safe_open(src, framework="pt", device="cpu") as f:
        for name in f.keys():
            t = f.get_tensor(name)
            if name not in hists:
                entries[name] = t
                continue
            if "." in name:
                raise ValueError(f"FP8 tensor names may not contain '.': {name}")
            b = t.view(torch.uint8)
            h = glob if glob is not None else hists[name]
            if matrices and b.dim() == 2 and b.shape[1] >= 2:
                e = encode_matrix(b.contiguous().to(device), h, alphabet=alphabet)
                kind, nbytes = "matrix", e.compressed_bytes()
            else:
                shp = _lane_shape(b.numel(), lane_elems)
                if shp is None:
                    entries[name] = t
                    continue
                K, N = shp
                x = b.reshape(K, N)
                enc = (encode_gpu(x.to(device), h, alphabet=alphabet) if str(device).startswith("cuda")
                       else encode(x, h, alphabet=alphabet))
                e = TansTensor.from_tuple(enc, K, N, alphabet)
                kind, nbytes = "lanes", e.compressed_bytes()
            entries[name] = e
            shapes[name] = {"shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", "")}
            report[name] = {"kind": kind, "shape": list(t.shape),
                            "bits_per_byte": nbytes * 8 / max(b.numel(), 1)}
    container.save(dst, entries, metadata={"shapes": json.dumps(shapes), "source": src})
    return report
