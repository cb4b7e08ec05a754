"""On-disk container for tANS-coded FP8 tensors (no counterpart in the
reference, which encodes in memory each run).

A container is one safetensors file, so it loads without executing anything
from the file.  For each encoded entry ``name`` it holds the tensors
``name.comp`` (uint8), ``name.states`` (uint16), ``name.offsets`` (int64),
``name.sm`` (uint8 tiles), ``name.freqs`` and ``name.spread`` (int32), and
the metadata key ``tans:name`` with a JSON description:

* ``{"kind": "lanes", "K", "N", "alphabet"}`` for a TansTensor (K lanes of N
  elements, the layout of gpu_tans_decode and fp8_vecadd_fused_tans);
* ``{"kind": "matrix", "rows", "cols", "segments", "seg_cols", "alphabet"}``
  for a TansMatrix (the layout of fp8_gemm_fused_tans).

Plain tensors (scales, unencoded weights) are stored under their own names;
``tans_format`` in the metadata names the layout version: v5 streams follow
the carry-driven refill schedule (segments of two steps for the pair
alphabet; 3, 3 and 2 steps for the nibble alphabet, whose tables give every
present symbol a frequency of at least 2) with a plain check before a last
16-element tile of one segment, or, for entries of lanes whose ``states``
part is empty, the packed layout of short streams (pair alphabet, N <= 64);
matrices use the 16-row matrix-core lane groups (include/tans_amd.h).  v4
files are v5 files without packed entries.  v3 files are read unless an
entry of lanes has such a last tile (N > 16 and N % 16 in 1..4 with pairs,
1..3 with nibbles: there v3 applied the final check), v2 files under the
same condition when all their entries use the pair alphabet; files of other
versions are refused.
"""
from __future__ import annotations

import json

import torch

from .tans_codec import TansMatrix, TansTensor

FORMAT = "tans-wave64-v5"
_NO_PACKED = "tans-wave64-v4"   # v5 without packed entries
_PREV = "tans-wave64-v3"        # differs only where _last_tile_rule_changed
_PAIR_ONLY = "tans-wave64-v2"   # pair entries: as v3


def _last_tile_rule_changed(desc: dict) -> bool:
    """An entry whose streams end in a 16-element tile of one refill segment
    (where v4 made the check before it the plain one).  Matrices never do:
    each lane holds a multiple of 8 elements."""
    if desc.get("kind") != "lanes":
        return False
    N = int(desc["N"])
    return N > 16 and 1 <= N % 16 <= (4 if desc.get("alphabet") == "pair" else 3)
_PARTS = ("comp", "states", "offsets", "sm", "freqs", "spread")


def save(path: str, entries: dict, metadata: dict | None = None) -> None:
    """Write ``entries`` (name -> TansTensor, TansMatrix or torch.Tensor) to
    ``path``.  Tensors are copied to the CPU; ``metadata`` adds string keys."""
    from safetensors.torch import save_file

    tensors: dict[str, torch.Tensor] = {}
    meta = {"tans_format": FORMAT}
    for k, v in (metadata or {}).items():
        if k.startswith("tans"):
            raise ValueError("metadata keys starting with 'tans' are reserved")
        meta[str(k)] = str(v)
    encoded = {n for n, e in entries.items() if isinstance(e, (TansTensor, TansMatrix))}
    for name, e in entries.items():
        if "." in name and name in encoded:
            raise ValueError(f"encoded entry names may not contain '.': {name}")
        stem, _, part = name.rpartition(".")
        if name not in encoded and stem in encoded and part in _PARTS:
            raise ValueError(f"plain tensor {name!r} would overwrite part {part!r} of the "
                             f"encoded entry {stem!r}")
        if isinstance(e, TansTensor):
            desc = {"kind": "lanes", "K": e.K, "N": e.N, "alphabet": e.alphabet}
        elif isinstance(e, TansMatrix):
            desc = {"kind": "matrix", "rows": e.rows, "cols": e.cols, "segments": e.segments,
                    "seg_cols": e.seg_cols, "alphabet": e.alphabet}
        elif isinstance(e, torch.Tensor):
            tensors[name] = e.detach().cpu().contiguous()
            continue
        else:
            raise TypeError(f"{name}: cannot store {type(e).__name__}")
        for part in _PARTS:
            tensors[f"{name}.{part}"] = getattr(e, part).detach().cpu().contiguous()
        meta[f"tans:{name}"] = json.dumps(desc)
    save_file(tensors, path, metadata=meta)


def load(path: str, device="cpu") -> dict:
    """Read a container: name -> TansTensor / TansMatrix / torch.Tensor, with
    every tensor on ``device``."""
    from safetensors import safe_open

    out: dict = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        fmt = meta.get("tans_format")
        if fmt not in (FORMAT, _NO_PACKED, _PREV, _PAIR_ONLY):
            raise ValueError(f"{path}: not a {FORMAT} container (format {fmt!r}); "
                             "re-encode it with this version")
        keys = set(f.keys())
        encoded = {k[len("tans:"):]: json.loads(v) for k, v in meta.items() if k.startswith("tans:")}
        if fmt == _PAIR_ONLY and any(d.get("alphabet") != "pair" for d in encoded.values()):
            raise ValueError(f"{path}: {fmt} container with nibble-alphabet entries, whose "
                             "streams follow the previous refill schedule; re-encode it with "
                             "this version")
        changed = [n for n, d in encoded.items() if _last_tile_rule_changed(d)]
        if fmt in (_PREV, _PAIR_ONLY) and changed:
            raise ValueError(f"{path}: {fmt} container whose entries {changed} end in a tile of "
                             "one refill segment, where that version's last check differs; "
                             "re-encode them with this version")
        for name, desc in encoded.items():
            parts = {p: f.get_tensor(f"{name}.{p}").to(device) for p in _PARTS}
            keys -= {f"{name}.{p}" for p in _PARTS}
            partial = torch.empty(0, dtype=torch.uint8, device=device)
            if desc["kind"] == "lanes":
                out[name] = TansTensor(parts["comp"], parts["states"], parts["offsets"], partial,
                                       parts["sm"], parts["freqs"], parts["spread"],
                                       K=int(desc["K"]), N=int(desc["N"]),
                                       alphabet=desc["alphabet"])
            elif desc["kind"] == "matrix":
                out[name] = TansMatrix(parts["comp"], parts["states"], parts["offsets"], partial,
                                       parts["sm"], parts["freqs"], parts["spread"],
                                       rows=int(desc["rows"]), cols=int(desc["cols"]),
                                       segments=int(desc["segments"]),
                                       seg_cols=int(desc["seg_cols"]), alphabet=desc["alphabet"])
            else:
                raise ValueError(f"{path}: entry {name} has unknown kind {desc['kind']}")
        for k in sorted(keys):
            out[k] = f.get_tensor(k).to(device)
    return out


def metadata(path: str) -> dict:
    """The user metadata of a container (without the reserved tans keys)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt", device="cpu") as f:
        return {k: v for k, v in (f.metadata() or {}).items() if not k.startswith("tans")}
