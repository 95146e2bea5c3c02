"""Candidate cache: on-disk store of each tensor's quantized candidates.

Same keys and file format as the reference's cache (``voodoo_quant/layers.py:
795-800, 884-944, 962-971, 1116-1155``; writer ``tools/precache.py:170-218``),
so caches built by either side are interchangeable:

* directory ``<root>/<tensor name with '.' and '/' -> '_'>/``
* combined file ``combined_{lazy|dequant}_w<sha16>_i<sha16|none>.pt`` holding
  ``{quant_type: tensor}``; per-type files ``<qt>_<mode>_w.._i...pt``
* ``<sha16>`` = first 16 hex digits of SHA-256 over the fp32 little-endian bytes
  of the (256-padded) weight or imatrix, streamed in 4M-element chunks
* lookups try the name with and without a ``model.`` prefix
* writes are atomic (temporary file + ``os.replace``)

The gated layers here keep candidates as packed bytes, i.e. the ``lazy``
entries (``uint8 [nblocks, block_bytes]``).  ``lazy`` entries hold llama.cpp
bytes only.  Candidates made by the non-ggml RTN encoder (no libggml on the
host) are stored under :data:`RTN_MODE` instead: same layout, a file name no
ggml-backed run (here or in the reference) ever looks up.  One root governs every path: the
module attribute :data:`CANDIDATE_CACHE_DIR` (or ``$VOODOO_CANDIDATE_CACHE_DIR``),
read at call time, so tests can point it at a temporary directory.
"""

from __future__ import annotations

import hashlib
import os
from pathlib import Path

import torch

CANDIDATE_CACHE_DIR = Path(
    os.environ.get("VOODOO_CANDIDATE_CACHE_DIR", Path(__file__).resolve().parent.parent / ".cache" / "mixed_quant_candidates")
)


# mode of the entries written from the RTN fallback encoder
RTN_MODE = "lazy_rtn"


def cache_root(root: Path | str | None = None) -> Path:
    return Path(root) if root is not None else Path(CANDIDATE_CACHE_DIR)


def tensor_hash(t: torch.Tensor | None) -> str:
    """First 16 hex digits of SHA-256 over the tensor's fp32 bytes ("none" for None)."""
    if t is None:
        return "none"
    flat = t.detach().contiguous().cpu().reshape(-1)
    h = hashlib.sha256()
    chunk = 1 << 22
    for i in range(0, flat.numel(), chunk):
        part = flat[i:i + chunk]
        if part.dtype != torch.float32:
            part = part.to(torch.float32)
        h.update(part.numpy().tobytes())
    return h.hexdigest()[:16]


def _safe_name(tensor_name: str) -> str:
    return tensor_name.replace(".", "_").replace("/", "_")


def candidate_cache_path(tensor_name: str, candidate_type: str, mode: str, weight_hash: str, imatrix_hash: str,
                         root: Path | str | None = None) -> Path:
    d = cache_root(root) / _safe_name(tensor_name)
    d.mkdir(parents=True, exist_ok=True)
    return d / f"{candidate_type}_{mode}_w{weight_hash}_i{imatrix_hash}.pt"


def combined_cache_path(tensor_name: str, mode: str, weight_hash: str, imatrix_hash: str,
                        root: Path | str | None = None) -> Path:
    d = cache_root(root) / _safe_name(tensor_name)
    d.mkdir(parents=True, exist_ok=True)
    return d / f"combined_{mode}_w{weight_hash}_i{imatrix_hash}.pt"


def atomic_torch_save(obj, path: Path) -> None:
    tmp = path.with_suffix(path.suffix + f".tmp{os.getpid()}")
    torch.save(obj, tmp)
    os.replace(tmp, path)


def _alt_name(name: str) -> str:
    return name.removeprefix("model.") if name.startswith("model.") else "model." + name


def load_candidates(tensor_name: str, candidate_types: list[str], mode: str, weight_hash: str, imatrix_hash: str,
                    root: Path | str | None = None) -> dict[str, torch.Tensor]:
    """Every cached candidate of ``candidate_types`` (combined file first, then
    per-type files).  Missing types are simply absent from the result."""
    found: dict[str, torch.Tensor] = {}
    for name in (tensor_name, _alt_name(tensor_name)):
        p = cache_root(root) / _safe_name(name) / f"combined_{mode}_w{weight_hash}_i{imatrix_hash}.pt"
        if p.exists():
            combined = torch.load(p, weights_only=True, map_location="cpu")
            for qt in candidate_types:
                if qt in combined and qt not in found:
                    found[qt] = combined[qt]
            break
    for qt in candidate_types:
        if qt in found:
            continue
        p = cache_root(root) / _safe_name(tensor_name) / f"{qt}_{mode}_w{weight_hash}_i{imatrix_hash}.pt"
        if p.exists():
            found[qt] = torch.load(p, weights_only=True, map_location="cpu")
    return found


def save_candidates(tensor_name: str, cands: dict[str, torch.Tensor], mode: str, weight_hash: str,
                    imatrix_hash: str, root: Path | str | None = None) -> Path:
    """Write (or extend) the combined file for this tensor."""
    p = combined_cache_path(tensor_name, mode, weight_hash, imatrix_hash, root)
    merged: dict[str, torch.Tensor] = {}
    if p.exists():
        merged.update(torch.load(p, weights_only=True, map_location="cpu"))
    merged.update({qt: t.detach().cpu().contiguous() for qt, t in cands.items()})
    atomic_torch_save(merged, p)
    return p


# Names used by the reference's layers module.
_tensor_hash = tensor_hash
_candidate_cache_path = candidate_cache_path
_combined_cache_path = combined_cache_path
_atomic_torch_save = atomic_torch_save
