"""Candidate-cache builder: quantize a model's selectable weights into the
on-disk candidate cache before training (reference
``voodoo_quant/tools/precache.py:88-229``).

A gated layer built over a tensor whose combined cache entry exists loads its
candidate bytes instead of quantizing them, so a precached model starts
training without the per-tensor quantization pass.

Selection follows the reference's rules (``precache.py:150-166``): every 2-D
parameter whose row length is a multiple of 32 or 256, except the recipe's
``in_proj_a``/``in_proj_b`` tensors (kept in F32), with the per-tensor menu
from :func:`voodoo_quant.layers.resolve_candidate_types` (attention and
non-attention menus).  Entries go under the keys :mod:`voodoo_quant.cache`
defines: ``combined_lazy_*`` holds packed llama.cpp bytes, ``combined_dequant_*``
their bf16 decodes.  A tensor whose combined file exists is skipped.  Without
libggml the candidates come from the labelled RTN encoder and are stored under
:data:`voodoo_quant.cache.RTN_MODE` (``dequant_rtn`` for decodes), keys that a
run with libggml, here or in the reference, never reads.

The gated layers load packed entries only (``combined_lazy_*``, or the RTN
key without libggml), so packed is the default here and on the command line;
decoded entries (``lazy=False``, ``--decoded``) are for other readers.
Decodes come from libggml's ``dequantize_row_*`` when it loads,
else from the HIP decoders on a ROCm device (bit-identical fp32, then bf16);
with neither the call raises.  Quantization runs on the CPU, one tensor at a
time (bounded memory), its candidate types in a thread pool: libggml's
quantizers and torch's kernels both run without the GIL.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

import torch
import torch.nn as nn

from voodoo_quant import cache, layers
from voodoo_quant.ggml import default_candidate_types, dequantize_tensor, find_libggml

# modules whose weights the recipe keeps in F32 (never gated, never cached)
_F32_SUFFIXES = (".in_proj_a", ".in_proj_b")
RTN_DEQUANT_MODE = "dequant_rtn"


@dataclass
class PrecacheReport:
    tensors: int = 0
    built: int = 0       # candidate entries quantized in this call
    cached: int = 0      # entries found in the cache already
    errors: list[str] = field(default_factory=list)
    source: str = ""     # "ggml" or "rtn"
    seconds: float = 0.0


def selectable_tensors(model: nn.Module, candidate_types: list[str],
                       attention_candidates: list[str] | None = None,
                       non_attention_candidates: list[str] | None = None) -> dict[str, list[str]]:
    """Module name (the parameter name without ``.weight``) -> its candidate
    types, for every tensor the gated layers would quantize."""
    out: dict[str, list[str]] = {}
    for pname, p in model.named_parameters():
        if p.dim() != 2 or (p.shape[1] % 256 and p.shape[1] % 32):
            continue
        name = pname[: -len(".weight")] if pname.endswith(".weight") else pname
        if name.endswith(_F32_SUFFIXES):
            continue
        types = layers.resolve_candidate_types(name, candidate_types, attention_candidates, non_attention_candidates)
        if types:
            out[name] = types
    return out


def _decode_bf16(qbytes: torch.Tensor, qt: str, out_f: int, in_pad: int, have_ggml: bool) -> torch.Tensor:
    if have_ggml:
        return dequantize_tensor(qbytes, qt, out_f, in_pad).to(torch.bfloat16)
    if not torch.cuda.is_available():
        raise RuntimeError("decoded (non-lazy) entries need libggml or a ROCm device for the HIP decoders")
    return layers.dequantize_tensor_gpu(qbytes, qt, out_f, in_pad, torch.device("cuda")).cpu()


def precache_model(model: nn.Module, candidate_types: list[str] | None = None,
                   attention_candidates: list[str] | None = None,
                   non_attention_candidates: list[str] | None = None, lazy: bool = True,
                   root: Path | str | None = None, workers: int | None = None,
                   log=None) -> PrecacheReport:
    """Write every selectable tensor's candidates into the cache at ``root``
    (default: the gated layers' cache directory).  Returns counts per entry;
    a candidate type that fails to quantize is reported in ``errors`` and the
    tensor's other types are still written."""
    t0 = time.monotonic()
    types = list(candidate_types) if candidate_types is not None else default_candidate_types()
    plan = selectable_tensors(model, types, attention_candidates, non_attention_candidates)
    root = Path(root) if root is not None else Path(layers.CANDIDATE_CACHE_DIR)
    have_ggml = find_libggml() is not None
    rep = PrecacheReport(tensors=len(plan), source="ggml" if have_ggml else "rtn")
    if have_ggml:
        mode = "lazy" if lazy else "dequant"
    else:
        mode = cache.RTN_MODE if lazy else RTN_DEQUANT_MODE
    if workers is None:
        workers = int(os.environ.get("VOODOO_QUANT_WORKERS", min(16, os.cpu_count() or 2)))
    params = dict(model.named_parameters())
    for i, (name, tensor_types) in enumerate(plan.items()):
        w = params[name + ".weight" if name + ".weight" in params else name].detach()
        padded, _, _ = layers.pad_weight_and_imatrix(w.to("cpu", torch.float32).contiguous(), None)
        out_f, in_pad = padded.shape
        wh = cache.tensor_hash(padded)
        if cache.combined_cache_path(name, mode, wh, "none", root).exists():
            rep.cached += len(tensor_types)
            continue

        def build(qt: str):
            made, _ = layers._quantize_candidates(padded, None, [qt])
            qb = made[qt]
            return qb if lazy else _decode_bf16(qb, qt, out_f, in_pad, have_ggml)

        entries: dict[str, torch.Tensor] = {}
        with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
            futs = {ex.submit(build, qt): qt for qt in tensor_types}
            for fut in concurrent.futures.as_completed(futs):
                qt = futs[fut]
                try:
                    entries[qt] = fut.result()
                except Exception as e:  # noqa: BLE001 - reported per entry, as the reference does
                    rep.errors.append(f"{name} {qt}: {e}")
        if entries:
            cache.save_candidates(name, entries, mode, wh, "none", root)
        rep.built += len(entries)
        if log is not None:
            log(f"[precache] {i + 1}/{len(plan)} {name}: {len(entries)} built, "
                f"{len(tensor_types) - len(entries)} failed")
    rep.seconds = time.monotonic() - t0
    return rep


def main(argv=None) -> int:
    """Command line of the reference's tool (``precache.py:88-103``): the
    architecture comes from ``--model``'s config (no weight download), the
    weights from ``--checkpoint`` (``model_state_dict``, loaded with
    ``weights_only=True``)."""
    ap = argparse.ArgumentParser(description="Pre-build the quant candidate cache (CPU quantization)")
    ap.add_argument("--checkpoint", required=True)
    ap.add_argument("--model", default=None,
                    help="HF model id or local config directory matching the checkpoint; "
                         "falls back to $VOODOO_PRECACHE_MODEL")
    ap.add_argument("--candidate_types", nargs="+", default=default_candidate_types())
    ap.add_argument("--attention_candidates", nargs="+", default=None)
    ap.add_argument("--non_attention_candidates", nargs="+", default=None)
    # The gated layers read only packed ("lazy") entries, so those are the
    # default; --lazy is accepted for the reference's command lines, and
    # --decoded writes bf16 decodes for other readers (with a warning)
    ap.add_argument("--lazy", dest="decoded", action="store_false")
    ap.add_argument("--decoded", dest="decoded", action="store_true",
                    help="write bf16 decodes (combined_dequant_*) instead of packed bytes; "
                         "MixedQuantLinear never reads them")
    ap.set_defaults(decoded=False)
    ap.add_argument("--device", default="cpu", help="unused: quantization runs on the CPU")
    args = ap.parse_args(argv)
    if args.decoded:
        print("precache: --decoded writes combined_dequant_* entries, which the gated layers never read "
              "(they load combined_lazy_* packed bytes only)", file=sys.stderr)
    base = args.model or os.environ.get("VOODOO_PRECACHE_MODEL")
    if not base:
        ap.error("--model is required (or set VOODOO_PRECACHE_MODEL)")
    from transformers import AutoConfig, AutoModelForCausalLM

    cfg = AutoConfig.from_pretrained(base, trust_remote_code=True)
    model = AutoModelForCausalLM.from_config(cfg, trust_remote_code=True).to(torch.bfloat16)
    ckpt = torch.load(args.checkpoint, weights_only=True, map_location="cpu", mmap=True)
    model.load_state_dict(ckpt["model_state_dict"], strict=False, assign=True)
    rep = precache_model(model, args.candidate_types, args.attention_candidates, args.non_attention_candidates,
                         lazy=not args.decoded, log=print)
    print(f"precache: {rep.tensors} tensors, {rep.built} entries built, {rep.cached} already cached, "
          f"{len(rep.errors)} errors, {rep.seconds:.1f} s (candidates from {rep.source})")
    for e in rep.errors:
        print(f"  error: {e}", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
