"""Write golden vectors of the reference's own GGUF block decoders.

Runs ONLY in the development container, where the reference checkout is
mounted (default ``/root/reference``; override with ``VOODOO_REFERENCE``).
It imports the reference's pure-torch decoders
``_dequantize_{q8_0,q4_K,q5_K,q6_K}_gpu`` (``voodoo_quant/layers.py:62-213``),
runs them on the CPU over seeded random valid blocks plus hand-made edge
blocks, and stores inputs and outputs in ``ref_decoders.npz``.  Nothing from
the reference is stored except those input/output arrays.

Why an import is needed: the closed forms in ``oracle/blocks.py`` pin each
decoder against a packer written from the format description, but only an
independent implementation pins the byte layout itself.  Q2_K and Q3_K have no
decoder in the reference, so they have no golden vectors here.

The IQ formats (``ref_iq_decoders.npz``) come from the reference's
``voodoo_quant/quants/gpu_dequant.py:53-519`` decoders, which it marks as
bit-identical to ggml's (``layers.py:217-225``).  Nothing else pins them: their
code books admit no closed form and the reference's own tests of them need a
libggml that is not present.

Usage:  python tests/golden/make_golden.py [k|iq|all]
"""

from __future__ import annotations

import os
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
REF = Path(os.environ.get("VOODOO_REFERENCE", "/root/reference"))

# Edge blocks: payload byte fill, fp16 scale bit patterns (d, dmin)
EDGE_CASES = [
    (0x00, 0x3C00, 0x3C00),  # all-zero payload, d = dmin = 1.0
    (0x00, 0xBC00, 0xBC00),  # all-zero payload, negative scales -> signed zeros
    (0xFF, 0x3C00, 0x3C00),  # all-ones payload
    (0xFF, 0x0001, 0x8001),  # smallest subnormal scales
    (0xA5, 0x7BFF, 0xFBFF),  # largest finite scales
    (0x5A, 0x0000, 0x8000),  # +0 / -0 scales
]


def _edge_blocks(blocks, qt: str, per_edge: int) -> list[np.ndarray]:
    out = []
    for fill, d, dmin in EDGE_CASES:
        blk = np.full((per_edge, blocks.BLOCK_BYTES[qt]), fill, np.uint8)
        for which, h in enumerate((d, dmin)[:max(len(blocks.F16_OFFSETS[qt]), 1)]):
            blocks.set_scale(qt, blk, h, which)
        out.append(blk)
    return out


def _vectors(torch, blocks, fns: dict, seed0: int, nb_rand: dict, dst: Path) -> None:
    out: dict[str, np.ndarray] = {}
    for seed, (qt, fn) in enumerate(fns.items()):
        rng = np.random.default_rng(seed0 + seed)
        rand = blocks.random_blocks(qt, nb_rand.get(qt, nb_rand["default"]), rng)
        edge = _edge_blocks(blocks, qt, 1 if qt != "Q8_0" else 8)
        qbytes = np.concatenate([rand] + edge, axis=0)
        n_weights = qbytes.shape[0] * blocks.BLOCK_SIZE[qt]
        rows = n_weights // 256
        y = fn(torch.from_numpy(qbytes.reshape(-1).copy()), rows, 256)
        out[f"{qt}_qbytes"] = qbytes
        out[f"{qt}_out"] = y.reshape(-1).numpy().astype(np.float32)
        print(f"{qt}: {qbytes.shape[0]} blocks -> {n_weights} weights")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({dst.stat().st_size} bytes)")


def main() -> None:
    which = sys.argv[1] if len(sys.argv) > 1 else "all"
    sys.dont_write_bytecode = True
    cache = tempfile.mkdtemp(prefix="vq_golden_")
    # the reference package sets these with setdefault at import time
    os.environ["TRITON_CACHE_DIR"] = os.path.join(cache, "triton")
    os.environ["TORCHINDUCTOR_CACHE_DIR"] = os.path.join(cache, "inductor")
    sys.path.insert(0, str(REF))
    sys.path.insert(1, str(REPO))
    import torch

    from voodoo_quant import layers as ref_layers  # the REFERENCE package
    from voodoo_quant.quants import gpu_dequant as ref_iq

    for mod in (ref_layers, ref_iq):
        assert Path(mod.__file__).resolve().is_relative_to(REF.resolve()), mod.__file__
    from oracle import blocks

    if which in ("k", "all"):
        fns = {
            "Q8_0": ref_layers._dequantize_q8_0_gpu,
            "Q4_K": ref_layers._dequantize_q4_K_gpu,
            "Q5_K": ref_layers._dequantize_q5_K_gpu,
            "Q6_K": ref_layers._dequantize_q6_K_gpu,
        }
        _vectors(torch, blocks, fns, 1000, {"default": 48, "Q8_0": 384}, HERE / "ref_decoders.npz")
    if which in ("iq", "all"):
        fns = {qt: getattr(ref_iq, f"_dequantize_{qt.lower()}_gpu") for qt in blocks.IQ_TYPES}
        _vectors(torch, blocks, fns, 2000, {"default": 128}, HERE / "ref_iq_decoders.npz")


if __name__ == "__main__":
    main()
