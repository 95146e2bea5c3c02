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

Usage:  python tests/golden/make_golden.py
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


def main() -> None:
    sys.dont_write_bytecode = True
    cache = tempfile.mkdtemp(prefix="vq_golden_")
    # the reference package sets these with setdefault at import time
    os.environ["TRITON_CACHE_DIR"] = os.path.join(cache, "triton")
    os.environ["TORCHINDUCTOR_CACHE_DIR"] = os.path.join(cache, "inductor")
    sys.path.insert(0, str(REF))
    sys.path.insert(1, str(REPO))
    import torch

    from voodoo_quant import layers as ref_layers  # the REFERENCE package

    assert Path(ref_layers.__file__).resolve().is_relative_to(REF.resolve()), ref_layers.__file__
    from oracle import blocks

    fns = {
        "Q8_0": ref_layers._dequantize_q8_0_gpu,
        "Q4_K": ref_layers._dequantize_q4_K_gpu,
        "Q5_K": ref_layers._dequantize_q5_K_gpu,
        "Q6_K": ref_layers._dequantize_q6_K_gpu,
    }
    out: dict[str, np.ndarray] = {}
    for seed, (qt, fn) in enumerate(fns.items()):
        rng = np.random.default_rng(1000 + seed)
        bb = blocks.BLOCK_BYTES[qt]
        nb_rand = 48 if qt != "Q8_0" else 384
        rand = blocks.random_blocks(qt, nb_rand, rng)
        per_edge = 1 if qt != "Q8_0" else 8
        edge = []
        for fill, d, dmin in EDGE_CASES:
            blk = np.full((per_edge, bb), fill, np.uint8)
            offs = blocks.F16_OFFSETS[qt]
            for off, h in zip(offs, (d, dmin)):
                blk[:, off] = h & 0xFF
                blk[:, off + 1] = h >> 8
            edge.append(blk)
        qbytes = np.concatenate([rand] + edge, axis=0)
        n_weights = qbytes.shape[0] * blocks.BLOCK_SIZE[qt]
        rows = n_weights // 256
        y = fn(torch.from_numpy(qbytes.reshape(-1).copy()), rows, 256)
        out[f"{qt}_qbytes"] = qbytes
        out[f"{qt}_out"] = y.reshape(-1).numpy().astype(np.float32)
        print(f"{qt}: {qbytes.shape[0]} blocks -> {n_weights} weights")
    dst = HERE / "ref_decoders.npz"
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({dst.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
