"""Quant-type registry and the bridge to llama.cpp's CPU quantizer (libggml-base).

Mirrors the reference's ``voodoo_quant/ggml.py`` (registry ``:30-66``, ladder
``:69-72``, library discovery ``:75-144``, ``quantize_tensor`` ``:171-221``,
``dequantize_tensor`` ``:224-269``) and adds the two K-quants the gated-Linear
path needs and the reference lacks:

* ``Q2_K``: ggml type 10, 256 weights per 84-byte block
* ``Q3_K``: ggml type 11, 256 weights per 110-byte block

(ids and sizes from the public ``ggml.h`` / ``ggml-common.h``; consistent with
the reference's Q4_K = 12, Q5_K = 13, Q6_K = 14 rows).

libggml stays the source of llama.cpp-exact candidate bytes when it can be
found (``$VOODOO_GGML_LIB`` first).  It is not present on every machine; the
gated layers then use the clearly labelled non-ggml encoder in
:mod:`voodoo_quant.rtn` (valid blocks, not llama.cpp-exact bytes).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np
import torch

QK_K = 256  # elements per K/IQ super-block


class QuantTypeInfo:
    def __init__(self, name: str, ggml_type: int, block_size: int, block_bytes: int, quant_func: str,
                 dequant_func: str):
        self.name = name
        self.ggml_type = ggml_type
        self.block_size = block_size
        self.block_bytes = block_bytes
        self.quant_func = quant_func
        self.dequant_func = dequant_func

    def bytes_per_weight(self) -> float:
        return self.block_bytes / self.block_size

    def __repr__(self) -> str:
        return f"QuantTypeInfo({self.name}, type={self.ggml_type}, {self.block_bytes}B/{self.block_size})"


def _info(name, ggml_type, block_size, block_bytes):
    low = name.lower() if not name.endswith("_K") else name[:-2].lower() + "_K"
    return QuantTypeInfo(name, ggml_type, block_size, block_bytes, f"quantize_{low}", f"dequantize_row_{low}")


_QUANT_REGISTRY: dict[str, QuantTypeInfo] = {
    "IQ1_S": _info("IQ1_S", 19, 256, 50),
    "IQ1_M": _info("IQ1_M", 29, 256, 56),
    "IQ2_XXS": _info("IQ2_XXS", 16, 256, 66),
    "IQ2_XS": _info("IQ2_XS", 17, 256, 74),
    "IQ2_S": _info("IQ2_S", 22, 256, 82),
    "IQ3_XXS": _info("IQ3_XXS", 18, 256, 98),
    "IQ3_S": _info("IQ3_S", 21, 256, 110),
    "IQ4_XS": _info("IQ4_XS", 23, 256, 136),
    "Q2_K": _info("Q2_K", 10, 256, 84),
    "Q3_K": _info("Q3_K", 11, 256, 110),
    "Q4_K": _info("Q4_K", 12, 256, 144),
    "Q5_K": _info("Q5_K", 13, 256, 176),
    "Q6_K": _info("Q6_K", 14, 256, 210),
    "Q8_0": _info("Q8_0", 8, 32, 34),
    "TQ1_0": _info("TQ1_0", 34, 256, 54),
    "TQ2_0": _info("TQ2_0", 35, 256, 66),
}

# The formats the HIP kernels decode (the gated-Linear candidate menu): every
# registry type but the ternary TQ1_0/TQ2_0, which the reference's default
# menu leaves out too (``ggml.py:156-158``).
HIP_TYPES: tuple[str, ...] = ("IQ1_S", "IQ1_M", "IQ2_XXS", "IQ2_XS", "IQ2_S", "Q2_K", "IQ3_XXS", "Q3_K", "IQ3_S",
                              "IQ4_XS", "Q4_K", "Q5_K", "Q6_K", "Q8_0")

# Quality ladder, coarsest to finest (reference ladder plus Q2_K/Q3_K at their
# bytes-per-weight positions).
QUANT_LADDER: list[str] = [
    "IQ1_S", "IQ1_M", "IQ2_XXS", "IQ2_XS", "IQ2_S", "Q2_K",
    "IQ3_XXS", "Q3_K", "IQ3_S", "IQ4_XS", "Q4_K", "Q5_K", "Q6_K", "Q8_0",
]

_LIB_NAME = "libggml-base.so"
_LIB = None


def _candidate_paths() -> list[Path]:
    paths: list[Path] = []
    env = os.environ.get("VOODOO_GGML_LIB")
    if env:
        paths.append(Path(env))
    root = Path(__file__).resolve().parent.parent
    paths.append(root / "third_party" / "llama.cpp" / "build" / "bin" / _LIB_NAME)
    for sibling in sorted(root.parent.glob("llama.cpp*")):
        paths.append(sibling / "build" / "bin" / _LIB_NAME)
    return paths


def find_libggml() -> Path | None:
    for p in _candidate_paths():
        if p.exists():
            return p
    try:
        ctypes.CDLL(_LIB_NAME)
        return Path(_LIB_NAME)
    except OSError:
        return None


def lib_path() -> str | None:
    p = find_libggml()
    return str(p) if p else None


def _load_lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    path = find_libggml()
    if path is None:
        raise RuntimeError(
            "libggml-base.so not found. Set VOODOO_GGML_LIB=/path/to/libggml-base.so or install llama.cpp."
        )
    try:
        L = ctypes.CDLL(str(path))
    except OSError:
        raise RuntimeError(f"Failed to load libggml-base from {path}; point VOODOO_GGML_LIB at a valid build.") from None
    L.ggml_quantize_init.argtypes = [ctypes.c_int]
    L.ggml_quantize_init.restype = None
    for info in _QUANT_REGISTRY.values():
        q = getattr(L, info.quant_func, None)
        if q is not None:
            q.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                          ctypes.POINTER(ctypes.c_float)]
            q.restype = ctypes.c_size_t
        dq = getattr(L, info.dequant_func, None)
        if dq is not None:
            dq.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int64]
            dq.restype = None
    _LIB = L
    return _LIB


def list_quant_types() -> list[str]:
    return list(_QUANT_REGISTRY.keys())


def default_candidate_types() -> list[str]:
    """All registry types except ternary ones (reference ``ggml.py:155-157``)."""
    return [qt for qt in list_quant_types() if not qt.startswith("TQ")]


def get_quant_info(quant_type: str) -> QuantTypeInfo:
    if quant_type not in _QUANT_REGISTRY:
        raise ValueError(f"Unknown quant type: {quant_type}. Supported: {list(_QUANT_REGISTRY.keys())}")
    return _QUANT_REGISTRY[quant_type]


def bytes_per_weight(quant_type: str) -> float:
    return get_quant_info(quant_type).bytes_per_weight()


def quantize_tensor(weight: torch.Tensor, quant_type: str, imatrix: torch.Tensor | None = None) -> torch.Tensor:
    """Quantize [out, in] weights with llama.cpp's own quantizer -> uint8 [nblocks, block_bytes].

    Always passes an importance matrix (all ones when None), as the reference
    does (``ggml.py:204-205``)."""
    info = get_quant_info(quant_type)
    L = _load_lib()
    L.ggml_quantize_init(info.ggml_type)
    weight = weight.float().contiguous()
    out_features, in_features = weight.shape
    if in_features % info.block_size != 0:
        raise ValueError(f"{quant_type} requires in_features % {info.block_size} == 0, got {in_features}")
    nblocks = out_features * (in_features // info.block_size)
    out_bytes = nblocks * info.block_bytes
    imatrix = torch.ones(in_features) if imatrix is None else imatrix.float().contiguous()
    if imatrix.numel() != in_features:
        raise ValueError(f"imatrix size {imatrix.numel()} != in_features {in_features}")
    dst = np.empty(out_bytes, dtype=np.uint8)
    fn = getattr(L, info.quant_func)
    res = fn(ctypes.cast(weight.data_ptr(), ctypes.POINTER(ctypes.c_float)), dst.ctypes.data, out_features,
             in_features, ctypes.cast(imatrix.data_ptr(), ctypes.POINTER(ctypes.c_float)))
    if res != out_bytes:
        raise RuntimeError(f"{info.quant_func} returned {res} bytes, expected {out_bytes}")
    return torch.from_numpy(dst).reshape(nblocks, info.block_bytes)


def dequantize_tensor(qweight: torch.Tensor, quant_type: str, out_features: int, in_features: int,
                      pin_memory: bool = False) -> torch.Tensor:
    """libggml CPU decode (reference ``ggml.py:224-269``).  For device tensors
    use :func:`voodoo_quant.layers.dequantize_tensor_gpu`."""
    info = get_quant_info(quant_type)
    if in_features % info.block_size != 0:
        raise ValueError(f"{quant_type} requires in_features % {info.block_size} == 0, got {in_features}")
    nblocks = out_features * (in_features // info.block_size)
    if qweight.numel() != nblocks * info.block_bytes:
        raise ValueError(f"qweight size {qweight.numel()} does not match {nblocks} blocks of "
                         f"{info.block_bytes} bytes for {quant_type}")
    L = _load_lib()
    qweight = qweight.reshape(-1).contiguous()
    out = torch.empty(out_features * in_features, dtype=torch.float32, pin_memory=pin_memory)
    getattr(L, info.dequant_func)(ctypes.c_void_p(qweight.data_ptr()),
                                  ctypes.cast(out.data_ptr(), ctypes.POINTER(ctypes.c_float)),
                                  out_features * in_features)
    return out.reshape(out_features, in_features)


def estimate_bytes(shape: tuple[int, ...], quant_type: str | None, source_dtype: torch.dtype = torch.bfloat16) -> int:
    numel = int(np.prod(shape))
    if quant_type is None:
        return numel * torch.finfo(source_dtype).bits // 8
    return int(numel * bytes_per_weight(quant_type))
