"""ctypes loader for the oracle's C decoders (test infrastructure only)."""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_dequant.so"
_LIB = None

# ggml type ids and bytes per 256 weights (Q8_0: eight 34-byte blocks)
GGML_TYPE = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ2_XXS": 16, "IQ2_XS": 17,
             "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29}
BYTES_PER_256 = {"Q8_0": 272, "Q2_K": 84, "Q3_K": 110, "Q4_K": 144, "Q5_K": 176, "Q6_K": 210, "IQ2_XXS": 66,
                 "IQ2_XS": 74, "IQ3_XXS": 98, "IQ1_S": 50, "IQ3_S": 110, "IQ2_S": 82, "IQ4_XS": 136, "IQ1_M": 56}


def build_oracle_lib(force: bool = False) -> Path:
    """Compile ``dequant_ref.c`` with the committed Makefile."""
    if force or not _LIB_PATH.exists():
        cmd = ["make", "-s", "-C", str(_HERE)] + (["-B"] if force else [])
        subprocess.run(cmd, check=True)
    return _LIB_PATH


def load_oracle_lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build_oracle_lib()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.oracle_dequant.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.oracle_dequant.restype = ctypes.c_int
        lib.oracle_dequant_parallel.argtypes = [
            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
        ]
        lib.oracle_dequant_parallel.restype = ctypes.c_int
        lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        lib.oracle_half_to_float.restype = ctypes.c_float
        _LIB = lib
    return _LIB


def _check(qtype: str, qbytes: np.ndarray, n_weights: int) -> np.ndarray:
    if qtype not in GGML_TYPE:
        raise ValueError(f"oracle: unsupported quant type {qtype}")
    if n_weights % 256:
        raise ValueError("oracle: weight count must be a multiple of 256")
    q = np.ascontiguousarray(qbytes, dtype=np.uint8).reshape(-1)
    if q.size != n_weights // 256 * BYTES_PER_256[qtype]:
        raise ValueError(f"oracle: {qtype} byte count {q.size} != {n_weights // 256 * BYTES_PER_256[qtype]}")
    return q


def oracle_dequant(qtype: str, qbytes: np.ndarray, n_weights: int) -> np.ndarray:
    """Single-threaded scalar decode of ``n_weights`` weights -> fp32 array."""
    q = _check(qtype, qbytes, n_weights)
    out = np.empty(n_weights, dtype=np.float32)
    rc = load_oracle_lib().oracle_dequant(GGML_TYPE[qtype], q.ctypes.data, out.ctypes.data, n_weights)
    if rc != 0:
        raise RuntimeError("oracle_dequant failed")
    return out


def oracle_dequant_parallel(qtype: str, qbytes: np.ndarray, n_weights: int, nthreads: int = 0) -> np.ndarray:
    """OpenMP decode (``nthreads`` <= 0 keeps the OpenMP default)."""
    q = _check(qtype, qbytes, n_weights)
    out = np.empty(n_weights, dtype=np.float32)
    rc = load_oracle_lib().oracle_dequant_parallel(
        GGML_TYPE[qtype], q.ctypes.data, out.ctypes.data, n_weights, int(nthreads)
    )
    if rc != 0:
        raise RuntimeError("oracle_dequant_parallel failed")
    return out


def half_to_float(h: int) -> float:
    return float(load_oracle_lib().oracle_half_to_float(ctypes.c_uint16(h)))


os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")
