"""Structured GGUF block packers and closed-form weight values (test infrastructure).

Every format is described here by its *fields* (fp16 scales, sub-block scales
and mins, quant codes) and by where each field lives in the block bytes.  Two
functions per format are independent of the byte decoders under test:

* ``pack_<fmt>(fields) -> uint8 [nb, block_bytes]`` writes the fields into the
  byte layout of the public GGUF format (llama.cpp ``ggml-common.h``; for
  Q8_0/Q4_K/Q5_K/Q6_K the same layout the reference decodes in
  ``voodoo_quant/layers.py:62-213``).
* ``value_<fmt>(fields) -> float32 [nb, 256 or 32]`` computes each weight
  straight from its fields with the same float operations ggml uses
  (``(d*sc)*q - (dmin*m)`` etc.), one numpy float32 op per C op, so results are
  bit-comparable.

A decoder that reads a wrong byte, bit or scale index disagrees with
``value_<fmt>`` on random fields.  Field placement is written per weight index
(``i -> byte, bit``), not by mirroring ggml's loop nest.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

BLOCK_BYTES = {"Q8_0": 34, "Q2_K": 84, "Q3_K": 110, "Q4_K": 144, "Q5_K": 176, "Q6_K": 210,
               "IQ1_S": 50, "IQ1_M": 56, "IQ2_XXS": 66, "IQ2_XS": 74, "IQ2_S": 82, "IQ3_XXS": 98, "IQ3_S": 110,
               "IQ4_XS": 136}
BLOCK_SIZE = {qt: 32 if qt == "Q8_0" else 256 for qt in BLOCK_BYTES}
# The IQ formats: sub-block scales times grid (code book) values; no closed-form
# packer here, their decoders are pinned by the reference's own outputs.
IQ_TYPES = ("IQ1_S", "IQ1_M", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S", "IQ4_XS")


def h2f(h: np.ndarray) -> np.ndarray:
    """Exact fp16 bit pattern -> float32."""
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def random_finite_f16(rng: np.random.Generator, shape, *, allow_subnormal=True, allow_negative=True) -> np.ndarray:
    h = rng.integers(0, 1 << 16, size=shape, dtype=np.uint32).astype(np.uint16)
    exp = (h >> 10) & 0x1F
    h = np.where(exp == 0x1F, h ^ np.uint16(0x4000), h).astype(np.uint16)  # no inf/nan
    if not allow_subnormal:
        exp = (h >> 10) & 0x1F
        h = np.where(exp == 0, h | np.uint16(0x0400), h).astype(np.uint16)
    if not allow_negative:
        h = (h & np.uint16(0x7FFF)).astype(np.uint16)
    return h


def _put16(dst: np.ndarray, off: int, h: np.ndarray) -> None:
    h = np.asarray(h, dtype=np.uint16)
    dst[:, off] = (h & 0xFF).astype(np.uint8)
    dst[:, off + 1] = (h >> 8).astype(np.uint8)


# --------------------------------------------------------------------------- Q8_0
def pack_q8_0(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    nb = d.shape[0]
    out = np.zeros((nb, 34), np.uint8)
    _put16(out, 0, d)
    out[:, 2:34] = q.astype(np.int8).view(np.uint8)
    return out


def value_q8_0(d, q):
    return q.astype(F32) * h2f(d)[:, None]


# --------------------------------------------------------------------------- K-quant index maps
def _idx_k4(i):
    """Q4_K/Q5_K: weight i -> (qs byte, nibble shift, sub-block, qh bit)."""
    c, r = i // 64, i % 64
    return 32 * c + (r % 32), 4 * (r // 32), i // 32, 2 * c + (r // 32)


def _idx_q6(i):
    """Q6_K: weight i -> (ql byte, ql shift, qh byte, qh shift, scale index)."""
    n, r = i // 128, i % 128
    t, l = r // 32, r % 32
    return 64 * n + l + 32 * (t & 1), 4 * (t >> 1), 32 * n + l, 2 * t, 8 * n + l // 16 + 2 * t


def _idx_q23(i):
    """Q2_K/Q3_K: weight i -> (qs byte, shift, hmask byte, hmask bit, scale index)."""
    n, r = i // 128, i % 128
    j, half, l = r // 32, (r % 32) // 16, r % 16
    return 32 * n + 16 * half + l, 2 * j, 16 * half + l, 4 * n + j, 8 * n + 2 * j + half


_I256 = np.arange(256)


def _pack_scales_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """8 six-bit scales and mins -> 12 bytes (Q4_K/Q5_K)."""
    nb = sc.shape[0]
    b = np.zeros((nb, 12), np.uint16)
    for j in range(4):
        b[:, j] = sc[:, j] | ((sc[:, j + 4] >> 4) << 6)
        b[:, j + 4] = m[:, j] | ((m[:, j + 4] >> 4) << 6)
        b[:, j + 8] = (sc[:, j + 4] & 0xF) | ((m[:, j + 4] & 0xF) << 4)
    return b.astype(np.uint8)


# --------------------------------------------------------------------------- Q4_K
def pack_q4_K(d, dmin, sc, m, q):
    nb = d.shape[0]
    out = np.zeros((nb, 144), np.uint8)
    _put16(out, 0, d)
    _put16(out, 2, dmin)
    out[:, 4:16] = _pack_scales_k4(sc.astype(np.uint16), m.astype(np.uint16))
    byte, shift, _, _ = _idx_k4(_I256)
    qs = np.zeros((nb, 128), np.uint16)
    for i in range(256):
        qs[:, byte[i]] |= (q[:, i].astype(np.uint16) & 0xF) << int(shift[i])
    out[:, 16:144] = qs.astype(np.uint8)
    return out


def value_q4_K(d, dmin, sc, m, q):
    _, _, sub, _ = _idx_k4(_I256)
    dl = h2f(d)[:, None] * sc[:, sub].astype(F32)
    ml = h2f(dmin)[:, None] * m[:, sub].astype(F32)
    return dl * q.astype(F32) - ml


# --------------------------------------------------------------------------- Q5_K
def pack_q5_K(d, dmin, sc, m, q):
    nb = d.shape[0]
    out = np.zeros((nb, 176), np.uint8)
    _put16(out, 0, d)
    _put16(out, 2, dmin)
    out[:, 4:16] = _pack_scales_k4(sc.astype(np.uint16), m.astype(np.uint16))
    byte, shift, _, hbit = _idx_k4(_I256)
    qs = np.zeros((nb, 128), np.uint16)
    qh = np.zeros((nb, 32), np.uint16)
    for i in range(256):
        qi = q[:, i].astype(np.uint16)
        qs[:, byte[i]] |= (qi & 0xF) << int(shift[i])
        qh[:, i % 64 % 32] |= ((qi >> 4) & 1) << int(hbit[i])
    out[:, 16:48] = qh.astype(np.uint8)
    out[:, 48:176] = qs.astype(np.uint8)
    return out


value_q5_K = value_q4_K  # same closed form, 5-bit codes


# --------------------------------------------------------------------------- Q6_K
def pack_q6_K(d, sc, q):
    nb = d.shape[0]
    out = np.zeros((nb, 210), np.uint8)
    lb, ls, hb, hs, _ = _idx_q6(_I256)
    ql = np.zeros((nb, 128), np.uint16)
    qh = np.zeros((nb, 64), np.uint16)
    for i in range(256):
        qi = q[:, i].astype(np.uint16)
        ql[:, lb[i]] |= (qi & 0xF) << int(ls[i])
        qh[:, hb[i]] |= ((qi >> 4) & 3) << int(hs[i])
    out[:, 0:128] = ql.astype(np.uint8)
    out[:, 128:192] = qh.astype(np.uint8)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    _put16(out, 208, d)
    return out


def value_q6_K(d, sc, q):
    _, _, _, _, si = _idx_q6(_I256)
    return (h2f(d)[:, None] * sc[:, si].astype(F32)) * (q.astype(np.int32) - 32).astype(F32)


# --------------------------------------------------------------------------- Q3_K
def pack_q3_K(d, sc, lo, h):
    """sc: 6-bit codes (value sc-32); lo: 2-bit codes; h: hmask bit (1 = no -4)."""
    nb = d.shape[0]
    out = np.zeros((nb, 110), np.uint8)
    qb, sh, hb, hbit, _ = _idx_q23(_I256)
    qs = np.zeros((nb, 64), np.uint16)
    hm = np.zeros((nb, 32), np.uint16)
    for i in range(256):
        qs[:, qb[i]] |= (lo[:, i].astype(np.uint16) & 3) << int(sh[i])
        hm[:, hb[i]] |= (h[:, i].astype(np.uint16) & 1) << int(hbit[i])
    out[:, 0:32] = hm.astype(np.uint8)
    out[:, 32:96] = qs.astype(np.uint8)
    s = sc.astype(np.uint16)
    b = np.zeros((nb, 12), np.uint16)
    for i in range(8):
        b[:, i] = (s[:, i] & 0xF) | ((s[:, i + 8] & 0xF) << 4)
    for t in range(4):
        for g in range(4):
            b[:, 8 + t] |= ((s[:, t + 4 * g] >> 4) & 3) << (2 * g)
    out[:, 96:108] = b.astype(np.uint8)
    _put16(out, 108, d)
    return out


def value_q3_K(d, sc, lo, h):
    _, _, _, _, si = _idx_q23(_I256)
    dl = h2f(d)[:, None] * (sc[:, si].astype(np.int32) - 32).astype(F32)
    qv = lo.astype(np.int32) - np.where(h.astype(bool), 0, 4)
    return dl * qv.astype(F32)


# --------------------------------------------------------------------------- Q2_K
def pack_q2_K(d, dmin, sc, m, q):
    nb = d.shape[0]
    out = np.zeros((nb, 84), np.uint8)
    out[:, 0:16] = ((sc.astype(np.uint16) & 0xF) | ((m.astype(np.uint16) & 0xF) << 4)).astype(np.uint8)
    qb, sh, _, _, _ = _idx_q23(_I256)
    qs = np.zeros((nb, 64), np.uint16)
    for i in range(256):
        qs[:, qb[i]] |= (q[:, i].astype(np.uint16) & 3) << int(sh[i])
    out[:, 16:80] = qs.astype(np.uint8)
    _put16(out, 80, d)
    _put16(out, 82, dmin)
    return out


def value_q2_K(d, dmin, sc, m, q):
    _, _, _, _, si = _idx_q23(_I256)
    dl = h2f(d)[:, None] * sc[:, si].astype(F32)
    ml = h2f(dmin)[:, None] * m[:, si].astype(F32)
    return dl * q.astype(F32) - ml


# --------------------------------------------------------------------------- random fields
def random_fields(qtype: str, nb: int, rng: np.random.Generator, **f16kw):
    """Random field set for ``nb`` blocks, returned as a dict of arrays."""
    rf = lambda: random_finite_f16(rng, nb, **f16kw)  # noqa: E731
    ri = lambda hi, n: rng.integers(0, hi, size=(nb, n))  # noqa: E731
    if qtype == "Q8_0":
        return dict(d=rf(), q=rng.integers(-128, 128, size=(nb, 32)))
    if qtype in ("Q4_K", "Q5_K"):
        return dict(d=rf(), dmin=rf(), sc=ri(64, 8), m=ri(64, 8), q=ri(16 if qtype == "Q4_K" else 32, 256))
    if qtype == "Q6_K":
        return dict(d=rf(), sc=rng.integers(-128, 128, size=(nb, 16)), q=ri(64, 256))
    if qtype == "Q3_K":
        return dict(d=rf(), sc=ri(64, 16), lo=ri(4, 256), h=ri(2, 256))
    if qtype == "Q2_K":
        return dict(d=rf(), dmin=rf(), sc=ri(16, 16), m=ri(16, 16), q=ri(4, 256))
    raise ValueError(qtype)


PACK = {"Q8_0": pack_q8_0, "Q2_K": pack_q2_K, "Q3_K": pack_q3_K, "Q4_K": pack_q4_K,
        "Q5_K": pack_q5_K, "Q6_K": pack_q6_K}
VALUE = {"Q8_0": value_q8_0, "Q2_K": value_q2_K, "Q3_K": value_q3_K, "Q4_K": value_q4_K,
         "Q5_K": value_q5_K, "Q6_K": value_q6_K}


def packed_and_values(qtype: str, nb: int, rng: np.random.Generator, **f16kw):
    f = random_fields(qtype, nb, rng, **f16kw)
    return PACK[qtype](**f), VALUE[qtype](**f)


# Byte offsets of the fp16 fields inside each block (d first, then dmin).
# IQ1_M has none: its fp16 scale is spread over the top nibbles of the four
# little-endian 16-bit scale words at bytes 48..55 (see set_iq1m_scale).
F16_OFFSETS = {"Q8_0": (0,), "Q2_K": (80, 82), "Q3_K": (108,), "Q4_K": (0, 2), "Q5_K": (0, 2), "Q6_K": (208,),
               "IQ1_S": (0,), "IQ1_M": (), "IQ2_XXS": (0,), "IQ2_XS": (0,), "IQ2_S": (0,), "IQ3_XXS": (0,),
               "IQ3_S": (0,), "IQ4_XS": (0,)}


def set_iq1m_scale(blk: np.ndarray, h: np.ndarray) -> None:
    """Write fp16 bit patterns ``h`` as IQ1_M super-block scales: nibble t of
    the scale is the top nibble of scale word t (bits 12..15 of the byte pair
    48 + 2t, 49 + 2t)."""
    h = np.asarray(h, dtype=np.uint16)
    for t in range(4):
        nib = ((h >> (4 * t)) & 0xF).astype(np.uint8)
        blk[:, 49 + 2 * t] = (blk[:, 49 + 2 * t] & 0x0F) | (nib << 4)


def set_scale(qtype: str, blk: np.ndarray, h, which: int = 0) -> None:
    """Write fp16 field ``which`` (0 = d, 1 = dmin) of every block."""
    if qtype == "IQ1_M":
        assert which == 0
        set_iq1m_scale(blk, np.broadcast_to(np.asarray(h, dtype=np.uint16), (blk.shape[0],)))
    else:
        _put16(blk, F16_OFFSETS[qtype][which], np.broadcast_to(np.asarray(h, dtype=np.uint16), (blk.shape[0],)))


def random_blocks(qtype: str, nb: int, rng: np.random.Generator, **f16kw) -> np.ndarray:
    """Uniformly random payload bytes with finite fp16 scale fields: every such
    block is a valid block of the format."""
    bb = BLOCK_BYTES[qtype]
    out = rng.integers(0, 256, size=(nb, bb), dtype=np.uint16).astype(np.uint8)
    for which in range(len(F16_OFFSETS[qtype]) or 1):
        set_scale(qtype, out, random_finite_f16(rng, nb, **f16kw), which)
    return out
