"""Round-to-nearest GGUF block encoder -- NOT llama.cpp's quantizer.

Used only when libggml-base cannot be loaded (the reference raises there,
``ggml.py:108-120``).  It writes *valid* blocks of the six formats the HIP
kernels decode, with the usual error ordering (Q2_K worst ... Q8_0 best), so
gated layers can be built and trained on any machine.  Bytes differ from
``llama-quantize`` output except for Q8_0, whose ggml quantizer is itself plain
round-to-nearest (amax / 127 scale, ``roundf`` codes).

Layouts (public GGUF format): Q8_0 {d; qs[32]}; Q2_K {scales[16]; qs[64]; d;
dmin}; Q3_K {hmask[32]; qs[64]; scales[12]; d}; Q4_K {d; dmin; scales[12];
qs[128]}; Q5_K {d; dmin; scales[12]; qh[32]; qs[128]}; Q6_K {ql[128]; qh[64];
scales[16]; d}.
"""

from __future__ import annotations

import numpy as np
import torch

BLOCK = {"Q8_0": (32, 34), "Q2_K": (256, 84), "Q3_K": (256, 110), "Q4_K": (256, 144), "Q5_K": (256, 176),
         "Q6_K": (256, 210)}


def _roundf(v: np.ndarray) -> np.ndarray:
    """C roundf: halves away from zero."""
    return np.trunc(v + np.copysign(np.float32(0.5), v)).astype(np.float32)


def _f16(v: np.ndarray):
    h = v.astype(np.float16)
    return h.view(np.uint16), h.astype(np.float32)


def _safe_div(a, b):
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(b != 0, a / np.where(b != 0, b, 1), 0)
    return r.astype(np.float32)


def _put16(out, off, h):
    out[:, off] = (h & 0xFF).astype(np.uint8)
    out[:, off + 1] = (h >> 8).astype(np.uint8)


# weight position tables within a 256-weight super-block
_I = np.arange(256)
# Q4_K / Q5_K: 64-weight chunks, low nibbles then high nibbles of 32 bytes
_K4_BYTE = 32 * (_I // 64) + (_I % 32)
_K4_SHIFT = 4 * ((_I % 64) // 32)
_K5_HBIT = 2 * (_I // 64) + (_I % 64) // 32
# Q6_K: 128-weight halves, 4 quarters of 32
_Q6_LBYTE = 64 * (_I // 128) + (_I % 32) + 32 * (((_I % 128) // 32) & 1)
_Q6_LSHIFT = 4 * (((_I % 128) // 32) >> 1)
_Q6_HBYTE = 32 * (_I // 128) + (_I % 32)
_Q6_HSHIFT = 2 * ((_I % 128) // 32)
_Q6_SCALE = 8 * (_I // 128) + (_I % 32) // 16 + 2 * ((_I % 128) // 32)
# Q2_K / Q3_K: 128-weight halves, 4 shifts x 2 sixteen-weight runs
_Q23_BYTE = 32 * (_I // 128) + 16 * ((_I % 32) // 16) + (_I % 16)
_Q23_SHIFT = 2 * ((_I % 128) // 32)
_Q3_HBYTE = 16 * ((_I % 32) // 16) + (_I % 16)
_Q3_HBIT = 4 * (_I // 128) + (_I % 128) // 32
_Q23_SCALE = 8 * (_I // 128) + 2 * ((_I % 128) // 32) + (_I % 32) // 16


def _scatter_bits(nb, nbytes, byte_idx, shift, codes):
    """OR codes[:, i] << shift[i] into byte byte_idx[i]."""
    acc = np.zeros((nb, nbytes), np.uint32)
    vals = codes.astype(np.uint32) << shift.astype(np.uint32)
    for b in range(nbytes):
        sel = byte_idx == b
        acc[:, b] = np.bitwise_or.reduce(vals[:, sel], axis=1)
    return acc.astype(np.uint8)


def _sub_of(sub_size):
    return _I // sub_size


def _encode_q8_0(x):
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = amax / np.float32(127)
    dh, _ = _f16(d)
    idv = _safe_div(np.ones_like(d), d)
    q = _roundf(xb * idv[:, None]).astype(np.int8)
    out = np.zeros((xb.shape[0], 34), np.uint8)
    _put16(out, 0, dh)
    out[:, 2:] = q.view(np.uint8)
    return out


def _affine_scales(xb, sub, levels, scale_levels):
    """Per-sub-block (scale, min) RTN with scale/min quantised to scale_levels."""
    nb = xb.shape[0]
    xs = xb.reshape(nb, 256 // sub, sub)
    xmin = np.minimum(xs.min(axis=2), 0).astype(np.float32)
    xmax = xs.max(axis=2).astype(np.float32)
    scale = (xmax - xmin) / np.float32(levels)
    mn = -xmin
    d = scale.max(axis=1) / np.float32(scale_levels)
    dmin = mn.max(axis=1) / np.float32(scale_levels)
    dh, df = _f16(d)
    mh, mf = _f16(dmin)
    sc = np.clip(_roundf(_safe_div(scale, df[:, None])), 0, scale_levels).astype(np.int32)
    m = np.clip(_roundf(_safe_div(mn, mf[:, None])), 0, scale_levels).astype(np.int32)
    dl = df[:, None] * sc.astype(np.float32)
    ml = mf[:, None] * m.astype(np.float32)
    s_of = _sub_of(sub)
    q = _roundf(_safe_div(xb + ml[:, s_of], dl[:, s_of]))
    q = np.clip(q, 0, levels).astype(np.int32)
    return dh, mh, sc, m, q


def _pack_k4_scales(sc, m):
    b = np.zeros((sc.shape[0], 12), np.int32)
    for j in range(4):
        b[:, j] = sc[:, j] | ((sc[:, j + 4] >> 4) << 6)
        b[:, j + 4] = m[:, j] | ((m[:, j + 4] >> 4) << 6)
        b[:, j + 8] = (sc[:, j + 4] & 0xF) | ((m[:, j + 4] & 0xF) << 4)
    return b.astype(np.uint8)


def _encode_q45_K(x, five):
    xb = x.reshape(-1, 256)
    nb = xb.shape[0]
    dh, mh, sc, m, q = _affine_scales(xb, 32, 31 if five else 15, 63)
    bb = 176 if five else 144
    out = np.zeros((nb, bb), np.uint8)
    _put16(out, 0, dh)
    _put16(out, 2, mh)
    out[:, 4:16] = _pack_k4_scales(sc, m)
    qs = _scatter_bits(nb, 128, _K4_BYTE, _K4_SHIFT, q & 0xF)
    if five:
        out[:, 16:48] = _scatter_bits(nb, 32, _I % 64 % 32, _K5_HBIT, (q >> 4) & 1)
        out[:, 48:176] = qs
    else:
        out[:, 16:144] = qs
    return out


def _encode_q2_K(x):
    xb = x.reshape(-1, 256)
    nb = xb.shape[0]
    dh, mh, sc, m, q = _affine_scales(xb, 16, 3, 15)
    out = np.zeros((nb, 84), np.uint8)
    out[:, 0:16] = (sc | (m << 4)).astype(np.uint8)
    # scale byte index of sub-block s is s itself (16-weight sub-blocks in order)
    out[:, 16:80] = _scatter_bits(nb, 64, _Q23_BYTE, _Q23_SHIFT, q)
    _put16(out, 80, dh)
    _put16(out, 82, mh)
    return out


def _symmetric_scales(xb, sub, qmax_neg, scale_max):
    """Per-sub-block signed scale: codes in [-qmax_neg, qmax_neg - 1]."""
    nb = xb.shape[0]
    xs = xb.reshape(nb, 256 // sub, sub)
    amax = np.abs(xs).max(axis=2).astype(np.float32)
    scale = amax / np.float32(qmax_neg)
    d = scale.max(axis=1) / np.float32(scale_max)
    dh, df = _f16(d)
    sc = np.clip(_roundf(_safe_div(scale, df[:, None])), 0, scale_max).astype(np.int32)
    dl = df[:, None] * sc.astype(np.float32)
    q = _roundf(_safe_div(xb, dl[:, _sub_of(sub)]))
    q = np.clip(q, -qmax_neg, qmax_neg - 1).astype(np.int32)
    return dh, sc, q


def _encode_q6_K(x):
    xb = x.reshape(-1, 256)
    nb = xb.shape[0]
    dh, sc, q = _symmetric_scales(xb, 16, 32, 127)
    u = q + 32
    out = np.zeros((nb, 210), np.uint8)
    out[:, 0:128] = _scatter_bits(nb, 128, _Q6_LBYTE, _Q6_LSHIFT, u & 0xF)
    out[:, 128:192] = _scatter_bits(nb, 64, _Q6_HBYTE, _Q6_HSHIFT, (u >> 4) & 3)
    # scale index of weight i is _Q6_SCALE[i]; sub-block s of 16 weights (in order) -> scale slot
    slot = np.zeros(16, np.int64)
    for s in range(16):
        slot[s] = _Q6_SCALE[16 * s]
    scales = np.zeros((nb, 16), np.int8)
    scales[:, slot] = sc.astype(np.int8)
    out[:, 192:208] = scales.view(np.uint8)
    _put16(out, 208, dh)
    return out


def _encode_q3_K(x):
    xb = x.reshape(-1, 256)
    nb = xb.shape[0]
    dh, sc, q = _symmetric_scales(xb, 16, 4, 31)
    out = np.zeros((nb, 110), np.uint8)
    out[:, 0:32] = _scatter_bits(nb, 32, _Q3_HBYTE, _Q3_HBIT, (q >= 0).astype(np.int32))
    out[:, 32:96] = _scatter_bits(nb, 64, _Q23_BYTE, _Q23_SHIFT, q & 3)
    slot = np.array([_Q23_SCALE[16 * s] for s in range(16)])
    s6 = np.zeros((nb, 16), np.int32)
    s6[:, slot] = sc + 32
    b = np.zeros((nb, 12), np.int32)
    for i in range(8):
        b[:, i] = (s6[:, i] & 0xF) | ((s6[:, i + 8] & 0xF) << 4)
    for t in range(4):
        for g in range(4):
            b[:, 8 + t] |= ((s6[:, t + 4 * g] >> 4) & 3) << (2 * g)
    out[:, 96:108] = b.astype(np.uint8)
    _put16(out, 108, dh)
    return out


_ENCODERS = {
    "Q8_0": _encode_q8_0,
    "Q2_K": _encode_q2_K,
    "Q3_K": _encode_q3_K,
    "Q4_K": lambda x: _encode_q45_K(x, False),
    "Q5_K": lambda x: _encode_q45_K(x, True),
    "Q6_K": _encode_q6_K,
}


def rtn_quantize_tensor(weight: torch.Tensor, quant_type: str, chunk_rows: int | None = None) -> torch.Tensor:
    """[out, in] float weights -> uint8 [nblocks, block_bytes] (non-ggml RTN;
    the IQ formats go to :func:`voodoo_quant.iq_encode.iq_quantize_tensor`)."""
    if quant_type.startswith("IQ"):
        from voodoo_quant.iq_encode import iq_quantize_tensor

        return iq_quantize_tensor(weight, quant_type, chunk_rows)
    if quant_type not in _ENCODERS:
        raise ValueError(f"the RTN encoder covers {sorted(_ENCODERS)}, not {quant_type}")
    bs, bb = BLOCK[quant_type]
    w = weight.detach().to(torch.float32).cpu().contiguous()
    out_f, in_f = w.shape
    if in_f % bs != 0:
        raise ValueError(f"{quant_type} requires in_features % {bs} == 0, got {in_f}")
    arr = w.numpy()
    rows = chunk_rows or max(1, (1 << 20) // max(in_f, 1))
    parts = [_ENCODERS[quant_type](arr[r:r + rows]) for r in range(0, out_f, rows)]
    return torch.from_numpy(np.concatenate(parts, axis=0).reshape(-1, bb))
