"""Round-to-nearest encoders for the GGUF IQ formats -- NOT llama.cpp's quantizer.

Used, like :mod:`voodoo_quant.rtn`, only when libggml-base cannot be loaded: it
writes *valid* blocks of the eight IQ formats so that gated layers with the
reference's IQ menus (``configs/qwen38_27b_voodoo30_tp4.sh:90-92``) can be
built and trained on any machine.  llama.cpp's IQ quantizers search scales
against an importance matrix; this one picks, per sub-block, the best of a few
scales by squared error and rounds every group of 4 or 8 weights to its
nearest code-book entry (signs stored separately; where the format stores 7
of 8 signs, the weight of least magnitude gives up its sign to make the count
of negatives even).  Bytes therefore differ from llama-quantize output.

The code books are read from ``csrc/vq_iq_grids.inc``, the same data the HIP
decoders use.  Block layouts (public GGUF format, decoded in the reference's
``voodoo_quant/quants/gpu_dequant.py:53-519``):

    IQ2_XXS {d; u16 qs[32]}                 per 32: 4 grid bytes, u32 (4 x 7 sign bits, 4-bit scale)
    IQ2_XS  {d; u16 qs[32]; scales[8]}      per 8: 9-bit grid index | 7 sign bits << 9
    IQ2_S   {d; qs[32]; signs[32]; qh[8]; scales[8]}
    IQ3_XXS {d; qs[64]; u32 sas[8]}         per 32: 8 grid bytes (4 values each), u32 signs + scale
    IQ3_S   {d; qs[64]; qh[8]; signs[32]; scales[4]}
    IQ1_S   {d; qs[32]; u16 qh[8]}          per 32: 3-bit scale, delta sign, 4 x 3 high index bits
    IQ1_M   {qs[32]; qh[16]; u16 sc[4]}     fp16 d in the top nibbles of sc
    IQ4_XS  {d; u16 scales_h; scales_l[4]; qs[128]}
"""

from __future__ import annotations

import re
from functools import lru_cache
from pathlib import Path

import numpy as np
import torch

IQ_BLOCK_BYTES = {"IQ1_S": 50, "IQ1_M": 56, "IQ2_XXS": 66, "IQ2_XS": 74, "IQ2_S": 82, "IQ3_XXS": 98,
                  "IQ3_S": 110, "IQ4_XS": 136}
IQ1_DELTA = 0.125
_INC = Path(__file__).resolve().parent.parent / "csrc" / "vq_iq_grids.inc"


@lru_cache(maxsize=None)
def tables() -> dict[str, np.ndarray]:
    """Code books: grids as uint8 [entries, 8 or 4] (iq1s_grid as int8), iq4nl_values int8 [16]."""
    text = _INC.read_text()
    out: dict[str, np.ndarray] = {}
    for ctype, name, n, body in re.findall(r"VQ_IQ_TABLE\((\w+), (\w+), (\d+)\) = \{(.*?)\};", text, re.S):
        vals = [int(v.strip().rstrip("ul"), 0) for v in body.split(",") if v.strip()]
        assert len(vals) == int(n), name
        if ctype == "uint64_t":
            arr = np.array(vals, dtype=np.uint64).astype("<u8").view(np.uint8).reshape(-1, 8)
        elif ctype == "uint32_t":
            arr = np.array(vals, dtype=np.uint32).astype("<u4").view(np.uint8).reshape(-1, 4)
        else:
            arr = np.array(vals, dtype=np.int8)
        out[name] = arr.view(np.int8) if name == "iq1s_grid" else arr
    return out


def _grid(name: str, device) -> torch.Tensor:
    return torch.from_numpy(tables()[name].astype(np.float32)).to(device)


def _f16(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(fp16 bit patterns as int32, their float32 values)."""
    h = v.to(torch.float16)
    return h.view(torch.int16).to(torch.int32) & 0xFFFF, h.to(torch.float32)


def _nearest(a: torch.Tensor, grid: torch.Tensor, chunk: int = 1 << 16) -> tuple[torch.Tensor, torch.Tensor]:
    """Index of the nearest grid row to each row of a [G, w] and the squared distance."""
    g2 = (grid * grid).sum(1)
    idx = torch.empty(a.shape[0], dtype=torch.int64, device=a.device)
    err = torch.empty(a.shape[0], dtype=torch.float32, device=a.device)
    for s in range(0, a.shape[0], chunk):
        blk = a[s:s + chunk]
        d = g2[None, :] - 2.0 * (blk @ grid.t())
        m, i = d.min(1)
        idx[s:s + chunk] = i
        err[s:s + chunk] = (m + (blk * blk).sum(1)).clamp_min(0)
    return idx, err


_SCALE_TRIES = (0.7, 0.8, 0.9, 1.0, 1.1)


def _signed_grid_fit(x: torch.Tensor, sub: int, w: int, grid_name: str, scale_of, s_max: int, parity: bool):
    """Magnitude-grid formats.  x [nb, 256] -> (d bits [nb], s [nb, 256/sub], idx [nb, 256/w],
    sign bytes [nb, 32]): weight = d * scale_of(s) * grid[idx] * sign."""
    nb = x.shape[0]
    grid = _grid(grid_name, x.device)
    gmax = float(grid.max())
    a = x.abs()
    neg = x < 0
    if parity:  # an even count of negatives per 8: flip the smallest weight of odd groups
        g8 = neg.view(nb, 32, 8)
        odd = (g8.sum(2) % 2) == 1
        jmin = a.view(nb, 32, 8).argmin(2)
        flip = torch.zeros_like(g8)
        flip.scatter_(2, jmin[..., None], odd[..., None])
        neg = (g8 ^ flip).view(nb, 256)
    # best continuous scale per sub-block among a few tries around amax / gmax
    asub = a.view(nb, 256 // sub, sub)
    amax = asub.amax(2).clamp_min(1e-30)
    best_err = torch.full_like(amax, float("inf"))
    best_db = amax / gmax
    for f in _SCALE_TRIES:
        db = amax / gmax * f
        q = (asub / db[..., None]).reshape(-1, w)
        _, e = _nearest(q, grid)
        e = (e.view(nb, 256 // sub, sub // w).sum(2)) * db * db
        better = e < best_err
        best_err = torch.where(better, e, best_err)
        best_db = torch.where(better, db, best_db)
    # quantised scales
    d = best_db.amax(1) / scale_of(torch.tensor(float(s_max), device=x.device))
    dh, df = _f16(d)
    df = torch.where(df > 0, df, torch.ones_like(df))
    s_cont = best_db / df[:, None]
    tries = torch.arange(s_max + 1, device=x.device, dtype=torch.float32)
    sv = scale_of(tries)  # [s_max + 1]
    s = (s_cont[..., None] - sv).abs().argmin(-1)
    db = df[:, None] * sv[s]
    q = (asub / db[..., None]).reshape(-1, w)
    idx, _ = _nearest(q, grid)
    bits = (neg.view(nb, 32, 8).to(torch.int32) << torch.arange(8, device=x.device, dtype=torch.int32)).sum(2)
    return dh, s.to(torch.int32), idx.view(nb, 256 // w).to(torch.int32), bits


def _put16(out: torch.Tensor, off: int, v: torch.Tensor) -> None:
    out[:, off] = (v & 0xFF).to(torch.uint8)
    out[:, off + 1] = ((v >> 8) & 0xFF).to(torch.uint8)


def _put32(out: torch.Tensor, off: int, v: torch.Tensor) -> None:
    for b in range(4):
        out[:, off + b] = ((v >> (8 * b)) & 0xFF).to(torch.uint8)


def _iq2_scale(s):
    return (0.5 + s) * 0.25


def _encode_iq2_xxs(x):
    nb = x.shape[0]
    dh, s, idx, sg = _signed_grid_fit(x, 32, 8, "iq2xxs_grid", _iq2_scale, 15, True)
    out = torch.zeros(nb, 66, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    s7 = (sg & 127).view(nb, 8, 4)
    for ib in range(8):
        for l in range(4):
            out[:, 2 + 8 * ib + l] = idx[:, 4 * ib + l].to(torch.uint8)
        aux = s7[:, ib, 0] | (s7[:, ib, 1] << 7) | (s7[:, ib, 2] << 14) | (s7[:, ib, 3] << 21) | (s[:, ib] << 28)
        _put32(out, 2 + 8 * ib + 4, aux)
    return out


def _encode_iq2_xs(x):
    nb = x.shape[0]
    dh, s, idx, sg = _signed_grid_fit(x, 16, 8, "iq2xs_grid", _iq2_scale, 15, True)
    out = torch.zeros(nb, 74, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    for j in range(32):
        _put16(out, 2 + 2 * j, idx[:, j] | ((sg[:, j] & 127) << 9))
    out[:, 66:74] = (s[:, 0::2] | (s[:, 1::2] << 4)).to(torch.uint8)
    return out


def _encode_iq2_s(x):
    nb = x.shape[0]
    dh, s, idx, sg = _signed_grid_fit(x, 16, 8, "iq2s_grid", _iq2_scale, 15, False)
    out = torch.zeros(nb, 82, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    out[:, 2:34] = (idx & 255).to(torch.uint8)
    out[:, 34:66] = sg.to(torch.uint8)
    hi = (idx >> 8).view(nb, 8, 4)
    out[:, 66:74] = (hi[..., 0] | (hi[..., 1] << 2) | (hi[..., 2] << 4) | (hi[..., 3] << 6)).to(torch.uint8)
    out[:, 74:82] = (s[:, 0::2] | (s[:, 1::2] << 4)).to(torch.uint8)
    return out


def _encode_iq3_xxs(x):
    nb = x.shape[0]
    dh, s, idx, sg = _signed_grid_fit(x, 32, 4, "iq3xxs_grid", lambda t: (0.5 + t) * 0.5, 15, True)
    out = torch.zeros(nb, 98, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    out[:, 2:66] = idx.to(torch.uint8)
    s7 = (sg & 127).view(nb, 8, 4)
    for ib in range(8):
        aux = s7[:, ib, 0] | (s7[:, ib, 1] << 7) | (s7[:, ib, 2] << 14) | (s7[:, ib, 3] << 21) | (s[:, ib] << 28)
        _put32(out, 66 + 4 * ib, aux)
    return out


def _encode_iq3_s(x):
    nb = x.shape[0]
    dh, s, idx, sg = _signed_grid_fit(x, 32, 4, "iq3s_grid", lambda t: 1.0 + 2.0 * t, 15, False)
    out = torch.zeros(nb, 110, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    out[:, 2:66] = (idx & 255).to(torch.uint8)
    hi = (idx >> 8).view(nb, 8, 8)
    out[:, 66:74] = (hi << torch.arange(8, device=x.device, dtype=torch.int32)).sum(2).to(torch.uint8)
    out[:, 74:106] = sg.to(torch.uint8)
    out[:, 106:110] = (s[:, 0::2] | (s[:, 1::2] << 4)).to(torch.uint8)
    return out


def _iq1_fit(x: torch.Tensor, sub: int, delta_per: int):
    """IQ1: weight = dl * (g + delta), g in the signed grid, delta = +-1/8 shared by
    `delta_per` weights, dl = d (2 s + 1) per `sub` weights.  Returns (d [nb] float
    target, s [nb, 256/sub], idx [nb, 32], delta_neg [nb, 256/delta_per])."""
    nb = x.shape[0]
    grid = _grid("iq1s_grid", x.device)  # [2048, 8] of -1, 0, 1
    xs = x.view(nb, 256 // sub, sub)
    amax = xs.abs().amax(2).clamp_min(1e-30)
    best = None
    for f in _SCALE_TRIES:
        dl = amax / (1.0 + IQ1_DELTA) * f
        y = (xs / dl[..., None]).reshape(nb, 256 // delta_per, delta_per)
        errs, idxs = [], []
        for sgn in (1.0, -1.0):
            q = (y - sgn * IQ1_DELTA).reshape(-1, 8)
            i, e = _nearest(q, grid)
            errs.append(e.view(nb, 256 // delta_per, delta_per // 8).sum(2))
            idxs.append(i.view(nb, 256 // delta_per, delta_per // 8))
        use_neg = errs[1] < errs[0]
        e = torch.where(use_neg, errs[1], errs[0])
        esub = e.view(nb, 256 // sub, -1).sum(2) * dl * dl if sub >= delta_per else None
        if esub is None:  # delta shared by more weights than a scale: not a layout this module needs
            raise AssertionError
        if best is None:
            best = [esub, dl]
        else:
            better = esub < best[0]
            best = [torch.where(better, esub, best[0]), torch.where(better, dl, best[1])]
    dl_c = best[1]
    d = dl_c.amax(1) / 15.0
    return d, dl_c, grid


def _iq1_final(x, sub, delta_per, d_f):
    """Quantised scales for fp16-rounded d_f, then the final grid/delta search."""
    nb = x.shape[0]
    grid = _grid("iq1s_grid", x.device)
    d_f = torch.where(d_f > 0, d_f, torch.ones_like(d_f))
    xs = x.view(nb, 256 // sub, sub)
    amax = xs.abs().amax(2)
    sv = 2.0 * torch.arange(8, device=x.device, dtype=torch.float32) + 1.0
    # scale code per sub-block: best of the 8 by squared error
    best_e, best_s = None, None
    for si in range(8):
        dl = d_f[:, None] * sv[si]
        y = (xs / dl[..., None]).reshape(nb, 256 // delta_per, delta_per)
        es = []
        for sgn in (1.0, -1.0):
            _, e = _nearest((y - sgn * IQ1_DELTA).reshape(-1, 8), grid)
            es.append(e.view(nb, 256 // delta_per, delta_per // 8).sum(2))
        e = torch.minimum(es[0], es[1]).view(nb, 256 // sub, -1).sum(2) * dl * dl
        if best_e is None:
            best_e, best_s = e, torch.zeros_like(e, dtype=torch.int64)
        else:
            better = e < best_e
            best_e = torch.where(better, e, best_e)
            best_s = torch.where(better, torch.full_like(best_s, si), best_s)
    del amax
    dl = d_f[:, None] * sv[best_s]
    y = (xs / dl[..., None]).reshape(nb, 256 // delta_per, delta_per)
    res = []
    for sgn in (1.0, -1.0):
        i, e = _nearest((y - sgn * IQ1_DELTA).reshape(-1, 8), grid)
        res.append((i.view(nb, 256 // delta_per, delta_per // 8), e.view(nb, 256 // delta_per, delta_per // 8).sum(2)))
    use_neg = res[1][1] < res[0][1]
    idx = torch.where(use_neg[..., None], res[1][0], res[0][0]).reshape(nb, 32)
    return best_s.to(torch.int32), idx.to(torch.int32), use_neg.to(torch.int32)


def _encode_iq1_s(x):
    nb = x.shape[0]
    d, _, _ = _iq1_fit(x, 32, 32)
    dh, df = _f16(d)
    s, idx, neg = _iq1_final(x, 32, 32, df)
    out = torch.zeros(nb, 50, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    out[:, 2:34] = (idx & 255).to(torch.uint8)
    hi = (idx >> 8).view(nb, 8, 4)
    qh = hi[..., 0] | (hi[..., 1] << 3) | (hi[..., 2] << 6) | (hi[..., 3] << 9) | (s << 12) | (neg[:, :] << 15)
    for ib in range(8):
        _put16(out, 34 + 2 * ib, qh[:, ib])
    return out


def _encode_iq1_m(x):
    nb = x.shape[0]
    d, _, _ = _iq1_fit(x, 16, 8)
    dh, df = _f16(d)
    s, idx, neg = _iq1_final(x, 16, 8, df)  # s [nb, 16], neg [nb, 32]
    out = torch.zeros(nb, 56, dtype=torch.uint8, device=x.device)
    out[:, 0:32] = (idx & 255).to(torch.uint8)
    hi = idx >> 8  # [nb, 32], group 4 ib + l
    for ib in range(8):
        for h in range(2):  # qh byte 2 ib + h holds groups l = 2 h (low nibble) and 2 h + 1 (high)
            l0, l1 = 4 * ib + 2 * h, 4 * ib + 2 * h + 1
            v = hi[:, l0] | (neg[:, l0] << 3) | (hi[:, l1] << 4) | (neg[:, l1] << 7)
            out[:, 32 + 2 * ib + h] = v.to(torch.uint8)
    for t in range(4):  # scale word t: sub-blocks 4 t .. 4 t + 3 (16 weights each), 3 bits each
        w = s[:, 4 * t] | (s[:, 4 * t + 1] << 3) | (s[:, 4 * t + 2] << 6) | (s[:, 4 * t + 3] << 9)
        w = w | (((dh >> (4 * t)) & 0xF) << 12)
        _put16(out, 48 + 2 * t, w)
    return out


def _encode_iq4_xs(x):
    nb = x.shape[0]
    kv = torch.from_numpy(tables()["iq4nl_values"].astype(np.float32)).to(x.device)
    xs = x.view(nb, 8, 32)
    # the weight of largest magnitude maps to -127 (the table's widest end)
    amax_i = xs.abs().argmax(2, keepdim=True)
    xm = xs.gather(2, amax_i).squeeze(2)
    best_e, best_dl = None, None
    for f in _SCALE_TRIES:
        dl = torch.where(xm != 0, -xm / 127.0 * f, torch.full_like(xm, 1e-30))
        q = (xs / dl[..., None])[..., None]
        e = ((q - kv).abs().amin(-1) ** 2).sum(2) * dl * dl
        if best_e is None:
            best_e, best_dl = e, dl
        else:
            better = e < best_e
            best_e, best_dl = torch.where(better, e, best_e), torch.where(better, dl, best_dl)
    d = best_dl.abs().amax(1) / 31.0
    dh, df = _f16(d)
    df = torch.where(df > 0, df, torch.ones_like(df))
    ls = torch.clamp(torch.round(best_dl / df[:, None]), -32, 31)
    dl = df[:, None] * ls
    q = torch.where(dl[..., None] != 0, xs / dl[..., None], torch.zeros_like(xs))
    code = (q[..., None] - kv).abs().argmin(-1).to(torch.int32)  # [nb, 8, 32]
    lsu = (ls + 32).to(torch.int32)
    out = torch.zeros(nb, 136, dtype=torch.uint8, device=x.device)
    _put16(out, 0, dh)
    sh = torch.zeros(nb, dtype=torch.int32, device=x.device)
    for ib in range(8):
        sh = sh | (((lsu[:, ib] >> 4) & 3) << (2 * ib))
    _put16(out, 2, sh)
    out[:, 4:8] = ((lsu[:, 0::2] & 15) | ((lsu[:, 1::2] & 15) << 4)).to(torch.uint8)
    out[:, 8:136] = (code[..., :16] | (code[..., 16:] << 4)).reshape(nb, 128).to(torch.uint8)
    return out


ENCODERS = {
    "IQ1_S": _encode_iq1_s,
    "IQ1_M": _encode_iq1_m,
    "IQ2_XXS": _encode_iq2_xxs,
    "IQ2_XS": _encode_iq2_xs,
    "IQ2_S": _encode_iq2_s,
    "IQ3_XXS": _encode_iq3_xxs,
    "IQ3_S": _encode_iq3_s,
    "IQ4_XS": _encode_iq4_xs,
}


def iq_quantize_tensor(weight: torch.Tensor, quant_type: str, chunk_rows: int | None = None) -> torch.Tensor:
    """[out, in] float weights -> uint8 [nblocks, block_bytes] (non-ggml IQ encoder).

    Runs on the weight's device (a GPU encodes a 27B-class tensor in seconds)."""
    if quant_type not in ENCODERS:
        raise ValueError(f"the IQ encoder covers {sorted(ENCODERS)}, not {quant_type}")
    w = weight.detach().to(torch.float32).contiguous()
    out_f, in_f = w.shape
    if in_f % 256 != 0:
        raise ValueError(f"{quant_type} requires in_features % 256 == 0, got {in_f}")
    rows = chunk_rows or max(1, (1 << 18) // in_f)
    parts = [ENCODERS[quant_type](w[r:r + rows].reshape(-1, 256)) for r in range(0, out_f, rows)]
    return torch.cat(parts, 0).cpu()
