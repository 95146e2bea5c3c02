"""Q8_0 teacher modules on the MI355X kernels.

Drop-in for the reference's ``voodoo_quant/training/q8_teacher.py``: the
teacher keeps every Linear/Embedding weight as llama.cpp Q8_0 bytes on the
device and decodes them when it runs.

* :class:`Q8Linear` (reference ``q8_teacher.py:62-128``) is the gated Linear
  with one candidate and probability 1: ``vq_gated_linear_fwd`` writes the
  bf16 decode of the bytes (``bf16(0 + 1 * w)``, the reference's
  ``dequantize_tensor_gpu`` value) and runs the MFMA GEMM on it, then the bias
  is added as in ``F.linear``.  With the decode kept (:func:`set_keep_decoded`)
  a forward is a plain bf16 GEMM over that decode, run by ``F.linear``
  (hipBLASLt).  The reference's row-blocked path for
  vocabulary-scale heads (``q8_teacher.py:39-59, 102-120``) exists to bound
  transients on 32 GB cards; here the whole bf16 weight is one transient
  buffer (2.5 GB for 248320 x 5120, against 288 GB of HBM).
* :class:`Q8Embedding` (``q8_teacher.py:131-173``) looks up the batch's unique
  rows with ``vq_embedding_rows_fwd`` routed to the one candidate, which gives
  ggml's values rounded to bf16 exactly as the reference's row decode.
* :func:`wrap_q8_teacher` (``q8_teacher.py:176-294``) swaps them into a model
  built from a Q8_0 teacher checkpoint.

Q8_0 stores 32-weight blocks; the kernels read rows as whole 256-weight groups
and the GEMM wants out_features % 8 == 0, so a tensor whose in_features is not
a multiple of 256 (or whose out_features is not a multiple of 8) is repacked
once into zero-padded rows (zero blocks decode to 0).  Inputs run in bf16, the
teacher's dtype in the reference's training runs; fp32 inputs are cast to bf16
for the GEMM and the result cast back.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from voodoo_quant import _hip
from voodoo_quant.layers import check_embedding_ids

_Q8_0 = 8            # ggml type id
_Q8_BLOCK = 32       # weights per block
_Q8_BLOCK_BYTES = 34  # fp16 scale + 32 int8

_KEEP_DECODED = False

# With the decode kept, a teacher forward is a plain bf16 GEMM, and it runs on
# hipBLASLt (as the student's plain output head does): its stream-K kernels
# measured as fast or faster at every teacher shape on MI355X at 8192 tokens,
# 1024 -> 151936 2.15 against 2.63 ms, 1024 -> 6144 88 against 109 us,
# 3072 -> 1024 48 against 53 us, 1024 -> 1536 and 1024 -> 1024 within 5%.
# Without the kept decode every forward decodes and mixes through the library
# (vq_gated_linear_fwd with one candidate), as the reference's teacher does.


def set_keep_decoded(enabled: bool) -> None:
    """Keep each Q8Linear's bf16 decode from one forward to the next.

    Off (the default, the reference's behaviour) every forward decodes the
    bytes and drops the result, bounding the teacher's memory to its Q8_0
    bytes.  On, the decode is made once and every later forward is only the
    GEMM: on a 288 GB device the decoded 0.8B-class teacher is 0.9 GB."""
    global _KEEP_DECODED
    _KEEP_DECODED = bool(enabled)


def _padded_q8(qbytes: torch.Tensor, rows: int, cols: int, rows_to: int) -> tuple[torch.Tensor, int]:
    """Q8_0 bytes of [rows, cols] as [rows_pad, d_pad] with d_pad = cols rounded
    up to 256 and rows_pad = rows rounded up to `rows_to` (zero blocks added)."""
    if cols % _Q8_BLOCK:
        raise ValueError(f"Q8_0 needs in_features % 32 == 0, got {cols}")
    nb = cols // _Q8_BLOCK
    if qbytes.numel() != rows * nb * _Q8_BLOCK_BYTES:
        raise ValueError(f"Q8_0 [{rows}, {cols}] holds {rows * nb * _Q8_BLOCK_BYTES} bytes, got {qbytes.numel()}")
    d_pad = (cols + 255) // 256 * 256
    rows_pad = (rows + rows_to - 1) // rows_to * rows_to
    flat = qbytes.reshape(-1)
    if d_pad == cols and rows_pad == rows:
        return (flat if flat.is_contiguous() else flat.contiguous()), d_pad
    out = torch.zeros(rows_pad, d_pad // _Q8_BLOCK, _Q8_BLOCK_BYTES, dtype=torch.uint8, device=qbytes.device)
    out[:rows, :nb] = flat.view(rows, nb, _Q8_BLOCK_BYTES)
    return out.reshape(-1), d_pad


class Q8Linear(nn.Module):
    """nn.Linear stand-in keeping Q8_0 bytes on the device (``qweight``),
    decoded on every forward (reference ``q8_teacher.py:62-128``)."""

    def __init__(self, qbytes: torch.Tensor, out_features: int, in_features: int,
                 bias: torch.Tensor | None = None, device: torch.device | None = None):
        super().__init__()
        self.out_features = out_features
        self.in_features = in_features
        dev = torch.device(device) if device is not None else qbytes.device
        self.register_buffer("qweight", qbytes.to(dev) if qbytes.device != dev else qbytes)
        self._w: torch.Tensor | None = None
        if bias is not None:
            self.bias = nn.Parameter(bias.to(dev).to(torch.bfloat16), requires_grad=False)
        else:
            self.register_parameter("bias", None)

    def _packed(self) -> tuple[torch.Tensor, int, int]:
        """(bytes in the kernels' row layout, rows, d_pad), repacked once if needed."""
        key = (self.qweight.data_ptr(), self.qweight.device)
        cached = self.__dict__.get("_pack")
        if cached is None or cached[0] != key:
            qb, d_pad = _padded_q8(self.qweight, self.out_features, self.in_features, 8)
            rows = qb.numel() // (d_pad // _Q8_BLOCK * _Q8_BLOCK_BYTES)
            cached = (key, qb, rows, d_pad)
            self.__dict__["_pack"] = cached
        return cached[1], cached[2], cached[3]

    def _decoded(self) -> torch.Tensor:
        """bf16 [rows, d_pad] decode of the (padded) bytes, kept in ``_w``'s storage."""
        qb, rows, d_pad = self._packed()
        full = self.__dict__.get("_w_full")
        if full is None or self._w is None or full.device != self.qweight.device:
            full = _hip.dequant_bf16(_Q8_0, qb, rows, d_pad)
            self.__dict__["_w_full"] = full
            self._w = full[: self.out_features, : self.in_features]
        return full

    def _weight(self) -> torch.Tensor:
        """bf16 [out, in] decode (the reference's dequant cache)."""
        if self.qweight.numel() == 0:
            raise RuntimeError(f"Q8Linear empty qweight: {self.out_features}x{self.in_features} "
                               "(offloaded, never reloaded)")
        if self._w is None or self._w.device != self.qweight.device:
            self._decoded()
        return self._w

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type != "cuda":
            raise RuntimeError(f"Q8Linear runs on a ROCm device only (got {x.device})")
        if self.qweight.numel() == 0:
            raise RuntimeError(f"Q8Linear empty qweight: {self.out_features}x{self.in_features} "
                               "(offloaded, never reloaded)")
        qb, rows, d_pad = self._packed()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.bfloat16:
            x2 = x2.to(torch.bfloat16)
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.contiguous().clone()
        m = x2.shape[0]
        dev = x2.device
        library = _KEEP_DECODED and m > 0
        if library:
            y = torch.nn.functional.linear(x2, self._decoded()[:, : self.in_features])
        else:
            y = torch.empty(m, rows, dtype=torch.bfloat16, device=dev)
        if m and not library:
            nbytes = _hip.fwd_workspace_bytes(m, rows, self.in_features)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes > 0 else None
            w = torch.empty(rows, d_pad, dtype=torch.bfloat16, device=dev)
            one = torch.ones(1, dtype=torch.float32, device=dev)
            _hip.gated_linear_fwd(x2, (_Q8_0,), [qb], one, rows, d_pad, w, y, ws)
        if rows != self.out_features:
            y = y[:, : self.out_features]
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        if not _KEEP_DECODED:
            self._w = None  # one-shot, as the reference's teacher forward
            self.__dict__["_w_full"] = None
        out = y.reshape(*lead, self.out_features)
        return out if out.dtype == x.dtype else out.to(x.dtype)


class Q8Embedding(nn.Module):
    """nn.Embedding stand-in keeping Q8_0 bytes on the device; a forward
    decodes only the batch's rows, one per position (reference
    ``q8_teacher.py:131-173``, which decodes the unique ids' rows and scatters
    them: the same values, without the sort).  ``id_check`` as in
    :class:`voodoo_quant.layers.MixedQuantEmbedding`."""

    id_check = "sync"

    def __init__(self, qbytes: torch.Tensor, num_embeddings: int, embedding_dim: int,
                 device: torch.device | None = None):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        dev = torch.device(device) if device is not None else qbytes.device
        self.register_buffer("qweight", qbytes.to(dev) if qbytes.device != dev else qbytes)
        self._w: torch.Tensor | None = None

    def _packed(self) -> tuple[torch.Tensor, int]:
        key = (self.qweight.data_ptr(), self.qweight.device)
        cached = self.__dict__.get("_pack")
        if cached is None or cached[0] != key:
            qb, d_pad = _padded_q8(self.qweight, self.num_embeddings, self.embedding_dim, 1)
            cached = (key, qb, d_pad)
            self.__dict__["_pack"] = cached
        return cached[1], cached[2]

    def _weight(self) -> torch.Tensor:
        """bf16 [num_embeddings, embedding_dim] decode of the whole table."""
        if self._w is None or self._w.device != self.qweight.device:
            qb, d_pad = self._packed()
            self._w = _hip.dequant_bf16(_Q8_0, qb, self.num_embeddings, d_pad)[:, : self.embedding_dim]
        return self._w

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type != "cuda":
            raise RuntimeError(f"Q8Embedding runs on a ROCm device only (got {x.device})")
        qb, d_pad = self._packed()
        rows = x.reshape(-1).to(device=qb.device, dtype=torch.int64).contiguous()
        check_embedding_ids(rows, self.num_embeddings, "Q8Embedding", self.id_check)
        dim8 = (self.embedding_dim + 7) // 8 * 8
        routing = torch.zeros_like(rows)  # every row from the one candidate: exact decode
        w_rows = _hip.embedding_rows_fwd((_Q8_0,), [qb], None, routing, rows, self.num_embeddings, dim8, d_pad)
        if dim8 != self.embedding_dim:
            w_rows = w_rows[:, : self.embedding_dim]
        return w_rows.reshape(*x.shape, self.embedding_dim)


_GROUP_DECODES: dict[tuple, torch.Tensor] = {}


def q8_linear_group(x: torch.Tensor, modules: list, stacked: bool = False):
    """Outputs of Q8Linears that all read `x`.  With kept decodes and no
    biases, their decodes are stacked once and the outputs come from ONE plain
    GEMM (on hipBLASLt, as Q8Linear's kept-decode forward); otherwise each
    module runs its own forward.
    stacked=True returns the stacked output [tokens, sum out_features] (None
    when the modules cannot be stacked)."""
    ok = (_KEEP_DECODED and len(modules) >= 2 and x.device.type == "cuda"
          and all(isinstance(m, Q8Linear) and m.bias is None and m.out_features % 8 == 0 for m in modules)
          and len({m.in_features for m in modules}) == 1)
    if not ok:
        return None if stacked else [m(x) for m in modules]
    key = tuple((id(m), m.qweight.data_ptr()) for m in modules)
    w = _GROUP_DECODES.get(key)
    if w is None:
        if len(_GROUP_DECODES) > 1024:
            _GROUP_DECODES.clear()
        w = torch.cat([m._decoded()[: m.out_features] for m in modules], 0).contiguous()
        _GROUP_DECODES[key] = w
    lead = x.shape[:-1]
    x2 = x.reshape(-1, modules[0].in_features)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous().clone()
    y = torch.nn.functional.linear(x2, w[:, : modules[0].in_features])
    if stacked:
        return y if x.dtype == torch.bfloat16 else y.to(x.dtype)
    outs = torch.split(y, [m.out_features for m in modules], dim=1)
    return [o.reshape(*lead, m.out_features).to(x.dtype) for m, o in zip(modules, outs)]


def _canonical(key: str) -> str:
    """A tensor or module name as the teacher checkpoint stores it: the text
    stack's leading ``model.`` removed (``lm_head`` and other top-level names
    are unchanged)."""
    return key[len("model."):] if key.startswith("model.") else key


def _layer_of(name: str) -> int | None:
    """N of the first ``layers.N`` in a dotted name (None outside the layers)."""
    parts = name.split(".")
    for a, b in zip(parts, parts[1:]):
        if a == "layers" and b.isdigit():
            return int(b)
    return None


def wrap_q8_teacher(model: nn.Module, teacher_state_dict: dict, quant_meta: dict,
                    layer_devices: dict[int, torch.device] | None = None) -> nn.Module:
    """Turn a freshly built model into the Q8_0 teacher, in place
    (the interface of the reference's ``q8_teacher.py:176-294``).

    The checkpoint contract: a Linear's or Embedding's weight stored as Q8_0
    is a 2-D ``uint8`` tensor under ``<module>.weight``, named the checkpoint
    way (:func:`_canonical`), with its ``out_features``/``in_features`` in
    ``quant_meta`` under the weight's or the module's name (either naming).
    Such a module becomes a :class:`Q8Linear` / :class:`Q8Embedding` over
    those bytes.  Every other checkpoint tensor (norms, biases, ...) is
    assigned to the model tensor with the same checkpoint name.  With
    ``layer_devices`` ({N: device}) everything under ``layers.N`` -- wrapped
    modules and carried tensors -- lives on that device.  A Q8_0 tensor with
    no metadata is left in place, with a warning."""
    import logging
    import warnings

    ckpt = {_canonical(k): v for k, v in teacher_state_dict.items()}
    shapes = {}
    for k, v in quant_meta.items():
        c = _canonical(k)
        shapes[c[: -len(".weight")] if c.endswith(".weight") else c] = v

    def device_of(name: str):
        n = _layer_of(name)
        return layer_devices.get(n) if layer_devices and n is not None else None

    # every Linear / Embedding with its parent, found before any is replaced
    sites = [(parent, attr, f"{pname}.{attr}" if pname else attr, child)
             for pname, parent in model.named_modules() for attr, child in parent.named_children()
             if isinstance(child, (nn.Linear, nn.Embedding))]
    consumed, wrapped = set(), 0
    for parent, attr, name, child in sites:
        key = _canonical(name)
        qb = ckpt.get(key + ".weight")
        if not (isinstance(qb, torch.Tensor) and qb.dtype == torch.uint8 and qb.dim() == 2):
            continue
        consumed.add(key + ".weight")  # Q8_0 bytes never load into a dense weight
        shape = shapes.get(key)
        if shape is None:
            warnings.warn(f"Q8_0 teacher: {name} has Q8_0 bytes but no quant_meta entry; kept as is")
            continue
        dev = device_of(name)
        if isinstance(child, nn.Linear):
            bias = child.bias.detach() if child.bias is not None else None
            q8 = Q8Linear(qb, shape["out_features"], shape["in_features"], bias, device=dev)
        else:
            q8 = Q8Embedding(qb, child.num_embeddings, child.embedding_dim, device=dev)
        setattr(parent, attr, q8)
        wrapped += 1

    # the remaining checkpoint tensors, under the model's own names
    by_canonical = {_canonical(k): k for k in model.state_dict()}
    carry, stray = {}, []
    for k, v in ckpt.items():
        if k in consumed:
            continue
        if k in by_canonical:
            carry[by_canonical[k]] = v
        else:
            stray.append(k)
    model.load_state_dict(carry, strict=False, assign=True)
    if stray:
        warnings.warn(f"Q8_0 teacher: {len(stray)} checkpoint tensors match no model tensor (e.g. {stray[:3]})")
    if layer_devices:
        for name, t in list(model.named_parameters()) + list(model.named_buffers()):
            dev = device_of(name)
            if dev is not None and t.device != torch.device(dev):
                t.data = t.data.to(dev)
    logging.getLogger(__name__).info("Q8_0 teacher: %d modules wrapped, %d tensors carried", wrapped, len(carry))
    return model
