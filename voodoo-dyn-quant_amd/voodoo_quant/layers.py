"""Gated-mixture layers on the MI355X kernels.

Drop-in for the gated-Linear path of the reference's ``voodoo_quant/layers.py``:
``MixedQuantLinear`` keeps the reference's constructor, attributes and methods
(``layers.py:1000-1557, 1640-1740``), the module walkers keep their signatures
(``layers.py:1845-2083``), and the trainer-facing helpers
(``set_temperature``, ``total_effective_bytes``, ``invalidate_candidate_cache``,
``get_assignment``) behave the same.  What changes is underneath:

* candidates stay packed (GGUF bytes, the reference's "lazy" layout) and live
  on the GPU next to the layer;
* the forward is one autograd Function, :class:`GatedLinearFunction`, whose
  forward calls ``vq_gated_linear_fwd`` (mix K candidates -> bf16 W_eff ->
  MFMA GEMM) and whose backward calls ``vq_gated_linear_bwd`` (dX GEMM, and the
  per-candidate gate gradients <dY^T X, W_k> with dW kept in registers).  The
  softmax Jacobian is applied by autograd, exactly as for the reference's
  ``_MixedWeightFunction`` (``layers.py:336-363``).

There is no CPU or PyTorch-op implementation of the mixture: inputs must be on
a ROCm device and ``libvoodoo_hip.so`` must be built.
"""

from __future__ import annotations

import os
import random
import sys
import time
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.autograd import Function

from voodoo_quant import _hip, cache
from voodoo_quant.ggml import HIP_TYPES, bytes_per_weight, find_libggml, get_quant_info, quantize_tensor
from voodoo_quant.rtn import rtn_quantize_tensor

CANDIDATE_CACHE_DIR = cache.CANDIDATE_CACHE_DIR
_tensor_hash = cache.tensor_hash
_candidate_cache_path = cache.candidate_cache_path
_combined_cache_path = cache.combined_cache_path
_atomic_torch_save = cache.atomic_torch_save


def _ggml_id(qt: str) -> int:
    return get_quant_info(qt).ggml_type


# ---------------------------------------------------------------------------
# straight-through Gumbel hardening and PTQR switches (reference layers.py:803-865)
# ---------------------------------------------------------------------------
class _STGumbelState:
    enabled: bool = False
    fraction: float = 0.0
    gs_tau: float = 1.0
    f_start: float | None = None
    f_end: float | None = None
    total_steps: int = 1
    step: int = 0


_ST_GUMBEL_STATE = _STGumbelState()


def set_st_gumbel(enabled: bool, fraction: float, gs_tau: float) -> None:
    _ST_GUMBEL_STATE.enabled = enabled
    _ST_GUMBEL_STATE.fraction = float(fraction)
    _ST_GUMBEL_STATE.gs_tau = float(gs_tau)


def set_st_gumbel_anneal(f_start: float, f_end: float, total_steps: int) -> None:
    _ST_GUMBEL_STATE.f_start = float(f_start)
    _ST_GUMBEL_STATE.f_end = float(f_end)
    _ST_GUMBEL_STATE.total_steps = max(int(total_steps), 1)


def st_gumbel_step(step: int) -> None:
    _ST_GUMBEL_STATE.step = int(step)


def _effective_fraction() -> float:
    st = _ST_GUMBEL_STATE
    if st.f_start is None:
        return st.fraction
    t = min(max(st.step / max(st.total_steps - 1, 1), 0.0), 1.0)
    return st.f_start + (st.f_end - st.f_start) * t


class _PTQRState:
    enabled: bool = False


_PTQR_STATE = _PTQRState()


def set_ptqr(enabled: bool) -> None:
    """Per-token quant routing switch (reference ``layers.py:864-865``): every
    token of every gated Linear runs through ONE candidate, sampled from the
    gate probabilities."""
    _PTQR_STATE.enabled = bool(enabled)


def _sample_token_routing(probs: torch.Tensor, num_tokens: int) -> torch.Tensor:
    """k(t) ~ Categorical(probs) for each token by the Gumbel-argmax trick
    (reference ``layers.py:868-881``): one uniform draw of [K, tokens] on
    probs' device, Gumbel noise -log(-log u) with the reference's 1e-9 clamps,
    argmax of log p + noise over the candidates.  The same draws give the same
    routing as the reference."""
    u = torch.rand(probs.shape[0], num_tokens, device=probs.device)
    noise = -torch.log((-torch.log(u.clamp_min(1e-9))).clamp_min(1e-9))
    return (torch.log(probs.clamp_min(1e-9)).unsqueeze(1) + noise).argmax(dim=0)


# ---------------------------------------------------------------------------
# embedding id checks
# ---------------------------------------------------------------------------
# Lookups whose id check is deferred: (module name, num_embeddings, pinned
# host flag, event after its copy).
_PENDING_ID_CHECKS: list = []
_MAX_PENDING_ID_CHECKS = 64


def check_embedding_ids(ids: torch.Tensor, num_embeddings: int, name: str, mode: str) -> None:
    """Raise IndexError for ids outside [0, num_embeddings) (torch's embedding
    message).  mode "sync" reads the ids' range on the host now, a device
    synchronisation.  mode "deferred" leaves an out-of-range flag on the
    device, copied into pinned host memory behind an event, and returns at
    once; :func:`raise_pending_id_errors` raises later.  The row kernels give
    zero rows for out-of-range ids in the meantime (they never read past the
    table).  A training loop that defers the check lets the host queue the
    next step while the device still runs the last one."""
    if ids.numel() == 0:
        return
    if mode == "sync":
        lo, hi = torch.aminmax(ids)
        lo, hi = torch.stack([lo, hi]).tolist()
        if lo < 0 or hi >= num_embeddings:
            raise IndexError(f"{name}: index out of range in self "
                             f"(ids span [{lo}, {hi}], num_embeddings={num_embeddings})")
        return
    if mode != "deferred":
        raise ValueError(f"{name}: id_check must be 'sync' or 'deferred', got {mode!r}")
    if len(_PENDING_ID_CHECKS) >= _MAX_PENDING_ID_CHECKS:
        # a caller that never collects: take the finished checks (no wait),
        # so the list stays bounded; an earlier bad id raises here
        raise_pending_id_errors(block=False)
    bad = ((ids < 0) | (ids >= num_embeddings)).any().reshape(1)
    host = torch.empty(1, dtype=torch.bool, pin_memory=True)
    host.copy_(bad, non_blocking=True)
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(ids.device))
    _PENDING_ID_CHECKS.append((name, num_embeddings, host, done))


def raise_pending_id_errors(block: bool = True) -> None:
    """Raise IndexError for the first deferred lookup that saw an out-of-range
    id (see :func:`check_embedding_ids`).  block=True waits for every pending
    check's copy; block=False looks only at the finished ones and keeps the
    rest pending."""
    keep = []
    err = None
    for entry in _PENDING_ID_CHECKS:
        name, num, host, done = entry
        if not block and not done.query():
            keep.append(entry)
            continue
        done.synchronize()
        if err is None and bool(host[0]):
            err = IndexError(f"{name}: index out of range in self (an id outside [0, {num}) in a deferred lookup)")
    _PENDING_ID_CHECKS[:] = keep
    if err is not None:
        raise err


# ---------------------------------------------------------------------------
# padding (reference layers.py:973-997)
# ---------------------------------------------------------------------------
def _pad_weight_and_imatrix(weight: torch.Tensor, imatrix: torch.Tensor | None):
    orig_in = weight.shape[1]
    if orig_in % 256 == 0:
        return weight, imatrix, orig_in
    pad = 256 - orig_in % 256
    padded = F.pad(weight, (0, pad), "constant", 0)
    if imatrix is not None:
        imatrix = F.pad(imatrix.to(torch.float32).contiguous(), (0, pad), "constant", 1.0)
    return padded, imatrix, orig_in


pad_weight_and_imatrix = _pad_weight_and_imatrix


# ---------------------------------------------------------------------------
# device dequant (reference layers.py:298-319)
# ---------------------------------------------------------------------------
def dequantize_tensor_gpu(qweight: torch.Tensor, quant_type: str, out_features: int, in_features: int,
                          device) -> torch.Tensor:
    """Decode packed bytes on the GPU with the HIP kernel -> bf16 [out, in].

    The fp32 intermediate is bit-identical to ggml's ``dequantize_row_*``."""
    if quant_type not in HIP_TYPES:
        raise NotImplementedError(f"{quant_type}: the HIP decoders cover {HIP_TYPES}")
    device = torch.device(device)
    qb = qweight.to(device).contiguous().reshape(-1)
    w = _hip.dequant(_ggml_id(quant_type), qb, out_features, in_features)
    return w[:, :in_features].to(torch.bfloat16)


def dequantize_tensor_gpu_fp32(qweight: torch.Tensor, quant_type: str, out_features: int, in_features: int,
                               device) -> torch.Tensor:
    if quant_type not in HIP_TYPES:
        raise NotImplementedError(f"{quant_type}: the HIP decoders cover {HIP_TYPES}")
    qb = qweight.to(torch.device(device)).contiguous().reshape(-1)
    return _hip.dequant(_ggml_id(quant_type), qb, out_features, in_features)


# ---------------------------------------------------------------------------
# autograd Functions
# ---------------------------------------------------------------------------
def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


# The fused few-token products (vq_gated_linear_fwd_fused / _dx_fused: W_eff
# built tile by tile in LDS, never written) replace mix + GEMM when a call
# has at most FUSED_MAX_TOKENS tokens and the tensor at most
# FUSED_MAX_WEIGHTS weights and FUSED_MAX_ROWS output rows.  Measured on
# MI355X, K = 6 (Q2_K..Q8_0), forward + dX at 1-32 tokens, the materialised
# path with the workspaces this module passes (K-split last tiles), both
# interleaved in one process, materialised time over fused:
#   out x in     1024x1024 1.22-1.29, 1024x2048 1.17-1.28, 1024x3072
#   1.06-1.17, 1024x4096 1.10-1.18, 2048x1024 1.04-1.14, 2048x2048
#   0.95-1.05, 3072x1024 0.97-1.07, 4096x1024 0.97-1.03;
# 4096 x 4096 and 5120 -> 6144 lose by 1.4-2x, and at 64 tokens fused loses
# from 3M weights on.  The fused forward and dX spread their work over the
# output rows, so it is the row count, not the size, that sets the edge:
# the limits sit at the last points where fused did not lose.
FUSED_MAX_TOKENS = 32
FUSED_MAX_WEIGHTS = 1 << 22
FUSED_MAX_ROWS = 2048
# The fused kernels build each W_eff tile as fma(p_k dl, u, acc) + p_k c, which
# is within one bf16 ulp of the reference's separately rounded fp32 mixture,
# not bitwise equal to it.  FUSED_PRODUCTS = False (or VOODOO_FUSED=0 in the
# environment) sends every call through the bit-exact mix + GEMM path, e.g.
# for parity checks that compare outputs bitwise across token counts.
FUSED_PRODUCTS = os.environ.get("VOODOO_FUSED", "1") not in ("0", "off", "false")


def use_fused(m: int, n: int, d_pad: int) -> bool:
    """Whether a gated product of m tokens over an [n, d_pad] tensor takes the
    fused path."""
    return FUSED_PRODUCTS and 0 < m <= FUSED_MAX_TOKENS and n <= FUSED_MAX_ROWS and n * d_pad <= FUSED_MAX_WEIGHTS


def _finish_on_gate_stream(stream, rows, grads, keep) -> None:
    """The gate gradients `grads`, reduced on `stream` by the library, are
    added to the sink rows there; every buffer that stream still reads or
    writes is marked in use by it, so the allocator does not hand it out again
    before the stream has passed it."""
    with torch.cuda.stream(stream):
        for row, g in zip(rows, grads):
            row.add_(g)
    for t in list(grads) + list(keep):
        if t is not None:
            t.record_stream(stream)


class GatedLinearFunction(Function):
    """y = x W_eff^T with W_eff = sum_k probs_k W_k, on libvoodoo_hip.

    forward(ctx, x [M, D] bf16, probs [K] fp32, meta, premixed, sink, *qbytes) -> y [M, N] bf16
    where meta = (ggml type ids, N, D_pad), premixed is None or this
    step's W_eff [N, D_pad] already mixed from probs (see
    :class:`MixPrefetch`), and sink is None or (row, stream): a deferred gate
    gradient (see ``trainer.GateBank``), finished on `stream` and added to
    `row` instead of being returned.  The backward returns dX and dL/dprobs;
    qbytes receive no gradient (they are constants, as the candidates are for
    the reference's ``_MixedWeightFunction``)."""

    @staticmethod
    def forward(ctx, x, probs, meta, premixed, sink, *qbytes):
        types, n, d_pad = meta
        x2 = _aligned(x)
        m, d = x2.shape
        p = probs.detach().to(device=x.device, dtype=torch.float32).contiguous()
        y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
        ctx.fused = premixed is None and use_fused(m, n, d_pad)
        if premixed is not None:  # W_eff mixed ahead on the prefetch stream: the GEMM only
            nbytes = _hip.fwd_workspace_bytes(m, n, d)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes > 0 else None
            if m > 0:
                _hip.linear_fwd(x2, premixed, n, y, ws)
            ctx.save_for_backward(x2, p, premixed)
        elif ctx.fused:
            # W_eff only ever exists tile by tile in LDS
            nbytes = _hip.fused_workspace_bytes(m, n, d, False)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes > 0 else None
            _hip.gated_linear_fwd_fused(x2, types, qbytes, p, n, d_pad, y, ws)
            ctx.save_for_backward(x2, p)
        else:
            w_eff = torch.empty(n, d_pad, dtype=torch.bfloat16, device=x.device)
            nbytes = _hip.fwd_workspace_bytes(m, n, d)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes > 0 else None
            _hip.gated_linear_fwd(x2, types, qbytes, p, n, d_pad, w_eff, y, ws)
            ctx.save_for_backward(x2, p, w_eff)
        ctx.meta = meta
        ctx.qbytes = qbytes
        ctx.probs_device = probs.device
        ctx.sink = sink
        return y

    @staticmethod
    def backward(ctx, dy):
        types, n, d_pad = ctx.meta
        sink = ctx.sink
        gs = sink[1] if sink is not None else None
        need_dx, need_dp = ctx.needs_input_grad[0], ctx.needs_input_grad[1] or sink is not None
        dy2 = _aligned(dy.to(torch.bfloat16))
        if ctx.fused:
            x2, p = ctx.saved_tensors
            m, d = x2.shape
            dx = dprobs = None
            if need_dx:  # dX through the fused kernel: W_eff never materialised
                dx = torch.empty_like(x2)
                nbytes = _hip.fused_workspace_bytes(m, n, d, True)
                ws = torch.empty(nbytes, dtype=torch.uint8, device=x2.device) if nbytes > 0 else None
                _hip.gated_linear_dx_fused(dy2, types, ctx.qbytes, p, d, d_pad, dx, ws)
            if need_dp:  # the gate product reads the packed candidates, never W_eff
                dprobs = torch.empty(len(types), dtype=torch.float32, device=x2.device)
                nbytes = _hip.bwd_workspace_bytes(m, n, d, d_pad, len(types), False)
                ws = torch.empty(nbytes, dtype=torch.uint8, device=x2.device)
                _hip.gated_linear_bwd(dy2, x2, types, ctx.qbytes, p, n, d_pad, None, None, dprobs, ws, gs)
                if sink is not None:
                    _finish_on_gate_stream(gs, [sink[0]], [dprobs], [ws])
                    dprobs = None
                else:
                    dprobs = dprobs.to(ctx.probs_device)
            return (dx, dprobs, None, None, None) + (None,) * len(ctx.qbytes)
        x2, p, w_eff = ctx.saved_tensors
        dx = torch.empty_like(x2) if need_dx else None
        dprobs = torch.empty(len(types), dtype=torch.float32, device=x2.device) if need_dp else None
        ws = None
        if need_dx or need_dp:  # gate partials and the K-split parts of dX's last tiles
            nbytes = _hip.bwd_workspace_bytes(x2.shape[0], n, x2.shape[1], d_pad, len(types), False)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x2.device)
        if need_dx or need_dp:
            _hip.gated_linear_bwd(dy2, x2, types, ctx.qbytes, p, n, d_pad, w_eff, dx, dprobs, ws,
                                  gs if dprobs is not None else None)
        if sink is not None and dprobs is not None:
            _finish_on_gate_stream(gs, [sink[0]], [dprobs], [ws])
            dprobs = None
        elif dprobs is not None:
            dprobs = dprobs.to(ctx.probs_device)
        return (dx, dprobs, None, None, None) + (None,) * len(ctx.qbytes)


class GatedLinearGroupFunction(Function):
    """Gated Linears that read the same input (q/k/v, gate/up) as ONE stacked
    product on libvoodoo_hip: every member's W_eff is mixed into its rows of a
    stacked [sum N, D_pad] weight, then one GEMM gives [M, sum N]; the
    backward is one launch for dX (which also sums the members' input
    gradients) and every member's gate gradients.

    forward(ctx, x [M, D] bf16, meta, premixed, sinks, *probs_then_qbytes) -> y [M, sum N] bf16
    with meta = (((ggml types, N) per member), D_pad), premixed None or the
    step's stacked W_eff [sum N, D_pad] mixed ahead (see :class:`MixPrefetch`),
    sinks None or one (row, stream) per member (deferred gate gradients, as
    for :class:`GatedLinearFunction`), then each member's probs [K_i] and
    finally every member's qbytes in order."""

    @staticmethod
    def forward(ctx, x, meta, premixed, sinks, *tensors):
        members, d_pad = meta
        nm = len(members)
        probs, qbytes = tensors[:nm], tensors[nm:]
        x2 = _aligned(x)
        dev = x2.device
        ps = [p.detach().to(device=dev, dtype=torch.float32).contiguous() for p in probs]
        spec, off = [], 0
        for types, n in members:
            spec.append((types, qbytes[off:off + len(types)], n))
            off += len(types)
        n_total = sum(n for _, n in members)
        y = torch.empty(x2.shape[0], n_total, dtype=torch.bfloat16, device=dev)
        nbytes = _hip.fwd_workspace_bytes(x2.shape[0], n_total, x2.shape[1])
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes > 0 else None
        if premixed is not None:  # mixed ahead on the prefetch stream: the GEMM only
            w_eff = premixed
            if x2.shape[0] > 0:
                _hip.linear_fwd(x2, w_eff, n_total, y, ws)
        else:
            w_eff = torch.empty(n_total, d_pad, dtype=torch.bfloat16, device=dev)
            _hip.gated_linear_group_fwd(x2, spec, ps, d_pad, w_eff, y, ws)
        ctx.save_for_backward(x2, w_eff)
        ctx.spec = spec
        ctx.meta = meta
        ctx.probs_devices = [p.device for p in probs]
        ctx.sinks = sinks
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, w_eff = ctx.saved_tensors
        members, d_pad = ctx.meta
        nm = len(members)
        sinks = ctx.sinks
        gs = sinks[0][1] if sinks is not None else None
        need_dx = ctx.needs_input_grad[0]
        need_dp = any(ctx.needs_input_grad[4:4 + nm]) or sinks is not None
        dx = torch.empty_like(x2) if need_dx else None
        dprobs = None
        if need_dp:
            dprobs = [torch.empty(len(t), dtype=torch.float32, device=x2.device) for t, _ in members]
        if need_dx or need_dp:
            dy2 = _aligned(dy.to(torch.bfloat16))
            nbytes = _hip.group_bwd_workspace_bytes(x2.shape[0], x2.shape[1], ctx.spec)
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x2.device)
            _hip.gated_linear_group_bwd(dy2, x2, ctx.spec, d_pad, w_eff if need_dx else None, dx, dprobs, ws,
                                        gs if dprobs is not None else None)
            if sinks is not None and dprobs is not None:
                _finish_on_gate_stream(gs, [r for r, _ in sinks], dprobs, [ws])
                dprobs = None
        grads_p = [None] * nm if dprobs is None else [g.to(d) for g, d in zip(dprobs, ctx.probs_devices)]
        n_q = sum(len(t) for t, _ in members)
        return (dx, None, None, None, *grads_p) + (None,) * n_q


class MixPrefetch:
    """Mixes the step's W_eff of the listed gated products on a second stream,
    a few products ahead of the forward that uses them.

    The mix is HBM- and VALU-bound, the GEMMs MFMA-bound, and a training step
    fixes every gate probability before its forward starts.  So while the
    forward runs product i, the mix of product i + ``ahead`` runs on a side
    stream (default priority), fenced by one event per product.  A gated
    forward that finds its product prefetched waits for that event only, runs
    the GEMM on the buffer (its backward reuses it), and issues the next mix.

    ``groups`` lists the products in forward order as the forward runs them: a
    list of :class:`MixedQuantLinear` that one stacked product reads, or a
    single module.  W_eff buffers live as long as the prefetcher (0.58 GB for
    the 0.8B-class decoder).  Launch arguments are marshalled once; each step
    copies the probabilities into persistent buffers with one multi-tensor
    copy, so issuing a mix is one C call and one event record.  Call
    :meth:`launch` after the step's probabilities are final (after
    ``GateBank.begin``).  The forward differentiates through the same
    probabilities, so W_eff, every output and every gradient are
    bit-identical to the unprefetched step's."""

    def __init__(self, groups: list, device=None, ahead: int = 8):
        self.groups = [list(g) if isinstance(g, (list, tuple)) else [g] for g in groups]
        dev = torch.device(device) if device is not None else self.groups[0][0].gates.device
        self.device = dev
        self.ahead = max(int(ahead), 1)
        self.stream = torch.cuda.Stream(device=dev)  # default priority
        self.buffers, self.events, self.probs, self._pbuf, self._calls = [], [], [], [], []
        self.pending = [False] * len(self.groups)
        self._next = 0  # the next product to mix in the current step
        sptr = self.stream.cuda_stream
        for gi, mods in enumerate(self.groups):
            d_pad = mods[0].padded_in_features
            if any(m.padded_in_features != d_pad for m in mods):
                raise ValueError("a prefetched product's members must share their input width")
            for m in mods:
                m._move_qbytes(dev)
            n_total = sum(m.out_features for m in mods)
            buf = torch.empty(n_total, d_pad, dtype=torch.bfloat16, device=dev)
            pbuf = [torch.zeros(m.num_candidates, dtype=torch.float32, device=dev) for m in mods]
            # the side stream writes both: when they are freed, the caching
            # allocator waits for the side stream's queued work too
            buf.record_stream(self.stream)
            for b in pbuf:
                b.record_stream(self.stream)
            self.buffers.append(buf)
            self._pbuf.append(pbuf)
            self.events.append(torch.cuda.Event())
            self.probs.append(None)
            self._calls.append(_hip.mix_only_call(
                [(m._ggml_types(), m._qbytes(), m.out_features) for m in mods], pbuf, d_pad, buf, sptr))
            for m in mods:
                m.__dict__["_prefetch"] = (self, gi)

    def _issue(self) -> None:
        gi = self._next
        if gi >= len(self.groups):
            return
        self._next += 1
        with torch.cuda.stream(self.stream):
            self._calls[gi]()
            self.events[gi].record(self.stream)
        self.pending[gi] = True

    def launch(self) -> None:
        main = torch.cuda.current_stream(self.device)
        probs = [[m.get_probs() for m in mods] for mods in self.groups]
        torch._foreach_copy_([b for pb in self._pbuf for b in pb],
                             [p.detach().to(torch.float32) for ps in probs for p in ps])
        ready = torch.cuda.Event()
        ready.record(main)  # the probabilities, and the previous step's use of the buffers
        self.stream.wait_event(ready)
        self.probs = probs
        self.pending = [False] * len(self.groups)
        self._next = 0
        for _ in range(min(self.ahead, len(self.groups))):
            self._issue()

    @staticmethod
    def take(modules: list):
        """(W_eff, probabilities) when `modules` are one prefetched product whose
        mix is pending: the current stream then waits for that mix, and the mix
        `ahead` products later is issued."""
        ref = modules[0].__dict__.get("_prefetch")
        if ref is None:
            return None
        pf, gi = ref
        mods = pf.groups[gi]
        if not pf.pending[gi] or len(mods) != len(modules) or any(a is not b for a, b in zip(mods, modules)):
            return None
        pf.pending[gi] = False
        pf._issue()
        torch.cuda.current_stream(pf.device).wait_event(pf.events[gi])
        return pf.buffers[gi], pf.probs[gi][:]

    def release(self) -> None:
        """Detach the prefetcher from its modules; the current stream waits
        for mixes still queued on the side stream."""
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        for mods in self.groups:
            for m in mods:
                m.__dict__.pop("_prefetch", None)
        self.pending = [False] * len(self.groups)


def groupable(modules: list) -> bool:
    """Whether gated Linears that read one input run as one stacked product:
    2 to 4 :class:`MixedQuantLinear` modules with the same input width,
    out_features multiples of 256, no sharding, PTQR off."""
    return (2 <= len(modules) <= 4 and not _PTQR_STATE.enabled
            and all(isinstance(m, MixedQuantLinear) for m in modules)
            and len({(m.in_features, m.padded_in_features) for m in modules}) == 1
            and all(m.out_features % 256 == 0 and m.shard_spec is None for m in modules))


def gated_linear_group(x: torch.Tensor, modules: list, stacked: bool = False):
    """Outputs of gated Linears that all read `x`, as one stacked product when
    they allow it: 2 to 4 :class:`MixedQuantLinear` modules with the same
    input width, out_features multiples of 256 and PTQR off.  Otherwise each
    module runs its own forward.  The outputs equal the modules' own forwards
    up to the GEMM's summation order.

    stacked=True returns the stacked output [tokens, sum out_features] itself
    (None when the modules cannot be stacked)."""
    if not (x.device.type == "cuda" and groupable(modules)):
        return None if stacked else [m(x) for m in modules]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    streamer = modules[0].__dict__.get("_streamer")
    if streamer is not None:
        if any(m.__dict__.get("_streamer") is not streamer for m in modules) or \
                any(m.__dict__.get("_gate_sink") is not None for m in modules):
            raise RuntimeError("a stacked product's members must share one candidate streamer and run without "
                               "deferred gate gradients")
        streamer.forward_fence(modules[0])
    pre = MixPrefetch.take(modules) if streamer is None else None
    # deferred gate gradients only when every member has a sink (else autograd
    # for all); the probabilities stay attached either way, so the product's
    # backward runs even when its input needs no gradient, and returns None
    # for them when deferring
    sinks = [m.__dict__.get("_gate_sink") for m in modules]
    sinks = None if any(sk is None for sk in sinks) else sinks
    probs, qbytes, members = [], [], []
    for i, m in enumerate(modules):
        m._move_qbytes(x.device)
        p = pre[1][i] if pre is not None else m.get_probs()
        probs.append(p if p.device == x.device else p.to(x.device))
        qbytes.extend(m._qbytes())
        members.append((m._ggml_types(), m.out_features))
    meta = (tuple(members), modules[0].padded_in_features)
    y = GatedLinearGroupFunction.apply(x2, meta, pre[0] if pre is not None else None, sinks, *probs, *qbytes)
    if streamer is not None:
        y = streamer.fenced(y, modules[0])
    if stacked:
        return y if x.dtype == torch.bfloat16 else y.to(x.dtype)
    outs = torch.split(y, [m.out_features for m in modules], dim=1)
    res = []
    for m, o in zip(modules, outs):
        o = o.reshape(*lead, m.out_features)
        res.append(o if x.dtype == torch.bfloat16 else o.to(x.dtype))
    return res


class RoutedLinearFunction(Function):
    """PTQR forward on libvoodoo_hip: y[t] = x[t] W_{k(t)}^T, tokens grouped by
    their routed candidate (reference ``_RoutedMixedLinear``,
    ``layers.py:366-429``).

    forward(ctx, x [M, D] bf16, probs [K] fp32, routing [M] int, meta,
    cand_bf16 (list of [N, D_pad] bf16 decodes), *qbytes) -> y [M, N] bf16.
    The backward is the straight-through mixture gradient at the routed point,
    the same as the gated Linear's: dX = dY W_eff and dL/dp_k = <dY^T X, W_k>,
    with W_eff re-mixed from the packed candidates."""

    @staticmethod
    def forward(ctx, x, probs, routing, meta, cand_bf16, *qbytes):
        types, n, d_pad = meta
        x2 = _aligned(x)
        k = len(types)
        r = routing.to(device=x2.device, dtype=torch.int64)
        perm = torch.argsort(r, stable=True).to(torch.int32)
        group_off = torch.zeros(k + 1, dtype=torch.int32, device=x2.device)
        group_off[1:] = torch.cumsum(torch.bincount(r, minlength=k), 0).to(torch.int32)
        y = torch.empty(x2.shape[0], n, dtype=torch.bfloat16, device=x2.device)
        _hip.routed_linear_fwd(x2, cand_bf16, perm, group_off, n, d_pad, y)
        p = probs.detach().to(device=x2.device, dtype=torch.float32).contiguous()
        ctx.save_for_backward(x2, p)
        ctx.meta = meta
        ctx.qbytes = qbytes
        ctx.probs_device = probs.device
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, p = ctx.saved_tensors
        types, n, d_pad = ctx.meta
        need_dx, need_dp = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dy2 = _aligned(dy.to(torch.bfloat16))
        dx = torch.empty_like(x2) if need_dx else None
        dprobs = torch.empty(len(types), dtype=torch.float32, device=x2.device) if need_dp else None
        if need_dx or need_dp:
            # no W_eff from the forward: the library re-mixes it into the workspace
            nbytes = _hip.bwd_workspace_bytes(x2.shape[0], n, x2.shape[1], d_pad, len(types), need_dx)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x2.device)
            _hip.gated_linear_bwd(dy2, x2, types, ctx.qbytes, p, n, d_pad, None, dx, dprobs, ws)
        if dprobs is not None:
            dprobs = dprobs.to(ctx.probs_device)
        return (dx, dprobs, None, None, None) + (None,) * len(ctx.qbytes)


class MixedWeightFunction(Function):
    """W_eff [N, D] in the source dtype, differentiable w.r.t. probs
    (reference ``_MixedWeightFunction``, ``layers.py:322-363``).  Serves the
    non-fused consumers of ``get_mixed_weight``; the gated Linear's own
    forward never materialises it outside its workspace."""

    @staticmethod
    def forward(ctx, probs, meta, *qbytes):
        types, n, d, d_pad, out_dtype = meta
        p = probs.detach().to(dtype=torch.float32).contiguous()
        w = _hip.mix_weight(types, qbytes, p, n, d_pad)[:, :d]
        ctx.meta = meta
        ctx.qbytes = qbytes
        return w.to(out_dtype)

    @staticmethod
    def backward(ctx, grad_w):
        types, n, d, d_pad, _ = ctx.meta
        g = grad_w.to(torch.float32)
        gp = torch.empty(len(types), dtype=torch.float32, device=grad_w.device)
        for k, (t, qb) in enumerate(zip(types, ctx.qbytes)):
            wk = _hip.dequant(t, qb.reshape(-1), n, d_pad)[:, :d]
            gp[k] = (g * wk).sum()
        return (gp, None) + (None,) * len(ctx.qbytes)


class EmbeddingRowsFunction(Function):
    """Row lookup of a gated embedding on libvoodoo_hip: only the requested
    rows of each packed candidate are decoded (reference
    ``_MixedEmbeddingRowFunctionLazy``, ``layers.py:670-750``; with a routing,
    its PTQR row selection, ``layers.py:712-716``).

    forward(ctx, probs [K] fp32, routing [R] int64 or None, row_ids [R] int64,
    meta, *qbytes) -> [R, dim] in meta's dtype (bf16 or fp32), where
    meta = (ggml type ids, num_embeddings, dim, d_pad, dtype).  Without a
    routing a row is the fp32 k-ordered mixture of the candidates' rows; with
    one, row r is candidate routing[r]'s row.  The backward is the full
    mixture gradient in both cases (straight-through under PTQR):
    dL/dp_k = sum_r <G[r], W_k[row_ids[r]]>."""

    @staticmethod
    def forward(ctx, probs, routing, row_ids, meta, *qbytes):
        types, vocab, dim, d_pad, dtype = meta
        p = probs.detach().to(device=row_ids.device, dtype=torch.float32).contiguous()
        out = _hip.embedding_rows_fwd(types, qbytes, p, routing, row_ids, vocab, dim, d_pad, dtype)
        ctx.save_for_backward(row_ids)
        ctx.meta = meta
        ctx.qbytes = qbytes
        ctx.probs_device = probs.device
        return out

    @staticmethod
    def backward(ctx, grad):
        (row_ids,) = ctx.saved_tensors
        types, vocab, dim, d_pad, dtype = ctx.meta
        dprobs = None
        if ctx.needs_input_grad[0]:
            g = _aligned(grad.to(dtype))
            dprobs = _hip.embedding_rows_bwd(types, ctx.qbytes, row_ids, vocab, dim, d_pad, g)
            dprobs = dprobs.to(ctx.probs_device)
        return (dprobs, None, None, None) + (None,) * len(ctx.qbytes)


# ---------------------------------------------------------------------------
# gated modules
# ---------------------------------------------------------------------------
class _MixedQuantBase(nn.Module):
    """Candidate production, storage and gate logic shared by gated layers
    (reference ``_MixedQuantBase``, ``layers.py:1000-1557``)."""

    def __init__(self, candidate_types: list[str], source_weight: torch.Tensor, out_features: int,
                 in_features: int, imatrix: torch.Tensor | None = None, device=None, lazy: bool = False,
                 tensor_name: str = "unknown", qbytes_device=None, shard_spec=None,
                 full_source_weight: torch.Tensor | None = None):
        super().__init__()
        if shard_spec is not None and full_source_weight is None:
            raise ValueError(f"{tensor_name}: shard_spec requires full_source_weight")
        self._setup(candidate_types, out_features, in_features, lazy, tensor_name, qbytes_device, shard_spec,
                    source_weight.device if device is None else device, source_weight.dtype)

        src = (full_source_weight if shard_spec is not None else source_weight).detach().to("cpu").contiguous()
        if imatrix is not None:
            imatrix = imatrix.detach().to(torch.float32).cpu()
        padded, padded_imatrix, _ = _pad_weight_and_imatrix(src.to(torch.float32), imatrix)
        self.padded_in_features = padded.shape[1]
        self._full_padded_in_features = self.padded_in_features
        weight_hash = cache.tensor_hash(padded)
        imatrix_hash = cache.tensor_hash(padded_imatrix) if imatrix is not None else "none"
        root = CANDIDATE_CACHE_DIR if CANDIDATE_CACHE_DIR != cache.CANDIDATE_CACHE_DIR else None
        # "lazy" entries hold llama.cpp bytes only (whoever wrote them); the
        # RTN fallback's bytes live under their own mode, read only while
        # libggml is absent, so a later libggml run never trains on them
        found = cache.load_candidates(tensor_name, self.candidate_types, "lazy", weight_hash, imatrix_hash, root)
        self.candidate_source = "cache"
        have_ggml = find_libggml() is not None
        if not have_ggml and len(found) < len(self.candidate_types):
            rest = [qt for qt in self.candidate_types if qt not in found]
            rtn_found = cache.load_candidates(tensor_name, rest, cache.RTN_MODE, weight_hash, imatrix_hash, root)
            if rtn_found:
                self.candidate_source = "cache_rtn"
                found.update(rtn_found)
        missing = [qt for qt in self.candidate_types if qt not in found]
        if missing:
            made, source = _quantize_candidates(padded, padded_imatrix, missing)
            self.candidate_source = source
            found.update(made)
            try:
                mode = "lazy" if source == "ggml" else cache.RTN_MODE
                cache.save_candidates(tensor_name, made, mode, weight_hash, imatrix_hash, root)
            except OSError as e:  # a read-only cache is not fatal
                print(f"  [cache] {tensor_name}: not saved ({e})", file=sys.stderr)
        full_out = shard_spec.full_out if shard_spec is not None else out_features
        for k, qt in enumerate(self.candidate_types):
            info = get_quant_info(qt)
            qb = found[qt].reshape(-1)
            expect = full_out * (self.padded_in_features // info.block_size) * info.block_bytes
            if qb.numel() != expect:
                raise ValueError(f"{tensor_name}: cached {qt} holds {qb.numel()} bytes, expected {expect}")
            self.register_buffer(f"_qweight_{k}", qb.contiguous(), persistent=False)
        if shard_spec is not None:
            self._apply_shard_to_candidates()
        self.imatrix = imatrix
        if self._qbytes_device is not None:
            self._move_qbytes(self._qbytes_device)

    def _setup(self, candidate_types, out_features, in_features, lazy, tensor_name, qbytes_device, shard_spec,
               device, source_dtype) -> None:
        self.candidate_types = list(candidate_types)
        bad = [qt for qt in self.candidate_types if qt not in HIP_TYPES]
        if bad:
            raise ValueError(f"{tensor_name}: candidate types {bad} have no HIP decoder (supported: {HIP_TYPES})")
        if not self.candidate_types:
            raise ValueError(f"{tensor_name}: empty candidate list")
        self.num_candidates = len(self.candidate_types)
        self.out_features = out_features
        self.in_features = in_features
        self.lazy = lazy
        self._tensor_name = tensor_name
        self._qbytes_device = torch.device(qbytes_device) if qbytes_device is not None else None
        self.shard_spec = shard_spec
        self._device = torch.device(device)
        self.gates = nn.Parameter(torch.zeros(self.num_candidates, device=self._device))
        self.temperature = 1.0
        self.source_dtype = source_dtype

    @classmethod
    def _from_packed(cls, candidate_types: list[str], qbytes: list[torch.Tensor], out_features: int,
                     in_features: int, source_dtype: torch.dtype, tensor_name: str, device=None):
        """A layer over candidate bytes that already exist (one packed
        [out_features, in_features rounded up to 256] stream per type): no
        quantization, no cache.  The bytes stay where they are."""
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        dev = qbytes[0].device if device is None else device
        obj._setup(candidate_types, out_features, in_features, True, tensor_name, None, None, dev, source_dtype)
        if len(qbytes) != obj.num_candidates:
            raise ValueError(f"{tensor_name}: {len(qbytes)} byte streams for {obj.num_candidates} candidates")
        obj.padded_in_features = (in_features + 255) // 256 * 256
        obj._full_padded_in_features = obj.padded_in_features
        obj.candidate_source = "packed"
        for k, qt in enumerate(obj.candidate_types):
            info = get_quant_info(qt)
            expect = out_features * (obj.padded_in_features // info.block_size) * info.block_bytes
            qb = qbytes[k].reshape(-1)
            if qb.dtype != torch.uint8 or qb.numel() != expect:
                raise ValueError(f"{tensor_name}: {qt} bytes must be uint8 x {expect}, got {qb.dtype} x {qb.numel()}")
            obj.register_buffer(f"_qweight_{k}", qb.contiguous(), persistent=False)
        obj.imatrix = None
        return obj

    # -- candidate storage ----------------------------------------------------
    def _qbytes(self) -> list[torch.Tensor]:
        streamer = self.__dict__.get("_streamer")
        if streamer is not None:  # views of this product's device slot (streaming.CandidateStreamer)
            return streamer.views(self)
        return [getattr(self, f"_qweight_{k}") for k in range(self.num_candidates)]

    def _move_qbytes(self, device) -> None:
        if self.__dict__.get("_streamer") is not None:  # the streamer stages the bytes
            return
        device = torch.device(device)
        for k in range(self.num_candidates):
            qb = getattr(self, f"_qweight_{k}")
            if qb.device != device:
                setattr(self, f"_qweight_{k}", qb.to(device, non_blocking=False).contiguous())

    def _ggml_types(self) -> tuple[int, ...]:
        return tuple(_ggml_id(qt) for qt in self.candidate_types)

    def _apply_shard_to_candidates(self) -> None:
        spec = self.shard_spec
        for k, qt in enumerate(self.candidate_types):
            qb = getattr(self, f"_qweight_{k}")
            setattr(self, f"_qweight_{k}", spec.slice_qbytes(qb, qt, self._full_padded_in_features).reshape(-1)
                    .contiguous())
        self.padded_in_features = spec.local_padded_in(self._full_padded_in_features, self.candidate_types)

    def __getattr__(self, name: str):
        # The reference's non-lazy modules expose decoded candidates as _w_{k}.
        if name.startswith("_w_") and name[3:].isdigit():
            return self._get_candidate(int(name[3:]))
        return super().__getattr__(name)

    def _get_candidate(self, k: int) -> torch.Tensor:
        qt = self.candidate_types[k]
        qb = getattr(self, f"_qweight_{k}")
        dev = qb.device if qb.device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
        w = dequantize_tensor_gpu_fp32(qb, qt, self.out_features, self.padded_in_features, dev)
        return w[:, : self.in_features].to(self.source_dtype)

    def invalidate_candidate_cache(self):
        """Drop the bf16 decodes the routed (PTQR) forward keeps (the trainer
        calls this, ``trainer.py:2502-2506``).  The mixture path caches
        nothing: its kernels decode the packed bytes directly."""
        self.__dict__["_bf16_cache"] = None

    def _bf16_candidates(self, device) -> list[torch.Tensor]:
        """bf16 [N, D_pad] decode of every candidate, kept until invalidated:
        candidates are constant, so the routed forward decodes them once (the
        reference's lazy path keeps the same per-candidate decodes)."""
        cache = self.__dict__.get("_bf16_cache")
        device = torch.device(device)
        if cache is None or cache[0].device != device:
            self._move_qbytes(device)
            cache = [_hip.dequant_bf16(_ggml_id(qt), getattr(self, f"_qweight_{k}"), self.out_features,
                                       self.padded_in_features)
                     for k, qt in enumerate(self.candidate_types)]
            self.__dict__["_bf16_cache"] = cache
        return cache

    # -- gates ----------------------------------------------------------------
    def set_temperature(self, temperature: float):
        self.temperature = max(temperature, 1e-6)

    def soft_probs(self) -> torch.Tensor:
        # a GateBank computes every bank member's softmax in one launch and
        # hands each module its row for the step
        override = self.__dict__.get("_probs_override")
        if override is not None:
            return override
        return F.softmax(self.gates / self.temperature, dim=0)

    def get_probs(self) -> torch.Tensor:
        probs = self.soft_probs()
        if _ST_GUMBEL_STATE.enabled and random.random() < _effective_fraction():
            u = torch.rand_like(probs)
            gumbel = -torch.log((-torch.log(u.clamp_min(1e-9))).clamp_min(1e-9))
            scores = (torch.log(probs.clamp_min(1e-9)) + gumbel) / max(_ST_GUMBEL_STATE.gs_tau, 1e-3)
            hard = F.one_hot(scores.argmax(dim=0), num_classes=probs.shape[0]).to(probs.dtype)
            return (hard - probs).detach() + probs
        return probs

    def get_mixed_weight(self) -> torch.Tensor:
        probs = self.get_probs()
        dev = self._compute_device()
        self._move_qbytes(dev)
        meta = (self._ggml_types(), self.out_features, self.in_features, self.padded_in_features, self.source_dtype)
        return MixedWeightFunction.apply(probs.to(dev), meta, *self._qbytes())

    def _compute_device(self) -> torch.device:
        qb = getattr(self, "_qweight_0")
        if qb.device.type == "cuda":
            return qb.device
        if self.gates.device.type == "cuda":
            return self.gates.device
        if not torch.cuda.is_available():
            raise RuntimeError(f"{self._tensor_name}: the gated layers run on ROCm devices only")
        return torch.device("cuda", torch.cuda.current_device())

    def _bytes_per_candidate(self) -> list[float]:
        """bpw_k * N * D with the full (unsharded) dims."""
        out_eff = getattr(self, "_full_out_features", None) or self.out_features
        in_eff = getattr(self, "_full_in_features", None) or self.in_features
        return [bytes_per_weight(qt) * in_eff * out_eff for qt in self.candidate_types]

    def effective_bytes(self) -> torch.Tensor:
        """sum_k p_k * bpw_k * N * D (reference ``layers.py:1537-1550``)."""
        probs = self.soft_probs()
        coef = torch.tensor(self._bytes_per_candidate(), dtype=probs.dtype).to(probs.device, non_blocking=True)
        return (probs * coef).sum()

    def get_assignment(self) -> str:
        return self.candidate_types[self.gates.argmax().item()]

    def get_assignment_prob(self) -> float:
        probs = self.soft_probs().detach()
        return probs[self.gates.argmax().item()].item()

    # -- tensor-parallel slicing (reference layers.py:1400-1472) ---------------
    def shard_rows(self, row_ranges: list[tuple[int, int]]) -> None:
        if getattr(self, "_full_out_features", None) is not None or getattr(self, "_full_in_features", None):
            raise RuntimeError(f"{self._tensor_name}: already row/col-sharded")
        shard_out = sum(e - s for s, e in row_ranges)
        if shard_out <= 0 or shard_out > self.out_features:
            raise ValueError(f"{self._tensor_name}: invalid row ranges {row_ranges} for out_features={self.out_features}")
        for k in range(self.num_candidates):
            q2d = getattr(self, f"_qweight_{k}").view(self.out_features, -1)
            setattr(self, f"_qweight_{k}", torch.cat([q2d[s:e] for s, e in row_ranges], 0).reshape(-1).contiguous())
        self._full_out_features = self.out_features
        self.out_features = shard_out
        self.invalidate_candidate_cache()

    def shard_cols(self, col_range: tuple[int, int]) -> None:
        if getattr(self, "_full_out_features", None) is not None or getattr(self, "_full_in_features", None):
            raise RuntimeError(f"{self._tensor_name}: already row/col-sharded")
        s, e = col_range
        if s < 0 or e > self.in_features or e <= s:
            raise ValueError(f"{self._tensor_name}: invalid column range {col_range} for in_features={self.in_features}")
        if s % 256 or e % 256:
            raise ValueError(f"{self._tensor_name}: column range {col_range} is not 256-aligned (gated layers "
                             "keep whole 256-weight groups)")
        for k, qt in enumerate(self.candidate_types):
            info = get_quant_info(qt)
            nbpr = self.padded_in_features // info.block_size
            b0, b1 = s // info.block_size, e // info.block_size
            q3 = getattr(self, f"_qweight_{k}").view(self.out_features, nbpr, info.block_bytes)[:, b0:b1, :]
            setattr(self, f"_qweight_{k}", q3.reshape(-1).contiguous())
        self._full_in_features = self.in_features
        self.in_features = e - s
        self.padded_in_features = e - s
        self.invalidate_candidate_cache()


def _quantize_candidates(padded: torch.Tensor, padded_imatrix: torch.Tensor | None,
                         types: list[str]) -> tuple[dict[str, torch.Tensor], str]:
    """Candidate bytes from libggml when it loads, else from the RTN encoder."""
    if find_libggml() is not None:
        return {qt: quantize_tensor(padded, qt, padded_imatrix) for qt in types}, "ggml"
    if not getattr(_quantize_candidates, "_warned", False):
        print("voodoo_quant: libggml-base not found; candidates come from the non-ggml RTN encoder "
              "(valid GGUF blocks, not llama.cpp-exact bytes)", file=sys.stderr)
        _quantize_candidates._warned = True
    return {qt: rtn_quantize_tensor(padded, qt) for qt in types}, "rtn"


class MixedQuantLinear(_MixedQuantBase):
    """Linear layer whose weight is a softmax mixture of K packed candidates
    (reference ``layers.py:1640-1740``)."""

    def __init__(self, in_features: int, out_features: int, candidate_types: list[str],
                 source_weight: torch.Tensor, imatrix: torch.Tensor | None = None, device=None, lazy: bool = False,
                 tensor_name: str = "unknown", qbytes_device=None, shard_spec=None,
                 full_source_weight: torch.Tensor | None = None):
        super().__init__(candidate_types=candidate_types, source_weight=source_weight, out_features=out_features,
                         in_features=in_features, imatrix=imatrix, device=device, lazy=lazy,
                         tensor_name=tensor_name, qbytes_device=qbytes_device, shard_spec=shard_spec,
                         full_source_weight=full_source_weight)
        if shard_spec is not None and getattr(shard_spec, "vocab_start", None) is not None:
            self.tp_vocab_start = shard_spec.vocab_start
            self.tp_vocab_end = shard_spec.vocab_start + out_features

    @classmethod
    def from_packed(cls, in_features: int, out_features: int, candidate_types: list[str],
                    qbytes: list[torch.Tensor], source_dtype: torch.dtype = torch.bfloat16,
                    tensor_name: str = "unknown", device=None) -> "MixedQuantLinear":
        """A gated Linear over existing candidate bytes (a candidate cache
        entry, another process's quantization, synthetic blocks)."""
        return cls._from_packed(candidate_types, qbytes, out_features, in_features, source_dtype, tensor_name,
                                device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.device.type != "cuda":
            raise RuntimeError(f"{self._tensor_name}: MixedQuantLinear runs on a ROCm device only (got {x.device})")
        self._move_qbytes(x.device)
        streamer = self.__dict__.get("_streamer")
        if streamer is not None:
            if _PTQR_STATE.enabled or self.__dict__.get("_gate_sink") is not None:
                raise RuntimeError(f"{self._tensor_name}: streamed candidates run without PTQR routing and "
                                   "without deferred gate gradients")
            streamer.forward_fence(self)
        pre = None if _PTQR_STATE.enabled or streamer is not None else MixPrefetch.take([self])
        probs = pre[1][0] if pre is not None else self.get_probs()
        if probs.device != x.device:
            probs = probs.to(x.device)
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype != torch.bfloat16:
            x2 = x2.to(torch.bfloat16)
        meta = (self._ggml_types(), self.out_features, self.padded_in_features)
        if _PTQR_STATE.enabled:
            routing = _sample_token_routing(probs.detach(), x2.shape[0])
            y = RoutedLinearFunction.apply(x2, probs, routing, meta, self._bf16_candidates(x.device),
                                           *self._qbytes())
        else:
            # with a sink the probabilities stay attached (so the backward runs
            # even when x needs no gradient); the backward returns None for them
            y = GatedLinearFunction.apply(x2, probs, meta, pre[0] if pre is not None else None,
                                          self.__dict__.get("_gate_sink"), *self._qbytes())
            if streamer is not None:
                y = streamer.fenced(y, self)
        if x.dtype != torch.bfloat16:
            y = y.to(x.dtype)
        out = y.reshape(*lead, self.out_features)
        spec = self.shard_spec
        if spec is not None and getattr(spec, "col_offset", None) is not None:
            raise NotImplementedError("row-parallel (column-sharded) gated Linear needs the TP all-reduce")
        return out

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"candidates={self.candidate_types}, source={self.candidate_source}")


class MixedQuantEmbedding(_MixedQuantBase):
    """Embedding whose weight is a softmax mixture of K packed candidates
    (reference ``layers.py:1743-1842``): the weight is the [num_embeddings,
    embedding_dim] matrix, padded along embedding_dim to a multiple of 256.

    Every lookup takes the reference's row-select route (``layers.py:1805-1828``),
    decoding only the looked-up rows of the candidates.  Under PTQR the batch's
    unique ids are looked up once, each taking one candidate sampled per row as
    there, and the rows are scattered back to the positions; without it every
    position decodes its own row (a repeated id gives the same row, and its
    gate-gradient terms add up as the reference's scattered rows do), so no
    sort and no host round trip is needed.  Rows come in fp32 when the source
    weight is fp32 (the mixture before the reference's final cast, and exact
    candidate values when routed) and as bf16 otherwise (then cast to the
    source dtype).

    ``id_check`` ("sync", the default, or "deferred"): when out-of-range ids
    raise IndexError (:func:`check_embedding_ids`)."""

    id_check = "sync"

    def __init__(self, num_embeddings: int, embedding_dim: int, candidate_types: list[str],
                 source_weight: torch.Tensor, imatrix: torch.Tensor | None = None, device=None, lazy: bool = False,
                 tensor_name: str = "unknown", qbytes_device=None, shard_spec=None,
                 full_source_weight: torch.Tensor | None = None):
        super().__init__(candidate_types=candidate_types, source_weight=source_weight, out_features=num_embeddings,
                         in_features=embedding_dim, imatrix=imatrix, device=device, lazy=lazy,
                         tensor_name=tensor_name, qbytes_device=qbytes_device, shard_spec=shard_spec,
                         full_source_weight=full_source_weight)
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        if shard_spec is not None and getattr(shard_spec, "vocab_start", None) is not None:
            self.tp_vocab_start = shard_spec.vocab_start
            self.tp_vocab_end = shard_spec.vocab_start + num_embeddings

    @classmethod
    def from_packed(cls, num_embeddings: int, embedding_dim: int, candidate_types: list[str],
                    qbytes: list[torch.Tensor], source_dtype: torch.dtype = torch.bfloat16,
                    tensor_name: str = "unknown", device=None) -> "MixedQuantEmbedding":
        """A gated embedding over existing candidate bytes."""
        obj = cls._from_packed(candidate_types, qbytes, num_embeddings, embedding_dim, source_dtype, tensor_name,
                               device)
        obj.num_embeddings = num_embeddings
        obj.embedding_dim = embedding_dim
        return obj

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        spec = self.shard_spec
        if spec is not None and getattr(spec, "vocab_start", None) is not None:
            raise NotImplementedError("vocab-parallel gated embedding needs the TP all-reduce")
        return self._embedding_lookup(input)

    def _row_dtype(self) -> torch.dtype:
        return torch.float32 if self.source_dtype == torch.float32 else torch.bfloat16

    def _embedding_lookup(self, input: torch.Tensor) -> torch.Tensor:
        if input.device.type != "cuda":
            raise RuntimeError(f"{self._tensor_name}: MixedQuantEmbedding runs on a ROCm device only "
                               f"(got {input.device})")
        dev = input.device
        self._move_qbytes(dev)
        ids = input.reshape(-1).to(torch.int64)
        if _PTQR_STATE.enabled:
            # one routing draw per distinct id, as the reference's lookup
            rows, inverse = torch.unique(ids, return_inverse=True)
        else:
            rows, inverse = ids.contiguous(), None
        check_embedding_ids(rows, self.num_embeddings, self._tensor_name, self.id_check)
        probs = self.get_probs()
        if probs.device != dev:
            probs = probs.to(dev)
        routing = _sample_token_routing(probs.detach(), rows.numel()) if _PTQR_STATE.enabled else None
        dim8 = (self.embedding_dim + 7) // 8 * 8  # the kernels store whole 8-weight runs
        meta = (self._ggml_types(), self.num_embeddings, dim8, self.padded_in_features, self._row_dtype())
        row_vals = EmbeddingRowsFunction.apply(probs, routing, rows, meta, *self._qbytes())
        if dim8 != self.embedding_dim:
            row_vals = row_vals[:, : self.embedding_dim]
        if inverse is not None:
            row_vals = row_vals[inverse]
        out = row_vals.reshape(*input.shape, self.embedding_dim)
        return out if out.dtype == self.source_dtype else out.to(self.source_dtype)

    def extra_repr(self) -> str:
        return (f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}, "
                f"candidates={self.candidate_types}, source={self.candidate_source}")


# ---------------------------------------------------------------------------
# module walkers (reference layers.py:1845-2160)
# ---------------------------------------------------------------------------
DEFAULT_ATTENTION_SEGMENTS: frozenset = frozenset({"self_attn", "linear_attn", "attn", "conv", "shortconv"})
_ATTENTION_SEGMENTS: frozenset = DEFAULT_ATTENTION_SEGMENTS


def resolve_candidate_types(tensor_name: str, base_candidates: list[str],
                            attention_candidates: list[str] | None = None,
                            non_attention_candidates: list[str] | None = None) -> list[str]:
    if attention_candidates is None and non_attention_candidates is None:
        return list(base_candidates)
    is_attn = any(seg in _ATTENTION_SEGMENTS for seg in tensor_name.split("."))
    group = attention_candidates if (is_attn and attention_candidates) else non_attention_candidates
    if not group:
        return list(base_candidates)
    base = set(base_candidates)
    return [qt for qt in group if qt in base]


def _count_selectable_linears(module: nn.Module, target_names: Optional[set[str]], skip_names: set[str]) -> int:
    total = 0
    for name, child in module.named_children():
        if name in skip_names:
            continue
        if isinstance(child, nn.Linear):
            if target_names is None or name in target_names:
                total += 1
        else:
            total += _count_selectable_linears(child, target_names, skip_names)
    return total


def replace_linear_with_mixed_quant(module: nn.Module, candidate_types: list[str] | None, prefix: str = "",
                                    target_names: Optional[set[str]] = None,
                                    skip_names: Optional[set[str]] = None,
                                    imatrix_dict: Optional[dict[str, torch.Tensor]] = None, device=None,
                                    lazy: bool = False, attention_candidates: Optional[list[str]] = None,
                                    non_attention_candidates: Optional[list[str]] = None,
                                    qbytes_device=None) -> dict[str, _MixedQuantBase]:
    """Recursively replace nn.Linear children with MixedQuantLinear; returns
    {full_name: module}.  Same arguments as the reference (``layers.py:1908-1920``)."""
    if candidate_types is None:
        candidate_types = list(HIP_TYPES)
    skip_names = skip_names or set()
    imatrix_dict = imatrix_dict or {}
    if prefix == "":
        total = _count_selectable_linears(module, target_names, skip_names)
        replace_linear_with_mixed_quant._mq_counter = 0
        replace_linear_with_mixed_quant._mq_start = time.monotonic()
        print(f"Preparing {total} selectable layers x {len(candidate_types)} candidates ...", flush=True)
    replaced: dict[str, _MixedQuantBase] = {}
    for name, child in list(module.named_children()):
        full_name = f"{prefix}.{name}" if prefix else name
        if name in skip_names:
            continue
        if isinstance(child, nn.Linear):
            if child.bias is not None:
                raise NotImplementedError(f"MixedQuantLinear does not support bias but {full_name} has one")
            if target_names is not None and name not in target_names:
                continue
            imatrix = imatrix_dict.get(full_name)
            if imatrix is None:
                imatrix = imatrix_dict.get(full_name + ".weight")
            new_child = MixedQuantLinear(
                in_features=child.in_features, out_features=child.out_features,
                candidate_types=resolve_candidate_types(full_name, candidate_types, attention_candidates,
                                                        non_attention_candidates),
                source_weight=child.weight.data, imatrix=imatrix, device=device, lazy=lazy, tensor_name=full_name,
                qbytes_device=qbytes_device, shard_spec=getattr(child, "tp_shard_spec", None),
                full_source_weight=getattr(child, "tp_full_weight", None))
            setattr(module, name, new_child)
            replaced[full_name] = new_child
            replace_linear_with_mixed_quant._mq_counter = getattr(replace_linear_with_mixed_quant, "_mq_counter", 0) + 1
        else:
            replaced.update(replace_linear_with_mixed_quant(
                child, candidate_types=candidate_types, prefix=full_name, target_names=target_names,
                skip_names=skip_names, imatrix_dict=imatrix_dict, device=device, lazy=lazy,
                attention_candidates=attention_candidates, non_attention_candidates=non_attention_candidates,
                qbytes_device=qbytes_device))
    return replaced


def replace_embedding_with_mixed_quant(module: nn.Module, candidate_types: list[str] | None, prefix: str = "",
                                       skip_names: Optional[set[str]] = None,
                                       imatrix_dict: Optional[dict[str, torch.Tensor]] = None, device=None,
                                       lazy: bool = False, qbytes_device=None,
                                       attention_candidates: Optional[list[str]] = None,
                                       non_attention_candidates: Optional[list[str]] = None
                                       ) -> dict[str, MixedQuantEmbedding]:
    """Replace every selected ``nn.Embedding`` below ``module`` by a
    :class:`MixedQuantEmbedding` (reference ``layers.py:2085-2153``)."""
    if candidate_types is None:
        candidate_types = list(HIP_TYPES)
    skip_names = set() if skip_names is None else skip_names
    imatrix_dict = {} if imatrix_dict is None else imatrix_dict
    replaced: dict[str, MixedQuantEmbedding] = {}
    for name, child in list(module.named_children()):
        full_name = f"{prefix}.{name}" if prefix else name
        if name in skip_names:
            continue
        if isinstance(child, nn.Embedding):
            imatrix = imatrix_dict.get(full_name)
            if imatrix is None:
                imatrix = imatrix_dict.get(full_name + ".weight")
            types = resolve_candidate_types(full_name, candidate_types, attention_candidates,
                                            non_attention_candidates)
            new = MixedQuantEmbedding(child.num_embeddings, child.embedding_dim, types, child.weight.data,
                                      imatrix=imatrix, device=device, lazy=lazy, tensor_name=full_name,
                                      qbytes_device=qbytes_device,
                                      shard_spec=getattr(child, "tp_shard_spec", None),
                                      full_source_weight=getattr(child, "tp_full_weight", None))
            setattr(module, name, new)
            replaced[full_name] = new
            print(f"  MixedQuantEmbedding init: {full_name} replaced", flush=True)
        else:
            replaced.update(replace_embedding_with_mixed_quant(
                child, candidate_types, prefix=full_name, skip_names=skip_names, imatrix_dict=imatrix_dict,
                device=device, lazy=lazy, qbytes_device=qbytes_device, attention_candidates=attention_candidates,
                non_attention_candidates=non_attention_candidates))
    return replaced


_BYTES_TABLES: dict[tuple, torch.Tensor] = {}


def total_effective_bytes(replaced: dict[str, _MixedQuantBase]) -> torch.Tensor:
    """sum over layers of effective_bytes() (reference ``layers.py:2156-2160``).

    Layers with the same candidate count, device and temperature are batched:
    one stack of their gates, one softmax and one weighted sum, instead of a
    handful of tiny launches per layer."""
    groups: dict[tuple, list[_MixedQuantBase]] = {}
    for layer in replaced.values():
        key = (layer.num_candidates, layer.gates.device, float(layer.temperature))
        groups.setdefault(key, []).append(layer)
    total = torch.tensor(0.0)
    for (_, dev, temp), mods in groups.items():
        tkey = (dev, tuple((id(m), tuple(m._bytes_per_candidate())) for m in mods))
        coef = _BYTES_TABLES.get(tkey)
        if coef is None:
            if len(_BYTES_TABLES) > 64:
                _BYTES_TABLES.clear()
            coef = torch.tensor([m._bytes_per_candidate() for m in mods], dtype=torch.float32).to(dev)
            _BYTES_TABLES[tkey] = coef
        probs = F.softmax(torch.stack([m.gates for m in mods]) / temp, dim=1)
        total = total + (probs * coef).sum()
    return total
