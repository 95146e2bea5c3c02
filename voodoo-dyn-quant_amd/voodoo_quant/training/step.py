"""Gate-training step of a decoder whose Linears and embedding are gated.

The step the reference's trainer runs per batch (``trainer.py:2498-2616``),
on a Llama/Qwen-style decoder (RMSNorm, RoPE, grouped-query attention,
SwiGLU MLP, tied embeddings):

* the student's seven Linears per layer are :class:`MixedQuantLinear` and its
  embedding a :class:`MixedQuantEmbedding`; with tied embeddings the student's
  lm_head stays a plain Linear over the source embedding weight, as in the
  reference (``trainer.py:2098-2101``);
* the teacher is the same architecture over Q8_0 bytes
  (:class:`Q8Linear`/:class:`Q8Embedding`, its tied lm_head a Q8Linear over the
  embedding's bytes) and runs without gradients;
* loss = CE + distill_weight * KL(teacher || student) + size_weight *
  dead-zone size penalty, backward, global clip 1.0, AdamW + cosine step on
  the gates only (every other weight is frozen), temperature annealed per step.

Only the gates train, so the backward runs dX through every layer and the
gate gradients of every gated tensor; no weight gradient is formed.  Causal
attention at head dim 64 runs ``vq_attention_fwd`` / ``vq_attention_bwd``,
fused with the rotary embedding into one autograd node that keeps K/V at
their own heads (the kernels read K/V head h / (Hq/Hkv)); other head dims use
torch's fused
scaled-dot-product kernels (flash or memory-efficient), and without one of
them the math path in fp32.
"""

from __future__ import annotations

import math
import warnings
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F

from voodoo_quant import _hip, layers
from voodoo_quant.ggml import get_quant_info
from voodoo_quant.training import trainer
from voodoo_quant.training.q8_teacher import Q8Embedding, Q8Linear, q8_linear_group, set_keep_decoded


@dataclass
class DecoderConfig:
    layers: int = 24
    hidden: int = 1024
    heads: int = 16
    kv_heads: int = 4
    head_dim: int = 64
    mlp: int = 3072
    vocab: int = 151936
    rope_theta: float = 1.0e6
    eps: float = 1.0e-6

    def linear_shapes(self) -> dict[str, tuple[int, int]]:
        """{name: (out_features, in_features)} of one layer's Linears."""
        h, q, kv, m = self.hidden, self.heads * self.head_dim, self.kv_heads * self.head_dim, self.mlp
        return {"self_attn.q_proj": (q, h), "self_attn.k_proj": (kv, h), "self_attn.v_proj": (kv, h),
                "self_attn.o_proj": (h, q), "mlp.gate_proj": (m, h), "mlp.up_proj": (m, h),
                "mlp.down_proj": (h, m)}

    def gated_weights(self) -> int:
        per_layer = sum(o * i for o, i in self.linear_shapes().values())
        return self.layers * per_layer + self.vocab * self.hidden  # tied: the embedding counted once


def _rope(s: int, head_dim: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    ang = torch.outer(torch.arange(s, dtype=torch.float32, device=device), inv)
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)


def _apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rot * sin


_SDPA_FUSED: bool | None = None
# head dim 64 on the GPU: causal attention on vq_attention_fwd / _bwd
HIP_ATTENTION = True
# False: the backward is torch's memory-efficient attention backward over the
# HIP forward's output and log-sum-exp (the kernel SDPA's own backward runs)
HIP_ATTENTION_BWD = True
# rotary embedding and HIP attention as one autograd node with K/V at their
# own heads (False: the rotary kernel writes each K/V head once per query head)
ROPE_ATTENTION = True


class _CausalAttention(torch.autograd.Function):
    """Causal attention with Hq == Hk: forward ``vq_attention_fwd`` (it saves
    the natural-log log-sum-exp per query); backward ``vq_attention_bwd``, or
    torch's ``aten::_scaled_dot_product_efficient_attention_backward``, which
    reads that log-sum-exp as SDPA's forward leaves it."""

    @staticmethod
    def forward(ctx, q, k, v):
        out, lse = _hip.attention_fwd(q, k, v, need_lse=True)
        ctx.save_for_backward(q, k, v, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        if HIP_ATTENTION_BWD:
            return _hip.attention_bwd(dout, q, k, v, out, lse)
        return _torch_attention_bwd(dout, q, k, v, out, lse)


def _torch_attention_bwd(dout, q, k, v, out, lse):
    """torch's memory-efficient attention backward (Hq == Hk) over the HIP
    forward's output and log-sum-exp."""
    zero = torch.zeros((), dtype=torch.int64)  # philox seed/offset: unused without dropout
    dq, dk, dv, _ = torch.ops.aten._scaled_dot_product_efficient_attention_backward(
        dout, q, k, v, None, out, lse, zero, zero, 0.0, [True, True, True, False], True,
        scale=1.0 / math.sqrt(q.shape[-1]))
    return dq, dk, dv


def _attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Causal attention, q [B, Hq, S, d], k/v [B, Hkv, S, d] (KV heads repeated)."""
    global _SDPA_FUSED
    rep = q.shape[1] // k.shape[1]
    if rep > 1:
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    if HIP_ATTENTION and q.is_cuda and q.dtype == torch.bfloat16 and q.shape[-1] == 64:
        if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
            return _CausalAttention.apply(q, k, v)
        return _hip.attention_fwd(q, k, v, need_lse=False)[0]
    from torch.nn.attention import SDPBackend, sdpa_kernel

    if _SDPA_FUSED is not False:
        try:
            # the memory-efficient backend first: on MI355X (torch 2.10, ROCm 7)
            # its backward is one fused kernel, 306 against 525 us for the
            # flash backend's at B 4, 16 heads, S 2048, d 64 (same forward
            # kernel, same error against fp32)
            with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION], set_priority=True):
                out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            _SDPA_FUSED = True
            return out
        except RuntimeError as e:
            if _SDPA_FUSED:
                raise
            warnings.warn(f"no fused attention kernel ({e}); using the fp32 math path")
            _SDPA_FUSED = False
    with sdpa_kernel([SDPBackend.MATH]):
        out = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
    return out.to(q.dtype)


GROUP_PROJECTIONS = True  # stack the projections that read one input into one product
FUSED_GLUE = True         # rotary embedding / SwiGLU on the stacked outputs in one kernel each


def _project(x: torch.Tensor, mods: list[nn.Module]) -> list[torch.Tensor]:
    if GROUP_PROJECTIONS and all(isinstance(m, layers.MixedQuantLinear) for m in mods):
        return layers.gated_linear_group(x, mods)
    if GROUP_PROJECTIONS and all(isinstance(m, Q8Linear) for m in mods):
        return q8_linear_group(x, mods)
    return [m(x) for m in mods]


def _project_stacked(x: torch.Tensor, mods: list[nn.Module]) -> torch.Tensor | None:
    """The stacked output [tokens, sum out] of projections that read x, or None."""
    if not (GROUP_PROJECTIONS and FUSED_GLUE and x.is_cuda):
        return None
    if all(isinstance(m, layers.MixedQuantLinear) for m in mods):
        return layers.gated_linear_group(x, mods, stacked=True)
    if all(isinstance(m, Q8Linear) for m in mods):
        return q8_linear_group(x, mods, stacked=True)
    return None


class _RopeQKV(torch.autograd.Function):
    """Stacked q/k/v projection output -> (q, k, v) as [B, Hq, S, D] views of
    [B, S, Hq, D] memory: rotary embedding on q and k, K/V heads repeated for
    grouped-query attention (``vq_rope_qkv_fwd/bwd``)."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, shape):
        b, s_, hq, hkv, d = shape
        q, k, v = _hip.rope_qkv_fwd(qkv.contiguous(), b, s_, hq, hkv, d, cos, sin)
        ctx.save_for_backward(cos, sin)
        ctx.shape = shape
        return tuple(t.view(b, s_, hq, d).transpose(1, 2) for t in (q, k, v))

    @staticmethod
    def backward(ctx, dq, dk, dv):
        cos, sin = ctx.saved_tensors
        b, s_, hq, hkv, d = ctx.shape
        zeros = None
        grads = []
        for g in (dq, dk, dv):
            if g is None:
                zeros = zeros if zeros is not None else torch.zeros(b, hq, s_, d, dtype=torch.bfloat16, device=cos.device)
                g = zeros
            grads.append(g.to(torch.bfloat16))
        return _hip.rope_qkv_bwd(*grads, b, s_, hq, hkv, d, cos, sin), None, None, None


class _RopeCausalAttention(torch.autograd.Function):
    """Rotary embedding of the stacked q/k/v projection output and causal
    attention over it as one autograd node, with K and V kept at their Hkv
    heads: ``vq_rope_qkv_fwd`` writes them unrepeated, ``vq_attention_fwd`` /
    ``_bwd`` read K/V head h / (Hq / Hkv) for query head h, and the backward's
    per-query-head dK/dV go straight into ``vq_rope_qkv_bwd``, which sums each
    group.  Bitwise the same as :class:`_RopeQKV` (heads repeated) followed by
    :class:`_CausalAttention`, without writing the repeated heads."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, shape):
        b, s_, hq, hkv, d = shape
        q, k, v = _hip.rope_qkv_fwd(qkv.contiguous(), b, s_, hq, hkv, d, cos, sin, repeat_kv=False)
        q = q.view(b, s_, hq, d).transpose(1, 2)
        k = k.view(b, s_, hkv, d).transpose(1, 2)
        v = v.view(b, s_, hkv, d).transpose(1, 2)
        out, lse = _hip.attention_fwd(q, k, v, need_lse=True)
        ctx.save_for_backward(q, k, v, out, lse, cos, sin)
        ctx.shape = shape
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, cos, sin = ctx.saved_tensors
        b, s_, hq, hkv, d = ctx.shape
        dout = dout.to(torch.bfloat16)
        if HIP_ATTENTION_BWD:
            dq, dk, dv = _hip.attention_bwd(dout, q, k, v, out, lse)
        else:  # torch's backward reads one K/V head per query head
            rep = hq // hkv
            grads = _torch_attention_bwd(dout, q, k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1),
                                         out, lse)
            # the rotary backward reads the three with one set of strides
            dq, dk, dv = (g.transpose(1, 2).contiguous().transpose(1, 2) for g in grads)
        return _hip.rope_qkv_bwd(dq, dk, dv, b, s_, hq, hkv, d, cos, sin), None, None, None


def _rope_attention(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, shape: tuple) -> torch.Tensor:
    """Causal attention [B, Hq, S, D] over the rotary-embedded stacked
    projection output qkv [B*S, (Hq + 2 Hkv) D] (HIP kernels, head dim 64),
    K/V at their Hkv heads; without a backward the log-sum-exp is not kept."""
    if torch.is_grad_enabled() and qkv.requires_grad:
        return _RopeCausalAttention.apply(qkv, cos, sin, shape)
    b, s_, hq, hkv, d = shape
    q, k, v = _hip.rope_qkv_fwd(qkv.contiguous(), b, s_, hq, hkv, d, cos, sin, repeat_kv=False)
    return _hip.attention_fwd(q.view(b, s_, hq, d).transpose(1, 2), k.view(b, s_, hkv, d).transpose(1, 2),
                              v.view(b, s_, hkv, d).transpose(1, 2), need_lse=False)[0]


class _SwiGLU(torch.autograd.Function):
    """silu(gate) * up from the stacked gate/up output [tokens, 2F] (``vq_swiglu_fwd/bwd``)."""

    @staticmethod
    def forward(ctx, gu):
        gu = gu.contiguous()
        ctx.save_for_backward(gu)
        return _hip.swiglu_fwd(gu)

    @staticmethod
    def backward(ctx, dy):
        (gu,) = ctx.saved_tensors
        return _hip.swiglu_bwd(gu, dy.to(torch.bfloat16).contiguous())


_ROPE_F32: dict[tuple, tuple[torch.Tensor, torch.Tensor]] = {}


def _rope_tables_f32(s: int, head_dim: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    key = (s, head_dim, theta, str(device))
    t = _ROPE_F32.get(key)
    if t is None:
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64, device=device) / head_dim))
        ang = torch.outer(torch.arange(s, dtype=torch.float64, device=device), inv)
        ang = torch.cat([ang, ang], dim=-1)
        t = (ang.cos().float().contiguous(), ang.sin().float().contiguous())
        _ROPE_F32[key] = t
    return t


class _AddRMSNorm(torch.autograd.Function):
    """(s, n) = (h + a, rms_norm(h + a) * w) in one HIP pass
    (``vq_add_rmsnorm_fwd``; a may be None for a plain RMSNorm, then s is h);
    the backward returns one gradient for both h and a.  The norm weight is
    frozen (the trainer trains gates only)."""

    @staticmethod
    def forward(ctx, h, a, w, eps):
        shape = h.shape
        h2 = h.reshape(-1, shape[-1])
        a2 = a.reshape(-1, shape[-1]) if a is not None else None
        # (grad mode is off inside forward; needs_input_grad says whether a
        # backward can come)
        s, n, rstd = _hip.add_rmsnorm_fwd(h2, a2, w, eps, need_backward=any(ctx.needs_input_grad[:2]))
        if s is None:
            s = h2
        ctx.save_for_backward(s, w, rstd)
        ctx.has_a = a is not None
        ctx.shape = shape
        return s.view(shape), n.view(shape)

    @staticmethod
    def backward(ctx, ds, dn):
        s, w, rstd = ctx.saved_tensors
        dim = ctx.shape[-1]
        ds2 = ds.reshape(-1, dim).contiguous() if ds is not None else None
        if dn is None:
            dh = ds2
        else:
            dh = _hip.rmsnorm_bwd(dn.reshape(-1, dim).contiguous(), ds2, s, w, rstd)
        dh = dh.view(ctx.shape) if dh is not None else None
        return dh, (dh if ctx.has_a else None), None, None


def _fused_norms(h: torch.Tensor, w) -> bool:
    return (FUSED_GLUE and h.is_cuda and h.dtype == torch.bfloat16 and h.shape[-1] % 8 == 0
            and not w.requires_grad)


class _Attention(nn.Module):
    def __init__(self, cfg: DecoderConfig, lin: dict[str, nn.Module]):
        super().__init__()
        self.cfg = cfg
        self.q_proj, self.k_proj = lin["self_attn.q_proj"], lin["self_attn.k_proj"]
        self.v_proj, self.o_proj = lin["self_attn.v_proj"], lin["self_attn.o_proj"]

    def forward(self, x, cos, sin):
        b, s, _ = x.shape
        c = self.cfg
        qkv = _project_stacked(x, [self.q_proj, self.k_proj, self.v_proj])
        if qkv is not None and c.head_dim % 16 == 0:
            cos32, sin32 = _rope_tables_f32(s, c.head_dim, c.rope_theta, x.device)
            shape = (b, s, c.heads, c.kv_heads, c.head_dim)
            if HIP_ATTENTION and ROPE_ATTENTION and qkv.dtype == torch.bfloat16 and c.head_dim == 64:
                a = _rope_attention(qkv.reshape(b * s, -1), cos32, sin32, shape)
                return self.o_proj(a.transpose(1, 2).reshape(b, s, c.heads * c.head_dim))
            q, k, v = _RopeQKV.apply(qkv.reshape(b * s, -1), cos32, sin32, shape)
        else:
            q, k, v = _project(x, [self.q_proj, self.k_proj, self.v_proj])
            q = q.view(b, s, c.heads, c.head_dim).transpose(1, 2)
            k = k.view(b, s, c.kv_heads, c.head_dim).transpose(1, 2)
            v = v.view(b, s, c.kv_heads, c.head_dim).transpose(1, 2)
            q, k = _apply_rope(q, cos, sin), _apply_rope(k, cos, sin)
        a = _attention(q, k, v).transpose(1, 2).reshape(b, s, c.heads * c.head_dim)
        return self.o_proj(a)


class _MLP(nn.Module):
    def __init__(self, lin: dict[str, nn.Module]):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = lin["mlp.gate_proj"], lin["mlp.up_proj"], lin["mlp.down_proj"]

    def forward(self, x):
        gu = _project_stacked(x, [self.gate_proj, self.up_proj])
        if gu is not None and gu.shape[-1] % 16 == 0:
            h = _SwiGLU.apply(gu.reshape(-1, gu.shape[-1])).view(*x.shape[:-1], gu.shape[-1] // 2)
        else:
            g, u = _project(x, [self.gate_proj, self.up_proj])
            h = F.silu(g) * u
        return self.down_proj(h)


class _Layer(nn.Module):
    def __init__(self, cfg: DecoderConfig, lin: dict[str, nn.Module], device):
        super().__init__()
        self.eps = cfg.eps
        self.self_attn = _Attention(cfg, lin)
        self.mlp = _MLP(lin)
        self.input_layernorm = nn.Parameter(torch.ones(cfg.hidden, dtype=torch.bfloat16, device=device),
                                            requires_grad=False)
        self.post_attention_layernorm = nn.Parameter(torch.ones(cfg.hidden, dtype=torch.bfloat16, device=device),
                                                     requires_grad=False)

    def forward(self, h, cos, sin):
        h = h + self.self_attn(F.rms_norm(h, (h.shape[-1],), self.input_layernorm, self.eps), cos, sin)
        return h + self.mlp(F.rms_norm(h, (h.shape[-1],), self.post_attention_layernorm, self.eps))


class _Body(nn.Module):
    def __init__(self, cfg: DecoderConfig, embed: nn.Module, layer_linears: list[dict[str, nn.Module]], device):
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = embed
        self.layers = nn.ModuleList([_Layer(cfg, lin, device) for lin in layer_linears])
        self.norm = nn.Parameter(torch.ones(cfg.hidden, dtype=torch.bfloat16, device=device), requires_grad=False)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        h = self.embed_tokens(input_ids).to(torch.bfloat16)
        cos, sin = _rope(input_ids.shape[1], self.cfg.head_dim, self.cfg.rope_theta, input_ids.device)
        if not _fused_norms(h, self.norm):
            for layer in self.layers:
                h = layer(h, cos, sin)
            return F.rms_norm(h, (h.shape[-1],), self.norm, self.cfg.eps)
        # each residual add runs fused with the RMSNorm that reads its result:
        # the attention add with the post-attention norm, the MLP add with the
        # next layer's input norm (the final norm after the last layer)
        eps = self.cfg.eps
        layers_ = list(self.layers)
        first = layers_[0].input_layernorm if layers_ else self.norm
        h = h.contiguous()
        _, n = _AddRMSNorm.apply(h, None, first, eps)
        for i, layer in enumerate(layers_):
            a = layer.self_attn(n, cos, sin)
            h, n = _AddRMSNorm.apply(h, a, layer.post_attention_layernorm, eps)
            m = layer.mlp(n)
            w_next = layers_[i + 1].input_layernorm if i + 1 < len(layers_) else self.norm
            h, n = _AddRMSNorm.apply(h, m, w_next, eps)
        return n


class Decoder(nn.Module):
    """``model`` (the text stack, returning final hidden states) + ``lm_head``."""

    def __init__(self, body: _Body, lm_head: nn.Module):
        super().__init__()
        self.model = body
        self.lm_head = lm_head

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.model(input_ids))


class _TiedHead(nn.Module):
    """Plain Linear over the (frozen) source embedding weight."""

    def __init__(self, weight: torch.Tensor):
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)

    def forward(self, h):
        return F.linear(h, self.weight)


# Smallest fp16 scale of the synthetic blocks, per format (scales are drawn
# from [base, 2 base)), chosen so that decoded weights stay within about
# +-0.2 (standard deviations 0.02-0.06).
_SYNTH_SCALE_BASE = {"Q8_0": 2.0 ** -11, "Q6_K": 2.0 ** -16, "Q5_K": 2.0 ** -15, "Q4_K": 2.0 ** -14,
                     "Q3_K": 2.0 ** -11, "Q2_K": 2.0 ** -9, "IQ1_S": 2.0 ** -8, "IQ1_M": 2.0 ** -8,
                     "IQ2_XXS": 2.0 ** -11, "IQ2_XS": 2.0 ** -11, "IQ2_S": 2.0 ** -11, "IQ3_XXS": 2.0 ** -13,
                     "IQ3_S": 2.0 ** -13, "IQ4_XS": 2.0 ** -16}
# fp16 scale fields; IQ1_M has none (its scale is spread over the top nibbles
# of bytes 49, 51, 53 and 55)
_F16_FIELDS = {"Q8_0": (0,), "Q2_K": (80, 82), "Q3_K": (108,), "Q4_K": (0, 2), "Q5_K": (0, 2), "Q6_K": (208,),
               "IQ1_S": (0,), "IQ1_M": (None,), "IQ2_XXS": (0,), "IQ2_XS": (0,), "IQ2_S": (0,), "IQ3_XXS": (0,),
               "IQ3_S": (0,), "IQ4_XS": (0,)}
# dmin / d of the formats with mins: the mean code, so weights centre on 0
_SYNTH_MIN_RATIO = {"Q2_K": 1.5, "Q4_K": 7.5, "Q5_K": 15.5}


def synthetic_candidate_bytes(qt: str, rows: int, cols: int, device, gen: torch.Generator) -> torch.Tensor:
    """Random valid blocks of an [rows, cols rounded up to 256] tensor,
    generated on `device`: random payload bytes and fp16 scale fields drawn
    uniformly from [base, 2 base) with a per-format base (normal or subnormal
    fp16, never inf or NaN)."""
    info = get_quant_info(qt)
    d_pad = (cols + 255) // 256 * 256
    nblocks = rows * d_pad // info.block_size
    q = torch.randint(0, 256, (nblocks, info.block_bytes), dtype=torch.uint8, device=device, generator=gen)
    for i, off in enumerate(_F16_FIELDS[qt]):
        base = _SYNTH_SCALE_BASE[qt] * (_SYNTH_MIN_RATIO[qt] if i == 1 else 1.0)
        d = base * (1.0 + torch.rand(nblocks, device=device, generator=gen))
        h = d.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
        if off is None:
            for t in range(4):
                b = q[:, 49 + 2 * t].to(torch.int32)
                q[:, 49 + 2 * t] = ((b & 0x0F) | (((h >> (4 * t)) & 0xF) << 4)).to(torch.uint8)
            continue
        q[:, off] = (h & 0xFF).to(torch.uint8)
        q[:, off + 1] = (h >> 8).to(torch.uint8)
    return q.reshape(-1)


def build_models(cfg: DecoderConfig, types: list[str], device, seed: int = 0, packed: bool = True):
    """(student, teacher, replaced): the gated student, the Q8_0 teacher and
    {tensor name: gated module}.

    packed=True takes candidates and teacher bytes from
    :func:`synthetic_candidate_bytes` (no quantization: the way to build a
    vocabulary-scale model in seconds); packed=False draws N(0, 0.02) source
    weights and quantizes them through the module constructors (the
    reference's path; CPU-bound, for small configurations)."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed)
    replaced: dict[str, nn.Module] = {}

    def gated_linear(name, out_f, in_f):
        if packed:
            qbs = [synthetic_candidate_bytes(qt, out_f, in_f, device, gen) for qt in types]
            mod = layers.MixedQuantLinear.from_packed(in_f, out_f, types, qbs, tensor_name=name, device=device)
        else:
            w = torch.randn(out_f, in_f, generator=cpu_gen) * 0.02
            mod = layers.MixedQuantLinear(in_f, out_f, types, w.to(torch.bfloat16), tensor_name=name,
                                          device=device).to(device)
        replaced[name] = mod
        return mod

    def teacher_linear(out_f, in_f):
        return Q8Linear(synthetic_candidate_bytes("Q8_0", out_f, in_f, device, gen), out_f, in_f)

    shapes = cfg.linear_shapes()
    s_layers, t_layers = [], []
    for li in range(cfg.layers):
        s_layers.append({n: gated_linear(f"model.layers.{li}.{n}", o, i) for n, (o, i) in shapes.items()})
        t_layers.append({n: teacher_linear(o, i) for n, (o, i) in shapes.items()})

    v, h = cfg.vocab, cfg.hidden
    src = (torch.randn(v, h, device=device, generator=gen) * 0.02).to(torch.bfloat16)
    if packed:
        qbs = [synthetic_candidate_bytes(qt, v, h, device, gen) for qt in types]
        emb = layers.MixedQuantEmbedding.from_packed(v, h, types, qbs, tensor_name="model.embed_tokens",
                                                     device=device)
    else:
        emb = layers.MixedQuantEmbedding(v, h, types, src.cpu(), tensor_name="model.embed_tokens",
                                         device=device).to(device)
    replaced["model.embed_tokens"] = emb
    student = Decoder(_Body(cfg, emb, s_layers, device), _TiedHead(src))

    set_keep_decoded(True)  # the teacher's weights never change: decode them once
    t_bytes = synthetic_candidate_bytes("Q8_0", v, h, device, gen)
    t_emb = Q8Embedding(t_bytes, v, h)
    teacher = Decoder(_Body(cfg, t_emb, t_layers, device), Q8Linear(t_bytes, v, h))
    teacher.requires_grad_(False)
    return student, teacher, replaced


@dataclass
class StepConfig:
    max_steps: int = 200
    lr: float = 0.05
    temp_start: float = 1.0
    temp_end: float = 0.1
    distill_weight: float = 1.0
    distill_temperature: float = 1.0
    size_weight: float = 10.0
    size_tolerance: float = 0.02
    target_fraction: float = 0.45   # of 8-bit bytes
    logits_chunk: int = 0
    fused_loss: bool = True         # CE + KL on the HIP kernels (full-logits path)
    gate_bank: bool = True          # one softmax launch for all gates (trainer.GateBank)
    # mix each W_eff a few products ahead on a second stream (layers.MixPrefetch).
    # Off by default: measured on MI355X the mixes then overlap the GEMMs
    # (1.4 ms of 2.1 ms per 0.8B step) but share their CUs, and the step time
    # does not move (60.8 ms both ways; stress step 157 ms both ways)
    prefetch_mix: bool = False
    # run the teacher's forward on a second stream (default priority) beside
    # the student's forward, fenced by events (_forwards); the step's values
    # do not change.  Measured on MI355X: the 0.8B-class decoder step 58.3 ->
    # 57.7 ms (its small products and attention leave room on the chip), the
    # SwiGLU stress stack 155.5 -> 156.9 ms (its teacher's 4096 x 14336
    # products fill the chip alone), so it is left to the caller
    teacher_stream: bool = False
    # finish the gated Linears' gate gradients on a second stream and apply
    # the softmax Jacobian once per bank after the backward (trainer.GateBank)
    defer_gate_grads: bool = False
    # keep the gated products' packed candidates in pinned host memory and
    # copy them into `stream_slots` device slots ahead of use
    # (streaming.CandidateStreamer): `stream_depth` products ahead on a copy
    # stream when stream_overlap, else in stream order before each product
    # (the reference's host -> device pattern).  For models whose candidates
    # do not fit in HBM; resident candidates need no copies at all.  Measured
    # on MI355X, the SwiGLU stress stack (16 products, 9.7 GB of copies per
    # step at 57 GB/s): in stream order 338 ms per step, 4 slots 3 ahead
    # 223-232 ms, 6 slots 5 ahead 194 ms, resident 153 ms.
    stream_candidates: bool = False
    stream_slots: int = 6
    stream_depth: int = 5
    stream_overlap: bool = True
    # run the plain GEMMs (the Q8_0 teacher's projections, the vocabulary
    # heads) with the library solutions PyTorch's TunableOp measured fastest
    # for these shapes on MI355X (use_tuned_gemms); process-wide, so off
    # unless asked for.  0.8B-class step: 42.0 -> 41.6 and 41.2 -> 40.9 ms (two boxes)
    tuned_gemms: bool = False
    stream_timeline: bool = False   # record timing events per copy and fence (CandidateStreamer.timeline_ms)
    # check the embeddings' ids on the device and raise an out-of-range id at
    # the next step (layers.check_embedding_ids) instead of reading the ids'
    # range on the host in every lookup: with no device synchronisation left
    # in the step, the host queues the next step's forward while the device
    # runs this step's backward.  Measured on MI355X, the 0.8B-class decoder
    # step 51.6 -> 49.3 ms.
    deferred_id_check: bool = True


def _embeddings(*models: nn.Module) -> list[nn.Module]:
    return [m for model in models for m in model.modules() if isinstance(m, (layers.MixedQuantEmbedding, Q8Embedding))]


# TunableOp results for the step's plain GEMMs on MI355X (ROCm 7, torch
# 2.10): the Q8_0 teacher's four projections and the vocabulary head at 8192
# tokens, forward (solutions measured by torch.cuda.tunable; a data file, not
# code)
GEMM_TUNING_FILE = Path(__file__).resolve().with_name("gemm_tuning_mi355x.csv")


def use_tuned_gemms(path: Path | str = GEMM_TUNING_FILE) -> bool:
    """Turn PyTorch's TunableOp on without tuning, with the results in `path`:
    GEMMs of the listed shapes then run the hipBLASLt / rocBLAS solution
    measured fastest for them, every other GEMM the library's default.
    Process-wide.  Returns False (and changes nothing) without a ROCm device,
    or when the file's validators (torch, HIP, hipBLASLt and rocBLAS
    versions, GPU architecture) differ from the running ones."""
    tun = getattr(torch.cuda, "tunable", None)
    if tun is None or not torch.cuda.is_available():
        return False
    want = {}
    for line in Path(path).read_text().splitlines():
        parts = line.split(",")
        if parts[0] == "Validator" and len(parts) >= 3:
            want[parts[1]] = ",".join(parts[2:])
    have = dict(tun.get_validators())
    if not want or any(have.get(k) != v for k, v in want.items()):
        warnings.warn(f"{path}: TunableOp validators differ from this runtime; GEMMs keep the library defaults")
        return False
    tun.tuning_enable(False)
    tun.enable(True)
    if not tun.read_file(str(path)):
        tun.enable(False)
        return False
    return True


class GateTrainer:
    """Runs the reference's per-batch gate-training step (``trainer.py:2498-2616``)."""

    def __init__(self, student: Decoder, teacher: Decoder, replaced: dict[str, nn.Module], cfg: StepConfig,
                 total_8bit_bytes: float, non_targeted_bytes: float = 0.0):
        self.student, self.teacher, self.replaced, self.cfg = student, teacher, replaced, cfg
        # whether the plain GEMMs run the tuned solutions (cfg.tuned_gemms)
        self.tuned_gemms = use_tuned_gemms() if cfg.tuned_gemms else False
        # the chunked loss runs one backward per chunk, so its probabilities
        # must come from each module's own graph
        self.bank = (trainer.GateBank(replaced.values(), cfg.defer_gate_grads)
                     if cfg.gate_bank and cfg.logits_chunk == 0 else None)
        self.trainable = self.bank.parameters() if self.bank else [m.gates for m in replaced.values()]
        self.opt, self.sched = trainer.build_gate_optimizer(self.trainable, cfg.lr, cfg.max_steps)
        self.target_bytes = cfg.target_fraction * total_8bit_bytes
        self.non_targeted_bytes = non_targeted_bytes
        self.step_index = 0
        # after the bank: the prefetch reads each module's probabilities row
        self.prefetch = _make_prefetch(cfg, student)
        self.t_stream = _make_teacher_stream(cfg, student)
        self.streamer = _make_streamer(cfg, student)
        if cfg.deferred_id_check:
            for m in _embeddings(student, teacher):
                m.id_check = "deferred"

    def step(self, x: torch.Tensor, y: torch.Tensor) -> dict[str, torch.Tensor]:
        """One optimizer step on batch (x, y); returns the detached losses (no
        host sync).  An out-of-range token id of the previous step raises
        IndexError here (StepConfig.deferred_id_check); waiting for that
        step's id checks also keeps the host at most about one step ahead."""
        c = self.cfg
        layers.raise_pending_id_errors()
        tau = trainer.anneal_temperature(self.step_index, c.max_steps, c.temp_start, c.temp_end)
        trainer.set_temperature_all(self.replaced, tau)
        dev = x.device
        t = c.distill_temperature
        bank_bytes = self.bank.begin(tau) if self.bank else None
        if self.prefetch:
            self.prefetch.launch()
        try:
            if c.logits_chunk > 0:
                lm, kl = trainer.chunked_forward_loss(self.student, self.teacher, x, y, t, c.logits_chunk)
                lm_loss, distill = torch.tensor(lm), torch.tensor(kl)
            else:
                logits, t_logits = _forwards(self.student, self.teacher, x, self.t_stream)
                fused = (c.fused_loss and logits.is_cuda and logits.dtype == torch.bfloat16
                         and logits.size(-1) % 8 == 0)
                losses = trainer.distill_losses_fused if fused else trainer.distill_losses
                lm_loss, distill = losses(logits, t_logits, y, t)
            gated = bank_bytes if bank_bytes is not None else layers.total_effective_bytes(self.replaced)
            current = gated.to(dev) + self.non_targeted_bytes
            size = trainer.size_loss(current, self.target_bytes, c.size_tolerance)
            if c.logits_chunk > 0:
                (c.size_weight * size).backward()
            else:
                loss = lm_loss + c.distill_weight * distill + c.size_weight * size
                loss.backward()
            if self.bank:
                self.bank.finish()
        finally:
            if self.bank:
                self.bank.end()
        trainer.gate_optimizer_step(self.trainable, self.opt, self.sched, max_norm=1.0)
        self.step_index += 1
        return {"lm": lm_loss.detach(), "kl": distill.detach(), "size": size.detach(), "tau": tau}


def prefetch_groups(model: nn.Module) -> list[list[nn.Module]]:
    """The gated products of `model` in forward order, as its forward runs
    them: q/k/v stacked, o, gate/up stacked, down per layer or block (products
    whose members are not all gated are left out)."""
    groups = []
    for mod in model.modules():
        if isinstance(mod, _Attention):
            cand = [[mod.q_proj, mod.k_proj, mod.v_proj], [mod.o_proj]]
        elif isinstance(mod, _MLP):
            cand = [[mod.gate_proj, mod.up_proj], [mod.down_proj]]
        else:
            continue
        for g in cand:
            if not all(isinstance(m, layers.MixedQuantLinear) for m in g):
                continue
            # the forward stacks a product only when it can; otherwise its members run singly
            groups += [g] if len(g) == 1 or (GROUP_PROJECTIONS and layers.groupable(g)) else [[m] for m in g]
    return groups


def _make_streamer(cfg: StepConfig, student: nn.Module):
    if not cfg.stream_candidates:
        return None
    if cfg.prefetch_mix or cfg.defer_gate_grads:
        raise ValueError("streamed candidates run without the mix prefetch and without deferred gate gradients")
    from voodoo_quant.streaming import CandidateStreamer

    dev = next(p for p in student.parameters()).device
    return CandidateStreamer(prefetch_groups(student), dev, slots=cfg.stream_slots, depth=cfg.stream_depth,
                             overlap=cfg.stream_overlap, timeline=cfg.stream_timeline)


def _make_teacher_stream(cfg: StepConfig, student: nn.Module):
    if not cfg.teacher_stream or cfg.logits_chunk > 0:
        return None
    dev = next(student.parameters()).device
    return torch.cuda.Stream(device=dev) if dev.type == "cuda" else None


def _forwards(student: nn.Module, teacher: nn.Module, x: torch.Tensor, t_stream):
    """The student's forward (recorded for autograd) and the teacher's (no
    grad).  With t_stream the teacher runs on that stream beside the student:
    the side stream first waits for the work queued before the step (x and
    anything that wrote the teacher's inputs), and the caller's stream waits
    for the teacher before it reads the teacher's output.  Both outputs are
    the ones the sequential order gives."""
    if t_stream is None:
        s_out = student(x)
        with torch.no_grad():
            t_out = teacher(x)
        return s_out, t_out
    cur = torch.cuda.current_stream(x.device)
    t_stream.wait_stream(cur)
    x.record_stream(t_stream)  # x may be freed by the caller before the teacher is done
    with torch.cuda.stream(t_stream), torch.no_grad():
        t_out = teacher(x)
    s_out = student(x)
    cur.wait_stream(t_stream)
    t_out.record_stream(cur)  # allocated on the side stream, read and freed on the caller's
    return s_out, t_out


def _make_prefetch(cfg: StepConfig, student: nn.Module):
    if not cfg.prefetch_mix or cfg.logits_chunk > 0:
        return None
    groups = prefetch_groups(student)
    if not groups or groups[0][0].gates.device.type != "cuda":
        return None
    return layers.MixPrefetch(groups)


def step_flops(cfg: DecoderConfig, tokens: int, seq: int) -> float:
    """Model FLOPs of one step: student gated Linears 6 M N D, its lm_head
    4 M V H (forward + dX), the teacher 2 M N D over all its Linears and head,
    and causal attention (QK^T and PV, forward 2 M S d per head halved by the
    mask, backward 2x the forward; the teacher forward once)."""
    per_layer = sum(o * i for o, i in cfg.linear_shapes().values())
    lin = cfg.layers * per_layer
    head = cfg.vocab * cfg.hidden
    attn_fwd = cfg.layers * 2 * 2 * tokens * seq * cfg.heads * cfg.head_dim / 2
    return 6 * tokens * lin + 4 * tokens * head + 2 * tokens * (lin + head) + attn_fwd * 3 + attn_fwd


# ---------------------------------------------------------------------------
# the wide-menu stress configuration: a stack of SwiGLU blocks
# ---------------------------------------------------------------------------
@dataclass
class StackConfig:
    blocks: int = 8
    hidden: int = 4096
    mlp: int = 14336
    eps: float = 1.0e-6

    def gated_weights(self) -> int:
        return self.blocks * 3 * self.hidden * self.mlp


class _SwiGLUBlock(nn.Module):
    """h + down(silu(gate(rmsnorm h)) * up(rmsnorm h))."""

    def __init__(self, cfg: StackConfig, lin: dict[str, nn.Module], device):
        super().__init__()
        self.eps = cfg.eps
        self.mlp = _MLP(lin)
        self.norm = nn.Parameter(torch.ones(cfg.hidden, dtype=torch.bfloat16, device=device), requires_grad=False)

    def forward(self, h):
        return h + self.mlp(F.rms_norm(h, (h.shape[-1],), self.norm, self.eps))


class SwiGLUStack(nn.Module):
    def __init__(self, cfg: StackConfig, block_linears: list[dict[str, nn.Module]], device):
        super().__init__()
        self.blocks = nn.ModuleList([_SwiGLUBlock(cfg, lin, device) for lin in block_linears])

    def forward(self, h):
        blocks = list(self.blocks)
        if not blocks or not _fused_norms(h, blocks[0].norm):
            for b in blocks:
                h = b(h)
            return h
        # each block's residual add fused with the next block's norm
        eps = blocks[0].eps
        h = h.contiguous()
        _, n = _AddRMSNorm.apply(h, None, blocks[0].norm, eps)
        for i, b in enumerate(blocks):
            m = b.mlp(n)
            if i + 1 < len(blocks):
                h, n = _AddRMSNorm.apply(h, m, blocks[i + 1].norm, eps)
            else:
                h = h + m
        return h


def build_stack(cfg: StackConfig, types: list[str], device, seed: int = 0):
    """(student, teacher, replaced) for the SwiGLU stack: every gate/up/down
    gated over `types` (a type may repeat: each entry is its own candidate),
    the teacher over Q8_0 bytes with kept decodes; candidates are synthetic
    valid blocks (see :func:`synthetic_candidate_bytes`)."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    replaced: dict[str, nn.Module] = {}
    shapes = {"mlp.gate_proj": (cfg.mlp, cfg.hidden), "mlp.up_proj": (cfg.mlp, cfg.hidden),
              "mlp.down_proj": (cfg.hidden, cfg.mlp)}
    s_blocks, t_blocks = [], []
    for bi in range(cfg.blocks):
        lin = {}
        for n, (o, i) in shapes.items():
            name = f"blocks.{bi}.{n}"
            qbs = [synthetic_candidate_bytes(qt, o, i, device, gen) for qt in types]
            lin[n] = layers.MixedQuantLinear.from_packed(i, o, types, qbs, tensor_name=name, device=device)
            replaced[name] = lin[n]
        s_blocks.append(lin)
        t_blocks.append({n: Q8Linear(synthetic_candidate_bytes("Q8_0", o, i, device, gen), o, i)
                         for n, (o, i) in shapes.items()})
    set_keep_decoded(True)
    teacher = SwiGLUStack(cfg, t_blocks, device)
    teacher.requires_grad_(False)
    return SwiGLUStack(cfg, s_blocks, device), teacher, replaced


class StackTrainer:
    """Gate training of the SwiGLU stack: loss = relative MSE of the output
    against the Q8_0 teacher's + size_weight * dead-zone size penalty;
    temperature annealed, clip 1.0, AdamW + cosine on the gates."""

    def __init__(self, student, teacher, replaced, cfg: StepConfig, total_8bit_bytes: float):
        self.student, self.teacher, self.replaced, self.cfg = student, teacher, replaced, cfg
        self.bank = trainer.GateBank(replaced.values(), cfg.defer_gate_grads) if cfg.gate_bank else None
        self.trainable = self.bank.parameters() if self.bank else [m.gates for m in replaced.values()]
        self.opt, self.sched = trainer.build_gate_optimizer(self.trainable, cfg.lr, cfg.max_steps)
        self.target_bytes = cfg.target_fraction * total_8bit_bytes
        self.step_index = 0
        self.prefetch = _make_prefetch(cfg, student)
        self.t_stream = _make_teacher_stream(cfg, student)
        self.streamer = _make_streamer(cfg, student)

    def step(self, x: torch.Tensor) -> dict[str, torch.Tensor]:
        c = self.cfg
        tau = trainer.anneal_temperature(self.step_index, c.max_steps, c.temp_start, c.temp_end)
        trainer.set_temperature_all(self.replaced, tau)
        bank_bytes = self.bank.begin(tau) if self.bank else None
        if self.prefetch:
            self.prefetch.launch()
        try:
            y, t = _forwards(self.student, self.teacher, x, self.t_stream)
            t = t.float()
            mse = ((y.float() - t) ** 2).mean() / (t ** 2).mean()
            gated = bank_bytes if bank_bytes is not None else layers.total_effective_bytes(self.replaced)
            size = trainer.size_loss(gated.to(x.device), self.target_bytes, c.size_tolerance)
            (mse + c.size_weight * size).backward()
            if self.bank:
                self.bank.finish()
        finally:
            if self.bank:
                self.bank.end()
        trainer.gate_optimizer_step(self.trainable, self.opt, self.sched, max_norm=1.0)
        self.step_index += 1
        return {"mse": mse.detach(), "size": size.detach(), "tau": tau}


def stack_flops(cfg: StackConfig, tokens: int) -> float:
    """6 M N D for the student's gated products (forward, dX, dW-gate) plus
    2 M N D for the teacher's forward."""
    return 8.0 * tokens * cfg.gated_weights()
