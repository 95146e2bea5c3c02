"""Torch CPU restatement of the gated-mixture Linear math (test infrastructure).

Follows, operation for operation where rounding matters:

* ``soft_probs``      -- ``voodoo_quant/layers.py:1342-1351``: softmax(gates / max(T, 1e-6))
* ``mix_weight``      -- ``voodoo_quant/layers.py:336-352``: ``mixed = 0; mixed = mixed + p_k * W_k``
                         in fp32, k-ordered (a multiply then an add, never fused),
                         then ``mixed.to(source_dtype)``
* ``forward``         -- ``voodoo_quant/layers.py:1729-1731``: ``F.linear(x, W_eff)``
* ``backward``        -- autograd of ``F.linear`` (dX = dY W_eff, dW = dY^T X) and
                         ``_MixedWeightFunction.backward`` (``layers.py:354-363``):
                         ``gp_k = sum(dW * W_k)``; the gates then receive the softmax
                         Jacobian ``(1/T) p * (gp - <p, gp>)`` (``tests/test_ptqr.py:161-172``
                         states the same identity at T = 1).
* ``effective_bytes`` -- ``layers.py:1537-1550``; ``anneal_temperature`` --
  ``training/trainer.py:199-203``; ``size_loss`` -- ``trainer.py:2585-2590``;
  ``make_gate_optimizer`` -- ``trainer.py:2378-2379`` (AdamW betas (0.9, 0.95),
  cosine to 1e-3) with the global clip of ``trainer.py:2612``.

Deliberate difference, stated once: the reference's non-lazy path stores each
candidate in the source dtype (bf16) before mixing (``layers.py:1311-1312``) and
its lazy path mixes in bf16 (``layers.py:514-556``).  This oracle mixes the
EXACT fp32 dequantised candidates, which is the "fp32 PyTorch path" the GPU
kernels are held to, and computes ``dW`` and ``gp`` in fp32 (``dtype`` below can
raise both to fp64 for the small cases the tests pin with finite differences).
"""

from __future__ import annotations

import math

import torch


def soft_probs(gates: torch.Tensor, temperature: float) -> torch.Tensor:
    return torch.softmax(gates / max(float(temperature), 1e-6), dim=0)


def mix_weight(cands: list[torch.Tensor], probs: torch.Tensor) -> torch.Tensor:
    """fp32 k-ordered mixture (each step rounds the product, then the sum)."""
    mixed = torch.zeros_like(cands[0], dtype=torch.float32)
    for k, c in enumerate(cands):
        mixed = mixed + probs[k].to(torch.float32) * c.to(torch.float32)
    return mixed


def forward(x: torch.Tensor, w_eff: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """Y = X W_eff^T accumulated in ``dtype``."""
    return x.to(dtype) @ w_eff.to(dtype).t()


def backward(dy: torch.Tensor, x: torch.Tensor, w_eff: torch.Tensor, cands: list[torch.Tensor],
             dtype=torch.float32):
    """Returns (dX, dW, gp) with gp_k = <dW, W_k>, all in ``dtype``."""
    dyf, xf = dy.to(dtype), x.to(dtype)
    dx = dyf @ w_eff.to(dtype)
    dw = dyf.t() @ xf
    gp = torch.stack([(dw * c.to(dtype)).sum() for c in cands])
    return dx, dw, gp


def gates_grad(gp: torch.Tensor, probs: torch.Tensor, temperature: float) -> torch.Tensor:
    """dL/dgates from dL/dprobs through softmax(g / T)."""
    t = max(float(temperature), 1e-6)
    p = probs.to(gp.dtype)
    return p * (gp - (p * gp).sum()) / t


def reference_step_fp32(x_bf16, dy_bf16, cands_f32, gates, temperature):
    """The timed CPU baseline: the reference's non-lazy gated Linear fwd+bwd in
    torch fp32 on the host (mixture, F.linear forward in the source dtype,
    autograd backward with a materialised dW, per-candidate reductions, softmax
    backward)."""
    g = gates.detach().clone().requires_grad_(True)
    probs = soft_probs(g, temperature)
    p_det = probs.detach()
    w_eff = mix_weight(cands_f32, p_det).to(torch.bfloat16)
    y = (x_bf16.float() @ w_eff.float().t()).to(torch.bfloat16)
    dx = (dy_bf16.float() @ w_eff.float()).to(torch.bfloat16)
    dw = dy_bf16.float().t() @ x_bf16.float()
    gp = torch.stack([(dw * c).sum() for c in cands_f32])
    probs.backward(gp)
    return y, dx, g.grad


# ----------------------------------------------------------------- budget and trainer math
def effective_bytes(probs: torch.Tensor, bytes_per_weight: list[float], n_weights: int) -> torch.Tensor:
    total = torch.tensor(0.0, dtype=probs.dtype)
    for k, bpw in enumerate(bytes_per_weight):
        total = total + probs[k] * bpw * n_weights
    return total


def anneal_temperature(step: int, max_steps: int, start: float, end: float) -> float:
    if max_steps <= 1:
        return end
    return start * (end / start) ** (step / (max_steps - 1))


def size_loss(current_bytes: torch.Tensor, target_bytes: float, tolerance: float) -> torch.Tensor:
    rel = torch.abs(current_bytes / target_bytes - 1.0)
    return torch.relu(rel - tolerance) ** 2


def make_gate_optimizer(params, lr: float, max_steps: int):
    opt = torch.optim.AdamW(params, lr=lr, betas=(0.9, 0.95))
    sched = torch.optim.lr_scheduler.CosineAnnealingLR(opt, T_max=max_steps, eta_min=1e-3)
    return opt, sched


def gated_linear_flops(m: int, n: int, d: int) -> float:
    """Algorithmic fwd+bwd FLOPs: Y, dX and dW, 2*M*N*D each."""
    return 6.0 * m * n * d


def relative_l2(a: torch.Tensor, b: torch.Tensor, floor: float = 0.0) -> float:
    a64, b64 = a.double(), b.double()
    den = max(float(b64.norm()), floor)
    if den == 0.0:
        return float((a64 - b64).norm())
    return float((a64 - b64).norm()) / den


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("math", "torch", "annotations")]
