"""The trainer's per-step calls into the gated layers.

Only the pieces of the reference's ``training/trainer.py`` that sit on the
gated-Linear path: the temperature schedule (``:199-203``), the 8-bit byte
budget (``:157-196``), the dead-zone size penalty (``:2585-2590``) and the gate
optimizer (AdamW betas (0.9, 0.95) + cosine to 1e-3, ``:2378-2379``; global
clip 1.0 then step, ``:2612-2616``).  Model building, data, losses over logits
and checkpointing stay with the caller.
"""

from __future__ import annotations

import torch


def anneal_temperature(step: int, max_steps: int, start: float, end: float) -> float:
    if max_steps <= 1:
        return end
    frac = step / (max_steps - 1)
    return start * (end / start) ** frac


def compute_total_8bit_bytes(state_dict_meta: dict[str, tuple[int, int]]) -> float:
    """Bytes at 8 bits per parameter, shared storages counted once."""
    seen: set[int] = set()
    total = 0.0
    for ptr, numel in state_dict_meta.values():
        if ptr not in seen:
            seen.add(ptr)
            total += numel * 1.0
    return total


def compute_non_targeted_8bit_bytes(state_dict_meta: dict[str, tuple[int, int]], targeted_keys: set[str]) -> float:
    ptr_bytes: dict[int, float] = {}
    ptr_targeted: dict[int, bool] = {}
    for k, (ptr, numel) in state_dict_meta.items():
        ptr_bytes[ptr] = numel * 1.0
        ptr_targeted.setdefault(ptr, False)
        if k in targeted_keys:
            ptr_targeted[ptr] = True
    return sum(b for ptr, b in ptr_bytes.items() if not ptr_targeted[ptr])


def size_loss(current_bytes: torch.Tensor, target_bytes: float, tolerance: float) -> torch.Tensor:
    """relu(|bytes / target - 1| - tol)^2."""
    rel = torch.abs(current_bytes / target_bytes - 1.0)
    return torch.relu(rel - tolerance) ** 2


def set_temperature_all(replaced: dict, tau: float) -> None:
    for layer in replaced.values():
        layer.set_temperature(tau)


def build_gate_optimizer(trainable: list[torch.nn.Parameter], lr: float, max_steps: int):
    opt = torch.optim.AdamW(trainable, lr=lr, betas=(0.9, 0.95))
    sched = torch.optim.lr_scheduler.CosineAnnealingLR(opt, T_max=max_steps, eta_min=1e-3)
    return opt, sched


def gate_optimizer_step(trainable, opt, sched, max_norm: float = 1.0) -> None:
    torch.nn.utils.clip_grad_norm_(trainable, max_norm=max_norm)
    opt.step()
    sched.step()
    opt.zero_grad()
