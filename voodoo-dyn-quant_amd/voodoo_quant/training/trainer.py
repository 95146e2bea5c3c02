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


def softmax_rows_backward(p: torch.Tensor, g: torch.Tensor, temperature: float) -> torch.Tensor:
    """Gradient w.r.t. the logits z of p = softmax(z / T) along dim 1, given
    dL/dp = g: (1/T) p (g - <p, g>) per row."""
    return p * (g - (p * g).sum(dim=1, keepdim=True)) / temperature


class GateBank:
    """The gate logits of many gated tensors as one [T, K] parameter per
    (candidate count, device) group.

    The reference trains one [K] parameter per gated tensor and each layer
    takes its own softmax (``layers.py:1729-1731``); with ~170 tensors that
    is ~170 softmaxes forward, ~170 backward and the scale ops around them,
    each a launch on a few bytes.  Here one softmax per group runs at the
    start of a step and each module reads its row (``soft_probs``); autograd
    brings the modules' gate gradients back as one stacked tensor.  The
    values and the optimizer update are the same elementwise: AdamW, the
    global-norm clip and the dead-zone size penalty see the same numbers.
    Each module's ``gates`` becomes a row view of its bank, so reading a
    module's gates (argmax, export) sees the trained values.

    defer_gate_grads (ROCm devices): the gated Linears' backwards leave their
    gate gradients to a second stream (default priority) -- the dot pass over
    dW parts and the fixed-order reduce, ~170 small launches per 0.8B-class
    step -- which adds each into a [T, K] buffer of the bank; :meth:`finish`,
    after ``backward()``, joins that stream and applies the softmax Jacobian
    (1/T) p (g - <p, g>) once per bank.  Those launches then overlap the next
    layer's backward instead of sitting between its products.  Modules that
    cannot defer (PTQR routing, embeddings) keep autograd through their row."""

    def __init__(self, modules, defer_gate_grads: bool = False) -> None:
        self.defer = bool(defer_gate_grads)
        self._streams: dict = {}
        self._pending: list = []
        groups: dict[tuple, list] = {}
        for m in modules:
            groups.setdefault((m.num_candidates, m.gates.device), []).append(m)
        self.groups = []
        for (_, dev), mods in groups.items():
            bank = torch.nn.Parameter(torch.stack([m.gates.detach() for m in mods]).contiguous())
            for i, m in enumerate(mods):
                m.gates = torch.nn.Parameter(bank.data[i], requires_grad=False)
            coef = torch.tensor([m._bytes_per_candidate() for m in mods], dtype=torch.float32).to(dev)
            self.groups.append((bank, mods, coef))

    def parameters(self) -> list:
        return [bank for bank, _, _ in self.groups]

    def begin(self, temperature: float) -> torch.Tensor:
        """Softmax every bank at `temperature`, hand each module its row, and
        return the differentiable effective bytes (sum of p_k * bytes_k)."""
        from voodoo_quant.layers import MixedQuantLinear

        total = None
        self._pending = []
        t = max(temperature, 1e-6)
        for bank, mods, coef in self.groups:
            probs = torch.nn.functional.softmax(bank / t, dim=1)
            for m, row in zip(mods, probs.unbind(0)):
                m._probs_override = row
            if self.defer and bank.device.type == "cuda":
                stream = self._streams.get(bank.device)
                if stream is None:
                    stream = self._streams[bank.device] = torch.cuda.Stream(device=bank.device)
                sink = torch.zeros(probs.shape, dtype=torch.float32, device=bank.device)
                for i, m in enumerate(mods):
                    if isinstance(m, MixedQuantLinear):
                        m._gate_sink = (sink[i], stream)
                self._pending.append((bank, probs.detach(), sink, t, stream))
            b = (probs * coef).sum()
            total = b if total is None else total + b
        return total if total is not None else torch.tensor(0.0)

    def finish(self) -> None:
        """After ``backward()``: add the deferred gate gradients, through the
        softmax Jacobian, to each bank's gradient (no-op without deferral)."""
        for bank, p, g, t, stream in self._pending:
            torch.cuda.current_stream(bank.device).wait_stream(stream)
            jac = softmax_rows_backward(p, g, t)
            if bank.grad is None:
                bank.grad = jac
            else:
                bank.grad.add_(jac)
        self._pending = []

    def end(self) -> None:
        for _, mods, _ in self.groups:
            for m in mods:
                m._probs_override = None
                m._gate_sink = None

    def release(self) -> None:
        """Give every module back an independent gates parameter (the bank's
        current values)."""
        self.end()
        for bank, mods, _ in self.groups:
            for i, m in enumerate(mods):
                m.gates = torch.nn.Parameter(bank.detach()[i].clone())
        self.groups = []


def gate_optimizer_step(trainable, opt, sched, max_norm: float = 1.0) -> None:
    torch.nn.utils.clip_grad_norm_(trainable, max_norm=max_norm)
    opt.step()
    sched.step()
    opt.zero_grad()


# ---------------------------------------------------------------------------
# losses over logits (reference trainer.py:2566-2575, 751-832)
# ---------------------------------------------------------------------------
def distill_losses(logits: torch.Tensor, teacher_logits: torch.Tensor, y: torch.Tensor, temperature: float):
    """(CE, KL): mean token cross-entropy against `y`, and the mean per-token
    KL(teacher || student) of the temperature-softened distributions times T^2
    (the reference's full-logits path, ``trainer.py:2566-2575``)."""
    import torch.nn.functional as F

    v = logits.size(-1)
    t = temperature
    lm_loss = F.cross_entropy(logits.view(-1, v), y.view(-1))
    student_log_probs = F.log_softmax(logits / t, dim=-1)
    teacher_probs = F.softmax(teacher_logits / t, dim=-1)
    per_token_kl = F.kl_div(student_log_probs.view(-1, v), teacher_probs.view(-1, v),
                            reduction="none").sum(dim=-1) * (t * t)
    return lm_loss, per_token_kl.mean()


class DistillLossFunction(torch.autograd.Function):
    """(CE, KL) of :func:`distill_losses` as one HIP pass over the logits and
    one for the gradient (``vq_distill_loss_fwd/bwd``).

    forward(ctx, logits [T, V] bf16, teacher_logits [T, V] bf16, labels [T]
    int64, temperature) -> fp32 [2] = (CE mean, KL mean); the backward gives
    the gradient of the logits only (the teacher runs without gradients)."""

    @staticmethod
    def forward(ctx, logits, teacher_logits, labels, temperature):
        from voodoo_quant import _hip

        out, ws = _hip.distill_loss_fwd(logits, teacher_logits, labels, temperature)
        ctx.save_for_backward(logits, teacher_logits, labels, ws)
        ctx.temperature = temperature
        return out

    @staticmethod
    def backward(ctx, grad_out):
        from voodoo_quant import _hip

        logits, teacher_logits, labels, ws = ctx.saved_tensors
        g = _hip.distill_loss_bwd(logits, teacher_logits, labels, ctx.temperature,
                                  grad_out.to(torch.float32).contiguous(), ws)
        return g, None, None, None


def distill_losses_fused(logits: torch.Tensor, teacher_logits: torch.Tensor, y: torch.Tensor, temperature: float):
    """:func:`distill_losses` on the GPU kernels: bf16 logits, vocabulary a
    multiple of 8.  The exponentials and sums run in fp32 (the per-token sums
    of the reference's bf16 tensors run in bf16) and the means in fp64."""
    v = logits.size(-1)
    out = DistillLossFunction.apply(logits.reshape(-1, v).contiguous(), teacher_logits.reshape(-1, v).contiguous(),
                                    y.reshape(-1).to(torch.int64).contiguous(), float(temperature))
    return out[0], out[1]


def _hidden(out) -> torch.Tensor:
    return out.last_hidden_state if hasattr(out, "last_hidden_state") else out


def chunked_forward_loss(student, teacher, x: torch.Tensor, y: torch.Tensor, temperature: float, chunk: int):
    """Token-chunked CE + KL with one backward through the student's text
    stack (reference ``_chunked_forward_loss``, ``trainer.py:751-832``).

    Each chunk's head forward, losses and head backward run on a detached copy
    of the final hidden states, and its input gradient is collected; one
    backward of the collected gradient then runs through the stack.  As in the
    reference, the chunk backward differentiates (CE + KL) / tokens, so the
    distillation weight is not applied on this path.  Returns (CE, KL) as
    floats, each a mean over tokens."""
    import torch.nn.functional as F

    hidden = _hidden(student.model(input_ids=x))
    with torch.no_grad():
        t_hidden = _hidden(teacher.model(input_ids=x))
    h = hidden.shape[-1]
    s_flat, t_flat, y_flat = hidden.reshape(-1, h), t_hidden.reshape(-1, h), y.reshape(-1)
    n_tok = s_flat.shape[0]
    t = temperature
    h_grad = torch.zeros_like(s_flat)
    lm_total = torch.zeros((), dtype=torch.float64, device=s_flat.device)
    kl_total = torch.zeros((), dtype=torch.float64, device=s_flat.device)
    for i in range(0, n_tok, chunk):
        h_c = s_flat[i:i + chunk].detach().requires_grad_(True)
        logits_c = student.lm_head(h_c)
        lm_c = F.cross_entropy(logits_c, y_flat[i:i + chunk], reduction="sum")
        student_log_probs = F.log_softmax(logits_c / t, dim=-1)
        del logits_c
        with torch.no_grad():
            teacher_probs = F.softmax(teacher.lm_head(t_flat[i:i + chunk]) / t, dim=-1)
        kl_c = F.kl_div(student_log_probs, teacher_probs, reduction="none").sum() * (t * t)
        del student_log_probs, teacher_probs
        ((lm_c + kl_c) / n_tok).backward()
        with torch.no_grad():
            if h_c.grad is not None:
                h_grad[i:i + chunk] = h_c.grad
        lm_total += lm_c.detach().double() / n_tok
        kl_total += kl_c.detach().double() / n_tok
    hidden.backward(h_grad.reshape(hidden.shape))
    return float(lm_total), float(kl_total)
