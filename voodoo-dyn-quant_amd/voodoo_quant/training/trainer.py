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
    """The model's size at one byte per parameter.

    `state_dict_meta` maps each state-dict key to (storage pointer, element
    count).  Keys that share a storage (tied embeddings) are one tensor, so
    each pointer's elements count once (reference ``trainer.py:157-176``)."""
    per_storage = {ptr: float(numel) for ptr, numel in state_dict_meta.values()}
    return float(sum(per_storage.values()))


def compute_non_targeted_8bit_bytes(state_dict_meta: dict[str, tuple[int, int]], targeted_keys: set[str]) -> float:
    """Bytes at one byte per parameter of the storages no gated tensor covers.

    A storage is targeted when any key that points at it is in
    `targeted_keys`; the rest keep their 8-bit size in the budget (reference
    ``trainer.py:178-196``)."""
    per_storage = {ptr: float(numel) for ptr, numel in state_dict_meta.values()}
    targeted = {ptr for key, (ptr, _) in state_dict_meta.items() if key in targeted_keys}
    return float(sum(b for ptr, b in per_storage.items() if ptr not in targeted))


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
                # the gate stream adds into the sink: the allocator must not
                # hand its memory to main-stream work before that stream is done
                sink.record_stream(stream)
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
        # a backward that raised leaves deferred work queued on the gate
        # streams: join them before the sinks are dropped
        for bank, _, _, _, stream in self._pending:
            torch.cuda.current_stream(bank.device).wait_stream(stream)
        self._pending = []
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


def _fused_loss_ok(logits: torch.Tensor) -> bool:
    return logits.is_cuda and logits.dtype == torch.bfloat16 and logits.size(-1) % 8 == 0


def chunk_loss_sums(logits: torch.Tensor, teacher_logits: torch.Tensor, labels: torch.Tensor,
                    temperature: float) -> torch.Tensor:
    """fp32 [2] = (CE summed over the labelled rows, T^2 KL(teacher || student)
    summed over all rows) of one block of rows, differentiable in `logits`.

    On a ROCm device with bf16 logits the sums come from the fused kernels
    (:class:`DistillLossFunction` returns the two means; each is scaled by
    its row count, which the backward turns into the kernel's gradient
    weights).  Elsewhere an fp32 torch restatement of the same sums runs."""
    labels = labels.reshape(-1)
    if _fused_loss_ok(logits):
        v = logits.size(-1)
        means = DistillLossFunction.apply(logits.reshape(-1, v).contiguous(),
                                          teacher_logits.reshape(-1, v).contiguous(),
                                          labels.to(torch.int64).contiguous(), float(temperature))
        labelled = (labels != -100).sum().to(torch.float32)
        # a block with no labelled row has CE mean 0/0; its sum is 0
        ce = torch.where(labelled > 0, means[0] * labelled, torch.zeros_like(means[0]))
        return torch.stack([ce, means[1] * float(labels.numel())])
    import torch.nn.functional as F

    s = logits.float().reshape(labels.numel(), -1)
    t = teacher_logits.float().reshape_as(s)
    ce = F.cross_entropy(s, labels, ignore_index=-100, reduction="sum")
    log_q = F.log_softmax(s / temperature, dim=-1)
    log_p = F.log_softmax(t / temperature, dim=-1)
    kl = (log_p.exp() * (log_p - log_q)).sum() * (temperature * temperature)
    return torch.stack([ce, kl])


class ChunkedDistillLoss:
    """CE + KL over the output head without the [tokens, vocab] logits of the
    whole batch (the reference's ``_chunked_forward_loss`` route,
    ``trainer.py:751-832``).

    The student's stack runs once and its final hidden states are taken out
    of the graph.  Rows are then processed `chunk` at a time: the student's
    and the teacher's heads give the block's logits, :func:`chunk_loss_sums`
    gives its loss sums, and ``torch.autograd.grad`` returns the gradient of
    (CE sum + KL sum) / tokens with respect to the block's hidden rows (and
    the head's own trainable parameters, which are accumulated into their
    ``.grad``).  The row gradients fill one buffer, and one backward carries
    it through the stack.

    Both terms are divided by the batch's token count and weighted 1: on this
    route the distillation weight of the full-logits loss is not applied, as
    in the reference (its chunk backward, ``trainer.py:812``), so that the
    gate gradients are the reference's."""

    def __init__(self, chunk: int, temperature: float) -> None:
        if chunk <= 0:
            raise ValueError("chunk must be positive")
        self.chunk = int(chunk)
        self.temperature = float(temperature)

    def __call__(self, student, teacher, x: torch.Tensor, y: torch.Tensor) -> tuple[float, float]:
        hidden = _hidden(student.model(input_ids=x))
        with torch.no_grad():
            teacher_rows = _hidden(teacher.model(input_ids=x)).reshape(-1, hidden.size(-1))
        rows = teacher_rows.size(0)
        student_rows = hidden.detach().reshape(rows, -1)
        labels = y.reshape(-1)
        head_params = [p for p in student.lm_head.parameters() if p.requires_grad]
        row_grad = torch.empty_like(student_rows)
        totals = torch.zeros(2, dtype=torch.float64, device=student_rows.device)
        for lo in range(0, rows, self.chunk):
            hi = min(rows, lo + self.chunk)
            leaf = student_rows[lo:hi].detach().requires_grad_(True)
            with torch.no_grad():
                t_logits = teacher.lm_head(teacher_rows[lo:hi])
            sums = chunk_loss_sums(student.lm_head(leaf), t_logits, labels[lo:hi], self.temperature)
            grads = torch.autograd.grad(sums.sum() / rows, [leaf] + head_params, allow_unused=True)
            row_grad[lo:hi].copy_(grads[0] if grads[0] is not None else torch.zeros_like(leaf))
            for p, g in zip(head_params, grads[1:]):
                if g is not None:
                    p.grad = g if p.grad is None else p.grad + g
            totals += sums.detach().double()
        hidden.backward(row_grad.view_as(hidden))
        means = (totals / rows).tolist()
        return float(means[0]), float(means[1])


def chunked_forward_loss(student, teacher, x: torch.Tensor, y: torch.Tensor, temperature: float, chunk: int):
    """Token-chunked CE + KL with one backward through the student's stack;
    returns (CE, KL) as floats, each a mean over tokens (see
    :class:`ChunkedDistillLoss`)."""
    return ChunkedDistillLoss(chunk, temperature)(student, teacher, x, y)
