"""The step's side streams leave the training step unchanged: the W_eff
prefetch (layers.MixPrefetch: every mix of a step on a second stream,
event-fenced ahead of its GEMMs) and the teacher's forward on a second stream
beside the student's (StepConfig.teacher_stream, step._forwards).

The mix is deterministic and the prefetched W_eff is the same buffer contents
the inline mix would write, and the teacher's output does not depend on the
stream it runs on, so on the SwiGLU stack (no attention) the gates after three
steps, and every loss on the way, must be bit-identical; so must the decoder
step's gates and losses (its attention kernels sum in a fixed order).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")


def _stack_run(prefetch: bool, steps: int = 3, teacher_stream: bool = False):
    from voodoo_quant.training import step as st

    dev = torch.device("cuda", 0)
    cfg = st.StackConfig(blocks=2, hidden=512, mlp=1024)
    types = ["Q2_K", "Q4_K", "Q6_K", "Q8_0"]
    student, teacher, replaced = st.build_stack(cfg, types, dev, seed=3)
    tr = st.StackTrainer(student, teacher, replaced,
                         st.StepConfig(max_steps=10, temp_start=2.0, temp_end=0.5, prefetch_mix=prefetch,
                                       teacher_stream=teacher_stream),
                         total_8bit_bytes=float(cfg.gated_weights()))
    assert (tr.prefetch is not None) == prefetch
    assert (tr.t_stream is not None) == teacher_stream
    x = torch.randn(256, cfg.hidden, device=dev, generator=torch.Generator(device=dev).manual_seed(4))
    x = x.to(torch.bfloat16)
    losses = []
    for _ in range(steps):
        out = tr.step(x)
        losses.append(torch.stack([out["mse"], out["size"]]))
    torch.cuda.synchronize()
    gates = torch.stack([m.gates.detach().clone() for m in replaced.values()])
    return gates, torch.stack(losses), tr


def test_prefetched_stack_step_is_bit_identical():
    _need_gpu()
    g0, l0, _ = _stack_run(False)
    g1, l1, tr = _stack_run(True)
    n_groups = len(tr.prefetch.groups)
    assert n_groups == 4  # gate/up stacked and down, per block
    assert torch.equal(l0.view(torch.int32), l1.view(torch.int32)), (l0, l1)
    assert torch.equal(g0.view(torch.int32), g1.view(torch.int32)), (g0 - g1).abs().max()
    assert not any(tr.prefetch.pending), "every prefetched product was consumed by its forward"


def test_prefetched_decoder_step_matches():
    _need_gpu()
    from voodoo_quant.training import step as st

    dev = torch.device("cuda", 0)
    cfg = st.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, mlp=512, vocab=1024)
    types = ["Q3_K", "Q4_K", "Q8_0"]
    res = []
    for prefetch in (False, True):
        student, teacher, replaced = st.build_models(cfg, types, dev, seed=7, packed=True)
        tr = st.GateTrainer(student, teacher, replaced,
                            st.StepConfig(max_steps=10, prefetch_mix=prefetch),
                            total_8bit_bytes=float(cfg.gated_weights()))
        assert (tr.prefetch is not None) == prefetch
        g = torch.Generator(device=dev).manual_seed(8)
        x = torch.randint(0, cfg.vocab, (2, 128), device=dev, generator=g)
        y = torch.randint(0, cfg.vocab, (2, 128), device=dev, generator=g)
        for _ in range(2):
            tr.step(x, y)
        torch.cuda.synchronize()
        res.append(torch.stack([m.gates.detach().clone().float() for m in replaced.values()]))
        if prefetch:
            # q alone (k/v have 128 rows, too few to stack), k, v, o, gate/up stacked, down
            assert len(tr.prefetch.groups) == 6 * cfg.layers
            assert not any(tr.prefetch.pending)
    diff = float((res[0] - res[1]).abs().max())
    print(f"[prefetch] decoder gates max |diff| {diff:.3e}", flush=True)
    assert torch.equal(res[0].view(torch.int32), res[1].view(torch.int32)), diff


def test_teacher_stream_stack_step_is_bit_identical():
    _need_gpu()
    g0, l0, _ = _stack_run(False)
    g1, l1, _ = _stack_run(False, teacher_stream=True)
    assert torch.equal(l0.view(torch.int32), l1.view(torch.int32)), (l0, l1)
    assert torch.equal(g0.view(torch.int32), g1.view(torch.int32)), (g0 - g1).abs().max()


def test_teacher_stream_decoder_step_matches():
    _need_gpu()
    from voodoo_quant.training import step as st

    dev = torch.device("cuda", 0)
    cfg = st.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, mlp=512, vocab=1024)
    types = ["Q3_K", "Q4_K", "Q8_0"]
    gates, losses = [], []
    for side in (False, True):
        student, teacher, replaced = st.build_models(cfg, types, dev, seed=7, packed=True)
        tr = st.GateTrainer(student, teacher, replaced, st.StepConfig(max_steps=10, teacher_stream=side),
                            total_8bit_bytes=float(cfg.gated_weights()))
        assert (tr.t_stream is not None) == side
        g = torch.Generator(device=dev).manual_seed(8)
        x = torch.randint(0, cfg.vocab, (2, 128), device=dev, generator=g)
        y = torch.randint(0, cfg.vocab, (2, 128), device=dev, generator=g)
        out = [tr.step(x, y) for _ in range(2)]
        torch.cuda.synchronize()
        gates.append(torch.stack([m.gates.detach().clone().float() for m in replaced.values()]))
        losses.append(torch.stack([torch.stack([o["lm"], o["kl"]]).float() for o in out]))
    diff = float((gates[0] - gates[1]).abs().max())
    ldiff = float((losses[0] - losses[1]).abs().max())
    print(f"[teacher stream] decoder gates max |diff| {diff:.3e}, losses {ldiff:.3e}", flush=True)
    assert torch.equal(gates[0].view(torch.int32), gates[1].view(torch.int32)), diff
    assert torch.equal(losses[0].view(torch.int32), losses[1].view(torch.int32)), ldiff


def _captured_grads(monkeypatch, make_trainer, run_step, steps: int = 2):
    """The bank gradients every optimizer step of `steps` sees, and the losses."""
    from voodoo_quant.training import trainer

    seen = []
    real = trainer.gate_optimizer_step

    def capture(trainable, opt, sched, max_norm=1.0):
        seen.append(torch.cat([p.grad.detach().reshape(-1).double().clone() for p in trainable]))
        real(trainable, opt, sched, max_norm=max_norm)

    monkeypatch.setattr(trainer, "gate_optimizer_step", capture)
    tr = make_trainer()
    losses = [run_step(tr) for _ in range(steps)]
    torch.cuda.synchronize()
    monkeypatch.setattr(trainer, "gate_optimizer_step", real)
    return seen, losses, tr


def test_deferred_gate_grads_stack_step_matches(monkeypatch):
    """Gate gradients finished on the bank's second stream: each step's bank
    gradient matches the in-order backward's to 1e-6 of its largest entry (the
    deferred dL/dp values are the same reduces; only the softmax Jacobian's
    arithmetic order differs), and the first step's losses are bit-equal."""
    _need_gpu()
    from voodoo_quant.training import step as st

    dev = torch.device("cuda", 0)
    cfg = st.StackConfig(blocks=2, hidden=512, mlp=1024)
    types = ["Q2_K", "Q4_K", "Q6_K", "Q8_0"]
    x = torch.randn(256, cfg.hidden, device=dev, generator=torch.Generator(device=dev).manual_seed(4))
    x = x.to(torch.bfloat16)
    res = []
    for defer in (False, True):
        student, teacher, replaced = st.build_stack(cfg, types, dev, seed=3)
        scfg = st.StepConfig(max_steps=10, temp_start=2.0, temp_end=0.5, defer_gate_grads=defer)
        seen, losses, tr = _captured_grads(
            monkeypatch,
            lambda: st.StackTrainer(student, teacher, replaced, scfg, total_8bit_bytes=float(cfg.gated_weights())),
            lambda tr: torch.stack([v.float() for k, v in tr.step(x).items() if k in ("mse", "size")]))
        assert bool(tr.bank._streams) == defer
        res.append((seen, losses))
    (g0, l0), (g1, l1) = res
    assert torch.equal(l0[0].view(torch.int32), l1[0].view(torch.int32)), (l0[0], l1[0])
    for a, b in zip(g0, g1):
        rel = float((a - b).abs().max() / a.abs().max())
        print(f"[defer] stack bank grad max rel diff {rel:.3e}", flush=True)
        assert rel < 1e-6


def test_deferred_gate_grads_decoder_step_matches(monkeypatch):
    """The same on the decoder step (stacked q/k/v and gate/up, single o and
    down, the parts path's dot pass; the embedding keeps autograd)."""
    _need_gpu()
    from voodoo_quant.training import step as st

    dev = torch.device("cuda", 0)
    cfg = st.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, mlp=512, vocab=1024)
    types = ["Q3_K", "Q4_K", "Q8_0"]
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randint(0, cfg.vocab, (2, 128), device=dev, generator=g)
    y = torch.randint(0, cfg.vocab, (2, 128), device=dev, generator=g)
    res = []
    for defer in (False, True):
        student, teacher, replaced = st.build_models(cfg, types, dev, seed=7, packed=True)
        scfg = st.StepConfig(max_steps=10, defer_gate_grads=defer)
        seen, losses, tr = _captured_grads(
            monkeypatch,
            lambda: st.GateTrainer(student, teacher, replaced, scfg, total_8bit_bytes=float(cfg.gated_weights())),
            lambda tr: torch.stack([v.float() for k, v in tr.step(x, y).items() if k in ("lm", "kl")]))
        assert bool(tr.bank._streams) == defer
        res.append((seen, losses))
    (g0, l0), (g1, l1) = res
    for a, b in zip(g0, g1):
        rel = float((a - b).abs().max() / a.abs().max())
        print(f"[defer] decoder bank grad max rel diff {rel:.3e}", flush=True)
        assert rel < 1e-5
    assert float((l0[0] - l1[0]).abs().max()) < 1e-5
