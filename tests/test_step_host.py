"""The training-step losses on the CPU, on a small decoder of plain torch
modules: the full-logits losses against their closed forms, and the chunked
path (reference ``trainer.py:751-832``) against the full-logits path
(``trainer.py:2566-2603``), which it must reproduce exactly when the
distillation weight is 1 (the chunk backward omits it, as in the reference)."""

import pytest
import torch
import torch.nn as nn

from voodoo_quant.training import step as st
from voodoo_quant.training import trainer

CFG = st.DecoderConfig(layers=2, hidden=64, heads=2, kv_heads=1, head_dim=32, mlp=96, vocab=50)


def _plain_decoder(seed, trainable=True):
    g = torch.Generator().manual_seed(seed)

    def lin(o, i):
        m = nn.Linear(i, o, bias=False)
        with torch.no_grad():
            m.weight.copy_(torch.randn(o, i, generator=g) * 0.1)
        m.to(torch.bfloat16).requires_grad_(trainable)
        return m

    layers = [{n: lin(o, i) for n, (o, i) in CFG.linear_shapes().items()} for _ in range(CFG.layers)]
    emb = nn.Embedding(CFG.vocab, CFG.hidden)
    with torch.no_grad():
        emb.weight.copy_(torch.randn(CFG.vocab, CFG.hidden, generator=g) * 0.5)
    emb.requires_grad_(False)
    head = st._TiedHead(emb.weight.detach().to(torch.bfloat16).clone())
    return st.Decoder(st._Body(CFG, emb, layers, "cpu"), head)


def _batch():
    g = torch.Generator().manual_seed(7)
    return torch.randint(0, CFG.vocab, (2, 12), generator=g), torch.randint(0, CFG.vocab, (2, 12), generator=g)


def test_full_logits_losses_closed_form():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(3, 5, 11, generator=g, dtype=torch.float64)
    t_logits = torch.randn(3, 5, 11, generator=g, dtype=torch.float64)
    y = torch.randint(0, 11, (3, 5), generator=g)
    temp = 1.7
    ce, kl = trainer.distill_losses(logits, t_logits, y, temp)
    lp = torch.log_softmax(logits.reshape(-1, 11), -1)
    assert float(ce) == pytest.approx(float(-lp[torch.arange(15), y.reshape(-1)].mean()), rel=1e-12)
    sp = torch.log_softmax(logits.reshape(-1, 11) / temp, -1)
    tp = torch.softmax(t_logits.reshape(-1, 11) / temp, -1)
    ref = (tp * (tp.log() - sp)).sum(-1).mean() * temp * temp
    assert float(kl) == pytest.approx(float(ref), rel=1e-10)
    # a planted sign error in the closed form must not pass
    assert float(kl) != pytest.approx(float((tp * (tp.log() + sp)).sum(-1).mean() * temp * temp), rel=1e-3)


def test_chunked_loss_matches_full_logits():
    x, y = _batch()
    temp = 1.3
    student, teacher = _plain_decoder(0), _plain_decoder(1, trainable=False)
    ce, kl = trainer.distill_losses(student(x), teacher(x), y, temp)
    (ce + kl).backward()
    full = {n: p.grad.clone() for n, p in student.named_parameters() if p.requires_grad}
    student.zero_grad()
    ce_c, kl_c = trainer.chunked_forward_loss(student, teacher, x, y, temp, chunk=5)
    chunked = {n: p.grad.clone() for n, p in student.named_parameters() if p.requires_grad}
    assert ce_c == pytest.approx(float(ce.detach()), rel=1e-2) and kl_c == pytest.approx(float(kl.detach()), rel=2e-2)
    for n, g in full.items():
        rel = float((chunked[n].float() - g.float()).norm() / g.float().norm())
        assert rel < 5e-2, (n, rel)


def test_step_flops_and_gated_weights():
    cfg = st.DecoderConfig()
    assert cfg.gated_weights() == 24 * 12_058_624 + 151936 * 1024
    fl = st.step_flops(cfg, 8192, 2048)
    assert 25e12 < fl < 35e12


def test_synthetic_candidates_are_valid_and_centred():
    from oracle import cdequant

    g = torch.Generator().manual_seed(0)
    for qt in ("Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"):
        qb = st.synthetic_candidate_bytes(qt, 16, 512, "cpu", g)
        w = torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), 16 * 512))
        assert torch.isfinite(w).all()
        assert abs(float(w.mean())) < 0.01 and 0.01 < float(w.std()) < 0.08 and float(w.abs().max()) < 0.2


def test_teacher_stream_is_opt_in_and_cpu_runs_in_order():
    """The teacher's side stream is off by default, and on a CPU model the
    forwards run in order (no stream), giving the two outputs unchanged."""
    assert st.StepConfig().teacher_stream is False
    student, teacher = nn.Linear(4, 3), nn.Linear(4, 3)
    assert st._make_teacher_stream(st.StepConfig(teacher_stream=True), student) is None
    x = torch.randn(2, 4)
    s_out, t_out = st._forwards(student, teacher, x, None)
    assert torch.equal(s_out, student(x)) and torch.equal(t_out, teacher(x))
    assert s_out.requires_grad and not t_out.requires_grad


def test_fused_path_region():
    """Few-token products take the fused kernels only up to 32 tokens, 2^22
    weights and 2048 output rows (the measured crossover against mix + GEMM)."""
    from voodoo_quant import layers

    assert layers.use_fused(1, 1024, 1024) and layers.use_fused(32, 2048, 2048)
    assert layers.use_fused(16, 1024, 4096)
    assert not layers.use_fused(33, 1024, 1024)
    assert not layers.use_fused(16, 3072, 1024) and not layers.use_fused(16, 4096, 1024)
    assert not layers.use_fused(16, 4096, 4096)
    assert not layers.use_fused(0, 1024, 1024)
    # the documented switch forces the bit-exact materialised path
    saved = layers.FUSED_PRODUCTS
    try:
        layers.FUSED_PRODUCTS = False
        assert not layers.use_fused(1, 1024, 1024)
    finally:
        layers.FUSED_PRODUCTS = saved


def test_softmax_rows_backward_matches_autograd():
    """The Jacobian the gate bank applies to deferred gate gradients equals
    autograd's through softmax(z / T), at the annealing schedule's ends."""
    from voodoo_quant.training import trainer

    g = torch.Generator().manual_seed(5)
    for t in (2.0, 1.0, 0.1):
        z = torch.randn(7, 6, generator=g, dtype=torch.float64, requires_grad=True)
        up = torch.randn(7, 6, generator=g, dtype=torch.float64)
        p = torch.softmax(z / t, dim=1)
        p.backward(up)
        got = trainer.softmax_rows_backward(p.detach(), up, t)
        assert torch.allclose(got, z.grad, rtol=1e-12, atol=1e-14), t
        # rows sum to zero: the softmax is shift-invariant
        assert float(got.sum(dim=1).abs().max()) < 1e-12


def test_gate_bank_defers_only_on_a_rocm_device():
    """Off the GPU a deferring bank sets no sinks and finish() is a no-op."""
    from voodoo_quant.training import trainer

    class _M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.num_candidates = 3
            self.gates = torch.nn.Parameter(torch.zeros(3))

        def _bytes_per_candidate(self):
            return [1.0, 2.0, 3.0]

    mods = [_M(), _M()]
    bank = trainer.GateBank(mods, defer_gate_grads=True)
    b = bank.begin(1.0)
    assert all(m.__dict__.get("_gate_sink") is None for m in mods)
    b.backward()
    bank.finish()
    bank.end()
    (param,) = bank.parameters()
    assert param.grad is not None and param.grad.shape == (2, 3)


def test_candidate_streamer_argument_checks():
    """The streamer needs 1 <= depth < slots (a prefetch must never reach a
    slot whose last user the fence has not covered) and a non-empty product
    list; the checks come before any device work."""
    from voodoo_quant.streaming import CandidateStreamer

    with pytest.raises(ValueError, match="depth"):
        CandidateStreamer([[object()]], "cpu", slots=2, depth=2)
    with pytest.raises(ValueError, match="depth"):
        CandidateStreamer([[object()]], "cpu", slots=4, depth=0)
    with pytest.raises(ValueError, match="no products"):
        CandidateStreamer([], "cpu")
    # streaming excludes the mix prefetch and deferred gate gradients
    with pytest.raises(ValueError, match="streamed candidates"):
        st._make_streamer(st.StepConfig(stream_candidates=True, prefetch_mix=True), nn.Linear(2, 2))


def test_embedding_id_check_modes_on_the_host():
    """check_embedding_ids: "sync" raises IndexError for ids outside the
    table (either end) and passes ids inside it; an unknown mode is a
    ValueError; the training harness defers the check by default."""
    from voodoo_quant import layers

    layers.check_embedding_ids(torch.tensor([0, 9, 3]), 10, "t", "sync")
    layers.check_embedding_ids(torch.empty(0, dtype=torch.int64), 10, "t", "bogus")  # nothing to check
    for bad in ([0, 10], [-1, 3]):
        with pytest.raises(IndexError, match="index out of range"):
            layers.check_embedding_ids(torch.tensor(bad), 10, "t", "sync")
    with pytest.raises(ValueError, match="id_check"):
        layers.check_embedding_ids(torch.tensor([1]), 10, "t", "bogus")
    assert st.StepConfig().deferred_id_check
    assert layers.MixedQuantEmbedding.id_check == "sync"
    layers.raise_pending_id_errors()  # nothing pending


def test_gemm_tuning_file_lists_the_step_shapes():
    """The TunableOp results file carries validators and one tuned solution
    for each plain forward GEMM of the 0.8B-class step (the Q8_0 teacher's four
    projections and the vocabulary head at 8192 tokens); without a ROCm device
    use_tuned_gemms changes nothing."""
    from voodoo_quant.training import step as st

    rows = [line.split(",") for line in st.GEMM_TUNING_FILE.read_text().splitlines()]
    validators = {r[1] for r in rows if r[0] == "Validator"}
    assert {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "GCN_ARCH_NAME", "ROCBLAS_VERSION"} <= validators
    ops = {r[1] for r in rows if r[0].startswith("GemmTunableOp_BFloat16")}
    for n, k in ((1536, 1024), (1024, 1024), (6144, 1024), (1024, 3072), (151936, 1024)):
        assert f"tn_{n}_8192_{k}_ld_{k}_{k}_{n}" in ops
    if not torch.cuda.is_available():
        assert st.use_tuned_gemms() is False


def test_use_tuned_gemms_refuses_other_runtimes(monkeypatch):
    """With validators that differ from the file's (another torch, ROCm or
    library build), use_tuned_gemms warns, returns False and leaves TunableOp
    off; with matching ones it enables it, tuning off, and reads the file."""
    from voodoo_quant.training import step as st

    calls = []

    class FakeTunable:
        def __init__(self, validators):
            self.validators = validators

        def get_validators(self):
            return self.validators

        def enable(self, on=True):
            calls.append(("enable", on))

        def tuning_enable(self, on=True):
            calls.append(("tuning", on))

        def read_file(self, path):
            calls.append(("read", path))
            return True

    rows = [line.split(",") for line in st.GEMM_TUNING_FILE.read_text().splitlines()]
    good = tuple((r[1], ",".join(r[2:])) for r in rows if r[0] == "Validator")
    bad = tuple((k, v + "-other") if k == "HIPBLASLT_VERSION" else (k, v) for k, v in good)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "tunable", FakeTunable(bad))
    with pytest.warns(UserWarning, match="validators"):
        assert st.use_tuned_gemms() is False
    assert calls == []
    monkeypatch.setattr(torch.cuda, "tunable", FakeTunable(good))
    assert st.use_tuned_gemms() is True
    assert ("tuning", False) in calls and ("enable", True) in calls
    assert ("read", str(st.GEMM_TUNING_FILE)) in calls
    assert calls.index(("tuning", False)) < calls.index(("enable", True))
