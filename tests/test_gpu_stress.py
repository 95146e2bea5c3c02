"""The wide-menu stress configuration at a size the oracle's CPU run covers:
a stack of 2 SwiGLU blocks (hidden 512, MLP 1024), every gate/up/down gated
over K = 8 candidates, temperature annealed 2.0 -> 0.1 over 200 steps.  Two
menus: repeated K-quants (Q2_K, Q3_K, Q4_K, Q4_K, Q5_K, Q6_K, Q6_K, Q8_0) and
eight distinct formats, four of them IQ (IQ1_S, IQ2_XXS, Q2_K, IQ3_S, IQ4_XS,
Q5_K, Q6_K, Q8_0).

The HIP side is the product's stress harness (``training.step.StackTrainer``:
stacked gate/up projections, the fused add + RMSNorm and SwiGLU kernels, the
gate bank, the Q8_0 teacher).  The oracle side restates the reference's step
on the CPU in the model's bf16 (``voodoo_quant/layers.py:336-363, 1729-1731``:
fp32 k-ordered mixture, cast to bf16, ``F.linear``; ``trainer.py:199-203,
2378-2379, 2577-2616``: anneal, dead-zone size loss, AdamW + cosine + clip
1.0), with the same candidate bytes and data.  The per-tensor argmax after
the run must be identical.

Candidates are the labelled non-ggml RTN encoder's bytes of one normal
source weight per tensor (std 0.01 in the first block, 0.05 in the second,
so the second block's error weighs more).  A repeated format's second copy
quantizes the source weight plus noise of 0.3 times its std: its own bytes,
the same byte cost, a larger error.  The teacher is the Q8_0 encoding of the
source weight.  The budget (45% of 8-bit) then gives the two blocks
different winners, and a size-only control run ends elsewhere, so the
GEMM gradients decide the result.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import cdequant, mixture
from voodoo_quant import ggml, rtn

TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q4_K", "Q5_K", "Q6_K", "Q6_K", "Q8_0"]
# eight distinct formats from 1.56 to 8.5 bits per weight, four of them IQ
IQ_TYPES = ["IQ1_S", "IQ2_XXS", "Q2_K", "IQ3_S", "IQ4_XS", "Q5_K", "Q6_K", "Q8_0"]
BLOCKS, HIDDEN, MLP = 2, 512, 1024
TOKENS = 256
STEPS, T0, T1 = 200, 2.0, 0.1
LR, SIZE_WEIGHT, SIZE_TOL, TARGET_FRAC = 0.05, 10.0, 0.02, 0.45
EPS = 1e-6
# source-weight scale per block: the second block's output dominates the
# residual stream, so its quantization error weighs more in the loss
STDS = (0.01, 0.05)
SHAPES = {"mlp.gate_proj": (MLP, HIDDEN), "mlp.up_proj": (MLP, HIDDEN), "mlp.down_proj": (HIDDEN, MLP)}


def _problem(seed=0, stds=STDS, types=TYPES):
    """{tensor name: (candidate bytes [K] (uint8, CPU), teacher Q8_0 bytes, (o, i))} and the input."""
    g = torch.Generator().manual_seed(seed)
    tensors = {}
    for b in range(BLOCKS):
        for n, (o, i) in SHAPES.items():
            w = torch.randn(o, i, generator=g) * stds[b]
            seen = set()
            qbs = []
            for qt in types:
                src = w if qt not in seen else w + torch.randn(o, i, generator=g) * (0.3 * stds[b])
                seen.add(qt)
                qbs.append(rtn.rtn_quantize_tensor(src, qt).reshape(-1))
            tensors[f"blocks.{b}.{n}"] = (qbs, rtn.rtn_quantize_tensor(w, "Q8_0").reshape(-1), (o, i))
    x = torch.randn(TOKENS, HIDDEN, generator=g).to(torch.bfloat16)
    return tensors, x


def _decode(qt, qb, o, i):
    return torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), o * i).reshape(o, i))


def _reference_run(tensors, x, steps=STEPS, with_mse=True, types=TYPES, cand_dtype=torch.float32):
    """The reference's step on the CPU in bf16; returns {name: final gates}.
    cand_dtype: the precision each decoded candidate is stored in before the
    mixture (bf16 is the reference's default non-lazy storage,
    ``layers.py:1308-1312``)."""
    cands = {nm: [_decode(qt, qb, *shape).to(cand_dtype).float() for qt, qb in zip(types, qbs)]
             for nm, (qbs, _, shape) in tensors.items()}
    teach = {nm: _decode("Q8_0", tq, *shape).to(torch.bfloat16) for nm, (_, tq, shape) in tensors.items()}
    norm = torch.ones(HIDDEN, dtype=torch.bfloat16)
    gates = {nm: torch.zeros(len(types), requires_grad=True) for nm in tensors}
    bpw = [ggml.bytes_per_weight(qt) for qt in types]
    n_weights = sum(o * i for _, _, (o, i) in tensors.values())
    target = TARGET_FRAC * n_weights  # of one byte per weight
    opt, sched = mixture.make_gate_optimizer(list(gates.values()), LR, steps)

    def model(weights):
        h = x
        for b in range(BLOCKS):
            n = F.rms_norm(h, (HIDDEN,), norm, EPS)
            wg, wu, wd = (weights[f"blocks.{b}.{k}"] for k in SHAPES)
            h = h + F.linear(F.silu(F.linear(n, wg)) * F.linear(n, wu), wd)
        return h

    with torch.no_grad():
        t = model(teach).float()
    for step in range(steps):
        tau = mixture.anneal_temperature(step, steps, T0, T1)
        weights, total = {}, 0.0
        for nm, (qbs, _, (o, i)) in tensors.items():
            p = mixture.soft_probs(gates[nm], tau)
            w_eff = torch.zeros(o, i)
            for k, c in enumerate(cands[nm]):
                w_eff = w_eff + p[k] * c
            weights[nm] = w_eff.to(torch.bfloat16)
            total = total + mixture.effective_bytes(p, bpw, o * i)
        y = model(weights)
        mse = ((y.float() - t) ** 2).mean() / (t ** 2).mean()
        loss = (mse if with_mse else 0.0) + SIZE_WEIGHT * mixture.size_loss(total, target, SIZE_TOL)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(list(gates.values()), max_norm=1.0)
        opt.step()
        sched.step()
        opt.zero_grad()
    return {nm: g.detach() for nm, g in gates.items()}


def _hip_run(tensors, x, steps=STEPS, types=TYPES):
    from voodoo_quant import layers
    from voodoo_quant.training import q8_teacher
    from voodoo_quant.training import step as st
    from voodoo_quant.training.q8_teacher import Q8Linear

    # the teacher as the product's stack builder runs it (decodes kept, gate/up
    # as one stacked GEMM), whatever an earlier caller left the switch at
    keep = q8_teacher._KEEP_DECODED
    q8_teacher.set_keep_decoded(True)
    try:
        return _hip_run_body(tensors, x, steps, types, layers, st, Q8Linear)
    finally:
        q8_teacher.set_keep_decoded(keep)


def _hip_run_body(tensors, x, steps, types, layers, st, Q8Linear):
    dev = torch.device("cuda", 0)
    cfg = st.StackConfig(blocks=BLOCKS, hidden=HIDDEN, mlp=MLP, eps=EPS)
    replaced, s_blocks, t_blocks = {}, [], []
    for b in range(BLOCKS):
        lin, tlin = {}, {}
        for n, (o, i) in SHAPES.items():
            nm = f"blocks.{b}.{n}"
            qbs, tq, _ = tensors[nm]
            lin[n] = layers.MixedQuantLinear.from_packed(i, o, types, [q.to(dev) for q in qbs], tensor_name=nm,
                                                         device=dev)
            replaced[nm] = lin[n]
            tlin[n] = Q8Linear(tq.to(dev), o, i)
        s_blocks.append(lin)
        t_blocks.append(tlin)
    student = st.SwiGLUStack(cfg, s_blocks, dev)
    teacher = st.SwiGLUStack(cfg, t_blocks, dev)
    teacher.requires_grad_(False)
    tr = st.StackTrainer(student, teacher, replaced,
                         st.StepConfig(max_steps=steps, lr=LR, temp_start=T0, temp_end=T1, size_weight=SIZE_WEIGHT,
                                       size_tolerance=SIZE_TOL, target_fraction=TARGET_FRAC),
                         total_8bit_bytes=float(cfg.gated_weights()))
    xd = x.to(dev)
    for _ in range(steps):
        tr.step(xd)
    torch.cuda.synchronize()
    return {nm: m.gates.detach().cpu() for nm, m in replaced.items()}


@pytest.mark.gpu
@pytest.mark.parametrize("cand_dtype", [torch.float32, torch.bfloat16], ids=["fp32-candidates", "bf16-candidates"])
@pytest.mark.parametrize("types", [TYPES, IQ_TYPES], ids=["repeated-k-quants", "iq-menu"])
def test_stress_stack_k8_argmax_matches_reference(types, cand_dtype):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    tensors, x = _problem(types=types)
    print(f"[stress] {types}, {cand_dtype} candidates: reference run on the CPU", flush=True)
    ref = _reference_run(tensors, x, types=types, cand_dtype=cand_dtype)
    print("[stress] HIP run", flush=True)
    got = _hip_run(tensors, x, types=types)
    worst = 0.0
    for nm in tensors:
        r, g = ref[nm], got[nm]
        d = float((r - g).abs().max())
        worst = max(worst, d)
        print(f"{nm}: reference {types[int(r.argmax())]}#{int(r.argmax())} {r.numpy().round(3)}  "
              f"hip {types[int(g.argmax())]}#{int(g.argmax())} {g.numpy().round(3)}  max|diff| {d:.2e}", flush=True)
    for nm in tensors:
        assert int(ref[nm].argmax()) == int(got[nm].argmax()), nm
    print(f"[stress] gates agree to {worst:.2e}", flush=True)
    assert worst < (GATE_TOL if cand_dtype == torch.float32 else GATE_TOL_BF16)
    if cand_dtype != torch.float32:
        return  # the control run below depends on the data only
    # not degenerate: more than one winner, and the loss's GEMM gradients decide
    assert len({int(r.argmax()) for r in ref.values()}) >= 2
    ctrl = _reference_run(tensors, x, with_mse=False, types=types)
    assert any(int(ref[nm].argmax()) != int(ctrl[nm].argmax()) for nm in tensors)


# largest gate difference accepted (gate logits are O(1), the winners' margins
# 0.07-0.3); measured on MI355X after the 200 steps: 6.5e-4 (repeated
# K-quants) and 2.1e-3 (IQ menu, whose winners sit closer together).  The
# teacher's GEMM order alone moves the IQ menu's figure between 8.8e-4 (one
# GEMM per projection) and 2.1e-3 (gate/up stacked).
GATE_TOL = 3e-3
# against bf16-stored candidates (the reference's default storage): on the CPU
# the bf16- and fp32-candidate reference runs end at most 1.2e-3 apart, on the
# same winners
GATE_TOL_BF16 = 1e-2


def reference_margins(types=TYPES, with_mse=True):
    """CPU-only helper: the reference run's winners and their logit margins."""
    tensors, x = _problem(types=types)
    ref = _reference_run(tensors, x, with_mse=with_mse, types=types)
    out = []
    for nm, r in ref.items():
        s = r.sort(descending=True).values
        out.append((nm, types[int(r.argmax())], int(r.argmax()), float(s[0] - s[1]), r.numpy().round(3)))
    return out
