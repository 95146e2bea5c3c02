"""Streamed candidates (``voodoo_quant.streaming.CandidateStreamer``): the
gated products' packed bytes in pinned host memory, copied into a ring of
device slots before each product, in stream order (the reference's host ->
device copies, ``layers.py:348, 362``) or ahead of use on a copy stream.

The kernels and bytes are the same as with resident candidates, so training
steps must be bit-identical: the SwiGLU stack (no attention) bitwise over
three steps, with two slots (every slot reused by three products, the
forward's last products reused by the backward, product 0 by the next step)
and with four slots three products ahead, and the decoder (its attention
kernels sum in a fixed order) bitwise over three steps.
"""

import pytest
import torch

from voodoo_quant.training import step as st

pytestmark = pytest.mark.gpu

TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q6_K", "Q8_0"]
STEPS = 3


def _stack_run(**stream):
    dev = torch.device("cuda", 0)
    cfg = st.StackConfig(blocks=3, hidden=512, mlp=1024)
    student, teacher, replaced = st.build_stack(cfg, TYPES, dev, seed=4)
    tr = st.StackTrainer(student, teacher, replaced,
                         st.StepConfig(max_steps=STEPS, temp_start=2.0, temp_end=0.1, **stream),
                         float(cfg.gated_weights()))
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(300, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    losses = []
    for _ in range(STEPS):
        out = tr.step(x)
        losses.append(torch.stack([out["mse"].float(), out["size"].float()]))
    torch.cuda.synchronize()
    gates = torch.cat([m.gates.detach().reshape(-1) for m in replaced.values()])
    return gates, torch.stack(losses), tr.streamer


def test_stack_steps_bit_identical_with_streamed_candidates():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    ref_g, ref_l, none = _stack_run()
    assert none is None
    copied = {}
    for kw in ({"stream_overlap": False, "stream_slots": 2, "stream_depth": 1},
               {"stream_slots": 2, "stream_depth": 1},
               {"stream_slots": 4, "stream_depth": 3}):
        g, losses, streamer = _stack_run(stream_candidates=True, **kw)
        print(f"[streaming] {kw}: {streamer.bytes_copied / 2**20:.1f} MiB copied over {STEPS} steps, "
              f"{len(streamer.products)} products", flush=True)
        assert torch.equal(g.view(torch.int32), ref_g.view(torch.int32)), kw
        assert torch.equal(losses.view(torch.int32), ref_l.view(torch.int32)), kw
        # the host holds the candidates; every product was copied at least
        # once, and slots still holding a product are reused (fewer copies
        # with more slots)
        assert all(not m._qweight_0.is_cuda and m._qweight_0.is_pinned()
                   for mods in streamer.products for m in mods)
        assert streamer.bytes_copied >= sum(streamer.product_bytes)
        copied[kw["stream_slots"]] = streamer.bytes_copied
    assert copied[4] < copied[2]


def test_decoder_steps_match_with_streamed_candidates():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    dev = torch.device("cuda", 0)
    cfg = st.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, mlp=512, vocab=1000)

    def run(**stream):
        torch.manual_seed(0)
        student, teacher, replaced = st.build_models(cfg, TYPES, dev, seed=6, packed=True)
        tr = st.GateTrainer(student, teacher, replaced, st.StepConfig(max_steps=STEPS, **stream),
                            float(cfg.gated_weights()))
        g = torch.Generator(device=dev).manual_seed(5)
        x = torch.randint(0, cfg.vocab, (2, 64), device=dev, generator=g)
        y = torch.randint(0, cfg.vocab, (2, 64), device=dev, generator=g)
        for _ in range(STEPS):
            tr.step(x, y)
        torch.cuda.synchronize()
        return torch.cat([m.gates.detach().reshape(-1) for m in replaced.values()])

    ref = run()
    got = run(stream_candidates=True, stream_slots=3, stream_depth=2)
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), float((got - ref).abs().max())


def test_streamed_modules_refuse_ptqr_and_release_back():
    """A streamed module refuses PTQR routing (its candidates live in the slots
    only while their product runs); release() gives every module resident
    device copies of its bytes back, bit-identical to the host copies, and
    the modules then run unstreamed with the same outputs."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import layers
    from voodoo_quant.streaming import CandidateStreamer

    dev = torch.device("cuda", 0)
    cfg = st.StackConfig(blocks=1, hidden=512, mlp=1024)
    student, _, replaced = st.build_stack(cfg, TYPES, dev, seed=8)
    mods = list(replaced.values())
    x = torch.randn(64, cfg.hidden, device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    x = x.to(torch.bfloat16)
    before = [m(x) for m in mods if m.in_features == cfg.hidden]
    streamer = CandidateStreamer([[m] for m in mods], dev, slots=2, depth=1)
    layers.set_ptqr(True)
    try:
        with pytest.raises(RuntimeError, match="PTQR"):
            mods[0](x)
    finally:
        layers.set_ptqr(False)
    host = [[getattr(m, f"_qweight_{k}").clone() for k in range(m.num_candidates)] for m in mods]
    streamer.release()
    torch.cuda.synchronize()
    for m, hq in zip(mods, host):
        assert m.__dict__.get("_streamer") is None
        for k, h in enumerate(hq):
            q = getattr(m, f"_qweight_{k}")
            assert q.is_cuda and torch.equal(q.cpu(), h)
    after = [m(x) for m in mods if m.in_features == cfg.hidden]
    assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(before, after))


def test_streamer_timeline():
    """timeline=True records every copy (end after start) and every fence
    (forward fences in product order, then backward fences in reverse), with
    the same results as without it; timeline_ms clears the record."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    ref_g, ref_l, _ = _stack_run(stream_candidates=True, stream_slots=4, stream_depth=3)
    dev = torch.device("cuda", 0)
    cfg = st.StackConfig(blocks=3, hidden=512, mlp=1024)
    student, teacher, replaced = st.build_stack(cfg, TYPES, dev, seed=4)
    tr = st.StackTrainer(student, teacher, replaced,
                         st.StepConfig(max_steps=STEPS, temp_start=2.0, temp_end=0.1, stream_candidates=True,
                                       stream_slots=4, stream_depth=3, stream_timeline=True),
                         float(cfg.gated_weights()))
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(300, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    origin = torch.cuda.Event(enable_timing=True)
    origin.record()
    for _ in range(STEPS):
        tr.step(x)
    torch.cuda.synchronize()
    gates = torch.cat([m.gates.detach().reshape(-1) for m in replaced.values()])
    assert torch.equal(gates.view(torch.int32), ref_g.view(torch.int32))
    events = tr.streamer.timeline_ms(origin)
    n = len(tr.streamer.products)
    copies = [e for e in events if e[0] == "copy"]
    assert copies and all(0.0 <= a <= b for _, _, a, b in copies)
    fwd = [i for kind, i, _, _ in events if kind == "forward"]
    bwd = [i for kind, i, _, _ in events if kind == "backward"]
    assert fwd == list(range(n)) * STEPS and bwd == list(range(n - 1, -1, -1)) * STEPS
    assert tr.streamer.timeline == []
