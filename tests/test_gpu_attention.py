"""The decoder step's causal attention forward (``vq_attention_fwd``) on the
GPU against an fp32 torch reference of softmax(q k^T * scale + causal mask) v
on the same bf16 inputs, and paired with torch's memory-efficient attention
backward through the log-sum-exp it saves.

Bars: the output within 1e-2 relative L2 of fp32 (and no worse than 1.5x
torch's own bf16 SDPA error on the same inputs + 1e-3); the log-sum-exp within
1e-4 (absolute, natural log) of fp32; the gradients from torch's backward over
this forward within 1e-2 relative L2 of fp32 autograd.
"""

import math

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")


def _inputs(B, Hq, Hk, S, layout, seed, mag=1.0):
    g = torch.Generator().manual_seed(seed)

    def mk(h):
        x = (torch.randn(B, S, h, 64, generator=g) * mag).to(torch.bfloat16).cuda()
        return x.transpose(1, 2) if layout == "bshd" else x.transpose(1, 2).contiguous()

    return mk(Hq), mk(Hk), mk(Hk)


def _ref(q, k, v, scale):
    """fp32 causal attention and its log-sum-exp, per batch to bound memory."""
    rep = q.shape[1] // k.shape[1]
    outs, lses = [], []
    S = q.shape[2]
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1)
    for b in range(q.shape[0]):
        qf = q[b].float()
        kf = k[b].float().repeat_interleave(rep, 0)
        vf = v[b].float().repeat_interleave(rep, 0)
        s = (qf @ kf.transpose(-1, -2)) * scale
        s = s.masked_fill(mask, float("-inf"))
        lses.append(torch.logsumexp(s, -1))
        outs.append(torch.softmax(s, -1) @ vf)
    return torch.stack(outs), torch.stack(lses)


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30))


CASES = [  # B, Hq, Hk, S, layout, magnitude
    (1, 1, 1, 1, "bhsd", 1.0),
    (1, 2, 2, 64, "bshd", 1.0),
    (2, 4, 1, 65, "bshd", 1.0),
    (1, 4, 4, 129, "bhsd", 1.0),
    (2, 8, 2, 300, "bshd", 2.0),
    (1, 16, 4, 1000, "bshd", 1.0),
    (1, 3, 3, 777, "bhsd", 4.0),  # peaked softmax: the running maximum moves
    (4, 16, 16, 2048, "bshd", 1.0),  # the 0.8B-class step: 4 x 2048, 16 heads of 64
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}_H{c[1]}_{c[2]}_S{c[3]}_{c[4]}" for c in CASES])
def test_attention_forward_matches_fp32(case):
    _need_gpu()
    from voodoo_quant import _hip

    B, Hq, Hk, S, layout, mag = case
    print(f"[attention] B={B} Hq={Hq} Hk={Hk} S={S} {layout} x{mag}", flush=True)
    q, k, v = _inputs(B, Hq, Hk, S, layout, seed=S + Hq, mag=mag)
    scale = 1.0 / math.sqrt(64)
    out, lse = _hip.attention_fwd(q, k, v)
    torch.cuda.synchronize()
    o_ref, lse_ref = _ref(q, k, v, scale)
    err = _rel(out, o_ref)
    rep = Hq // Hk
    torch_out = F.scaled_dot_product_attention(q, k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1),
                                               is_causal=True)
    torch_err = _rel(torch_out, o_ref)
    lse_err = float((lse - lse_ref).abs().max())
    print(f"[attention] out rel {err:.2e} (torch {torch_err:.2e}), lse max abs {lse_err:.2e}", flush=True)
    assert err < 1e-2 and err <= 1.5 * torch_err + 1e-3
    assert lse_err < 1e-4 * max(1.0, float(lse_ref.abs().max()))
    assert out.shape == (B, Hq, S, 64) and out.transpose(1, 2).is_contiguous()


def test_attention_forward_without_lse_and_custom_scale():
    _need_gpu()
    from voodoo_quant import _hip

    q, k, v = _inputs(2, 4, 2, 200, "bshd", seed=3)
    out, lse = _hip.attention_fwd(q, k, v, scale=0.05, need_lse=False)
    assert lse is None
    o_ref, _ = _ref(q, k, v, 0.05)
    assert _rel(out, o_ref) < 1e-2
    # bit-identical with and without the saved log-sum-exp
    out2, _ = _hip.attention_fwd(q, k, v, scale=0.05)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("S", [300, 2048])
def test_attention_forward_pairs_with_torch_backward(S):
    """Gradients of torch's memory-efficient backward over this forward's
    output and log-sum-exp match fp32 autograd (and torch's own pairing)."""
    _need_gpu()
    from voodoo_quant import _hip

    B, H = 2, 8
    print(f"[attention] backward pairing S={S}", flush=True)
    q, k, v = _inputs(B, H, H, S, "bshd", seed=11 + S)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(B, S, H, 64, generator=g).to(torch.bfloat16).cuda().transpose(1, 2)
    scale = 1.0 / math.sqrt(64)
    out, lse = _hip.attention_fwd(q, k, v)
    seed0 = torch.zeros((), dtype=torch.int64)
    dq, dk, dv, _ = torch.ops.aten._scaled_dot_product_efficient_attention_backward(
        dout, q, k, v, None, out, lse, seed0, seed0, 0.0, [True, True, True, False], True, scale=scale)
    qf, kf, vf = (t.detach().float().requires_grad_(True) for t in (q, k, v))
    mask = torch.ones(S, S, dtype=torch.bool, device="cuda").triu(1)
    s = (qf @ kf.transpose(-1, -2)) * scale
    o = torch.softmax(s.masked_fill(mask, float("-inf")), -1) @ vf
    o.backward(dout.float())
    for name, got, want in (("dq", dq, qf.grad), ("dk", dk, kf.grad), ("dv", dv, vf.grad)):
        err = _rel(got, want)
        print(f"[attention] {name} rel {err:.2e}", flush=True)
        assert err < 1e-2, name


def test_step_attention_matches_sdpa_forward_and_backward():
    """The decoder step's attention (HIP forward and backward; HIP forward with
    torch's backward) against torch's SDPA forward and backward, all against
    fp32 autograd; grouped-query heads are repeated before each."""
    _need_gpu()
    from voodoo_quant.training import step as st

    B, Hq, Hk, S = 2, 8, 2, 512
    q, k, v = _inputs(B, Hq, Hk, S, "bshd", seed=21)
    g = torch.Generator().manual_seed(2)
    dout = torch.randn(B, Hq, S, 64, generator=g).to(torch.bfloat16).cuda()
    res = {}
    saved = st.HIP_ATTENTION, st.HIP_ATTENTION_BWD
    try:
        for flag in ("hip", "hip_fwd", False):
            st.HIP_ATTENTION = bool(flag)
            st.HIP_ATTENTION_BWD = flag == "hip"
            qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
            out = st._attention(qq, kk, vv)
            out.backward(dout)
            res[flag] = (out.detach(), qq.grad, kk.grad, vv.grad)
            with torch.no_grad():  # the teacher's path: no log-sum-exp, same output
                assert torch.equal(st._attention(q, k, v), out.detach()) or not flag
    finally:
        st.HIP_ATTENTION, st.HIP_ATTENTION_BWD = saved
    qf, kf, vf = (t.detach().float().requires_grad_(True) for t in (q, k, v))
    rep = Hq // Hk
    mask = torch.ones(S, S, dtype=torch.bool, device="cuda").triu(1)
    s = (qf @ kf.repeat_interleave(rep, 1).transpose(-1, -2)) / 8.0
    o = torch.softmax(s.masked_fill(mask, float("-inf")), -1) @ vf.repeat_interleave(rep, 1)
    o.backward(dout.float())
    want = (o.detach(), qf.grad, kf.grad, vf.grad)
    for i, name in enumerate(("out", "dq", "dk", "dv")):
        torch_err = _rel(res[False][i], want[i])
        for mode in ("hip", "hip_fwd"):
            hip_err = _rel(res[mode][i], want[i])
            print(f"[attention] step {name} ({mode}): {hip_err:.2e}, torch {torch_err:.2e}", flush=True)
            assert hip_err < 1e-2 and hip_err <= 1.5 * torch_err + 1e-3, (name, mode)


BWD_CASES = [  # B, H, S, magnitude
    (1, 1, 1, 1.0),
    (1, 2, 64, 1.0),
    (2, 3, 65, 1.0),
    (1, 4, 129, 2.0),
    (2, 8, 300, 1.0),
    (1, 3, 777, 4.0),  # peaked softmax
    (4, 16, 2048, 1.0),  # the 0.8B-class step
]


@pytest.mark.parametrize("case", BWD_CASES, ids=[f"B{c[0]}_H{c[1]}_S{c[2]}_x{c[3]}" for c in BWD_CASES])
def test_attention_backward_matches_fp32(case):
    """vq_attention_bwd's dq, dk, dv against fp32 autograd of the causal
    softmax attention on the same bf16 inputs, and no worse than 1.5x torch's
    memory-efficient backward on the same forward (+ 1e-3); bit-identical when
    run twice (no atomics)."""
    _need_gpu()
    from voodoo_quant import _hip

    B, H, S, mag = case
    print(f"[attention] backward B={B} H={H} S={S} x{mag}", flush=True)
    q, k, v = _inputs(B, H, H, S, "bshd", seed=7 * S + H, mag=mag)
    g = torch.Generator().manual_seed(S)
    dout = torch.randn(B, S, H, 64, generator=g).to(torch.bfloat16).cuda().transpose(1, 2)
    scale = 1.0 / math.sqrt(64)
    out, lse = _hip.attention_fwd(q, k, v)
    dq, dk, dv = _hip.attention_bwd(dout, q, k, v, out, lse)
    again = _hip.attention_bwd(dout, q, k, v, out, lse)
    assert all(torch.equal(a, b) for a, b in zip((dq, dk, dv), again))
    zero = torch.zeros((), dtype=torch.int64)
    tq, tk, tv, _ = torch.ops.aten._scaled_dot_product_efficient_attention_backward(
        dout, q, k, v, None, out, lse, zero, zero, 0.0, [True, True, True, False], True, scale=scale)
    want = []
    for b in range(B):  # fp32 autograd per batch to bound memory
        qf, kf, vf = (t[b].detach().float().requires_grad_(True) for t in (q, k, v))
        mask = torch.ones(S, S, dtype=torch.bool, device="cuda").triu(1)
        s = (qf @ kf.transpose(-1, -2)) * scale
        o = torch.softmax(s.masked_fill(mask, float("-inf")), -1) @ vf
        o.backward(dout[b].float())
        want.append((qf.grad, kf.grad, vf.grad))
    for i, (name, got, ref_t) in enumerate((("dq", dq, tq), ("dk", dk, tk), ("dv", dv, tv))):
        w = torch.stack([x[i] for x in want])
        # relative L2 with a floor of 1e-3 on the reference's norm: at S = 1
        # dq and dk are zero and both sides leave ~1e-7 of fp32 cancellation
        den = max(float(w.float().norm()), 1e-3)
        err = float((got.float() - w).norm()) / den
        terr = float((ref_t.float() - w).norm()) / den
        print(f"[attention] {name} rel {err:.2e} (torch {terr:.2e})", flush=True)
        assert err < 1e-2 and err <= 1.5 * terr + 1e-3, name


GQA_CASES = [  # B, Hq, Hk, S, magnitude
    (1, 4, 1, 65, 1.0),
    (2, 8, 2, 300, 1.0),
    (1, 6, 3, 777, 4.0),
    (4, 16, 4, 2048, 1.0),  # the 0.8B-class step's heads
]


@pytest.mark.parametrize("case", GQA_CASES, ids=[f"B{c[0]}_H{c[1]}_{c[2]}_S{c[3]}_x{c[4]}" for c in GQA_CASES])
def test_attention_backward_grouped_kv(case):
    """vq_attention_bwd with Hk < Hq K/V heads: dq and the per-query-head dk,
    dv bit for bit those of the same call on K/V repeated to Hq heads; the
    group sums of dk, dv against fp32 autograd through the repeat (1e-2
    relative L2)."""
    _need_gpu()
    from voodoo_quant import _hip

    B, Hq, Hk, S, mag = case
    rep = Hq // Hk
    print(f"[attention] grouped backward B={B} Hq={Hq} Hk={Hk} S={S} x{mag}", flush=True)
    q, k, v = _inputs(B, Hq, Hk, S, "bshd", seed=3 * S + Hq, mag=mag)
    g = torch.Generator().manual_seed(S + 1)
    dout = torch.randn(B, S, Hq, 64, generator=g).to(torch.bfloat16).cuda().transpose(1, 2)
    out, lse = _hip.attention_fwd(q, k, v)
    grads = _hip.attention_bwd(dout, q, k, v, out, lse)
    kr, vr = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
    out_r, lse_r = _hip.attention_fwd(q, kr, vr)
    assert torch.equal(out, out_r) and torch.equal(lse, lse_r)
    grads_r = _hip.attention_bwd(dout, q, kr, vr, out_r, lse_r)
    for name, a, b_ in zip(("dq", "dk", "dv"), grads, grads_r):
        assert a.shape == (B, Hq, S, 64), name
        assert torch.equal(a, b_), name
    scale = 1.0 / math.sqrt(64)
    mask = torch.ones(S, S, dtype=torch.bool, device="cuda").triu(1)
    for bi in range(B):  # fp32 autograd per batch to bound memory
        qf, kf, vf = (t[bi].detach().float().requires_grad_(True) for t in (q, k, v))
        s_ = (qf @ kf.repeat_interleave(rep, 0).transpose(-1, -2)) * scale
        o = torch.softmax(s_.masked_fill(mask, float("-inf")), -1) @ vf.repeat_interleave(rep, 0)
        o.backward(dout[bi].float())
        for name, got, want in (("dq", grads[0][bi], qf.grad),
                                ("dk", grads[1][bi].float().unflatten(0, (Hk, rep)).sum(1), kf.grad),
                                ("dv", grads[2][bi].float().unflatten(0, (Hk, rep)).sum(1), vf.grad)):
            err = float((got.float() - want).norm()) / max(float(want.norm()), 1e-3)
            print(f"[attention] batch {bi} {name} rel {err:.2e}", flush=True)
            assert err < 1e-2, (bi, name)


def test_step_rope_attention_node_matches_unfused():
    """The decoder step's rotary + attention node (K/V at their own heads)
    against the rotary node with repeated heads followed by the attention
    node: output and the stacked projection's gradient bit for bit with the
    HIP backward, and the no-grad path's output the same; with torch's
    backward, within 1e-2 of fp32 autograd."""
    _need_gpu()
    from voodoo_quant.training import step as st

    b, s, hq, hkv, d = 2, 300, 8, 2, 64
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(b * s, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).cuda()
    dout = torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16).cuda()
    cos, sin = st._rope_tables_f32(s, d, 1.0e6, "cuda")
    shape = (b, s, hq, hkv, d)

    def fused():
        x = qkv.detach().clone().requires_grad_(True)
        out = st._rope_attention(x, cos, sin, shape)
        out.backward(dout)
        return out.detach(), x.grad

    def unfused():
        x = qkv.detach().clone().requires_grad_(True)
        q, k, v = st._RopeQKV.apply(x, cos, sin, shape)
        out = st._CausalAttention.apply(q, k, v)
        out.backward(dout)
        return out.detach(), x.grad

    saved = st.HIP_ATTENTION_BWD
    try:
        st.HIP_ATTENTION_BWD = True
        (o1, g1), (o2, g2) = fused(), unfused()
        assert torch.equal(o1, o2) and torch.equal(g1, g2)
        with torch.no_grad():
            assert torch.equal(st._rope_attention(qkv, cos, sin, shape), o1)
        st.HIP_ATTENTION_BWD = False
        o3, g3 = fused()
        assert torch.equal(o3, o1)
    finally:
        st.HIP_ATTENTION_BWD = saved
    # fp32 autograd of rotary + attention with the K/V heads repeated
    xr = qkv.float().cpu().requires_grad_(True)
    c, sn = cos.cpu(), sin.cpu()
    half = d // 2

    def rope(t):
        return t * c + torch.cat([-t[..., half:], t[..., :half]], dim=-1) * sn

    qr = rope(xr[:, : hq * d].view(b, s, hq, d).transpose(1, 2))
    kr = rope(xr[:, hq * d:(hq + hkv) * d].view(b, s, hkv, d).transpose(1, 2)).repeat_interleave(hq // hkv, 1)
    vr = xr[:, (hq + hkv) * d:].view(b, s, hkv, d).transpose(1, 2).repeat_interleave(hq // hkv, 1)
    mask = torch.ones(s, s, dtype=torch.bool).triu(1)
    o = torch.softmax(((qr @ kr.transpose(-1, -2)) / 8.0).masked_fill(mask, float("-inf")), -1) @ vr
    o.backward(dout.float().cpu())
    for name, got in (("HIP backward", g1), ("torch backward", g3)):
        err = _rel(got.cpu(), xr.grad)
        print(f"[attention] rotary + attention node, {name}: dqkv rel {err:.2e}", flush=True)
        assert err < 1e-2, name
