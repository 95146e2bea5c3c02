"""The decoder glue kernels of the step harness (rotary embedding with
grouped-query K/V expansion, SwiGLU, residual add + RMSNorm) against fp32
torch, forward and backward.  Bar: 1e-2 relative L2 (bf16 inputs and
outputs, fp32 inside); the residual add is torch's bf16 add bit for bit."""

import pytest
import torch

from voodoo_quant.training import step as st

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float((a.double() - b.double()).norm() / max(float(b.double().norm()), 1e-30))


def _rope_ref(x, cos, sin):
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rot * sin


@pytest.mark.parametrize("b,s,hq,hkv,d", [(2, 48, 8, 2, 64), (1, 33, 4, 4, 32), (3, 16, 6, 3, 128)])
def test_rope_qkv_matches_torch(b, s, hq, hkv, d):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    print(f"[rope] b={b} s={s} hq={hq} hkv={hkv} d={d}", flush=True)
    g = torch.Generator().manual_seed(s)
    w = (hq + 2 * hkv) * d
    qkv = torch.randn(b * s, w, generator=g).to(torch.bfloat16)
    cos, sin = st._rope_tables_f32(s, d, 1.0e6, "cuda")
    # fused
    x = qkv.cuda().requires_grad_(True)
    q, k, v = st._RopeQKV.apply(x, cos, sin, (b, s, hq, hkv, d))
    gq, gk, gv = (torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16) for _ in range(3))
    (q.float() * gq.cuda().float()).sum().add((k.float() * gk.cuda().float()).sum()).add(
        (v.float() * gv.cuda().float()).sum()).backward()
    # reference in fp32
    xr = qkv.float().requires_grad_(True)
    qr = xr[:, : hq * d].view(b, s, hq, d).transpose(1, 2)
    kr = xr[:, hq * d:(hq + hkv) * d].view(b, s, hkv, d).transpose(1, 2)
    vr = xr[:, (hq + hkv) * d:].view(b, s, hkv, d).transpose(1, 2)
    c, sn = cos.cpu(), sin.cpu()
    qr, kr = _rope_ref(qr, c, sn), _rope_ref(kr, c, sn)
    rep = hq // hkv
    kr, vr = kr.repeat_interleave(rep, 1), vr.repeat_interleave(rep, 1)
    (qr * gq.float()).sum().add((kr * gk.float()).sum()).add((vr * gv.float()).sum()).backward()
    assert _rel(q.cpu(), qr.detach()) < 1e-2 and _rel(k.cpu(), kr.detach()) < 1e-2
    assert torch.equal(v.cpu().float(), vr.detach())  # a copy, exact
    assert _rel(x.grad.cpu(), xr.grad) < 1e-2


@pytest.mark.parametrize("b,s,hq,hkv,d", [(2, 48, 8, 2, 64), (1, 33, 4, 4, 32)])
def test_rope_qkv_unrepeated_kv_matches_repeated(b, s, hq, hkv, d):
    """kv_heads_out = Hkv writes each K/V head once: bit for bit every copy
    of it in the repeated output, with q unchanged."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    g = torch.Generator().manual_seed(s + hq)
    qkv = torch.randn(b * s, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).cuda()
    cos, sin = st._rope_tables_f32(s, d, 1.0e6, "cuda")
    q1, k1, v1 = _hip.rope_qkv_fwd(qkv, b, s, hq, hkv, d, cos, sin)
    q2, k2, v2 = _hip.rope_qkv_fwd(qkv, b, s, hq, hkv, d, cos, sin, repeat_kv=False)
    rep = hq // hkv
    assert k2.shape == (b * s, hkv, d) and v2.shape == (b * s, hkv, d)
    assert torch.equal(q1, q2)
    for full, one in ((k1, k2), (v1, v2)):
        assert torch.equal(full.view(b * s, hkv, rep, d), one.unsqueeze(2).expand(b * s, hkv, rep, d))


@pytest.mark.parametrize("t,f", [(100, 64), (4096, 3072)])
def test_swiglu_matches_torch(t, f):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    g = torch.Generator().manual_seed(t)
    gu = (torch.randn(t, 2 * f, generator=g) * 3).to(torch.bfloat16)
    dy = torch.randn(t, f, generator=g).to(torch.bfloat16)
    x = gu.cuda().requires_grad_(True)
    y = st._SwiGLU.apply(x)
    y.backward(dy.cuda())
    xr = gu.float().requires_grad_(True)
    yr = torch.nn.functional.silu(xr[:, :f]) * xr[:, f:]
    yr.backward(dy.float())
    assert _rel(y.cpu(), yr.detach()) < 1e-2
    assert _rel(x.grad.cpu(), xr.grad) < 1e-2


@pytest.mark.parametrize("rows,dim,with_add", [(300, 1024, True), (7, 4096, True), (65, 1032, False), (1, 8, True),
                                                (33, 2048, True)])
def test_add_rmsnorm_matches_torch(rows, dim, with_add):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    print(f"[add_rmsnorm] rows={rows} dim={dim} add={with_add}", flush=True)
    g = torch.Generator().manual_seed(rows + dim)
    eps = 1e-6
    h = torch.randn(rows, dim, generator=g).to(torch.bfloat16).cuda()
    a = torch.randn(rows, dim, generator=g).to(torch.bfloat16).cuda() if with_add else None
    w = (1.0 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16).cuda()
    hh = h.clone().requires_grad_(True)
    aa = a.clone().requires_grad_(True) if with_add else None
    s, n = st._AddRMSNorm.apply(hh, aa, w, eps)
    s_ref = h + a if with_add else h
    assert torch.equal(s.detach(), s_ref)  # torch's bf16 add, bit for bit
    x = s_ref.float().requires_grad_(True)
    n_ref = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()
    assert _rel(n.detach().float(), n_ref.detach()) < 1e-2
    # backward: ds from the residual path, dn from the normed output
    ds = torch.randn(rows, dim, generator=g).to(torch.bfloat16).cuda()
    dn = torch.randn(rows, dim, generator=g).to(torch.bfloat16).cuda()
    (s.float() * ds.float()).sum().add((n.float() * dn.float()).sum()).backward()
    (n_ref * dn.float()).sum().backward()
    dh_ref = x.grad + ds.float()  # s is h itself without the add
    assert _rel(hh.grad.float(), dh_ref) < 1e-2
    if with_add:
        assert torch.equal(aa.grad, hh.grad)


def test_fused_norm_body_matches_unfused(monkeypatch):
    """The decoder body with every residual add fused into the following
    RMSNorm gives the unfused body's output and gate gradients."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    import copy
    cfg = st.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, mlp=512, vocab=1000)
    torch.manual_seed(0)
    student, _, replaced = st.build_models(cfg, ["Q2_K", "Q4_K", "Q8_0"], torch.device("cuda", 0), seed=4, packed=False)
    other = copy.deepcopy(student)
    ids = torch.randint(0, cfg.vocab, (2, 64), device="cuda", generator=torch.Generator(device="cuda").manual_seed(1))
    out_f = student(ids)
    out_f.float().pow(2).mean().backward()
    with monkeypatch.context() as mp:
        mp.setattr(st, "_fused_norms", lambda h, w: False)
        out_u = other(ids)
        out_u.float().pow(2).mean().backward()
    assert _rel(out_f.detach().float(), out_u.detach().float()) < 1e-2
    names = list(replaced)
    mods_o = dict(other.named_modules())
    gf = torch.cat([replaced[nm].gates.grad for nm in names])
    gu = torch.cat([mods_o[nm].gates.grad for nm in names])
    assert _rel(gf, gu) < 3e-2
