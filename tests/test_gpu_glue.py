"""The decoder glue kernels of the step harness (rotary embedding with
grouped-query K/V expansion, SwiGLU) against fp32 torch, forward and
backward.  Bar: 1e-2 relative L2 (bf16 inputs and outputs, fp32 inside)."""

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
