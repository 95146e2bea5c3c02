"""Gated Linears that read one input, stacked into one product
(``vq_gated_linear_group_fwd/bwd``), against the oracle and against the
members run one by one.

Bars (as for a single gated Linear): each member's rows of the stacked W_eff
bit-exact to the oracle's mixture; Y, dX (the members' input gradients
summed) within 1e-2 relative L2 of fp64; each member's dL/dp_k within 1e-4
relative L2 of fp64 <dY_i^T X, W_ik>.
"""

import numpy as np
import pytest
import torch

from oracle import cdequant, mixture
from voodoo_quant import layers

pytestmark = pytest.mark.gpu

GGML = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
TOL = 1e-2


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _rtn(types, n, d_pad, seed):
    from voodoo_quant import rtn

    w = torch.randn(n, d_pad, generator=torch.Generator().manual_seed(seed)) * 0.02
    qbs = [rtn.rtn_quantize_tensor(w, qt).reshape(-1) for qt in types]
    ws = [torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), n * d_pad).reshape(n, d_pad))
          for qt, qb in zip(types, qbs)]
    return qbs, ws


GROUPS = [
    # (name, m, d, d_pad, [(types, n)])
    ("qkv", 777, 1024, 1024, [(["Q8_0", "Q4_K", "Q2_K", "Q6_K"], 1024), (["Q3_K", "Q5_K"], 256),
                              (["Q2_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q3_K"], 256)]),
    ("gate-up", 512, 1000, 1024, [(["Q4_K", "Q8_0"], 768), (["Q2_K", "Q3_K", "Q6_K"], 512)]),
    ("four", 300, 256, 256, [(["Q8_0"], 256), (["Q4_K", "Q6_K"], 512), (["Q2_K"], 256), (["Q5_K", "Q3_K"], 256)]),
]


@pytest.mark.parametrize("case", GROUPS, ids=[g[0] for g in GROUPS])
def test_group_matches_oracle(hip, case):
    name, m, d, d_pad, members = case
    print(f"[group] {name} m={m} d={d} members={[(len(t), n) for t, n in members]}", flush=True)
    g = torch.Generator().manual_seed(m)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    n_total = sum(n for _, n in members)
    dy = torch.randn(m, n_total, generator=g).to(torch.bfloat16)
    spec, refs, probs = [], [], []
    for i, (types, n) in enumerate(members):
        qbs, ws = _rtn(types, n, d_pad, seed=100 * i + m)
        spec.append((tuple(GGML[t] for t in types), [q.cuda() for q in qbs], n))
        p = torch.softmax(torch.randn(len(types), generator=g), 0)
        probs.append(p)
        refs.append((ws, mixture.mix_weight(ws, p).to(torch.bfloat16)))
    xd, dyd = x.cuda(), dy.cuda()
    w_eff = torch.empty(n_total, d_pad, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(m, n_total, dtype=torch.bfloat16, device="cuda")
    fws = torch.empty(max(hip.fwd_workspace_bytes(m, n_total, d), 16), dtype=torch.uint8, device="cuda")
    hip.gated_linear_group_fwd(xd, spec, [p.cuda() for p in probs], d_pad, w_eff, y, fws)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device="cuda")
    dps = [torch.empty(len(t), dtype=torch.float32, device="cuda") for t, _ in members]
    ws = torch.empty(hip.group_bwd_workspace_bytes(m, d, spec), dtype=torch.uint8, device="cuda")
    hip.gated_linear_group_bwd(dyd, xd, spec, d_pad, w_eff, dx, dps, ws)
    torch.cuda.synchronize()

    w_all = torch.cat([r[1] for r in refs], 0)
    assert torch.equal(w_eff.cpu().view(torch.int16), w_all.view(torch.int16)), "stacked W_eff not bit-exact"
    wd = w_all[:, :d]
    assert mixture.relative_l2(y.cpu().double(), mixture.forward(x, wd, torch.float64)) < TOL
    dx_ref = dy.double() @ wd.double()
    assert mixture.relative_l2(dx.cpu().double(), dx_ref) < TOL
    off = 0
    for (types, n), (cands, _), dp in zip(members, refs, dps):
        dyi = dy[:, off:off + n]
        gp_ref = torch.stack([(dyi.double().t() @ x.double() * c[:, :d].double()).sum() for c in cands])
        assert mixture.relative_l2(dp.cpu().double(), gp_ref) < 1e-4, (name, types)
        off += n


def test_group_module_path_matches_members(hip):
    """layers.gated_linear_group on modules: outputs and gate gradients match
    each module run alone."""
    torch.manual_seed(1)
    d = 512
    mods = [layers.MixedQuantLinear(d, n, t, torch.randn(n, d) * 0.02, tensor_name=f"grp.{i}").cuda()
            for i, (t, n) in enumerate([(["Q4_K", "Q8_0"], 512), (["Q2_K", "Q6_K", "Q8_0"], 256),
                                        (["Q3_K", "Q5_K"], 256)])]
    for m in mods:
        with torch.no_grad():
            m.gates.copy_(torch.randn(m.num_candidates))
    x = torch.randn(3, 40, d, device="cuda").to(torch.bfloat16)
    gys = [torch.randn(3, 40, m.out_features, device="cuda").to(torch.bfloat16) for m in mods]

    xa = x.clone().requires_grad_(True)
    outs = layers.gated_linear_group(xa, mods)
    sum((o.float() * gy.float()).sum() for o, gy in zip(outs, gys)).backward()
    ga = [m.gates.grad.clone() for m in mods]
    for m in mods:
        m.gates.grad = None
    xb = x.clone().requires_grad_(True)
    outs_b = [m(xb) for m in mods]
    sum((o.float() * gy.float()).sum() for o, gy in zip(outs_b, gys)).backward()
    for o, ob in zip(outs, outs_b):
        assert o.shape == ob.shape
        assert float((o.float() - ob.float()).norm() / ob.float().norm()) < 1e-2
    assert float((xa.grad.float() - xb.grad.float()).norm() / xb.grad.float().norm()) < 1e-2
    for a, m in zip(ga, mods):
        assert float((a - m.gates.grad).norm() / m.gates.grad.norm()) < 1e-3


def test_group_rejects_unaligned_members(hip):
    spec = [((12,), [torch.zeros(136 * 144, dtype=torch.uint8, device="cuda")], 136),
            ((12,), [torch.zeros(256 * 144, dtype=torch.uint8, device="cuda")], 256)]
    x = torch.zeros(8, 256, dtype=torch.bfloat16, device="cuda")
    w = torch.empty(392, 256, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(8, 392, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="multiple of 256"):
        hip.gated_linear_group_fwd(x, spec, [torch.ones(1, device="cuda")] * 2, 256, w, y)
