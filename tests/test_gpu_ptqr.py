"""Per-token quant routing (PTQR) on the HIP path, against the oracle.

Ports the reference's tests/test_ptqr.py:46-91 (routed linear: every row from
exactly its routed candidate; straight-through gradients) and :121-186 (module
toggle) onto libvoodoo_hip, plus the bf16 candidate decode and multi-tile
routed shapes with empty and full groups.  Floating-point bar: 1e-2 relative
(bf16 operands); a row must also sit clearly farther from every non-routed
candidate's output than from its own.
"""

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture
from voodoo_quant import layers

pytestmark = pytest.mark.gpu

GGML = dict(cdequant.GGML_TYPE)
SIX = ["Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
TOL = 1e-2


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _rel(a, b):
    return float((a.double() - b.double()).norm() / max(float(b.double().norm()), 1e-30))


def _rtn(types, n, d_pad, seed):
    from voodoo_quant import rtn

    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, d_pad, generator=g) * 0.02
    qbs = [rtn.rtn_quantize_tensor(w, qt) for qt in types]
    ws = [torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), n * d_pad).reshape(n, d_pad))
          for qt, qb in zip(types, qbs)]
    return qbs, ws


@pytest.mark.parametrize("qt", SIX)
def test_dequant_bf16_is_torch_rounding_of_ggml_values(hip, qt):
    rng = np.random.default_rng(5)
    groups = 40
    per = 8 if qt == "Q8_0" else 1
    qb = blocks.random_blocks(qt, groups * per, rng)
    ref = torch.from_numpy(cdequant.oracle_dequant(qt, qb, groups * 256)).to(torch.bfloat16)
    got = hip.dequant_bf16(GGML[qt], torch.from_numpy(qb.reshape(-1)).cuda(), groups, 256)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().reshape(-1).view(torch.int16), ref.view(torch.int16))


def _routed(hip, types, qbs, x, routing, n, d_pad):
    """Run the routed forward through the C ABI (host permutation as the module builds it)."""
    cands = [hip.dequant_bf16(GGML[t], q.reshape(-1).cuda(), n, d_pad) for t, q in zip(types, qbs)]
    fn = layers.RoutedLinearFunction
    meta = (tuple(GGML[t] for t in types), n, d_pad)
    return fn, meta, cands


@pytest.mark.parametrize("m,n,d,d_pad,types,mode", [
    (10, 8 * 4, 256, 256, ["IQ2_XXS", "IQ3_XXS", "Q4_K", "Q8_0"], "random"),  # test_ptqr.py:46-91, its menu
    (10, 8 * 4, 256, 256, ["Q2_K", "Q3_K", "Q4_K", "Q8_0"], "random"),
    (1000, 520, 1000, 1024, SIX, "random"),                                # multi-tile, ragged groups
    (777, 264, 512, 512, ["Q2_K", "Q6_K", "Q8_0"], "one-empty"),            # a candidate with no tokens
    (300, 256, 256, 256, ["Q4_K", "Q8_0"], "all-one"),                      # every token to one candidate
    # groups of more than 8 tile-rows run in blocks of 8 tile-rows (the last block shorter)
    (2600, 264, 256, 256, ["Q4_K", "Q8_0"], "all-one"),                     # one group of 11 tile-rows
    (3000, 264, 256, 256, ["Q2_K", "Q5_K", "Q8_0"], "skewed"),              # 85% of the tokens to one candidate
])
def test_routed_linear_forward_and_backward(hip, m, n, d, d_pad, types, mode):
    print(f"[ptqr] m={m} n={n} d={d} types={types} mode={mode}", flush=True)
    qbs, ws = _rtn(types, n, d_pad, seed=m)
    g = torch.Generator().manual_seed(m + 1)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    k = len(types)
    if mode == "random":
        routing = torch.randint(0, k, (m,), generator=g)
    elif mode == "one-empty":
        routing = torch.randint(0, k - 1, (m,), generator=g)  # candidate k-1 gets no token
    elif mode == "skewed":
        routing = torch.where(torch.rand(m, generator=g) < 0.85, torch.tensor(1),
                              torch.randint(0, k, (m,), generator=g))
    else:
        routing = torch.full((m,), k - 1, dtype=torch.int64)
    probs = torch.softmax(torch.randn(k, generator=g), 0)
    fn, meta, cands = _routed(hip, types, qbs, x, routing, n, d_pad)

    xd = x.cuda().requires_grad_(True)
    pd = probs.cuda().requires_grad_(True)
    y = fn.apply(xd, pd, routing.cuda(), meta, cands, *[q.reshape(-1).cuda() for q in qbs])
    torch.cuda.synchronize()
    yc = y.detach().cpu().double()

    # forward: each row from ITS routed candidate (bf16 operands), far from the others
    xf = x.double()
    outs = [xf @ w[:, :d].double().t() for w in ws]
    for t in range(m):
        own = outs[int(routing[t])][t]
        err = float((yc[t] - own).norm() / max(float(own.norm()), 1e-30))
        assert err < TOL, (t, err)
        if k > 1 and t < 64:
            others = [float((yc[t] - outs[j][t]).norm() / max(float(own.norm()), 1e-30))
                      for j in range(k) if j != int(routing[t])]
            assert min(others) > 3 * err, (t, err, others)

    # backward: the straight-through mixture gradient at the routed point
    gy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    y.backward(gy.cuda())
    torch.cuda.synchronize()
    gf = gy.double()
    gp_ref = torch.stack([(gf * o).sum() for o in outs])
    w_mix = mixture.mix_weight(ws, probs).to(torch.bfloat16).double()[:, :d]
    dx_ref = gf @ w_mix
    assert _rel(pd.grad.cpu(), gp_ref) < TOL
    assert _rel(xd.grad.cpu(), dx_ref) < TOL


def _oracle_candidates(mod, ncols):
    """The module's candidates decoded by the oracle from its packed bytes
    (fp32 [out, ncols]), not by the kernels under test."""
    rows, dp = mod.out_features if hasattr(mod, "out_features") else mod.num_embeddings, mod.padded_in_features
    return [torch.from_numpy(cdequant.oracle_dequant(qt, getattr(mod, f"_qweight_{k}").cpu().numpy(), rows * dp))
            .reshape(rows, dp)[:, :ncols] for k, qt in enumerate(mod.candidate_types)]


def test_module_toggle(hip):
    """Port of tests/test_ptqr.py:121-186 (linear part) on the HIP module, with its menu."""
    types = ["IQ2_XXS", "IQ3_XXS", "Q8_0"]
    in_f, out_f = 256, 64
    g = torch.Generator().manual_seed(23)
    lin = layers.MixedQuantLinear(in_f, out_f, types, torch.randn(out_f, in_f, generator=g) * 0.02,
                                  tensor_name="tests.ptqr.linear").cuda()
    x = torch.randn(16, in_f, generator=g).to(torch.bfloat16).cuda()
    cands = [c.cuda() for c in _oracle_candidates(lin, in_f)]
    outs = [x.float() @ c.t() for c in cands]
    layers.set_ptqr(True)
    try:
        torch.manual_seed(0)
        y = lin(x).float()
        for t in range(x.shape[0]):
            errs = [float((y[t] - o[t]).norm() / o[t].norm()) for o in outs]
            assert sum(e < TOL for e in errs) == 1, errs  # exactly one candidate
        lin.zero_grad()
        y2 = lin(x)
        gy = torch.randn_like(y2)
        y2.backward(gy)
        gp = torch.stack([(gy.float() * o).sum() for o in outs]).cpu()
        p = lin.soft_probs().detach().cpu()
        gates_ref = (torch.diag(p) - torch.outer(p, p)) @ gp.double().float()
        assert _rel(lin.gates.grad.cpu(), gates_ref) < TOL
    finally:
        layers.set_ptqr(False)
    # toggled off: the soft mixture again
    y_mix = lin(x).float()
    p = lin.soft_probs().detach()
    w_mix = sum(p[k] * cands[k] for k in range(len(types)))
    assert _rel(y_mix.cpu(), (x.float() @ w_mix.t()).cpu()) < TOL


def test_routed_forward_ignores_out_of_range_map_entries(hip):
    """A routing map entry outside [0, m) reads zero rows and writes nothing,
    and group offsets are clamped to [0, m] and made non-decreasing, so a bad
    map or bad offsets cannot make the kernel touch memory outside x and y."""
    m, n, d = 100, 264, 256
    types = ["Q4_K", "Q6_K", "Q8_0"]
    qbs, ws = _rtn(types, n, d, seed=5)
    x = torch.randn(m, d, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    cands = [w.to(torch.bfloat16).cuda() for w in ws]
    perm = torch.arange(m, dtype=torch.int32)
    perm[7] = -5
    perm[60] = m + 3
    goff = torch.tensor([0, 50, 30, 200], dtype=torch.int32)  # clamped: [0, 50), empty, [50, 100)
    sentinel = torch.full((m, n), 7.0, dtype=torch.bfloat16)
    y = sentinel.cuda()
    hip.routed_linear_fwd(x.cuda(), cands, perm.cuda(), goff.cuda(), n, d, y)
    torch.cuda.synchronize()
    yc = y.cpu().double()
    for r in range(m):
        if r in (7, 60):  # no map entry names these rows: left as they were
            assert torch.equal(y[r].cpu(), sentinel[r]), r
            continue
        w = ws[0] if r < 50 else ws[2]
        ref = x[r].double() @ w.to(torch.bfloat16).double().t()
        assert _rel(yc[r], ref) < TOL, r
