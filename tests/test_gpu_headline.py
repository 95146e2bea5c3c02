"""GPU parity at the Linear shapes the benchmark times (needs an MI355X).

8192 tokens through each of the four projection shapes of a 27B-class layer
(hidden 5120: q 5120 -> 6144, o 6144 -> 5120, gate/up 5120 -> 17408,
down 17408 -> 5120), K = 6 candidates (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0),
and 2 x 8192 tokens through one SwiGLU block of the stress stack (hidden
4096, MLP 14336: 4096 -> 14336 and 14336 -> 4096) with its K = 8 menu (Q2_K,
IQ2_XXS, Q3_K, IQ3_S, Q4_K, Q5_K, Q6_K, Q8_0), through the C ABI with the forward's split-tail workspace on, so every work
plan the benchmark runs (whole-tile rounds, K-split tail tiles on every XCD,
the dual dX + gate launch) is compared with the oracle:

* W_eff bit-exact against ``mixture.mix_weight`` of the oracle's C decodes;
* Y and dX: every 256 x 256 tile within 1e-2 relative L2 of an fp32 product
  of the same bf16 operands (the reference's fp32 PyTorch path), and 64+
  sampled rows, including rows of every K-split tail tile, against fp64;
* dL/dp_k = <dY^T X, W_k> within 1e-4 of the fp32/fp64 evaluation of the
  reference's formula (``voodoo_quant/layers.py:354-363``), and the gate
  gradient through the softmax within 1e-2.

The last test runs the gate product over a Q8_0 candidate larger than 2 GiB
(a vocabulary-scale head, reference ``layers.py:1560-1637``), whose rows past
the 2 GiB mark must reach the gate gradient.
"""

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture

pytestmark = pytest.mark.gpu

TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]
# the stress stack's wide menu: eight distinct formats, two of them IQ
STRESS_TYPES = ["Q2_K", "IQ2_XXS", "Q3_K", "IQ3_S", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]
GGML = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ2_XXS": 16, "IQ3_S": 21}
TOL = 1e-2
M = 8192
SHAPES = [  # (name, in_features D, out_features N, tokens M, candidate menu)
    ("q_5120x6144", 5120, 6144, M, TYPES),
    ("o_6144x5120", 6144, 5120, M, TYPES),
    ("up_5120x17408", 5120, 17408, M, TYPES),
    ("down_17408x5120", 17408, 5120, M, TYPES),
    # one SwiGLU block of the stress stack: hidden 4096, MLP 14336, 2 x 8192 tokens, K = 8
    ("stress_up_4096x14336_k8", 4096, 14336, 2 * M, STRESS_TYPES),
    ("stress_down_14336x4096_k8", 14336, 4096, 2 * M, STRESS_TYPES),
]


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _say(msg):
    print(msg, flush=True)


def _random_candidate(qt, n, d_pad, rng):
    """Random valid blocks: random payload bytes, fp16 scale fields with
    random sign and mantissa and an exponent in 8..15 (normal numbers,
    weights of magnitude ~1e-2 .. 1)."""
    per_group = 8 if qt == "Q8_0" else 1
    nb = n * d_pad // 256 * per_group
    qb = rng.integers(0, 256, size=(nb, blocks.BLOCK_BYTES[qt]), dtype=np.uint8)
    for off in blocks.F16_OFFSETS[qt]:
        qb[:, off + 1] = (qb[:, off + 1] & 0x83) | (0x20 + (rng.integers(0, 8, size=nb, dtype=np.uint8) << 2))
    return qb


# ---------------------------------------------------------------- the kernels' work plan
# A restatement of the launch plan (xcd_plan / tile_coords in csrc/vq_gemm_impl.h),
# used only to aim the sampled rows at the K-split tail tiles.
def _xcd_plan(x, total, cus_per_xcd, ksteps, split_ok, min_saved, max_split=8):
    base, rem = divmod(total, 8)
    tiles = base + (1 if x < rem else 0)
    t0 = x * base + min(x, rem)
    t = tiles % cus_per_xcd
    sp = min(cus_per_xcd // t if t else 1, max_split, ksteps // 4)
    if sp >= 2 and ksteps - (ksteps + sp - 1) // sp < min_saved:
        sp = 1
    if not split_ok or t == 0 or sp < 2:
        return t0, tiles, 0, 1
    return t0, tiles - t, t, sp


def _tile_coords(tile, tiles_m, tiles_n, group_m=8):
    size = group_m * tiles_n
    first = tile // size * group_m
    gm = min(tiles_m - first, group_m)
    return first + tile % size % gm, tile % size // gm


def _tail_tiles(i, j, k, cus_per_xcd, min_saved):
    tm_, tn_ = i // 256, j // 256
    out = []
    for x in range(8):
        t0, full, tail, sp = _xcd_plan(x, tm_ * tn_, cus_per_xcd, (k + 63) // 64, True, min_saved)
        out += [(_tile_coords(t0 + full + t, tm_, tn_), sp) for t in range(tail)]
    return out


def _tile_rel(got, ref):
    """Per 256 x 256 tile relative L2 (fp64) of two [R, C] device tensors."""
    r, c = got.shape
    g = got.double().reshape(r // 256, 256, c // 256, 256)
    f = ref.double().reshape(r // 256, 256, c // 256, 256)
    num = (g - f).pow(2).sum(dim=(1, 3)).sqrt()
    den = f.pow(2).sum(dim=(1, 3)).sqrt().clamp_min(1e-30)
    return num / den


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_linear_shape_at_benchmark_tokens(hip, shape):
    name, d, n, M, types = shape
    d_pad = d
    k_ = len(types)
    _say(f"[headline] {name}: M={M} D={d} N={n} K={k_}: building candidates")
    rng = np.random.default_rng(d * 7 + n)
    qbs = [_random_candidate(qt, n, d_pad, rng) for qt in types]
    cands = [torch.from_numpy(cdequant.oracle_dequant_parallel(qt, qb, n * d_pad).reshape(n, d_pad))
             for qt, qb in zip(types, qbs)]
    g = torch.Generator().manual_seed(n + d)
    probs = torch.softmax(torch.randn(k_, generator=g), 0)
    x = torch.randn(M, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(M, n, generator=g).to(torch.bfloat16)

    dev = torch.device("cuda", 0)
    qd = [torch.from_numpy(q.reshape(-1)).to(dev) for q in qbs]
    ids = [GGML[t] for t in types]
    xd, dyd, pd = x.to(dev), dy.to(dev), probs.to(dev)
    w_eff = torch.empty(n, d_pad, dtype=torch.bfloat16, device=dev)
    y = torch.empty(M, n, dtype=torch.bfloat16, device=dev)
    fws = torch.empty(max(hip.fwd_workspace_bytes(M, n, d), 256), dtype=torch.uint8, device=dev)
    _say(f"[headline] {name}: forward")
    hip.gated_linear_fwd(xd, ids, qd, pd, n, d_pad, w_eff, y, fws)
    dx = torch.empty(M, d, dtype=torch.bfloat16, device=dev)
    dp = torch.empty(k_, dtype=torch.float32, device=dev)
    ws = torch.empty(hip.bwd_workspace_bytes(M, n, d, d_pad, k_, False), dtype=torch.uint8, device=dev)
    _say(f"[headline] {name}: backward (dX + gate in one launch)")
    hip.gated_linear_bwd(dyd, xd, ids, qd, pd, n, d_pad, w_eff, dx, dp, ws)
    torch.cuda.synchronize()

    # the oracle's k-ordered fp32 mixture (a multiply kernel, then an add
    # kernel, per candidate: the same separately rounded IEEE operations on
    # the device as on the host)
    _say(f"[headline] {name}: W_eff against the oracle mixture")
    ref_w = mixture.mix_weight([c.to(dev) for c in cands], pd).to(torch.bfloat16)
    assert torch.equal(w_eff.view(torch.int16), ref_w.view(torch.int16)), \
        f"W_eff not bit-exact: {int((w_eff.view(torch.int16) != ref_w.view(torch.int16)).sum())} weights differ"
    del ref_w

    # every tile of Y and dX against fp32 products of the same bf16 operands
    _say(f"[headline] {name}: Y and dX tiles against fp32")
    wf = w_eff[:, :d].float()
    y_ref = xd.float() @ wf.t()
    ty = _tile_rel(y, y_ref)
    assert float(ty.max()) < TOL, f"worst Y tile {float(ty.max()):.3e} at {divmod(int(ty.argmax()), ty.shape[1])}"
    del y_ref
    dx_ref = dyd.float() @ wf
    tdx = _tile_rel(dx, dx_ref)
    assert float(tdx.max()) < TOL, f"worst dX tile {float(tdx.max()):.3e} at {divmod(int(tdx.argmax()), tdx.shape[1])}"
    del dx_ref

    # sampled rows against fp64 on the host: rows of every XCD's split tail tiles
    cus = torch.cuda.get_device_properties(dev).multi_processor_count // 8
    tails_y = _tail_tiles(M, n, d, cus, 14)
    tails_dx = _tail_tiles(M, d, n, cus, 14)
    tails_gate = _tail_tiles(d, n, M, cus, 0)
    _say(f"[headline] {name}: split tails fwd {len(tails_y)} dX {len(tails_dx)} gate {len(tails_gate)}")
    rows = {tm * 256 + int(rng.integers(256)) for (tm, _), _ in tails_y + tails_dx}
    while len(rows) < 64:
        rows.add(int(rng.integers(M)))
    rows = sorted(rows)
    wd = w_eff[:, :d].cpu().double()
    ri = torch.tensor(rows)
    ey = mixture.relative_l2(y.cpu()[ri].double(), x[ri].double() @ wd.t())
    edx = mixture.relative_l2(dx.cpu()[ri].double(), dy[ri].double() @ wd)
    _say(f"[headline] {name}: {len(rows)} sampled rows vs fp64: Y {ey:.2e} dX {edx:.2e}")
    assert ey < TOL and edx < TOL
    del wd

    # dL/dp_k = <dY^T X, W_k>: dW in fp32 on the device, the dots in fp64
    _say(f"[headline] {name}: gate gradients")
    dw = (dyd.float().t() @ xd.float()).double()
    gp_ref = torch.stack([(dw * c[:, :d].to(dev, torch.float64)).sum() for c in cands]).cpu()
    del dw
    e_gp = mixture.relative_l2(dp.cpu().double(), gp_ref)
    dg = mixture.gates_grad(dp.cpu().double(), probs.double(), 1.0)
    dg_ref = mixture.gates_grad(gp_ref, probs.double(), 1.0)
    e_dg = mixture.relative_l2(dg, dg_ref, floor=1e-6 * float(gp_ref.abs().max()))
    _say(f"[headline] {name}: dL/dp rel {e_gp:.2e}, dL/dg rel {e_dg:.2e}; tiles Y {float(ty.max()):.2e} "
         f"dX {float(tdx.max()):.2e}")
    assert e_gp < 1e-4
    assert e_dg < TOL


def test_gate_gradient_candidate_past_2gib(hip):
    """A Q8_0 candidate of 262144 x 8192 (2.28 GB, a vocabulary-scale head) and
    a Q4_K one (1.21 GB): the gate epilogue must read rows past the 2 GiB mark.
    dY is nonzero only on a set of output rows S (among them the rows right
    after the 2 GiB boundary and the last rows), so the oracle needs the bytes
    of those rows only: dL/dp_k = sum_{n in S} <dY[:, n]^T X, W_k[n]>."""
    dev = torch.device("cuda", 0)
    n, d, m = 262144, 8192, 256
    types = ["Q4_K", "Q8_0"]
    row_bytes = {qt: d // 256 * blocks.BLOCK_BYTES[qt] * (8 if qt == "Q8_0" else 1) for qt in types}
    assert n * row_bytes["Q8_0"] > 2 ** 31
    g = torch.Generator(device=dev).manual_seed(31)
    qd = []
    for qt in types:
        bb = blocks.BLOCK_BYTES[qt]
        q = torch.randint(0, 256, (n * row_bytes[qt] // bb, bb), dtype=torch.uint8, device=dev, generator=g)
        for off in blocks.F16_OFFSETS[qt]:  # normal fp16 scales, exponent 8..15
            h = torch.randint(0, 1 << 16, (q.shape[0],), dtype=torch.int32, device=dev, generator=g)
            h = (h & 0x83FF) | (0x2000 + ((h >> 10) & 0x7) * 0x0400)
            q[:, off] = (h & 0xFF).to(torch.uint8)
            q[:, off + 1] = ((h >> 8) & 0xFF).to(torch.uint8)
        qd.append(q.reshape(-1))
    boundary = 2 ** 31 // row_bytes["Q8_0"]
    rng = np.random.default_rng(5)
    sel = set(range(boundary - 40, boundary + 300)) | set(range(n - 256, n)) | set(range(0, 64))
    sel |= {int(r) for r in rng.choice(n, size=256, replace=False)}
    sel = torch.tensor(sorted(sel))
    _say(f"[2GiB] boundary row {boundary}, {sel.numel()} nonzero dY columns")
    gx = torch.Generator().manual_seed(32)
    x = torch.randn(m, d, generator=gx).to(torch.bfloat16)
    dys = torch.randn(m, sel.numel(), generator=gx).to(torch.bfloat16)
    dy = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
    dy[:, sel.to(dev)] = dys.to(dev)
    probs = torch.tensor([0.4, 0.6], device=dev)
    dp = torch.empty(2, dtype=torch.float32, device=dev)
    ws = torch.empty(hip.bwd_workspace_bytes(m, n, d, d, 2, False), dtype=torch.uint8, device=dev)
    hip.gated_linear_bwd(dy, x.to(dev), [GGML[t] for t in types], qd, probs, n, d, None, None, dp, ws)
    torch.cuda.synchronize()
    dw = dys.double().t() @ x.double()  # [|S|, d]
    past = sel >= boundary
    ref, ref_past = [], []
    for qt, q in zip(types, qd):
        rb = row_bytes[qt]
        qrows = q.view(n, rb)[sel.to(dev)].cpu().numpy()
        w = torch.from_numpy(cdequant.oracle_dequant(qt, qrows, sel.numel() * d).reshape(-1, d)).double()
        per_row = (dw * w).sum(dim=1)
        ref.append(per_row.sum())
        ref_past.append(per_row[past].sum())
    ref, ref_past = torch.stack(ref), torch.stack(ref_past)
    err = mixture.relative_l2(dp.cpu().double(), ref)
    _say(f"[2GiB] dL/dp {dp.cpu().tolist()} vs {ref.tolist()} (rows past 2 GiB: {ref_past.tolist()}): rel {err:.2e}")
    # the rows past the boundary carry far more than the bar: losing them fails it
    assert float(ref_past.norm()) > 100 * 1e-4 * float(ref.norm())
    assert err < 1e-4


def test_vocab_head_module_matches_oracle(hip):
    """A vocabulary-scale gated head (151936 x 1024, 155.6M weights per
    candidate, K = 6 including two IQ formats) through MixedQuantLinear and
    autograd, 512 tokens.  The reference routes heads of 64M+ elements to
    _BlockedCandidateLinear (layers.py:1560-1637), Y = sum_k p_k X W_k^T in
    row blocks; here the same mixture goes through the one fused path.  Y on
    sampled rows and dX against fp64 of the oracle's W_eff; gates.grad against
    the softmax Jacobian of <dY^T X, W_k> evaluated on the device in fp32 over
    the oracle's decodes (layers.py:354-363)."""
    from voodoo_quant import layers

    dev = torch.device("cuda", 0)
    n, d, m = 151936, 1024, 512
    types = ["Q8_0", "Q6_K", "Q4_K", "IQ4_XS", "Q2_K", "IQ2_XXS"]
    rng = np.random.default_rng(77)
    qbs, cands = [], []
    for qt in types:
        per = 8 if qt == "Q8_0" else 1
        qb = blocks.random_blocks(qt, n * d // 256 * per, rng)
        for which in range(len(blocks.F16_OFFSETS[qt]) or 1):  # scales in [2^-8, 2^-5)
            blocks.set_scale(qt, qb, (0x1C00 + rng.integers(0, 0x0C00, size=qb.shape[0])).astype(np.uint16), which)
        qbs.append(torch.from_numpy(qb.reshape(-1)))
        cands.append(torch.from_numpy(cdequant.oracle_dequant_parallel(qt, qb, n * d)).reshape(n, d))
    lin = layers.MixedQuantLinear.from_packed(d, n, types, [q.to(dev) for q in qbs], tensor_name="tests.vocab_head",
                                              device=dev)
    with torch.no_grad():
        lin.gates.copy_(torch.tensor([0.4, -0.1, 0.3, 0.0, -0.3, 0.2]))
    lin.set_temperature(0.8)
    g = torch.Generator().manual_seed(78)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    y = lin(x)
    G = torch.randn(m, n, generator=g).to(torch.bfloat16).to(dev)
    y.backward(G)
    torch.cuda.synchronize()
    p = lin.soft_probs().detach().cpu()
    w_eff = mixture.mix_weight(cands, p).to(torch.bfloat16)  # the reference's fp32 mixture, source dtype
    rows = torch.from_numpy(np.sort(rng.choice(m, size=64, replace=False)))
    y_ref = x.detach().cpu()[rows].double() @ w_eff.double().t()
    e_y = mixture.relative_l2(y.detach().cpu()[rows].double(), y_ref)
    wd = w_eff.to(dev)
    e_dx = mixture.relative_l2(x.grad.double(), G.double() @ wd.double())
    # <dY^T X, W_k>: dW once in fp32 on the device, then one dot per oracle decode
    dw = G.float().t() @ x.detach().float()  # [n, d]
    gp = torch.stack([(dw * c.to(dev)).sum(dtype=torch.float64) for c in cands]).cpu()
    pd = p.double()
    ref = (torch.diag(pd) - torch.outer(pd, pd)) @ gp / 0.8
    e_g = mixture.relative_l2(lin.gates.grad.double().cpu(), ref)
    _say(f"[vocab-head] Y {e_y:.2e} dX {e_dx:.2e} gates.grad {e_g:.2e}")
    assert e_y < TOL and e_dx < TOL and e_g < TOL
