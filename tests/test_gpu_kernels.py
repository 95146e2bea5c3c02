"""GPU parity of libvoodoo_hip against the oracle (needs an MI355X).

Bars: dequant and the W_eff mixture bit-exact; Y, dX and dL/dp within 1e-2
relative L2 of the fp32/fp64 oracle (bf16 products; the path's stated tolerance).
Every call goes through the C ABI (ctypes binding of include/voodoo_hip.h).
"""

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture

pytestmark = pytest.mark.gpu

SIX = ["Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
GGML = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
TOL = 1e-2  # relative L2 bar for Y, dX and the gate gradients


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _gpu_dequant(hip, qt, qb, n_weights):
    rows = n_weights // 256
    out = hip.dequant(GGML[qt], _dev(qb.reshape(-1)), rows, 256)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(-1)


def _edge_blocks(qt):
    bb = blocks.BLOCK_BYTES[qt]
    per = 8 if qt == "Q8_0" else 1
    out = []
    for fill, d, dmin in [(0x00, 0x3C00, 0x3C00), (0x00, 0xBC00, 0xBC00), (0xFF, 0x3C00, 0x3C00),
                          (0xFF, 0x0001, 0x8001), (0xA5, 0x7BFF, 0xFBFF), (0x5A, 0x0000, 0x8000),
                          (0x33, 0x03FF, 0x83FF)]:
        b = np.full((per, bb), fill, np.uint8)
        for off, h in zip(blocks.F16_OFFSETS[qt], (d, dmin)):
            b[:, off], b[:, off + 1] = h & 0xFF, h >> 8
        out.append(b)
    return np.concatenate(out)


@pytest.mark.parametrize("qt", SIX)
@pytest.mark.parametrize("groups", [1, 15, 16, 17, 333])
def test_dequant_bit_exact_random_and_edge(hip, qt, groups):
    print(f"[dequant] {qt} groups={groups}", flush=True)
    rng = np.random.default_rng(groups)
    per_group = 8 if qt == "Q8_0" else 1
    edge = _edge_blocks(qt)
    n_rand = max(groups * per_group - edge.shape[0], 0)
    qb = np.concatenate([edge, blocks.random_blocks(qt, n_rand, rng)])[: groups * per_group]
    n = groups * 256
    ref = cdequant.oracle_dequant(qt, qb, n)
    got = _gpu_dequant(hip, qt, qb, n)
    assert np.array_equal(_bits(got), _bits(ref)), f"{qt}: {np.sum(_bits(got) != _bits(ref))} mismatches"


@pytest.mark.parametrize("qt", ["Q8_0", "Q4_K", "Q5_K", "Q6_K"])
def test_dequant_matches_reference_golden(hip, qt):
    from pathlib import Path

    g = np.load(Path(__file__).resolve().parent / "golden" / "ref_decoders.npz")
    qb, ref = g[f"{qt}_qbytes"], g[f"{qt}_out"]
    got = _gpu_dequant(hip, qt, qb, ref.size)
    assert np.array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("qt", SIX)
def test_dequant_full_size_4096x14336(hip, qt):
    """The dequant microbench shape: every weight compared bit for bit."""
    print(f"[dequant-full] {qt}", flush=True)
    rng = np.random.default_rng(7)
    nrows, ncols = 4096, 14336
    per_group = 8 if qt == "Q8_0" else 1
    qb = blocks.random_blocks(qt, nrows * ncols // 256 * per_group, rng)
    ref = cdequant.oracle_dequant_parallel(qt, qb, nrows * ncols)
    out = hip.dequant(GGML[qt], _dev(qb.reshape(-1)), nrows, ncols)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(-1)
    assert np.array_equal(_bits(got), _bits(ref))


def test_dequant_rejects_misaligned(hip):
    qb = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        hip.dequant(GGML["Q4_K"], qb, 4, 200)
    with pytest.raises(ValueError):
        hip.dequant(99, qb, 4, 256)


# ------------------------------------------------------------------ mixture, fwd, bwd
def _candidates(types, n, d_pad, rng):
    """Random valid blocks of each type -> (packed numpy, fp32 torch [n, d_pad])."""
    qbs, ws = [], []
    for qt in types:
        per_group = 8 if qt == "Q8_0" else 1
        qb = blocks.random_blocks(qt, n * d_pad // 256 * per_group, rng, allow_subnormal=False)
        # keep magnitudes O(1): clamp the fp16 scales' exponent field
        for off in blocks.F16_OFFSETS[qt]:
            h = qb[:, off].astype(np.uint16) | (qb[:, off + 1].astype(np.uint16) << 8)
            h = (h & 0x83FF) | (np.uint16(0x2000) + ((h >> 10) & 0x7) * np.uint16(0x0400))
            qb[:, off], qb[:, off + 1] = (h & 0xFF).astype(np.uint8), (h >> 8).astype(np.uint8)
        qbs.append(qb)
        ws.append(torch.from_numpy(cdequant.oracle_dequant(qt, qb, n * d_pad).reshape(n, d_pad)))
    return qbs, ws


def _rtn_candidates(types, n, d_pad, seed):
    import voodoo_quant.rtn as rtn

    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, d_pad, generator=g) * 0.02
    qbs = [rtn.rtn_quantize_tensor(w, qt).numpy() for qt in types]
    ws = [torch.from_numpy(cdequant.oracle_dequant(qt, qb, n * d_pad).reshape(n, d_pad)) for qt, qb in zip(types, qbs)]
    return qbs, ws


@pytest.mark.parametrize("types", [SIX, ["Q4_K"], ["Q8_0", "Q3_K", "Q8_0"]])
def test_mix_weight_bit_exact(hip, types):
    rng = np.random.default_rng(11)
    n, d_pad = 264, 768
    qbs, ws = _candidates(types, n, d_pad, rng)
    probs = torch.softmax(torch.randn(len(types), generator=torch.Generator().manual_seed(1)), 0)
    ref = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    got = hip.mix_weight([GGML[t] for t in types], [_dev(q.reshape(-1)) for q in qbs], probs.cuda(), n, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


def test_mix_weight_bit_exact_large(hip):
    """A large tensor (4104 x 1280 = 20520 groups, 1283 workgroups of 16
    groups) with a ragged last workgroup of 8 groups."""
    rng = np.random.default_rng(12)
    n, d_pad = 4104, 1280
    qbs, ws = _candidates(SIX, n, d_pad, rng)
    probs = torch.softmax(torch.randn(len(SIX), generator=torch.Generator().manual_seed(2)), 0)
    ref = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    got = hip.mix_weight([GGML[t] for t in SIX], [_dev(q.reshape(-1)) for q in qbs], probs.cuda(), n, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


def test_mix_weight_bit_exact_odd_tail(hip):
    """263 groups: the last 16-group workgroup stages 7 groups, so the Q3_K
    and Q6_K byte ranges end inside a 16-byte chunk (770 and 1470 bytes) and
    their last bytes take the byte-copy path after the direct-to-LDS chunks."""
    rng = np.random.default_rng(13)
    n, d_pad = 263, 256
    qbs, ws = _candidates(SIX, n, d_pad, rng)
    probs = torch.softmax(torch.randn(len(SIX), generator=torch.Generator().manual_seed(3)), 0)
    ref = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    got = hip.mix_weight([GGML[t] for t in SIX], [_dev(q.reshape(-1)) for q in qbs], probs.cuda(), n, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("qt", SIX)
def test_mix_weight_bit_exact_edge_scales(hip, qt):
    """Full finite fp16 scale range (subnormal, negative, huge) plus all-0x00
    and all-0xFF payloads: the mixture decodes candidates with a single
    rounding per weight and a hardware fp16 conversion, so every exactly
    representable ggml value must come out identical."""
    rng = np.random.default_rng(23)
    n, d_pad = 48, 512
    per_group = 8 if qt == "Q8_0" else 1
    nb = n * d_pad // 256 * per_group
    a = blocks.random_blocks(qt, nb, rng)  # any finite scale, subnormals included
    a[: nb // 8, :] = 0
    a[nb // 8: nb // 4, :] = 0xFF
    for off in blocks.F16_OFFSETS[qt]:  # keep fields finite after the fills
        h = a[:, off].astype(np.uint16) | (a[:, off + 1].astype(np.uint16) << 8)
        h = np.where(((h >> 10) & 0x1F) == 0x1F, h ^ np.uint16(0x4000), h).astype(np.uint16)
        a[:, off], a[:, off + 1] = (h & 0xFF).astype(np.uint8), (h >> 8).astype(np.uint8)
    b = blocks.random_blocks(qt, nb, rng, allow_subnormal=False)
    ws = [torch.from_numpy(cdequant.oracle_dequant(qt, q, n * d_pad).reshape(n, d_pad)) for q in (a, b)]
    probs = torch.tensor([0.3, 0.7])
    ref = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    got = hip.mix_weight([GGML[qt]] * 2, [_dev(q.reshape(-1)) for q in (a, b)], probs.cuda(), n, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


def _run_fwd_bwd(hip, types, m, n, d, d_pad, qbs, probs, x, dy):
    dev_q = [_dev(q.reshape(-1)) for q in qbs]
    ids = [GGML[t] for t in types]
    xd, dyd, pd = x.cuda(), dy.cuda(), probs.cuda()
    w_eff = torch.empty(n, d_pad, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    fws = torch.empty(max(hip.fwd_workspace_bytes(m, n, d), 16), dtype=torch.uint8, device="cuda")
    hip.gated_linear_fwd(xd, ids, dev_q, pd, n, d_pad, w_eff, y, fws)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device="cuda")
    dp = torch.empty(len(types), dtype=torch.float32, device="cuda")
    ws = torch.empty(hip.bwd_workspace_bytes(m, n, d, d_pad, len(types), False), dtype=torch.uint8, device="cuda")
    hip.gated_linear_bwd(dyd, xd, ids, dev_q, pd, n, d_pad, w_eff, dx, dp, ws)
    torch.cuda.synchronize()
    return w_eff.cpu(), y.cpu(), dx.cpu(), dp.cpu()


CASES = [
    # (name, types, m, n, d, d_pad)
    ("cfg1", ["Q8_0", "Q6_K", "Q4_K", "Q3_K"], 512, 1024, 1024, 1024),
    # 512 tiles of 256x256: the large-product tile configuration and split tails
    ("large-tiles", ["Q4_K", "Q8_0"], 4096, 8192, 512, 512),
    ("ragged", ["Q2_K", "Q5_K", "Q8_0"], 37, 136, 264, 512),
    ("single-token", ["Q6_K", "Q4_K"], 1, 256, 256, 256),
    ("multi-tile", SIX, 300, 520, 1000, 1024),
    # 208 ragged 256x256 tiles (the 8-wave forward; rows, columns and k all
    # partial at the edges)
    ("large-ragged", ["Q3_K", "Q6_K", "Q8_0"], 4000, 3080, 520, 768),
    # 336 forward tiles: one full round and a K-split tail (the split refill
    # path with partial k ranges and the fixup); dX splits too (16 tiles per
    # XCD, 2 parts), the gate's 21 tiles per XCD run whole (its 3-way splits
    # run in tests/test_gpu_headline.py at 8192 x 5120 -> 17408)
    ("split-tails", ["Q4_K", "Q6_K"], 4096, 5376, 2048, 2048),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_gated_linear_matches_oracle(hip, case):
    name, types, m, n, d, d_pad = case
    print(f"[fwd/bwd] {name} m={m} n={n} d={d} K={len(types)}", flush=True)
    qbs, ws = _rtn_candidates(types, n, d_pad, seed=m + n)
    g = torch.Generator().manual_seed(2)
    probs = torch.softmax(torch.randn(len(types), generator=g), 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    w_eff, y, dx, dp = _run_fwd_bwd(hip, types, m, n, d, d_pad, qbs, probs, x, dy)

    ref_w = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    assert torch.equal(w_eff.view(torch.int16), ref_w.view(torch.int16)), "W_eff not bit-exact"
    wd = ref_w[:, :d]
    y_ref = mixture.forward(x, wd, torch.float64)
    dx_ref, _, gp_ref = mixture.backward(dy, x, wd, [w[:, :d] for w in ws], torch.float64)
    assert mixture.relative_l2(y.double(), y_ref) < TOL
    assert mixture.relative_l2(dx.double(), dx_ref) < TOL
    # gate gradient through the softmax, as autograd applies it (T = 1)
    dg = mixture.gates_grad(dp.double(), probs.double(), 1.0)
    dg_ref = mixture.gates_grad(gp_ref, probs.double(), 1.0)
    assert mixture.relative_l2(dp.double(), gp_ref) < 1e-4
    assert mixture.relative_l2(dg, dg_ref, floor=1e-6 * float(gp_ref.abs().max())) < TOL


def test_gate_gradient_deterministic(hip):
    types = ["Q8_0", "Q4_K", "Q2_K"]
    m, n, d = 256, 512, 512
    qbs, _ = _rtn_candidates(types, n, d, seed=3)
    g = torch.Generator().manual_seed(9)
    probs = torch.softmax(torch.randn(3, generator=g), 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    a = _run_fwd_bwd(hip, types, m, n, d, d, qbs, probs, x, dy)
    b = _run_fwd_bwd(hip, types, m, n, d, d, qbs, probs, x, dy)
    for u, v in zip(a, b):
        assert torch.equal(u.view(torch.uint8) if u.dtype != torch.float32 else u, v.view(torch.uint8)
                           if v.dtype != torch.float32 else v)


def _oracle_candidates(mod, ncols):
    """The module's candidates decoded by the oracle from its packed bytes
    (fp32 [out, ncols]), not by the kernels under test."""
    rows, dp = mod.out_features if hasattr(mod, "out_features") else mod.num_embeddings, mod.padded_in_features
    return [torch.from_numpy(cdequant.oracle_dequant(qt, getattr(mod, f"_qweight_{k}").cpu().numpy(), rows * dp))
            .reshape(rows, dp)[:, :ncols] for k, qt in enumerate(mod.candidate_types)]


def test_module_gates_grad_matches_softmax_jacobian(hip):
    """Port of tests/test_ptqr.py:161-186 (soft mixture) onto the HIP module."""
    from voodoo_quant.layers import MixedQuantLinear

    torch.manual_seed(23)
    in_f, out_f = 512, 64
    qts = ["Q3_K", "Q5_K", "Q8_0"]
    lin = MixedQuantLinear(in_features=in_f, out_features=out_f, candidate_types=qts,
                           source_weight=torch.randn(out_f, in_f) * 0.02, tensor_name="tests.gpu.linear",
                           device="cuda")
    with torch.no_grad():
        lin.gates.copy_(torch.tensor([0.3, -0.2, 0.5]))
    lin.set_temperature(0.7)
    x = torch.randn(6, in_f).to(torch.bfloat16).cuda()
    y = lin(x)
    G = torch.randn_like(y)
    y.backward(G)
    cands = [c.double() for c in _oracle_candidates(lin, in_f)]
    xf, Gf = x.double().cpu(), G.double().cpu()
    gp = torch.stack([(Gf * (xf @ c.t())).sum() for c in cands])
    p = lin.soft_probs().detach().double().cpu()
    ref = (torch.diag(p) - torch.outer(p, p)) @ gp / 0.7
    assert mixture.relative_l2(lin.gates.grad.double().cpu(), ref) < TOL
    # forward equals x @ (sum p_k W_k)^T
    mix = sum(p[k] * cands[k] for k in range(3))
    assert mixture.relative_l2(y.double().cpu(), xf @ mix.t()) < TOL
