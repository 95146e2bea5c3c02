"""GPU parity of the IQ decoders (IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS, IQ2_S,
IQ3_XXS, IQ3_S, IQ4_XS) on every path that decodes candidates, through the C
ABI, against the oracle.

Bars, as for the K-quants:
* dequant bit-exact: against the reference's own decoders
  (quants/gpu_dequant.py:53-519, golden vectors) and against the oracle on
  random and edge blocks, up to the 4096 x 14336 microbench shape;
* the W_eff mixture bit-exact (every IQ weight is exact in fp32, so the
  separately rounded k-ordered mixture must match to the bit);
* Y, dX and dL/dp within 1e-2 relative L2 of the fp64 oracle products;
* embedding rows bit-exact, their dL/dp within 1e-5 relative.

Menus: the reference's 27B recipe (configs/qwen38_27b_voodoo30_tp4.sh:90-92:
all, attention and non-attention candidates), every decodable type (14) and
16 candidates (the library's maximum).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture

pytestmark = pytest.mark.gpu

GGML = dict(cdequant.GGML_TYPE)
IQ = list(blocks.IQ_TYPES)
SIX = ["Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
RECIPE = ["Q8_0", "Q5_K", "IQ3_S", "IQ2_S", "IQ2_XXS", "IQ1_S"]
RECIPE_ATTN = ["Q5_K", "IQ3_S", "IQ2_S", "IQ2_XXS"]
RECIPE_MLP = ["IQ4_XS", "IQ3_S", "IQ2_S", "IQ2_XXS", "IQ1_S"]
ALL14 = ["IQ1_S", "IQ1_M", "IQ2_XXS", "IQ2_XS", "IQ2_S", "Q2_K", "IQ3_XXS", "Q3_K", "IQ3_S", "IQ4_XS", "Q4_K", "Q5_K",
         "Q6_K", "Q8_0"]
SIXTEEN = ALL14 + ["IQ2_XXS", "IQ4_XS"]
TOL = 1e-2


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


def _moderate_blocks(qt, nb, rng):
    """Random valid blocks whose fp16 scales lie in [2^-8, 2^-5): O(1) weights."""
    qb = blocks.random_blocks(qt, nb, rng)
    for which in range(len(blocks.F16_OFFSETS[qt]) or 1):
        h = (0x1C00 + rng.integers(0, 0x0C00, size=nb)).astype(np.uint16)
        blocks.set_scale(qt, qb, h, which)
    return qb


def _cands(types, n, d_pad, rng):
    qbs, ws = [], []
    for qt in types:
        per = 8 if qt == "Q8_0" else 1
        qb = _moderate_blocks(qt, n * d_pad // 256 * per, rng)
        qbs.append(qb)
        ws.append(torch.from_numpy(cdequant.oracle_dequant_parallel(qt, qb, n * d_pad).reshape(n, d_pad)))
    return qbs, ws


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("qt", IQ)
def test_iq_dequant_matches_reference_golden(hip, qt):
    g = np.load(Path(__file__).resolve().parent / "golden" / "ref_iq_decoders.npz")
    qb, ref = g[f"{qt}_qbytes"], g[f"{qt}_out"]
    out = hip.dequant(GGML[qt], _dev(qb.reshape(-1)), ref.size // 256, 256)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(-1)
    assert np.array_equal(_bits(got), _bits(ref)), f"{qt}: {np.sum(_bits(got) != _bits(ref))} mismatches"


@pytest.mark.parametrize("qt", IQ)
@pytest.mark.parametrize("groups", [1, 17, 333])
def test_iq_dequant_random_and_edge(hip, qt, groups):
    print(f"[iq-dequant] {qt} groups={groups}", flush=True)
    rng = np.random.default_rng(100 + groups)
    edge = []
    for fill, h in [(0x00, 0x3C00), (0xFF, 0x3C00), (0xFF, 0x0001), (0xA5, 0x7BFF), (0x5A, 0x8000), (0x33, 0xBC00)]:
        b = np.full((1, blocks.BLOCK_BYTES[qt]), fill, np.uint8)
        blocks.set_scale(qt, b, h)
        edge.append(b)
    qb = np.concatenate(edge + [blocks.random_blocks(qt, groups, rng)])[:groups]
    ref = cdequant.oracle_dequant(qt, qb, groups * 256)
    out = hip.dequant(GGML[qt], _dev(qb.reshape(-1)), groups, 256)
    bf = hip.dequant_bf16(GGML[qt], _dev(qb.reshape(-1)), groups, 256)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(-1)
    assert np.array_equal(_bits(got), _bits(ref)), f"{qt}: {np.sum(_bits(got) != _bits(ref))} mismatches"
    ref_bf = torch.from_numpy(ref).to(torch.bfloat16)
    assert torch.equal(bf.cpu().reshape(-1).view(torch.int16), ref_bf.view(torch.int16))


@pytest.mark.parametrize("qt", ["IQ1_M", "IQ2_XXS", "IQ3_S", "IQ4_XS"])
def test_iq_dequant_full_size_4096x14336(hip, qt):
    print(f"[iq-dequant-full] {qt}", flush=True)
    rng = np.random.default_rng(7)
    nrows, ncols = 4096, 14336
    qb = blocks.random_blocks(qt, nrows * ncols // 256, rng)
    ref = cdequant.oracle_dequant_parallel(qt, qb, nrows * ncols)
    out = hip.dequant(GGML[qt], _dev(qb.reshape(-1)), nrows, ncols)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out.cpu().numpy().reshape(-1)), _bits(ref))


# ------------------------------------------------------------------ mixture
MENUS = {"recipe": RECIPE, "recipe-attn": RECIPE_ATTN, "recipe-mlp": RECIPE_MLP, "all14": ALL14,
         "sixteen": SIXTEEN, "iq8": IQ,
         # 16 x 16 Q8_0 groups staged per workgroup: 68 KiB of LDS (past the 64 KiB default)
         "q8x16": ["Q8_0"] * 16}


@pytest.mark.parametrize("menu", list(MENUS))
def test_iq_mix_weight_bit_exact(hip, menu):
    types = MENUS[menu]
    print(f"[iq-mix] {menu} K={len(types)}", flush=True)
    rng = np.random.default_rng(len(types))
    n, d_pad = 263, 768
    qbs, ws = _cands(types, n, d_pad, rng)
    probs = torch.softmax(torch.randn(len(types), generator=torch.Generator().manual_seed(5)), 0)
    ref = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    got = hip.mix_weight([GGML[t] for t in types], [_dev(q.reshape(-1)) for q in qbs], probs.cuda(), n, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu().view(torch.int16), ref.view(torch.int16))


def test_seventeen_candidates_rejected(hip):
    types = SIXTEEN + ["Q8_0"]
    with pytest.raises(ValueError):
        hip.validate_candidates([GGML[t] for t in types], 256, 256, 256)


# ------------------------------------------------------------------ forward / backward
CASES = [
    # (name, types, m, n, d, d_pad)
    ("recipe", RECIPE, 512, 1024, 1024, 1024),
    ("recipe-mlp-ragged", RECIPE_MLP, 300, 520, 1000, 1024),
    ("all14", ALL14, 256, 512, 768, 768),
    ("sixteen-split", SIXTEEN, 2048, 2048, 2048, 2048),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_iq_gated_linear_matches_oracle(hip, case):
    name, types, m, n, d, d_pad = case
    print(f"[iq-fwd/bwd] {name} m={m} n={n} d={d} K={len(types)}", flush=True)
    rng = np.random.default_rng(m + n)
    qbs, ws = _cands(types, n, d_pad, rng)
    g = torch.Generator().manual_seed(2)
    probs = torch.softmax(torch.randn(len(types), generator=g), 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    ids = [GGML[t] for t in types]
    dq = [_dev(q.reshape(-1)) for q in qbs]
    xd, dyd, pd = x.cuda(), dy.cuda(), probs.cuda()
    w_eff = torch.empty(n, d_pad, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    fws = torch.empty(max(hip.fwd_workspace_bytes(m, n, d), 16), dtype=torch.uint8, device="cuda")
    hip.gated_linear_fwd(xd, ids, dq, pd, n, d_pad, w_eff, y, fws)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device="cuda")
    dp = torch.empty(len(types), dtype=torch.float32, device="cuda")
    ws_b = torch.empty(hip.bwd_workspace_bytes(m, n, d, d_pad, len(types), False), dtype=torch.uint8, device="cuda")
    hip.gated_linear_bwd(dyd, xd, ids, dq, pd, n, d_pad, w_eff, dx, dp, ws_b)
    torch.cuda.synchronize()
    ref_w = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    assert torch.equal(w_eff.cpu().view(torch.int16), ref_w.view(torch.int16)), "W_eff not bit-exact"
    wd = ref_w[:, :d]
    y_ref = mixture.forward(x, wd, torch.float64)
    dx_ref, _, gp_ref = mixture.backward(dy, x, wd, [w[:, :d] for w in ws], torch.float64)
    e_y = mixture.relative_l2(y.cpu().double(), y_ref)
    e_dx = mixture.relative_l2(dx.cpu().double(), dx_ref)
    e_gp = mixture.relative_l2(dp.cpu().double(), gp_ref)
    print(f"[iq-fwd/bwd] {name}: Y {e_y:.2e} dX {e_dx:.2e} dL/dp {e_gp:.2e}", flush=True)
    assert e_y < TOL and e_dx < TOL
    assert e_gp < 1e-4


@pytest.mark.parametrize("m", [1, 16, 32])
def test_iq_fused_matches_oracle(hip, m):
    types = RECIPE
    n, d = 2048, 1536
    print(f"[iq-fused] m={m} n={n} d={d}", flush=True)
    rng = np.random.default_rng(40 + m)
    qbs, ws = _cands(types, n, d, rng)
    g = torch.Generator().manual_seed(m)
    probs = torch.softmax(torch.randn(len(types), generator=g), 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    ids = [GGML[t] for t in types]
    dq = [_dev(q.reshape(-1)) for q in qbs]
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    dx = torch.full((m, d), float("nan"), dtype=torch.bfloat16, device="cuda")
    wsf = torch.empty(max(hip.fused_workspace_bytes(m, n, d, False), 16), dtype=torch.uint8, device="cuda")
    wsd = torch.empty(max(hip.fused_workspace_bytes(m, n, d, True), 16), dtype=torch.uint8, device="cuda")
    hip.gated_linear_fwd_fused(x.cuda(), ids, dq, probs.cuda(), n, d, y, wsf)
    hip.gated_linear_dx_fused(dy.cuda(), ids, dq, probs.cuda(), d, d, dx, wsd)
    torch.cuda.synchronize()
    ref_w = mixture.mix_weight(ws, probs).to(torch.bfloat16)
    e_y = mixture.relative_l2(y.cpu().double(), mixture.forward(x, ref_w, torch.float64))
    e_dx = mixture.relative_l2(dx.cpu().double(), dy.double() @ ref_w.double())
    print(f"[iq-fused] m={m}: Y {e_y:.2e} dX {e_dx:.2e}", flush=True)
    assert e_y < TOL and e_dx < TOL


def test_iq_embedding_rows(hip):
    types = RECIPE_MLP
    vocab, dim = 304, 512
    rng = np.random.default_rng(9)
    qbs, ws = _cands(types, vocab, dim, rng)
    probs = torch.softmax(torch.randn(len(types), generator=torch.Generator().manual_seed(9)), 0)
    ids = torch.from_numpy(rng.integers(0, vocab, size=77)).to(torch.int64)
    dq = [_dev(q.reshape(-1)) for q in qbs]
    gids = [GGML[t] for t in types]
    rows = hip.embedding_rows_fwd(gids, dq, probs.cuda(), None, ids.cuda(), vocab, dim, dim, torch.float32)
    grad = torch.randn(ids.numel(), dim, generator=torch.Generator().manual_seed(3))
    dp = hip.embedding_rows_bwd(gids, dq, ids.cuda(), vocab, dim, dim, grad.cuda())
    torch.cuda.synchronize()
    ref_rows = mixture.mix_weight(ws, probs)[ids]
    assert torch.equal(rows.cpu().view(torch.int32), ref_rows.view(torch.int32))
    ref_dp = torch.stack([(grad.double() * w[ids].double()).sum() for w in ws])
    scale = torch.stack([(grad.double() * w[ids].double()).abs().sum() for w in ws])
    assert float(((dp.cpu().double() - ref_dp).abs() / scale).max()) < 1e-5


def test_module_with_recipe_menu(hip):
    """A gated Linear over the 27B recipe's menu, candidates from the package's
    encoders: Y, dX and gates.grad match the oracle (decoded by the oracle)."""
    from voodoo_quant import layers

    torch.manual_seed(31)
    in_f, out_f = 768, 512
    lin = layers.MixedQuantLinear(in_features=in_f, out_features=out_f, candidate_types=RECIPE,
                                  source_weight=torch.randn(out_f, in_f) * 0.02, tensor_name="tests.iq.recipe")
    cands = [torch.from_numpy(cdequant.oracle_dequant(qt, getattr(lin, f"_qweight_{k}").numpy(), out_f * in_f))
             .reshape(out_f, in_f).double() for k, qt in enumerate(RECIPE)]
    lin = lin.to("cuda")
    with torch.no_grad():
        lin.gates.copy_(torch.linspace(-0.5, 0.5, len(RECIPE)))
    lin.set_temperature(0.8)
    for tokens in (8, 96):  # the fused path and the materialising one
        lin.gates.grad = None
        x = torch.randn(tokens, in_f).to(torch.bfloat16).cuda().requires_grad_(True)
        y = lin(x)
        G = torch.randn_like(y)
        y.backward(G)
        xf, Gf = x.detach().double().cpu(), G.double().cpu()
        p = lin.soft_probs().detach().double().cpu()
        mix = sum(p[k] * cands[k] for k in range(len(RECIPE)))
        gp = torch.stack([(Gf * (xf @ c.t())).sum() for c in cands])
        ref = (torch.diag(p) - torch.outer(p, p)) @ gp / 0.8
        assert mixture.relative_l2(y.detach().double().cpu(), xf @ mix.t()) < TOL
        assert mixture.relative_l2(x.grad.double().cpu(), Gf @ mix) < TOL
        assert mixture.relative_l2(lin.gates.grad.double().cpu(), ref) < TOL
