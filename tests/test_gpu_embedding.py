"""Gated embedding rows and the Q8_0 teacher on the HIP path, against the oracle.

Bars:
* mixture rows bit-exact: fp32 rows equal the oracle's k-ordered fp32 mixture
  of ggml's values, bf16 rows equal its round-to-nearest-even, and both equal
  the same rows of ``vq_mix_weight``'s W_eff;
* routed (PTQR) rows bit-exact to the routed candidate's ggml values (fp32) and
  their bf16 rounding;
* dL/dp_k = sum_r <G[r], W_k[ids[r]]> within 1e-5 of the fp64 sum, relative
  to sum |G W_k| (fp32 products and partial sums, fp64 block reduction);
* the Q8_0 teacher: embedding rows bit-exact to the bf16 decode, Linear
  outputs within 1e-2 relative L2 of the fp64 product of the bf16 decode.

Ports the reference's tests/test_ptqr.py:93-119 (routed embedding rows),
:121-186 (module toggle, embedding part) and :187-219 (routed lazy embedding
on the GPU), with the reference's own menus (IQ2_XXS/Q4_K and
IQ2_XXS/IQ3_XXS/Q8_0).
"""

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture
from voodoo_quant import layers

pytestmark = pytest.mark.gpu

SIX = ["Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
GGML = dict(cdequant.GGML_TYPE)


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _table(types, vocab, d_pad, seed):
    """Random valid candidate bytes of a [vocab, d_pad] table and ggml's fp32 values."""
    rng = np.random.default_rng(seed)
    qbs, ws = [], []
    for qt in types:
        per = 8 if qt == "Q8_0" else 1
        qb = blocks.random_blocks(qt, vocab * d_pad // 256 * per, rng)
        qbs.append(torch.from_numpy(qb.reshape(-1)).cuda())
        ws.append(torch.from_numpy(cdequant.oracle_dequant(qt, qb, vocab * d_pad).reshape(vocab, d_pad)))
    return qbs, ws


def _bits(t):
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


CASES = [  # (types, vocab, dim, d_pad)
    (SIX, 50, 256, 256),
    (SIX, 37, 1000, 1024),                       # ragged: the last group is cut at 1000
    (["Q3_K", "Q6_K", "Q2_K"], 20, 5120, 5120),  # 20 groups: two segments of 10
    (["Q8_0", "Q4_K"], 9, 4352, 4352),           # 17 groups: segments of 9 and 8
    (["Q3_K"], 33, 256, 256),                    # 110-byte rows: no row starts 16-byte aligned
]


@pytest.mark.parametrize("types,vocab,dim,d_pad", CASES)
def test_mixture_rows_bit_exact(hip, types, vocab, dim, d_pad):
    print(f"[emb mix] types={types} vocab={vocab} dim={dim}", flush=True)
    qbs, ws = _table(types, vocab, d_pad, seed=vocab * 7 + dim)
    g = torch.Generator().manual_seed(vocab)
    probs = torch.softmax(torch.randn(len(types), generator=g), 0)
    ids = torch.cat([torch.randint(0, vocab, (61,), generator=g), torch.tensor([0, vocab - 1, 3, 3])])
    mixed = mixture.mix_weight(ws, probs)  # fp32 [vocab, d_pad]
    ref32 = mixed[ids][:, :dim]
    ggml = tuple(GGML[t] for t in types)
    pd, idd = probs.cuda(), ids.cuda()
    got32 = hip.embedding_rows_fwd(ggml, qbs, pd, None, idd, vocab, dim, d_pad, torch.float32)
    got16 = hip.embedding_rows_fwd(ggml, qbs, pd, None, idd, vocab, dim, d_pad, torch.bfloat16)
    w_eff = hip.mix_weight(ggml, qbs, pd, vocab, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got32.cpu()), _bits(ref32))
    assert torch.equal(_bits(got16.cpu()), _bits(ref32.to(torch.bfloat16)))
    assert torch.equal(_bits(got16.cpu()), _bits(w_eff.cpu()[ids][:, :dim]))


@pytest.mark.parametrize("types,vocab,dim,d_pad", CASES)
def test_routed_rows_bit_exact(hip, types, vocab, dim, d_pad):
    print(f"[emb routed] types={types} vocab={vocab} dim={dim}", flush=True)
    qbs, ws = _table(types, vocab, d_pad, seed=vocab * 11 + dim)
    g = torch.Generator().manual_seed(vocab + 1)
    ids = torch.randint(0, vocab, (70,), generator=g)
    routing = torch.randint(0, len(types), (70,), generator=g)
    ref32 = torch.stack([ws[int(routing[r])][int(ids[r]), :dim] for r in range(70)])
    ggml = tuple(GGML[t] for t in types)
    got32 = hip.embedding_rows_fwd(ggml, qbs, None, routing.cuda(), ids.cuda(), vocab, dim, d_pad, torch.float32)
    got16 = hip.embedding_rows_fwd(ggml, qbs, None, routing.cuda(), ids.cuda(), vocab, dim, d_pad)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got32.cpu()), _bits(ref32))
    assert torch.equal(_bits(got16.cpu()), _bits(ref32.to(torch.bfloat16)))


@pytest.mark.parametrize("types,vocab,dim,d_pad", CASES)
@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float32])
def test_rows_backward(hip, types, vocab, dim, d_pad, gdtype):
    print(f"[emb bwd] types={types} vocab={vocab} dim={dim} grad={gdtype}", flush=True)
    qbs, ws = _table(types, vocab, d_pad, seed=vocab * 13 + dim)
    g = torch.Generator().manual_seed(vocab + 2)
    ids = torch.randint(0, vocab, (45,), generator=g)
    grad = torch.randn(45, dim, generator=g).to(gdtype)
    ggml = tuple(GGML[t] for t in types)
    got = hip.embedding_rows_bwd(ggml, qbs, ids.cuda(), vocab, dim, d_pad, grad.cuda())
    again = hip.embedding_rows_bwd(ggml, qbs, ids.cuda(), vocab, dim, d_pad, grad.cuda())
    torch.cuda.synchronize()
    gd = grad.double()
    for k, w in enumerate(ws):
        terms = gd * w[ids][:, :dim].double()
        ref, scale = float(terms.sum()), float(terms.abs().sum())
        assert abs(float(got[k]) - ref) <= 1e-5 * scale + 1e-30, (types[k], float(got[k]), ref)
    assert torch.equal(got.cpu(), again.cpu())  # fixed-order reduction


def test_out_of_range_rows_and_routes_are_zero(hip):
    types, vocab, dim = ["Q4_K", "Q8_0"], 12, 512
    qbs, ws = _table(types, vocab, dim, seed=3)
    ggml = (GGML["Q4_K"], GGML["Q8_0"])
    ids = torch.tensor([-1, 0, vocab, 5, 2 ** 40, 11], device="cuda")
    probs = torch.tensor([0.25, 0.75], device="cuda")
    out = hip.embedding_rows_fwd(ggml, qbs, probs, None, ids, vocab, dim, dim, torch.float32).cpu()
    bad = [0, 2, 4]
    assert torch.count_nonzero(out[bad]) == 0
    routing = torch.tensor([0, 1, 0, 2, 1, -1], device="cuda")
    routed = hip.embedding_rows_fwd(ggml, qbs, None, routing, ids, vocab, dim, dim, torch.float32).cpu()
    assert torch.count_nonzero(routed[bad + [3, 5]]) == 0
    assert torch.equal(routed[1], ws[1][0])
    grad = torch.ones(6, dim, device="cuda")
    dp = hip.embedding_rows_bwd(ggml, qbs, ids, vocab, dim, dim, grad).cpu().double()
    for k in range(2):
        ref = float(ws[k][[0, 5, 11]].double().sum())
        assert abs(float(dp[k]) - ref) <= 1e-5 * float(ws[k][[0, 5, 11]].double().abs().sum())


def test_no_rows(hip):
    types, vocab, dim = ["Q2_K", "Q6_K"], 4, 256
    qbs, _ = _table(types, vocab, dim, seed=4)
    ggml = (GGML["Q2_K"], GGML["Q6_K"])
    ids = torch.empty(0, dtype=torch.int64, device="cuda")
    out = hip.embedding_rows_fwd(ggml, qbs, torch.ones(2, device="cuda") / 2, None, ids, vocab, dim, dim)
    assert out.shape == (0, dim)
    dp = hip.embedding_rows_bwd(ggml, qbs, ids, vocab, dim, dim, torch.empty(0, dim, dtype=torch.bfloat16,
                                                                            device="cuda"))
    assert torch.equal(dp.cpu(), torch.zeros(2))


def test_rejects_bad_arguments(hip):
    qbs, _ = _table(["Q4_K"], 4, 256, seed=5)
    ids = torch.zeros(3, dtype=torch.int64, device="cuda")
    p = torch.ones(1, device="cuda")
    with pytest.raises(ValueError, match="multiple of 8"):
        hip.embedding_rows_fwd((12,), qbs, p, None, ids, 4, 100, 256)
    with pytest.raises(ValueError, match="exceeds d_pad"):
        hip.embedding_rows_fwd((12,), qbs, p, None, ids, 4, 512, 256)
    with pytest.raises(ValueError, match="int64"):
        hip.embedding_rows_fwd((12,), qbs, p, None, ids.int(), 4, 256, 256)
    with pytest.raises(ValueError, match="unsupported"):
        hip.embedding_rows_fwd((9,), qbs, p, None, ids, 4, 256, 256)


# ----------------------------------------------------------------------------- ports of tests/test_ptqr.py
def _rtn_cands(types, vocab, dim, weight):
    from voodoo_quant import rtn

    qbs = [rtn.rtn_quantize_tensor(weight, qt) for qt in types]
    cands = [torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), vocab * dim).reshape(vocab, dim))
             for qt, qb in zip(types, qbs)]
    return qbs, cands


def test_routed_embedding_rows(hip):
    """Port of tests/test_ptqr.py:93-119 (menu IQ2_XXS/Q4_K)."""
    torch.manual_seed(11)
    vocab, dim = 64, 256
    qts = ["IQ2_XXS", "Q4_K"]
    weight = torch.randn(vocab, dim, dtype=torch.float32)
    qbs, cands = _rtn_cands(qts, vocab, dim, weight)
    base = torch.softmax(torch.randn(len(qts)), dim=0)
    probs = base.detach().clone().cuda().requires_grad_(True)
    ids = torch.randint(0, vocab, (12,))
    routing = layers._sample_token_routing(probs.detach(), 12)
    meta = (tuple(GGML[t] for t in qts), vocab, dim, dim, torch.float32)
    y = layers.EmbeddingRowsFunction.apply(probs, routing, ids.cuda(), meta, *[q.reshape(-1).cuda() for q in qbs])
    ref = torch.stack([cands[int(routing[t])][ids[t]] for t in range(12)])
    assert torch.allclose(y.cpu(), ref, rtol=0, atol=0)
    G = torch.randn_like(y)
    y.backward(G)
    gp_ref = torch.stack([(G.cpu() * c[ids]).sum() for c in cands])
    assert torch.allclose(probs.grad.cpu(), gp_ref, rtol=1e-5, atol=1e-5)


def _oracle_candidates(mod, ncols):
    """The module's candidates decoded by the oracle from its packed bytes
    (fp32 [out, ncols]), not by the kernels under test."""
    rows, dp = mod.out_features if hasattr(mod, "out_features") else mod.num_embeddings, mod.padded_in_features
    return [torch.from_numpy(cdequant.oracle_dequant(qt, getattr(mod, f"_qweight_{k}").cpu().numpy(), rows * dp))
            .reshape(rows, dp)[:, :ncols] for k, qt in enumerate(mod.candidate_types)]


def test_module_toggle_embedding(hip):
    """Port of tests/test_ptqr.py:121-186, embedding part (menu IQ2_XXS/IQ3_XXS/Q8_0),
    plus the gate gradient through the softmax and the toggled-off mixture."""
    torch.manual_seed(23)
    in_f = 256
    qts = ["IQ2_XXS", "IQ3_XXS", "Q8_0"]
    emb = layers.MixedQuantEmbedding(num_embeddings=64, embedding_dim=in_f, candidate_types=qts,
                                     source_weight=torch.randn(64, in_f, dtype=torch.float32),
                                     tensor_name="tests.ptqr.embedding").cuda()
    ids = torch.randint(0, 64, (6,)).cuda()
    cands = [c.cuda() for c in _oracle_candidates(emb, in_f)]
    layers.set_ptqr(True)
    try:
        ey = emb(ids)
        outs = [c[ids] for c in cands]
        for t in range(ids.numel()):
            matches = [torch.allclose(ey[t], o[t], rtol=1e-5, atol=1e-4) for o in outs]
            assert sum(matches) == 1, "some embedding row not from exactly one candidate"
        emb.zero_grad()
        ey = emb(ids)
        G = torch.randn_like(ey)
        ey.backward(G)
        gp = torch.stack([(G * o).sum() for o in outs])
        p = emb.soft_probs().detach()
        gates_ref = (torch.diag(p) - torch.outer(p, p)) @ gp
        assert torch.allclose(emb.gates.grad, gates_ref, rtol=1e-4, atol=1e-4)
    finally:
        layers.set_ptqr(False)
    y_mix = emb(ids)
    p = emb.get_probs().detach()
    mix = sum(p[k] * cands[k] for k in range(len(qts)))
    assert torch.allclose(y_mix, mix[ids], rtol=1e-5, atol=1e-5)


def test_lazy_embedding_routing(hip):
    """Port of tests/test_ptqr.py:187-219 (lazy routed embedding on the GPU)."""
    torch.manual_seed(31)
    dev = torch.device("cuda")
    vocab, dim = 64, 256
    qts = ["Q4_K", "Q8_0"]
    emb = layers.MixedQuantEmbedding(num_embeddings=vocab, embedding_dim=dim, candidate_types=qts,
                                     source_weight=torch.randn(vocab, dim, dtype=torch.float32), device=dev,
                                     lazy=True, qbytes_device=dev, tensor_name="tests.ptqr.embedding_lazy")
    cands = [torch.from_numpy(cdequant.oracle_dequant(qt, getattr(emb, f"_qweight_{k}").cpu().numpy(), vocab * dim))
             .reshape(vocab, dim).to(dev) for k, qt in enumerate(qts)]
    ids = torch.randint(0, vocab, (9,), device=dev)
    layers.set_ptqr(True)
    try:
        y = emb(ids)
        for t in range(ids.numel()):
            matches = [torch.allclose(y[t], c[ids[t]], rtol=1e-2, atol=1e-2) for c in cands]
            assert sum(matches) >= 1, "lazy routed embedding row not from any single candidate"
    finally:
        layers.set_ptqr(False)


def test_bf16_module_rows_and_duplicates(hip):
    """A bf16 source weight: rows are the bf16 mixture (the W_eff rows), the
    lookup keeps the input's shape, and duplicate ids share one row."""
    torch.manual_seed(5)
    vocab, dim = 300, 1000
    qts = ["Q4_K", "Q6_K", "Q8_0"]
    emb = layers.MixedQuantEmbedding(vocab, dim, qts, (torch.randn(vocab, dim) * 0.02).to(torch.bfloat16),
                                     tensor_name="tests.emb.bf16").cuda()
    ids = torch.randint(0, vocab, (4, 33)).cuda()
    ids[1, 5] = ids[0, 0]
    y = emb(ids)
    assert y.shape == (4, 33, dim) and y.dtype == torch.bfloat16
    w_eff = emb.get_mixed_weight().detach()
    assert torch.equal(_bits(y.reshape(-1, dim)), _bits(w_eff[ids.reshape(-1)]))
    with pytest.raises(IndexError):
        emb(torch.tensor([0, vocab], device="cuda"))


def test_mixture_gate_gradient_with_repeated_ids(hip):
    """Without PTQR every position decodes its own row: a repeated id's
    gate-gradient terms add up, dL/dp_k = sum_t <G_t, W_k[id_t]>, as the
    reference's unique-row lookup scattered back (layers.py:670-750)."""
    torch.manual_seed(29)
    vocab, dim = 40, 512
    qts = ["Q3_K", "Q5_K", "IQ4_XS"]
    emb = layers.MixedQuantEmbedding(vocab, dim, qts, torch.randn(vocab, dim, dtype=torch.float32) * 0.05,
                                     tensor_name="tests.emb.repeats").cuda()
    ids = torch.randint(0, 6, (3, 50)).cuda()  # every id repeated many times
    cands = [c.cuda().double() for c in _oracle_candidates(emb, dim)]
    y = emb(ids)
    G = torch.randn_like(y)
    y.backward(G)
    flat = ids.reshape(-1)
    gp = torch.stack([(G.reshape(-1, dim).double() * c[flat]).sum() for c in cands])
    p = emb.soft_probs().detach().double()
    gates_ref = (torch.diag(p) - torch.outer(p, p)) @ gp
    err = float((emb.gates.grad.double() - gates_ref).norm() / gates_ref.norm())
    assert err < 1e-5, err


def test_deferred_id_check(hip):
    """id_check = "deferred": the lookup returns at once (zero rows for the
    out-of-range ids, as the row kernels give), and raise_pending_id_errors
    raises the IndexError afterwards; valid lookups leave nothing pending."""
    from voodoo_quant.training.q8_teacher import Q8Embedding

    torch.manual_seed(31)
    vocab, dim = 50, 256
    emb = layers.MixedQuantEmbedding(vocab, dim, ["Q4_K", "Q8_0"], torch.randn(vocab, dim) * 0.05,
                                     tensor_name="tests.emb.deferred").cuda()
    qb, _ = _q8_bytes(vocab, dim, seed=7)
    q8 = Q8Embedding(qb.cuda(), vocab, dim)
    layers.raise_pending_id_errors()
    for mod in (emb, q8):
        with pytest.raises(IndexError):
            mod(torch.tensor([1, vocab], device="cuda"))
        mod.id_check = "deferred"
        try:
            y = mod(torch.tensor([[1, vocab], [-1, 2]], device="cuda"))
            assert y.shape == (2, 2, dim)
            assert torch.count_nonzero(y[0, 1]) == 0 and torch.count_nonzero(y[1, 0]) == 0
            assert torch.count_nonzero(y[0, 0]) > 0
            with pytest.raises(IndexError, match="index out of range"):
                layers.raise_pending_id_errors()
            mod(torch.tensor([0, vocab - 1], device="cuda"))
            layers.raise_pending_id_errors()  # nothing pending raises
        finally:
            mod.id_check = "sync"
    assert not layers._PENDING_ID_CHECKS
    # a caller that never collects: finished checks are taken along the way
    emb.id_check = "deferred"
    try:
        ids = torch.tensor([0, 1, 2], device="cuda")
        for _ in range(3 * layers._MAX_PENDING_ID_CHECKS):
            emb(ids)
            torch.cuda.synchronize()
        assert len(layers._PENDING_ID_CHECKS) <= layers._MAX_PENDING_ID_CHECKS
        layers.raise_pending_id_errors()
    finally:
        emb.id_check = "sync"
    assert not layers._PENDING_ID_CHECKS


# ----------------------------------------------------------------------------- Q8_0 teacher
def _q8_bytes(rows, cols, seed):
    from voodoo_quant import rtn

    w = torch.randn(rows, cols, generator=torch.Generator().manual_seed(seed)) * 0.05
    qb = rtn.rtn_quantize_tensor(w, "Q8_0").reshape(-1)
    n = rows * cols
    extra = (-n) % 256 // 32  # zero blocks so the oracle sees whole 256-weight groups
    padded = np.concatenate([qb.numpy(), np.zeros(extra * 34, np.uint8)])
    dec = torch.from_numpy(cdequant.oracle_dequant("Q8_0", padded, n + extra * 32)[:n].reshape(rows, cols))
    return qb, dec


@pytest.mark.parametrize("out_f,in_f,bias", [(13, 160, True), (512, 1024, False), (264, 5120, True)])
def test_q8_linear(hip, out_f, in_f, bias):
    from voodoo_quant.training.q8_teacher import Q8Linear, set_keep_decoded

    set_keep_decoded(False)
    print(f"[q8 linear] out={out_f} in={in_f} bias={bias}", flush=True)
    qb, dec = _q8_bytes(out_f, in_f, seed=out_f)
    g = torch.Generator().manual_seed(in_f)
    b = torch.randn(out_f, generator=g) if bias else None
    lin = Q8Linear(qb.cuda(), out_f, in_f, b)
    x = torch.randn(3, 7, in_f, generator=g).to(torch.bfloat16)
    y = lin(x.cuda())
    torch.cuda.synchronize()
    assert y.shape == (3, 7, out_f) and y.dtype == torch.bfloat16
    w16 = dec.to(torch.bfloat16).double()
    ref = x.double().reshape(-1, in_f) @ w16.t()
    if bias:
        ref = ref + b.to(torch.bfloat16).double()
    got = y.reshape(-1, out_f).cpu().double()
    assert float((got - ref).norm() / ref.norm()) < 1e-2
    assert torch.equal(_bits(lin._weight().cpu()), _bits(dec.to(torch.bfloat16)))
    yf = lin(x.float().cuda())
    assert yf.dtype == torch.float32
    # the decode kept between forwards (a plain GEMM on it, on hipBLASLt) gives
    # the same product within bf16 rounding, the same bits on every call
    from voodoo_quant.training import q8_teacher

    q8_teacher.set_keep_decoded(True)
    try:
        y1, y2 = lin(x.cuda()), lin(x.cuda())
    finally:
        q8_teacher.set_keep_decoded(False)
    assert torch.equal(_bits(y1), _bits(y2))
    g1 = y1.reshape(-1, out_f).cpu().double()
    assert float((g1 - ref).norm() / ref.norm()) < 1e-2
    assert float((g1 - got).norm() / got.norm()) < 1e-2


def test_q8_linear_vocabulary_width_head(hip):
    """A vocabulary-width Q8Linear: the decode-every-forward path (the library's
    mixture with one candidate and its GEMM) and the kept decode (a plain GEMM
    on hipBLASLt) give the same product within bf16 rounding, and of fp64."""
    from voodoo_quant.training import q8_teacher
    from voodoo_quant.training.q8_teacher import Q8Linear

    out_f, in_f = 32768 + 264, 512
    print(f"[q8 linear] vocabulary-width head out={out_f} in={in_f}", flush=True)
    qb, dec = _q8_bytes(out_f, in_f, seed=3)
    lin = Q8Linear(qb.cuda(), out_f, in_f)
    x = torch.randn(5, 33, in_f, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    q8_teacher.set_keep_decoded(False)
    y_lib = lin(x.cuda())
    q8_teacher.set_keep_decoded(True)
    try:
        y_keep = lin(x.cuda())
    finally:
        q8_teacher.set_keep_decoded(False)
    torch.cuda.synchronize()
    assert y_keep.shape == (5, 33, out_f)
    ref = x.double().reshape(-1, in_f) @ dec.to(torch.bfloat16).double().t()
    for y in (y_lib, y_keep):
        got = y.reshape(-1, out_f).cpu().double()
        assert float((got - ref).norm() / ref.norm()) < 1e-2
    assert float((y_keep.float() - y_lib.float()).norm() / y_lib.float().norm()) < 1e-2


@pytest.mark.parametrize("vocab,dim", [(100, 160), (57, 512)])
def test_q8_embedding_rows_exact(hip, vocab, dim):
    from voodoo_quant.training.q8_teacher import Q8Embedding

    qb, dec = _q8_bytes(vocab, dim, seed=vocab)
    emb = Q8Embedding(qb.cuda(), vocab, dim)
    ids = torch.randint(0, vocab, (2, 9), generator=torch.Generator().manual_seed(1))
    ids[1, 3] = ids[0, 0]
    y = emb(ids.cuda())
    assert y.shape == (2, 9, dim) and y.dtype == torch.bfloat16
    assert torch.equal(_bits(y.cpu().reshape(-1, dim)), _bits(dec.to(torch.bfloat16)[ids.reshape(-1)]))
