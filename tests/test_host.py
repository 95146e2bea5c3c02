"""Host logic of the drop-in package (CPU only): registry, RTN candidate bytes,
candidate cache, module construction, budget, temperature, ST-Gumbel, menus,
TP slicing and the refusal to run the mixture off-GPU.

Ports of the reference's CPU assertions: tests/test_ggml.py:13-33,
tests/test_invariants.py:20-52, 57-128."""

import numpy as np
import pytest
import torch

from oracle import cdequant
from voodoo_quant import cache, ggml, layers, rtn
from voodoo_quant.training import trainer

SIX = ["Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]


def test_registry_and_ladder():
    types = ggml.list_quant_types()
    assert "IQ4_XS" in types and "Q8_0" in types and "Q2_K" in types and "Q3_K" in types
    ladder = ggml.QUANT_LADDER
    assert set(ladder) <= set(types)
    bpw = [ggml.bytes_per_weight(qt) for qt in ladder]
    assert bpw == sorted(bpw)
    assert ggml.get_quant_info("Q2_K").ggml_type == 10 and ggml.get_quant_info("Q2_K").block_bytes == 84
    assert ggml.get_quant_info("Q3_K").ggml_type == 11 and ggml.get_quant_info("Q3_K").block_bytes == 110
    assert ggml.get_quant_info("Q3_K").dequant_func == "dequantize_row_q3_K"


def test_default_candidates_exclude_ternary():
    cands = ggml.default_candidate_types()
    assert "TQ1_0" not in cands and "TQ2_0" not in cands
    assert cands[0] == "IQ1_S" and cands[-1] == "Q8_0"


def test_bytes_per_weight_matches_registry():
    assert ggml.bytes_per_weight("Q8_0") == pytest.approx(34 / 32)
    assert ggml.bytes_per_weight("Q2_K") == pytest.approx(84 / 256)
    with pytest.raises(ValueError):
        ggml.get_quant_info("NOT_A_QUANT")


@pytest.mark.parametrize("qt", SIX)
def test_rtn_blocks_are_valid_and_accurate(qt):
    torch.manual_seed(0)
    w = torch.randn(8, 512)
    qb = rtn.rtn_quantize_tensor(w, qt)
    bs, bb = rtn.BLOCK[qt]
    assert qb.shape == (8 * 512 // bs, bb)
    y = torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), w.numel()).reshape(w.shape))
    err = ((y - w).abs().mean() / w.abs().mean()).item()
    ceil = {"Q8_0": 0.02, "Q6_K": 0.05, "Q5_K": 0.08, "Q4_K": 0.12, "Q3_K": 0.25, "Q2_K": 0.45}[qt]
    assert err < ceil, f"{qt} roundtrip error {err:.3f}"


IQ_CEIL = {"IQ1_S": 0.55, "IQ1_M": 0.5, "IQ2_XXS": 0.45, "IQ2_XS": 0.4, "IQ2_S": 0.35, "IQ3_XXS": 0.25,
           "IQ3_S": 0.2, "IQ4_XS": 0.12}


@pytest.mark.parametrize("qt", list(IQ_CEIL))
def test_iq_encoder_blocks_are_valid_and_accurate(qt):
    """Relative L2 round trip on 8 x 512 N(0, 1) weights (the reference's
    tests/test_ggml.py:38-49 bars: IQ4_XS < 0.12, IQ2_XXS < 0.45, measured with
    llama.cpp's quantizer at 0.080 and 0.352), decoded by the oracle."""
    from voodoo_quant import iq_encode

    torch.manual_seed(0)
    w = torch.randn(8, 512)
    qb = rtn.rtn_quantize_tensor(w, qt)
    assert qb.dtype == torch.uint8 and qb.shape == (8 * 2, iq_encode.IQ_BLOCK_BYTES[qt])
    y = torch.from_numpy(cdequant.oracle_dequant(qt, qb.numpy(), w.numel()).reshape(w.shape))
    assert torch.isfinite(y).all()
    rel = float((y - w).norm() / w.norm())
    assert rel < IQ_CEIL[qt], f"{qt} roundtrip error {rel:.3f}"


def test_iq_encoder_zero_rows_and_scale_invariance():
    """All-zero rows decode to zeros; scaling the weights by 2 scales every
    decoded weight by 2 (the encoder's choices depend only on ratios)."""
    torch.manual_seed(2)
    w = torch.randn(4, 256)
    w[1] = 0
    for qt in IQ_CEIL:
        y1 = cdequant.oracle_dequant(qt, rtn.rtn_quantize_tensor(w, qt).numpy(), w.numel()).reshape(4, 256)
        y2 = cdequant.oracle_dequant(qt, rtn.rtn_quantize_tensor(2 * w, qt).numpy(), w.numel()).reshape(4, 256)
        assert np.all(np.abs(y1[1]) < 1e-20), qt
        assert np.array_equal(y2, 2 * y1), qt


def test_iq_code_books_parse():
    from voodoo_quant import iq_encode

    t = iq_encode.tables()
    assert t["iq2xxs_grid"].shape == (256, 8) and set(np.unique(t["iq2xxs_grid"])) == {8, 25, 43}
    assert t["iq2xs_grid"].shape == (512, 8) and t["iq2s_grid"].shape == (1024, 8)
    assert t["iq3xxs_grid"].shape == (256, 4) and t["iq3s_grid"].shape == (512, 4)
    assert t["iq1s_grid"].shape == (2048, 8) and set(np.unique(t["iq1s_grid"])) == {-1, 0, 1}
    assert t["iq4nl_values"].tolist()[:2] == [-127, -104] and len(t["iq4nl_values"]) == 16
    # every grid row is distinct (a decoder indexing a wrong table would repeat rows)
    for name in ("iq2xxs_grid", "iq2xs_grid", "iq2s_grid", "iq3xxs_grid", "iq3s_grid", "iq1s_grid"):
        assert len({r.tobytes() for r in t[name]}) == t[name].shape[0], name


def test_rtn_error_ladder_is_monotone():
    torch.manual_seed(1)
    w = torch.randn(16, 1024) * 0.02
    errs = []
    for qt in ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]:
        y = cdequant.oracle_dequant(qt, rtn.rtn_quantize_tensor(w, qt).numpy(), w.numel())
        errs.append(float(np.abs(y - w.numpy().reshape(-1)).mean()))
    assert errs == sorted(errs, reverse=True)


def test_rtn_q8_0_is_ggml_round_to_nearest():
    """Q8_0 codes are roundf(x / (amax / 127)) with d stored as fp16."""
    x = torch.tensor([[0.5, -1.0, 0.25, 0.0] * 8])
    qb = rtn.rtn_quantize_tensor(x, "Q8_0").numpy()[0]
    d = np.frombuffer(qb[:2].tobytes(), np.float16)[0]
    assert d == np.float16(1.0 / 127)
    q = qb[2:].view(np.int8)
    assert list(q[:4]) == [64, -127, 32, 0]


def test_rtn_rejects_unaligned():
    with pytest.raises(ValueError):
        rtn.rtn_quantize_tensor(torch.randn(4, 100), "Q4_K")


def test_shape_validation_matches_reference():
    with pytest.raises(ValueError):
        ggml.quantize_tensor(torch.randn(4, 100), "Q4_K") if ggml.find_libggml() else \
            rtn.rtn_quantize_tensor(torch.randn(4, 100), "Q4_K")


# ------------------------------------------------------------------ cache
def test_tensor_hash_is_sha256_of_fp32_bytes():
    import hashlib

    t = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    assert cache.tensor_hash(t) == hashlib.sha256(t.numpy().tobytes()).hexdigest()[:16]
    assert cache.tensor_hash(t.to(torch.bfloat16)) == cache.tensor_hash(t.to(torch.bfloat16).float())
    assert cache.tensor_hash(None) == "none"


def test_cache_paths_and_roundtrip(tmp_path):
    p = cache.combined_cache_path("model.layers.0.mlp.up_proj", "lazy", "w" * 16, "none", tmp_path)
    assert p.parent.name == "model_layers_0_mlp_up_proj"
    assert p.name == f"combined_lazy_w{'w' * 16}_inone.pt"
    cands = {"Q4_K": torch.arange(144, dtype=torch.uint8).reshape(1, 144)}
    cache.save_candidates("layers.0.mlp.up_proj", cands, "lazy", "a" * 16, "none", tmp_path)
    # found under the name with the `model.` prefix too (reference layers.py:1116-1121)
    got = cache.load_candidates("model.layers.0.mlp.up_proj", ["Q4_K", "Q8_0"], "lazy", "a" * 16, "none", tmp_path)
    assert list(got) == ["Q4_K"] and torch.equal(got["Q4_K"], cands["Q4_K"])
    # per-type files are read when the combined file lacks a type
    pt = cache.candidate_cache_path("layers.0.mlp.up_proj", "Q8_0", "lazy", "a" * 16, "none", tmp_path)
    cache.atomic_torch_save(torch.zeros(8, 34, dtype=torch.uint8), pt)
    got = cache.load_candidates("layers.0.mlp.up_proj", ["Q4_K", "Q8_0"], "lazy", "a" * 16, "none", tmp_path)
    assert set(got) == {"Q4_K", "Q8_0"}
    assert not list(tmp_path.rglob("*.tmp*"))


# ------------------------------------------------------------------ module (host side)
@pytest.fixture
def isolated_cache(tmp_path, monkeypatch):
    monkeypatch.setattr(layers, "CANDIDATE_CACHE_DIR", tmp_path)
    return tmp_path


def _lin(types=("Q2_K", "Q4_K", "Q8_0"), out_f=64, in_f=512, name="test.proj", seed=0):
    g = torch.Generator().manual_seed(seed)
    return layers.MixedQuantLinear(in_f, out_f, list(types), torch.randn(out_f, in_f, generator=g) * 0.02,
                                   tensor_name=name)


def test_module_construction_and_cache_reuse(isolated_cache):
    lin = _lin()
    assert lin.num_candidates == 3 and lin.gates.shape == (3,)
    assert lin.padded_in_features == 512
    assert lin.candidate_source in ("rtn", "ggml")
    assert list(isolated_cache.rglob("combined_lazy_*.pt"))
    lin2 = _lin()
    assert lin2.candidate_source == ("cache" if lin.candidate_source == "ggml" else "cache_rtn")
    for k in range(3):
        assert torch.equal(getattr(lin, f"_qweight_{k}"), getattr(lin2, f"_qweight_{k}"))
    assert "_qweight_0" not in lin.state_dict()  # packed bytes are not checkpointed


def test_rtn_candidates_never_land_under_the_ggml_key(isolated_cache, monkeypatch):
    """Candidates from the RTN fallback are cached under their own mode: a run
    (here or the reference's) that looks up llama.cpp bytes finds nothing."""
    monkeypatch.setattr(layers, "find_libggml", lambda: None)
    lin = _lin(name="rtn.proj", seed=3)
    assert lin.candidate_source == "rtn"
    padded, _, _ = layers.pad_weight_and_imatrix(
        torch.randn(64, 512, generator=torch.Generator().manual_seed(3)) * 0.02, None)
    wh = cache.tensor_hash(padded)
    assert cache.load_candidates("rtn.proj", lin.candidate_types, "lazy", wh, "none", isolated_cache) == {}
    rtn_hit = cache.load_candidates("rtn.proj", lin.candidate_types, cache.RTN_MODE, wh, "none", isolated_cache)
    assert set(rtn_hit) == set(lin.candidate_types)
    # without libggml the RTN entry is reused ...
    assert _lin(name="rtn.proj", seed=3).candidate_source == "cache_rtn"
    # ... and with libggml it is ignored: the candidates are quantized afresh
    made = {}
    monkeypatch.setattr(layers, "find_libggml", lambda: "libggml-base.so")
    monkeypatch.setattr(layers, "quantize_tensor",
                        lambda w, qt, im=None: made.setdefault(qt, rtn.rtn_quantize_tensor(w, qt)))
    assert _lin(name="rtn.proj", seed=3).candidate_source == "ggml"
    assert set(made) == set(lin.candidate_types)
    assert set(cache.load_candidates("rtn.proj", lin.candidate_types, "lazy", wh, "none", isolated_cache)) == set(made)


def test_padding_to_256(isolated_cache):
    lin = _lin(in_f=300, name="pad.proj")
    assert lin.padded_in_features == 512 and lin.in_features == 300
    w, im, orig = layers.pad_weight_and_imatrix(torch.ones(2, 300), torch.ones(300) * 2)
    assert w.shape == (2, 512) and orig == 300 and float(w[:, 300:].abs().sum()) == 0
    assert float(im[300:].min()) == 1.0 and float(im[:300].max()) == 2.0


def test_rejects_types_without_hip_decoder(isolated_cache):
    with pytest.raises(ValueError, match="HIP decoder"):
        _lin(types=("TQ2_0", "Q8_0"), name="bad.proj")


def test_effective_bytes_and_assignment(isolated_cache):
    lin = _lin()
    p = lin.soft_probs().detach()
    expect = sum(float(p[k]) * ggml.bytes_per_weight(qt) * 64 * 512 for k, qt in enumerate(lin.candidate_types))
    assert float(lin.effective_bytes()) == pytest.approx(expect, rel=1e-6)
    with torch.no_grad():
        lin.gates.copy_(torch.tensor([0.0, 2.0, 1.0]))
    assert lin.get_assignment() == "Q4_K"
    assert lin.get_assignment_prob() == pytest.approx(float(torch.softmax(lin.gates, 0)[1]))
    total = layers.total_effective_bytes({"a": lin, "b": _lin(name="b.proj")})
    assert float(total) > float(lin.effective_bytes())


def test_temperature(isolated_cache):
    lin = _lin()
    lin.set_temperature(0.0)
    assert lin.temperature == 1e-6
    with torch.no_grad():
        lin.gates.copy_(torch.tensor([0.0, 0.1, 0.0]))
    lin.set_temperature(0.01)
    assert float(lin.soft_probs()[1]) > 0.99


def test_st_gumbel_hardening(isolated_cache):
    """Port of tests/test_invariants.py:88-118."""
    lin = _lin()
    try:
        layers.set_st_gumbel(False, 0.0, 1.0)
        assert torch.allclose(lin.get_probs(), torch.softmax(lin.gates / lin.temperature, 0))
        layers.set_st_gumbel(True, 1.0, 0.5)
        for _ in range(10):
            p = lin.get_probs()
            assert p.sum() == 1 and ((p == 0) | (p == 1)).all()
        c = torch.tensor([0.1, 0.9, -0.4])
        (lin.get_probs() * c).sum().backward()
        hard = lin.gates.grad.clone()
        lin.gates.grad = None
        layers.set_st_gumbel(False, 0.0, 1.0)
        (lin.get_probs() * c).sum().backward()
        assert torch.allclose(hard, lin.gates.grad, atol=1e-6)
    finally:
        layers.set_st_gumbel(False, 0.0, 1.0)


def test_role_menus():
    base = ["Q8_0", "Q5_K", "Q3_K", "Q2_K"]
    attn = ["Q5_K", "Q3_K", "Q2_K"]
    assert "Q8_0" not in layers.resolve_candidate_types("layers.0.self_attn.q_proj", base, attn, None)
    assert layers.resolve_candidate_types("layers.0.mlp.up_proj", base, attn, None) == base


def test_forward_refuses_cpu(isolated_cache):
    lin = _lin()
    with pytest.raises(RuntimeError, match="ROCm"):
        lin(torch.randn(2, 512))


def test_row_slice_bit_identical(isolated_cache):
    """Row slices of candidates equal quantizing the slice (test_invariants.py:20-31)."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(8, 1024, generator=g)
    lin = layers.MixedQuantLinear(1024, 8, ["Q4_K", "Q6_K"], w, tensor_name="slice.proj")
    lin.shard_rows([(2, 5)])
    for k, qt in enumerate(["Q4_K", "Q6_K"]):
        direct = rtn.rtn_quantize_tensor(w[2:5].contiguous(), qt) if lin.candidate_source != "ggml" \
            else ggml.quantize_tensor(w[2:5].contiguous(), qt)
        assert torch.equal(getattr(lin, f"_qweight_{k}").reshape(-1), direct.reshape(-1))
    assert lin.out_features == 3 and lin._full_out_features == 8


def test_col_slice_alignment(isolated_cache):
    lin = layers.MixedQuantLinear(1024, 8, ["Q4_K"], torch.randn(8, 1024), tensor_name="cols.proj")
    with pytest.raises(ValueError):
        lin.shard_cols((128, 384))
    lin.shard_cols((256, 512))
    assert lin.in_features == 256 and lin.padded_in_features == 256


def test_replace_linear_walker(isolated_cache):
    net = torch.nn.Sequential(torch.nn.Linear(512, 64, bias=False), torch.nn.ReLU(),
                              torch.nn.Sequential(torch.nn.Linear(64 * 4, 32, bias=False)))
    # second Linear's in_features (256) after padding stays 256
    net[2][0] = torch.nn.Linear(256, 32, bias=False)
    replaced = layers.replace_linear_with_mixed_quant(net, ["Q4_K", "Q8_0"])
    assert set(replaced) == {"0", "2.0"}
    assert isinstance(net[0], layers.MixedQuantLinear) and isinstance(net[2][0], layers.MixedQuantLinear)
    with pytest.raises(NotImplementedError):
        layers.replace_linear_with_mixed_quant(torch.nn.Sequential(torch.nn.Linear(256, 8)), ["Q4_K"])


def test_trainer_calls():
    assert trainer.anneal_temperature(0, 200, 2.0, 0.1) == 2.0
    assert trainer.anneal_temperature(199, 200, 2.0, 0.1) == pytest.approx(0.1)
    meta = {"a": (1, 10), "b": (1, 10), "c": (2, 5)}
    assert trainer.compute_total_8bit_bytes(meta) == 15.0
    assert trainer.compute_non_targeted_8bit_bytes(meta, {"a"}) == 5.0
    assert float(trainer.size_loss(torch.tensor(100.0), 100.0, 0.02)) == 0.0
    p = torch.nn.Parameter(torch.zeros(3))
    opt, sched = trainer.build_gate_optimizer([p], lr=0.5, max_steps=10)
    p.grad = torch.tensor([1.0, -1.0, 0.0])
    trainer.gate_optimizer_step([p], opt, sched)
    assert float(p[0]) < 0 < float(p[1]) and p.grad is None or float(p.grad.abs().sum()) == 0


def test_router_shares():
    """Port of tests/test_ptqr.py:29-44: token shares track the probabilities,
    and a seeded draw is reproducible."""
    torch.manual_seed(0)
    for pv in ([0.25, 0.75], [0.1, 0.2, 0.3, 0.4], [0.05, 0.05, 0.9]):
        routing = layers._sample_token_routing(torch.tensor(pv), 200_000)
        for k, p in enumerate(pv):
            assert abs(float((routing == k).float().mean()) - p) <= 0.01
    torch.manual_seed(0)
    a = layers._sample_token_routing(torch.tensor([0.5, 0.5]), 64)
    torch.manual_seed(0)
    b = layers._sample_token_routing(torch.tensor([0.5, 0.5]), 64)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ gated embedding and the Q8_0 teacher (host side)
def test_embedding_module_construction(isolated_cache):
    g = torch.Generator().manual_seed(3)
    emb = layers.MixedQuantEmbedding(100, 1000, ["Q2_K", "Q8_0"], torch.randn(100, 1000, generator=g) * 0.02,
                                     tensor_name="tok_embeddings")
    assert emb.num_embeddings == 100 and emb.embedding_dim == 1000 and emb.padded_in_features == 1024
    assert emb.out_features == 100 and emb.in_features == 1000
    for k, qt in enumerate(["Q2_K", "Q8_0"]):
        info = ggml.get_quant_info(qt)
        assert getattr(emb, f"_qweight_{k}").numel() == 100 * 1024 // info.block_size * info.block_bytes
    expect = 0.5 * (ggml.bytes_per_weight("Q2_K") + ggml.bytes_per_weight("Q8_0")) * 100 * 1000
    assert float(emb.effective_bytes().detach()) == pytest.approx(expect, rel=1e-6)
    with pytest.raises(RuntimeError, match="ROCm"):
        emb(torch.tensor([1, 2]))


def test_replace_embedding_walker(isolated_cache):
    net = torch.nn.Module()
    net.embed_tokens = torch.nn.Embedding(50, 256)
    net.inner = torch.nn.Sequential(torch.nn.Embedding(20, 512), torch.nn.Linear(512, 8))
    net.skipme = torch.nn.Embedding(10, 256)
    replaced = layers.replace_embedding_with_mixed_quant(net, ["Q4_K", "Q8_0"], skip_names={"skipme"})
    assert set(replaced) == {"embed_tokens", "inner.0"}
    assert isinstance(net.embed_tokens, layers.MixedQuantEmbedding)
    assert isinstance(net.inner[1], torch.nn.Linear) and isinstance(net.skipme, torch.nn.Embedding)
    assert replaced["inner.0"].candidate_types == ["Q4_K", "Q8_0"]


def _q8_teacher_checkpoint():
    """A tiny HF-style model and a checkpoint with stripped names, Q8_0 bytes
    for its Linears/Embedding and plain tensors for the rest."""
    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.up = torch.nn.Linear(64, 32, bias=True)
            self.norm = torch.nn.LayerNorm(64)

    class Body(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.embed_tokens = torch.nn.Embedding(40, 64)
            self.layers = torch.nn.ModuleList([Block(), Block()])

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.model = Body()
            self.lm_head = torch.nn.Linear(64, 40, bias=False)

    g = torch.Generator().manual_seed(9)
    sd, meta = {}, {}
    for name, (o, i) in {"embed_tokens": (40, 64), "layers.0.up": (32, 64), "layers.1.up": (32, 64),
                         "lm_head": (40, 64)}.items():
        sd[name + ".weight"] = rtn.rtn_quantize_tensor(torch.randn(o, i, generator=g), "Q8_0")
        meta[name + ".weight"] = {"out_features": o, "in_features": i}
    for li in range(2):
        sd[f"layers.{li}.up.bias"] = torch.randn(32, generator=g)
        sd[f"layers.{li}.norm.weight"] = torch.full((64,), 2.0 + li)
        sd[f"layers.{li}.norm.bias"] = torch.zeros(64)
    return Model(), sd, meta


def test_wrap_q8_teacher():
    from voodoo_quant.training.q8_teacher import Q8Embedding, Q8Linear, wrap_q8_teacher

    model, sd, meta = _q8_teacher_checkpoint()
    wrap_q8_teacher(model, sd, meta)
    assert isinstance(model.model.embed_tokens, Q8Embedding) and isinstance(model.lm_head, Q8Linear)
    assert all(isinstance(blk.up, Q8Linear) for blk in model.model.layers)
    up = model.model.layers[0].up
    assert torch.equal(up.qweight, sd["layers.0.up.weight"])
    assert up.out_features == 32 and up.in_features == 64
    assert torch.equal(up.bias.detach(), sd["layers.0.up.bias"])  # carried over the constructor's copy
    # non-Q8 tensors are carried over under the model's names
    assert torch.equal(model.model.layers[1].norm.weight, torch.full((64,), 3.0))
    assert model.model.embed_tokens.num_embeddings == 40
    with pytest.raises(RuntimeError, match="ROCm"):
        model.lm_head(torch.randn(2, 64))


def test_wrap_q8_teacher_metadata_naming_and_strays():
    """quant_meta may name the module instead of its weight, and with the
    `model.` prefix; bytes without metadata stay put; checkpoint tensors the
    model lacks are reported, not loaded."""
    from voodoo_quant.training.q8_teacher import Q8Embedding, Q8Linear, wrap_q8_teacher

    model, sd, meta = _q8_teacher_checkpoint()
    meta = {("model." + k[: -len(".weight")]) if k.startswith("layers") else k: v for k, v in meta.items()}
    del meta["model.layers.1.up"]
    sd["layers.9.extra.weight"] = torch.zeros(3)
    with pytest.warns(UserWarning) as rec:
        wrap_q8_teacher(model, sd, meta)
    msgs = " ".join(str(w.message) for w in rec)
    assert "layers.1.up" in msgs and "layers.9.extra.weight" in msgs
    assert isinstance(model.model.layers[0].up, Q8Linear) and isinstance(model.model.embed_tokens, Q8Embedding)
    assert isinstance(model.model.layers[1].up, torch.nn.Linear)


def test_q8_padding_repacks_rows():
    from voodoo_quant.training.q8_teacher import _padded_q8

    w = torch.randn(8, 96)
    qb = rtn.rtn_quantize_tensor(w, "Q8_0").reshape(-1)
    padded, d_pad = _padded_q8(qb, 8, 96, 16)
    assert d_pad == 256 and padded.numel() == 16 * 8 * 34
    vals = cdequant.oracle_dequant("Q8_0", padded.numpy(), 16 * 256).reshape(16, 256)
    ref = cdequant.oracle_dequant("Q8_0", qb.numpy(), 8 * 96).reshape(8, 96)
    assert np.array_equal(vals[:8, :96], ref)
    assert not vals[8:].any() and not vals[:, 96:].any()
    same, d = _padded_q8(rtn.rtn_quantize_tensor(torch.randn(8, 256), "Q8_0"), 8, 256, 8)
    assert d == 256 and same.numel() == 8 * 8 * 34
    with pytest.raises(ValueError):
        _padded_q8(qb, 8, 80, 8)


def test_total_effective_bytes_batches_like_the_per_layer_sum(isolated_cache):
    mods = {f"l{i}": _lin(types=t, out_f=16, in_f=256, name=f"eb.{i}", seed=i)
            for i, t in enumerate([("Q2_K", "Q4_K", "Q8_0"), ("Q3_K", "Q6_K"), ("Q2_K", "Q5_K", "Q8_0")])}
    g = torch.Generator().manual_seed(4)
    for i, m in enumerate(mods.values()):
        with torch.no_grad():
            m.gates.copy_(torch.randn(m.num_candidates, generator=g))
        m.set_temperature(0.5 + i)
    total = layers.total_effective_bytes(mods)
    ref = sum(float(m.effective_bytes()) for m in mods.values())
    assert float(total) == pytest.approx(ref, rel=1e-6)
    total.backward()
    for m in mods.values():
        p = m.soft_probs().detach().double()
        c = torch.tensor(m._bytes_per_candidate(), dtype=torch.float64)
        grad_ref = (torch.diag(p) - torch.outer(p, p)) @ c / m.temperature
        assert torch.allclose(m.gates.grad.double(), grad_ref, rtol=1e-4)


def test_gate_bank_rows_bytes_and_release(isolated_cache):
    """GateBank: one [T, K] parameter per candidate count; each module's
    soft_probs is its row of one softmax, the bank's bytes equal the
    per-layer sum, gradients land in the bank, and release() gives each
    module an independent parameter with the trained values."""
    from voodoo_quant.training import trainer

    mods = {f"l{i}": _lin(types=t, out_f=16, in_f=256, name=f"gb.{i}", seed=i)
            for i, t in enumerate([("Q2_K", "Q4_K", "Q8_0"), ("Q3_K", "Q6_K"), ("Q2_K", "Q5_K", "Q8_0")])}
    g = torch.Generator().manual_seed(5)
    for m in mods.values():
        with torch.no_grad():
            m.gates.copy_(torch.randn(m.num_candidates, generator=g))
        m.set_temperature(0.7)
    expect_probs = {n: m.soft_probs().detach().clone() for n, m in mods.items()}
    expect_bytes = float(layers.total_effective_bytes(mods))
    bank = trainer.GateBank(mods.values())
    assert sorted(p.shape for p in bank.parameters()) == [(1, 2), (2, 3)]
    total = bank.begin(0.7)
    assert float(total) == pytest.approx(expect_bytes, rel=1e-6)
    for n, m in mods.items():
        assert torch.allclose(m.soft_probs(), expect_probs[n], rtol=1e-6, atol=1e-7)
    total.backward()
    bank.end()
    assert all(m.__dict__.get("_probs_override") is None for m in mods.values())
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in bank.parameters())
    with torch.no_grad():
        for p in bank.parameters():
            p.mul_(2.0)
    doubled = {n: m.gates.detach().clone() for n, m in mods.items()}
    bank.release()
    for n, m in mods.items():
        assert m.gates.requires_grad and torch.equal(m.gates.detach(), doubled[n])


# ------------------------------------------------------------------ precache (reference tools/precache.py:88-229)
class _TinyDecoder(torch.nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(7)
        layer = torch.nn.Module()
        layer.self_attn = torch.nn.Module()
        layer.self_attn.q_proj = torch.nn.Linear(512, 64, bias=False)
        layer.mlp = torch.nn.Module()
        layer.mlp.up_proj = torch.nn.Linear(512, 128, bias=False)
        layer.linear_attn = torch.nn.Module()
        layer.linear_attn.in_proj_a = torch.nn.Linear(512, 32, bias=False)  # kept F32 by the recipe
        layer.norm = torch.nn.LayerNorm(512)                                # 1-D: never gated
        layer.odd = torch.nn.Linear(100, 16, bias=False)                    # rows of 100: not block-aligned
        self.model = torch.nn.Module()
        self.model.layers = torch.nn.ModuleList([layer])
        for p in self.parameters():
            if p.dim() == 2:
                p.data = torch.randn(p.shape, generator=g) * 0.02


def test_precache_selection_and_reuse(isolated_cache, monkeypatch):
    from voodoo_quant import precache

    monkeypatch.setattr(layers, "find_libggml", lambda: None)
    monkeypatch.setattr(precache, "find_libggml", lambda: None)
    model = _TinyDecoder()
    plan = precache.selectable_tensors(model, ["Q8_0", "Q4_K"], attention_candidates=["Q8_0"])
    assert plan == {"model.layers.0.self_attn.q_proj": ["Q8_0"], "model.layers.0.mlp.up_proj": ["Q8_0", "Q4_K"]}
    rep = precache.precache_model(model, ["Q8_0", "Q4_K"], attention_candidates=["Q8_0"], workers=2)
    assert (rep.tensors, rep.built, rep.cached, rep.errors, rep.source) == (2, 3, 0, [], "rtn")
    # RTN bytes sit under their own key only, and equal the encoder's output
    w = model.model.layers[0].mlp.up_proj.weight.detach()
    wh = cache.tensor_hash(w)
    assert cache.load_candidates("model.layers.0.mlp.up_proj", ["Q8_0"], "lazy", wh, "none", isolated_cache) == {}
    hit = cache.load_candidates("model.layers.0.mlp.up_proj", ["Q8_0", "Q4_K"], cache.RTN_MODE, wh, "none",
                                isolated_cache)
    for qt in ("Q8_0", "Q4_K"):
        assert torch.equal(hit[qt].reshape(-1), rtn.rtn_quantize_tensor(w.float(), qt).reshape(-1))
    # a gated layer over the same weight loads the precached bytes
    lin = layers.MixedQuantLinear(512, 128, ["Q8_0", "Q4_K"], w.clone(), tensor_name="model.layers.0.mlp.up_proj")
    assert lin.candidate_source == "cache_rtn"
    assert torch.equal(lin._qweight_1, hit["Q4_K"].reshape(-1))
    # a second pass finds everything
    rep2 = precache.precache_model(model, ["Q8_0", "Q4_K"], attention_candidates=["Q8_0"])
    assert (rep2.built, rep2.cached) == (0, 3)


def test_precache_reports_failed_types(isolated_cache, monkeypatch):
    from voodoo_quant import precache

    monkeypatch.setattr(layers, "find_libggml", lambda: None)
    monkeypatch.setattr(precache, "find_libggml", lambda: None)
    real = layers._quantize_candidates

    def flaky(padded, imatrix, types):
        if types == ["Q4_K"]:
            raise ValueError("quantizer failed")
        return real(padded, imatrix, types)

    monkeypatch.setattr(layers, "_quantize_candidates", flaky)
    rep = precache.precache_model(_TinyDecoder(), ["Q8_0", "Q4_K"])
    assert rep.built == 2 and len(rep.errors) == 2 and all("Q4_K" in e for e in rep.errors)
    # decoded entries need libggml or a ROCm device
    if not torch.cuda.is_available():
        rep = precache.precache_model(_TinyDecoder(), ["Q8_0"], lazy=False, root=isolated_cache / "dq")
        assert rep.built == 0 and len(rep.errors) == 2 and "ROCm" in rep.errors[0]
