"""The libggml bridge (``voodoo_quant/ggml.py``) driven through a real shared
library on the CPU.

llama.cpp's ``libggml-base.so`` is not available here, so these tests build
``tests/ggml_stand_in/ggml_stand_in.c``: a TEST-ONLY stand-in that exports the
part of ggml's C ABI the bridge binds (``ggml_quantize_init``,
``quantize_q8_0``/``quantize_q4_K``, ``dequantize_row_<t>``) and records the
arguments it receives.  Its bytes are not llama.cpp's (its Q8_0 is ggml's
round-to-nearest, its Q4_K the labelled RTN encoder's, its decoders the
oracle's), so what is tested is the plumbing, not llama.cpp parity:

* discovery through ``$VOODOO_GGML_LIB`` and the errors for a missing or
  unloadable library (reference ``ggml.py:103-144``);
* ``quantize_tensor``'s argument passing (rows, row length, data, the
  all-ones importance matrix when none is given, ``ggml.py:204-205``), its
  block-alignment ``ValueError`` and its returned-size check
  (``ggml.py:171-221``);
* ``dequantize_tensor``'s call and size checks (``ggml.py:224-269``);
* the gated layers' ``"ggml"`` candidate branch, which writes the ``lazy``
  cache key that the reference and a later run read, and the precache tool's
  default output, which a gated layer then loads.
"""

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant
from voodoo_quant import cache, ggml, layers, rtn

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "ggml_stand_in" / "ggml_stand_in.c"


@pytest.fixture(scope="module")
def stand_in_path(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is needed to build the stand-in library")
    out = tmp_path_factory.mktemp("ggml_stand_in") / "libggml-base.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fopenmp", str(SRC),
                    str(ROOT / "oracle" / "dequant_ref.c"), "-o", str(out), "-lm"], check=True)
    return out


@pytest.fixture
def stand_in(stand_in_path, monkeypatch, tmp_path):
    """The bridge bound to the stand-in (a fresh load), with an isolated cache."""
    monkeypatch.setenv("VOODOO_GGML_LIB", str(stand_in_path))
    monkeypatch.setattr(ggml, "_LIB", None)
    monkeypatch.setattr(layers, "CANDIDATE_CACHE_DIR", tmp_path / "cache")
    probe = ctypes.CDLL(str(stand_in_path))
    for name, res in (("stand_in_init_type", ctypes.c_int), ("stand_in_init_calls", ctypes.c_int),
                      ("stand_in_rows", ctypes.c_int64), ("stand_in_cols", ctypes.c_int64),
                      ("stand_in_imatrix_null", ctypes.c_int), ("stand_in_imatrix_sum", ctypes.c_double)):
        getattr(probe, name).restype = res
    probe.stand_in_set_size_skew.argtypes = [ctypes.c_int64]
    probe.stand_in_reset()
    yield probe
    probe.stand_in_reset()


def _weights(rows, cols, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, cols, generator=g) * 0.02


def test_discovery_prefers_the_environment(stand_in, stand_in_path):
    assert ggml.find_libggml() == stand_in_path
    assert ggml.lib_path() == str(stand_in_path)


def test_missing_and_unloadable_libraries_raise(monkeypatch, tmp_path):
    monkeypatch.setattr(ggml, "_LIB", None)
    monkeypatch.setattr(ggml, "_candidate_paths", lambda: [tmp_path / "absent.so"])
    monkeypatch.setattr(ggml, "_LIB_NAME", "libggml-base-absent-for-test.so")
    assert ggml.find_libggml() is None
    with pytest.raises(RuntimeError, match="not found"):
        ggml.quantize_tensor(_weights(4, 256), "Q8_0")
    junk = tmp_path / "libggml-base.so"
    junk.write_bytes(b"not a shared object")
    monkeypatch.setattr(ggml, "_candidate_paths", lambda: [junk])
    with pytest.raises(RuntimeError, match="Failed to load"):
        ggml.quantize_tensor(_weights(4, 256), "Q8_0")


def test_quantize_passes_rows_data_and_an_all_ones_imatrix(stand_in):
    w = _weights(24, 512)
    qb = ggml.quantize_tensor(w, "Q8_0")
    assert stand_in.stand_in_init_type() == 8 and stand_in.stand_in_init_calls() == 1
    assert (stand_in.stand_in_rows(), stand_in.stand_in_cols()) == (24, 512)
    # no importance matrix given: the bridge passes ones, never NULL
    assert stand_in.stand_in_imatrix_null() == 0 and stand_in.stand_in_imatrix_sum() == 512.0
    assert qb.dtype == torch.uint8 and tuple(qb.shape) == (24 * 512 // 32, 34)
    # the stand-in's Q8_0 is ggml's round-to-nearest, which the RTN encoder also writes
    assert torch.equal(qb.reshape(-1), rtn.rtn_quantize_tensor(w, "Q8_0").reshape(-1))


def test_quantize_passes_a_given_imatrix_and_k_quant_blocks(stand_in):
    w = _weights(16, 768, seed=1)
    imatrix = torch.linspace(0.5, 2.0, 768)
    qb = ggml.quantize_tensor(w, "Q4_K", imatrix)
    assert stand_in.stand_in_init_type() == 12
    assert (stand_in.stand_in_rows(), stand_in.stand_in_cols()) == (16, 768)
    assert stand_in.stand_in_imatrix_null() == 0
    assert stand_in.stand_in_imatrix_sum() == pytest.approx(float(imatrix.double().sum()), rel=1e-6)
    assert tuple(qb.shape) == (16 * 3, 144)
    assert torch.equal(qb.reshape(-1), rtn.rtn_quantize_tensor(w, "Q4_K").reshape(-1))
    with pytest.raises(ValueError, match="imatrix size"):
        ggml.quantize_tensor(w, "Q4_K", torch.ones(767))


def test_block_misalignment_raises_before_the_library_is_called(stand_in):
    with pytest.raises(ValueError, match=r"Q4_K requires in_features % 256 == 0, got 288"):
        ggml.quantize_tensor(_weights(4, 288), "Q4_K")
    assert stand_in.stand_in_rows() == -1
    with pytest.raises(ValueError, match=r"requires in_features % 32 == 0"):
        ggml.dequantize_tensor(torch.zeros(34, dtype=torch.uint8), "Q8_0", 1, 48)


def test_returned_size_is_checked(stand_in):
    stand_in.stand_in_set_size_skew(-34)
    with pytest.raises(RuntimeError, match=r"quantize_q8_0 returned \d+ bytes, expected \d+"):
        ggml.quantize_tensor(_weights(4, 256), "Q8_0")


@pytest.mark.parametrize("qt", ["Q8_0", "Q4_K", "Q2_K", "Q6_K", "IQ4_XS"])
def test_dequantize_calls_the_row_decoder(stand_in, qt):
    rows, cols = 6, 512
    if qt in ("Q8_0", "Q4_K"):
        qb = ggml.quantize_tensor(_weights(rows, cols, seed=2), qt)
    else:
        qb = torch.from_numpy(blocks.random_blocks(qt, rows * cols // 256, np.random.default_rng(3)).reshape(-1))
    got = ggml.dequantize_tensor(qb, qt, rows, cols)
    assert got.shape == (rows, cols) and got.dtype == torch.float32
    ref = cdequant.oracle_dequant(qt, qb.numpy().reshape(-1), rows * cols)
    assert np.array_equal(got.numpy().reshape(-1).view(np.uint32), ref.view(np.uint32))
    with pytest.raises(ValueError, match="does not match"):
        ggml.dequantize_tensor(qb.reshape(-1)[:-1], qt, rows, cols)


def test_gated_layer_takes_candidates_from_the_library(stand_in):
    """With libggml present the layer quantizes through it, stores the bytes
    under the ``lazy`` key, and a second layer over the same weight loads them."""
    w = _weights(64, 300, seed=4)
    lin = layers.MixedQuantLinear(300, 64, ["Q8_0", "Q4_K"], w, tensor_name="model.layers.0.mlp.up_proj")
    assert lin.candidate_source == "ggml" and lin.padded_in_features == 512
    assert (stand_in.stand_in_rows(), stand_in.stand_in_cols()) == (64, 512)
    padded, _, _ = layers.pad_weight_and_imatrix(w, None)
    for k, qt in enumerate(["Q8_0", "Q4_K"]):
        assert torch.equal(getattr(lin, f"_qweight_{k}"), rtn.rtn_quantize_tensor(padded, qt).reshape(-1))
    wh = cache.tensor_hash(padded)
    hit = cache.load_candidates("model.layers.0.mlp.up_proj", ["Q8_0", "Q4_K"], "lazy", wh, "none",
                                layers.CANDIDATE_CACHE_DIR)
    assert set(hit) == {"Q8_0", "Q4_K"}
    assert cache.load_candidates("model.layers.0.mlp.up_proj", ["Q8_0"], cache.RTN_MODE, wh, "none",
                                 layers.CANDIDATE_CACHE_DIR) == {}
    calls = stand_in.stand_in_init_calls()
    again = layers.MixedQuantLinear(300, 64, ["Q8_0", "Q4_K"], w, tensor_name="model.layers.0.mlp.up_proj")
    assert again.candidate_source == "cache" and stand_in.stand_in_init_calls() == calls
    assert torch.equal(again._qweight_1, lin._qweight_1)


def test_precache_cli_default_output_is_what_the_layers_load(stand_in, tmp_path, monkeypatch):
    """``python -m voodoo_quant.precache`` without flags writes packed entries,
    and a gated layer over a precached weight loads them without quantizing."""
    transformers = pytest.importorskip("transformers")
    from voodoo_quant import precache

    cfg = transformers.LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                                   num_attention_heads=4, num_key_value_heads=2, vocab_size=64)
    cfg_dir = tmp_path / "cfg"
    cfg.save_pretrained(cfg_dir)
    torch.manual_seed(0)
    model = transformers.AutoModelForCausalLM.from_config(cfg).to(torch.bfloat16)
    ckpt = tmp_path / "ckpt.pt"
    torch.save({"model_state_dict": model.state_dict()}, ckpt)
    assert precache.main(["--checkpoint", str(ckpt), "--model", str(cfg_dir),
                          "--candidate_types", "Q8_0", "Q4_K"]) == 0
    name = "model.layers.0.mlp.up_proj"
    w = model.state_dict()[name + ".weight"]
    calls = stand_in.stand_in_init_calls()
    lin = layers.MixedQuantLinear(256, 512, ["Q8_0", "Q4_K"], w.clone(), tensor_name=name)
    assert lin.candidate_source == "cache" and stand_in.stand_in_init_calls() == calls
    assert list(Path(layers.CANDIDATE_CACHE_DIR).rglob("combined_lazy_*.pt"))
    assert not list(Path(layers.CANDIDATE_CACHE_DIR).rglob("combined_dequant_*.pt"))
