"""The C ABI library loads and exports every entry point of include/voodoo_hip.h;
host-side validation returns the documented error codes (no GPU work)."""

import ctypes
import re
from pathlib import Path

import pytest

from voodoo_quant import _hip

HEADER = Path(__file__).resolve().parent.parent / "include" / "voodoo_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in voodoo_hip.h but not exported"
    assert set(names) == set(_hip.EXPORTED), "ctypes binding and header disagree"


def _declarations():
    """{name: (return type, [parameter types])} of the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"\b((?:const\s+)?[a-z0-9_]+\s*\**)\s*\b(vq_[a-z0-9_]+)\s*\(([^)]*)\)\s*;",
                                        text):
        params = [q.strip() for q in params.split(",") if q.strip() and q.strip() != "void"]
        types = [re.sub(r"\s*\b[A-Za-z_][A-Za-z0-9_]*(\s*\[\])?$", "", q) for q in params]
        out[name] = (ret.replace(" ", ""), types)
    return out


def _ctype_of(c_type: str):
    c = c_type.replace("const", "").replace(" ", "")
    if "*" in c:
        return ctypes.c_char_p if c == "char*" else ctypes.c_void_p
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float, "void": None}[c]


def test_ctypes_signatures_match_the_header():
    """Every ctypes signature the bindings set has the header's parameter
    count, parameter types and return type (a pointer is c_void_p, except
    the error string's char*)."""
    decl = _declarations()
    assert set(decl) == set(declared_functions())
    for name, res, args in _hip._SIGNATURES:
        ret, params = decl[name]
        assert res is _ctype_of(ret), (name, ret)
        assert len(args) == len(params), (name, len(args), params)
        for i, (a, c_type) in enumerate(zip(args, params)):
            assert a is _ctype_of(c_type), (name, i, c_type)


def test_version_and_group_bytes():
    lib = _hip.lib()
    assert lib.vq_version() >= 100
    expect = {8: 272, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 16: 66, 17: 74, 18: 98, 19: 50, 21: 110, 22: 82,
              23: 136, 29: 56}
    for t, gb in expect.items():
        assert _hip.group_bytes(t) == gb
    assert _hip.group_bytes(34) == 0  # TQ1_0: no HIP decoder
    assert _hip.group_bytes(35) == 0  # TQ2_0


def test_qbytes_size_matches_reference_arithmetic():
    from voodoo_quant.ggml import get_quant_info

    for qt in ("Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ1_S", "IQ1_M", "IQ2_XXS", "IQ2_XS", "IQ2_S",
               "IQ3_XXS", "IQ3_S", "IQ4_XS"):
        info = get_quant_info(qt)
        assert _hip.qbytes_size(info.ggml_type, 17, 1024) == 17 * 1024 // info.block_size * info.block_bytes
    with pytest.raises(ValueError, match="in_features"):
        _hip.qbytes_size(12, 4, 100)  # Q4_K needs 256-aligned rows (ggml.py:195-198)


def test_validate_candidates_errors():
    lib = _hip.lib()
    ok = (ctypes.c_int * 2)(8, 12)
    assert lib.vq_validate_candidates(2, ok, 64, 512, 512) == _hip.VQ_OK
    assert lib.vq_validate_candidates(2, ok, 64, 512, 500) == _hip.VQ_ERR_ALIGN
    assert b"256" in lib.vq_last_error_string()
    bad = (ctypes.c_int * 2)(8, 34)  # TQ1_0: no HIP decoder
    assert lib.vq_validate_candidates(2, bad, 64, 512, 512) == _hip.VQ_ERR_QTYPE
    assert lib.vq_validate_candidates(0, ok, 64, 512, 512) == _hip.VQ_ERR_SHAPE
    assert lib.vq_validate_candidates(2, ok, 64, 768, 512) == _hip.VQ_ERR_SHAPE
    assert lib.vq_validate_candidates(2, ok, 60, 512, 512) == _hip.VQ_ERR_ALIGN
    assert lib.vq_validate_candidates(2, None, 64, 512, 512) == _hip.VQ_ERR_NULL
    with pytest.raises(ValueError):
        _hip.validate_candidates([8, 99], 64, 512, 512)


def test_null_pointers_rejected_before_any_gpu_work():
    lib = _hip.lib()
    types = (ctypes.c_int * 1)(8)
    assert lib.vq_dequant(8, None, None, 4, 256, None) == _hip.VQ_ERR_NULL
    assert lib.vq_dequant(99, None, None, 4, 256, None) == _hip.VQ_ERR_QTYPE
    assert lib.vq_mix_weight(1, types, None, None, 8, 256, None, None) == _hip.VQ_ERR_NULL
    assert lib.vq_gated_linear_fwd(None, 4, 8, 256, 256, 1, types, None, None, None, None, None, 0,
                                   None) == _hip.VQ_ERR_NULL


def test_embedding_rows_argument_checks():
    lib = _hip.lib()
    types = (ctypes.c_int * 1)(12)
    ptrs = (ctypes.c_void_p * 1)(None)
    # a NULL candidate pointer, an unsupported type and bad sizes fail before any GPU work
    assert lib.vq_embedding_rows_fwd(1, types, ptrs, None, None, None, 4, 10, 256, 256, None, 0,
                                     None) == _hip.VQ_ERR_NULL
    bad = (ctypes.c_int * 1)(9)
    assert lib.vq_embedding_rows_fwd(1, bad, ptrs, None, None, None, 4, 10, 256, 256, None, 0,
                                     None) == _hip.VQ_ERR_QTYPE
    fake = (ctypes.c_void_p * 1)(4096)  # never dereferenced: the checks fail first
    assert lib.vq_embedding_rows_fwd(1, types, fake, None, None, None, 4, 10, 100, 256, None, 0,
                                     None) == _hip.VQ_ERR_ALIGN
    assert lib.vq_embedding_rows_fwd(1, types, fake, None, None, None, 4, 10, 512, 256, None, 0,
                                     None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_embedding_rows_fwd(1, types, fake, None, None, None, 4, 10, 256, 256, None, 0,
                                     None) == _hip.VQ_ERR_NULL  # ids
    assert lib.vq_embedding_rows_bwd(1, types, fake, None, 0, 10, 256, 256, None, 0, None, None, 0,
                                     None) == _hip.VQ_ERR_NULL  # dprobs
    # workspace: one fp32 partial per (row, segment of <= 16 groups) and candidate
    assert lib.vq_embedding_rows_bwd_workspace(100, 5120, 6) == 100 * 2 * 6 * 4 + 64
    assert lib.vq_embedding_rows_bwd_workspace(0, 256, 1) == 0
    assert lib.vq_embedding_rows_bwd_workspace(4, 256, 17) == -1  # more than 16 candidates


def test_linear_fwd_argument_checks():
    lib = _hip.lib()
    assert lib.vq_linear_fwd(None, 4, 8, 256, None, 256, None, None, 0, None) == _hip.VQ_ERR_NULL
    assert lib.vq_linear_fwd(None, 4, 12, 256, None, 256, None, None, 0, None) == _hip.VQ_ERR_ALIGN
    assert lib.vq_linear_fwd(None, 4, 8, 256, None, 128, None, None, 0, None) == _hip.VQ_ERR_SHAPE  # ldw < d


def test_forward_workspace_size():
    # 8192 x 17408 tiles: 2176 over 8 XCDs of 32 CUs -> each XCD splits its last 16 tiles in 2
    n = _hip.fwd_workspace_bytes(8192, 17408, 5120)
    assert n == 8 * 16 * 2 * 256 * 256 * 4
    assert _hip.fwd_workspace_bytes(8192, 8192, 4096) == 0  # 1024 tiles: whole rounds only
    with pytest.raises(ValueError):
        _hip.fwd_workspace_bytes(-1, 64, 256)


def test_workspace_size():
    n = _hip.bwd_workspace_bytes(8192, 17408, 5120, 5120, 6, False)
    tiles = (17408 // 256) * (5120 // 256)
    assert n >= tiles * 6 * 4 and n % 256 == 0
    assert _hip.bwd_workspace_bytes(8192, 17408, 5120, 5120, 6, True) >= n + 17408 * 5120 * 2
    assert _hip.bwd_workspace_bytes(0, 64, 256, 256, 2, False) > 0


TILE = 256 * 256 * 4  # one fp32 dW tile


@pytest.mark.parametrize("m, n, d", [(8192, 1024, 1024), (8192, 1536, 1024), (8192, 1024, 3072), (2048, 1024, 1024),
                                     (8000, 1000, 1024)])
def test_backward_workspace_holds_gate_parts_at_few_tile_shapes(m, n, d):
    """Few dW tiles (the plan splits each 4 ways or more): the workspace holds
    at least two fp32 parts per tile and at most 64 MiB of them (the CU count
    falls back to 256, MI355X's, without a device)."""
    tiles = ((n + 255) // 256) * ((d + 255) // 256)
    ws = _hip.bwd_workspace_bytes(m, n, d, (d + 255) // 256 * 256, 6, False)
    assert 2 * tiles * TILE <= ws <= (64 << 20) + (8 << 20)
    # a group of the same total rows sizes the same parts
    g = _hip.group_bwd_workspace_bytes(m, d, [((8,), [], n)])
    assert 2 * tiles * TILE <= g


@pytest.mark.parametrize("m, n, d", [(8192, 17408, 5120), (8192, 6144, 5120), (8192, 5120, 6144),
                                     (8192, 5120, 17408), (256, 1024, 1024)])
def test_backward_workspace_keeps_the_fused_gate_elsewhere(m, n, d):
    """Many tiles, or too few tokens to split: no parts, only the partials and
    dX's split-tail tiles (at these shapes less than two fp32 tiles per dW
    tile would take)."""
    ws = _hip.bwd_workspace_bytes(m, n, d, d, 6, False)
    tiles = ((n + 255) // 256) * ((d + 255) // 256)
    assert ws < 2 * tiles * TILE


def test_attention_fwd_argument_checks():
    """vq_attention_fwd refuses other head dims, a query-head count that the
    key/value heads do not divide, missing pointers and unaligned strides
    before any device work."""
    import ctypes

    lib = _hip.lib()
    st = (ctypes.c_int64 * 3)(64 * 16 * 8, 64 * 16, 64)
    bad = (ctypes.c_int64 * 3)(64 * 16 * 8, 64 * 16 + 4, 64)
    p = 4096  # never dereferenced: every call below fails its checks first
    assert lib.vq_attention_fwd(p, p, p, p, None, 1, 8, 16, 4, 128, st, st, st, st, 0.125, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_attention_fwd(p, p, p, p, None, 1, 8, 16, 5, 64, st, st, st, st, 0.125, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_attention_fwd(p, p, p, p, None, 1, 8, 16, 4, 64, st, st, st, st, -1.0, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_attention_fwd(None, p, p, p, None, 1, 8, 16, 4, 64, st, st, st, st, 0.125, None) == _hip.VQ_ERR_NULL
    assert lib.vq_attention_fwd(p, p, p, p, None, 1, 8, 16, 4, 64, st, bad, st, st, 0.125, None) == _hip.VQ_ERR_ALIGN
    assert lib.vq_attention_fwd(p + 8, p, p, p, None, 1, 8, 16, 4, 64, st, st, st, st, 0.125, None) == _hip.VQ_ERR_ALIGN
    # nothing to do: no pointer is needed
    assert lib.vq_attention_fwd(None, None, None, None, None, 0, 8, 16, 4, 64, None, None, None, None, 0.125,
                                None) == _hip.VQ_OK


def test_attention_bwd_argument_checks():
    """vq_attention_bwd refuses other head dims, K/V head counts that do not
    divide the query heads, a short workspace and unaligned strides before
    any device work; its workspace holds two floats per query padded to 128
    queries."""
    import ctypes

    lib = _hip.lib()
    assert lib.vq_attention_bwd_workspace(2, 100, 16) == 2 * 16 * 128 * 8
    assert lib.vq_attention_bwd_workspace(-1, 100, 16) == -1
    st = (ctypes.c_int64 * 24)(*([64 * 16 * 8, 64 * 16, 64] * 8))
    bad = (ctypes.c_int64 * 24)(*([64 * 16 * 8, 64 * 16 + 4, 64] * 8))
    p = 4096
    args = [p] * 6 + [p] * 3
    need = lib.vq_attention_bwd_workspace(1, 8, 16)
    assert lib.vq_attention_bwd(*args, 1, 8, 16, 4, 128, st, 0.125, p, need, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_attention_bwd(*args, 1, 8, 16, 3, 64, st, 0.125, p, need, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_attention_bwd(*args, 1, 8, 16, 0, 64, st, 0.125, p, need, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_attention_bwd(*args, 1, 8, 16, 4, 64, bad, 0.125, p, need, None) == _hip.VQ_ERR_ALIGN
    assert lib.vq_attention_bwd(*args, 1, 8, 16, 4, 64, st, 0.125, p, need - 1, None) == _hip.VQ_ERR_WORKSPACE
    assert lib.vq_attention_bwd(*args, 1, 8, 16, 4, 64, st, 0.125, None, need, None) == _hip.VQ_ERR_WORKSPACE
    assert lib.vq_attention_bwd(None, *args[1:], 1, 8, 16, 16, 64, st, 0.125, p, need, None) == _hip.VQ_ERR_NULL


def test_rope_qkv_fwd_argument_checks():
    """vq_rope_qkv_fwd takes K/V output heads of Hq (each head repeated) or
    Hkv and refuses any other count, and a head count that does not divide,
    before any device work."""
    lib = _hip.lib()
    p = 4096
    assert lib.vq_rope_qkv_fwd(p, 1, 8, 16, 4, 8, 64, p, p, p, p, p, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_rope_qkv_fwd(p, 1, 8, 16, 3, 16, 64, p, p, p, p, p, None) == _hip.VQ_ERR_SHAPE
    assert lib.vq_rope_qkv_fwd(p, 1, 8, 16, 4, 4, 40, p, p, p, p, p, None) == _hip.VQ_ERR_ALIGN
    assert lib.vq_rope_qkv_fwd(p, 1, 8, 16, 4, 16, 64, None, p, p, p, p, None) == _hip.VQ_ERR_NULL
    # nothing to do at B = 0: no pointer is needed
    assert lib.vq_rope_qkv_fwd(None, 0, 8, 16, 4, 4, 64, p, p, None, None, None, None) == _hip.VQ_OK


def test_attention_bwd_wrapper_head_checks():
    """The Python wrapper refuses K/V head counts that do not divide the query
    heads (zero included) with ValueError, before any device work."""
    import torch

    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16)
    lse = torch.zeros(1, 4, 8)
    for hk in (0, 3):
        kv = torch.zeros(1, hk, 8, 64, dtype=torch.bfloat16)
        with pytest.raises(ValueError):
            _hip.attention_bwd(q, q, kv, kv, q, lse)
