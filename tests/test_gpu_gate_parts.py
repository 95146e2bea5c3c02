"""The gate product's dW-parts path at decoder sizes (needs an MI355X).

When a gate product has few 256 x 256 dW tiles, the fused plan splits every
tile along the tokens, and each part then repeats the K-candidate decode of
its epilogue. The 0.8B-class decoder's 1024-wide products at 8192 tokens are
such a case. There the parts write their fp32 tiles, and one pass over the
summed parts takes dL/dp_k = <dY^T X, W_k> (``gate_dot_kernel``,
csrc/vq_dequant.hip). These tests run shapes that take that path, through
the C ABI:

* dL/dp within 1e-4 relative L2 of the fp32/fp64 evaluation of the
  reference's formula (voodoo_quant/layers.py:354-363). This covers single
  tensors, the gate product alone and inside the dual dX + gate launch,
  stacked groups with IQ menus, and a ragged D whose padded weights must
  carry no gradient;
* the fused epilogue, which vq_gated_linear_bwd_static keeps, agrees to 1e-5;
* dL/dp is bitwise the same on a second run and from the gate product alone
  (the last dot block to finish runs one fixed-order reduce);
* dX within 1e-2 of an fp32 product of the same bf16 operands;
* the workspace holds the parts, so these shapes do take the path, and the
  27B-class shapes do not.
"""

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture

pytestmark = pytest.mark.gpu

GGML = dict(cdequant.GGML_TYPE)
SIX = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]
TOL = 1e-2
TILE_BYTES = 256 * 256 * 4


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _say(msg):
    print(msg, flush=True)


def _cands(types, n, d_pad, rng):
    """Random valid blocks with fp16 scales in [2^-8, 2^-5) (O(1) weights) and
    the oracle's fp32 decodes of them."""
    qbs, ws = [], []
    for qt in types:
        nb = n * d_pad // 256 * (8 if qt == "Q8_0" else 1)
        qb = blocks.random_blocks(qt, nb, rng)
        for which in range(len(blocks.F16_OFFSETS[qt]) or 1):
            blocks.set_scale(qt, qb, (0x1C00 + rng.integers(0, 0x0C00, size=nb)).astype(np.uint16), which)
        qbs.append(qb)
        ws.append(torch.from_numpy(cdequant.oracle_dequant_parallel(qt, qb, n * d_pad).reshape(n, d_pad)))
    return qbs, ws


def _gp_ref(dy, x, cands, d):
    """<dY^T X, W_k> with dW in fp32 on the device and the dots in fp64."""
    dw = (dy.float().t() @ x.float()).double()
    return torch.stack([(dw * c[:, :d].to(dw.device, torch.float64)).sum() for c in cands]).cpu()


def _tiles(n, d):
    return ((n + 255) // 256) * ((d + 255) // 256)


SINGLE = [  # (name, m, d, d_pad, n, types)
    ("o_1024x1024", 8192, 1024, 1024, 1024, SIX),
    ("down_3072x1024", 8192, 3072, 3072, 1024, SIX),
    ("o_2048_tokens", 2048, 1024, 1024, 1024, SIX),
    ("ragged_d1000", 8192, 1000, 1024, 1024, ["Q8_0", "Q4_K", "Q2_K", "Q6_K"]),
    ("recipe_iq", 8192, 1024, 1024, 1536, ["Q8_0", "Q5_K", "IQ3_S", "IQ2_S", "IQ2_XXS", "IQ1_S"]),
    # ragged output rows (the last tile column half full) and a token count that
    # splits into uneven K parts (8000 = 125 steps of 64)
    ("ragged_n1000_m8000", 8000, 1024, 1024, 1000, ["Q6_K", "Q3_K", "Q8_0"]),
]


@pytest.mark.parametrize("case", SINGLE, ids=[c[0] for c in SINGLE])
def test_parts_single_matches_oracle(hip, case):
    name, m, d, d_pad, n, types = case
    k_ = len(types)
    _say(f"[parts] {name}: M={m} D={d} d_pad={d_pad} N={n} K={k_}")
    rng = np.random.default_rng(m + d + n)
    qbs, cands = _cands(types, n, d_pad, rng)
    g = torch.Generator().manual_seed(n + d)
    probs = torch.softmax(torch.randn(k_, generator=g), 0)
    dev = torch.device("cuda", 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16).to(dev)
    qd = [torch.from_numpy(q.reshape(-1)).to(dev) for q in qbs]
    ids = [GGML[t] for t in types]
    pd = probs.to(dev)

    ws_bytes = hip.bwd_workspace_bytes(m, n, d, d_pad, k_, False)
    assert ws_bytes >= 2 * _tiles(n, d) * TILE_BYTES, f"{name}: workspace {ws_bytes} holds no dW parts"
    w_eff = torch.empty(n, d_pad, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    hip.gated_linear_fwd(x, ids, qd, pd, n, d_pad, w_eff, y)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    dp = torch.empty(k_, dtype=torch.float32, device=dev)
    _say(f"[parts] {name}: dual dX + gate (parts)")
    hip.gated_linear_bwd(dy, x, ids, qd, pd, n, d_pad, w_eff, dx, dp, ws)
    dp_again = torch.empty(k_, dtype=torch.float32, device=dev)
    hip.gated_linear_bwd(dy, x, ids, qd, pd, n, d_pad, w_eff, dx, dp_again, ws)
    dp_gate = torch.empty(k_, dtype=torch.float32, device=dev)
    _say(f"[parts] {name}: gate product alone (parts)")
    hip.gated_linear_bwd(dy, x, ids, qd, pd, n, d_pad, w_eff, None, dp_gate, ws)
    dx_f = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    dp_f = torch.empty(k_, dtype=torch.float32, device=dev)
    _say(f"[parts] {name}: fused epilogue (static entry point)")
    hip.gated_linear_bwd_static(dy, x, ids, qd, n, d_pad, w_eff, dx_f, dp_f)
    torch.cuda.synchronize()

    gp_ref = _gp_ref(dy, x, cands, d)
    e_dual = mixture.relative_l2(dp.cpu().double(), gp_ref)
    e_gate = mixture.relative_l2(dp_gate.cpu().double(), gp_ref)
    e_fused = mixture.relative_l2(dp.cpu().double(), dp_f.cpu().double())
    dx_ref = dy.float() @ w_eff[:, :d].float()
    e_dx = mixture.relative_l2(dx.double(), dx_ref.double())
    _say(f"[parts] {name}: dL/dp dual {e_dual:.2e} gate-only {e_gate:.2e} vs fused {e_fused:.2e}; dX {e_dx:.2e}")
    assert e_dual < 1e-4 and e_gate < 1e-4
    assert e_fused < 1e-5
    # whichever dot block finishes last, the reduce runs in one fixed order
    assert torch.equal(dp.view(torch.int32), dp_again.view(torch.int32)), "dL/dp differs between two runs"
    assert torch.equal(dp.view(torch.int32), dp_gate.view(torch.int32)), "dual and gate-only dL/dp differ"
    assert e_dx < TOL
    assert torch.equal(dx.view(torch.int16), dx_f.view(torch.int16)), "dX depends on the gate path"


GROUPS = [  # (name, m, d, [(types, n)])
    ("qkv_iq", 8192, 1024, [(["Q8_0", "Q5_K", "IQ3_S", "IQ2_S"], 1024), (["IQ2_XXS", "Q4_K"], 256),
                            (["Q6_K", "IQ1_S", "IQ4_XS", "Q3_K", "Q2_K"], 256)]),
    ("kv_iq", 8192, 1024, [(SIX, 512), (["IQ4_XS", "IQ3_S", "IQ2_S", "IQ2_XXS", "IQ1_S"], 512)]),
]


@pytest.mark.parametrize("case", GROUPS, ids=[c[0] for c in GROUPS])
def test_parts_group_matches_oracle(hip, case):
    name, m, d, members = case
    d_pad = d
    n_total = sum(n for _, n in members)
    _say(f"[parts] group {name}: M={m} D={d} members {[(len(t), n) for t, n in members]}")
    rng = np.random.default_rng(m + n_total)
    g = torch.Generator().manual_seed(n_total)
    dev = torch.device("cuda", 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(m, n_total, generator=g).to(torch.bfloat16).to(dev)
    spec, cands_all, probs = [], [], []
    for types, n in members:
        qbs, cands = _cands(types, n, d_pad, rng)
        spec.append((tuple(GGML[t] for t in types), [torch.from_numpy(q.reshape(-1)).to(dev) for q in qbs], n))
        cands_all.append(cands)
        probs.append(torch.softmax(torch.randn(len(types), generator=g), 0).to(dev))
    ws_bytes = hip.group_bwd_workspace_bytes(m, d, spec)
    assert ws_bytes >= 2 * _tiles(n_total, d) * TILE_BYTES, f"{name}: workspace {ws_bytes} holds no dW parts"
    w_eff = torch.empty(n_total, d_pad, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n_total, dtype=torch.bfloat16, device=dev)
    hip.gated_linear_group_fwd(x, spec, probs, d_pad, w_eff, y)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    dps = [torch.empty(len(t), dtype=torch.float32, device=dev) for t, _ in members]
    hip.gated_linear_group_bwd(dy, x, spec, d_pad, w_eff, dx, dps, ws)
    dps_gate = [torch.empty(len(t), dtype=torch.float32, device=dev) for t, _ in members]
    hip.gated_linear_group_bwd(dy, x, spec, d_pad, None, None, dps_gate, ws)
    torch.cuda.synchronize()
    off = 0
    for (types, n), cands, dp, dpg in zip(members, cands_all, dps, dps_gate):
        gp_ref = _gp_ref(dy[:, off:off + n], x, cands, d)
        e, eg = mixture.relative_l2(dp.cpu().double(), gp_ref), mixture.relative_l2(dpg.cpu().double(), gp_ref)
        _say(f"[parts] group {name}: member {types} dL/dp dual {e:.2e} gate-only {eg:.2e}")
        assert e < 1e-4 and eg < 1e-4, (name, types)
        off += n
    e_dx = mixture.relative_l2(dx.double(), (dy.float() @ w_eff[:, :d].float()).double())
    assert e_dx < TOL


def test_parts_group_with_wider_padding_keeps_fused_path(hip):
    """A group whose d_pad exceeds D rounded up to 256 runs the fused epilogue
    (its workspace, sized from D, still suffices) and stays exact."""
    m, d, d_pad = 8192, 1024, 1280
    members = [(["Q8_0", "Q4_K", "Q2_K"], 1024), (["Q6_K", "Q3_K"], 256)]
    n_total = sum(n for _, n in members)
    rng = np.random.default_rng(7)
    g = torch.Generator().manual_seed(7)
    dev = torch.device("cuda", 0)
    x = torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(m, n_total, generator=g).to(torch.bfloat16).to(dev)
    spec, cands_all, probs = [], [], []
    for types, n in members:
        qbs, cands = _cands(types, n, d_pad, rng)
        spec.append((tuple(GGML[t] for t in types), [torch.from_numpy(q.reshape(-1)).to(dev) for q in qbs], n))
        cands_all.append(cands)
        probs.append(torch.softmax(torch.randn(len(types), generator=g), 0).to(dev))
    w_eff = torch.empty(n_total, d_pad, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n_total, dtype=torch.bfloat16, device=dev)
    hip.gated_linear_group_fwd(x, spec, probs, d_pad, w_eff, y)
    ws = torch.empty(hip.group_bwd_workspace_bytes(m, d, spec), dtype=torch.uint8, device=dev)
    dps = [torch.empty(len(t), dtype=torch.float32, device=dev) for t, _ in members]
    hip.gated_linear_group_bwd(dy, x, spec, d_pad, w_eff, None, dps, ws)
    torch.cuda.synchronize()
    off = 0
    for (types, n), cands, dp in zip(members, cands_all, dps):
        e = mixture.relative_l2(dp.cpu().double(), _gp_ref(dy[:, off:off + n], x, cands, d))
        _say(f"[parts] padded group: member {types} dL/dp {e:.2e}")
        assert e < 1e-4
        off += n


@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120), (5120, 6144)])
def test_many_tile_shapes_keep_the_fused_epilogue(hip, shape):
    """Many tiles: no dW parts in the workspace (the tiles run whole or split
    fewer than 4 ways, or their parts would pass 64 MiB).  At these shapes dX's
    split-tail tiles are smaller than the smallest parts buffer (two per
    tile), so the workspace size tells the two paths apart."""
    d, n = shape
    assert hip.bwd_workspace_bytes(8192, n, d, d, 6, False) < 2 * _tiles(n, d) * TILE_BYTES
