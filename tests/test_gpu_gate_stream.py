"""Backward entry points that finish the gate gradient on a second stream
(vq_gated_linear_bwd_gate_stream, vq_gated_linear_group_bwd_gate_stream; needs
an MI355X).

The products run on the caller's stream and the dot pass and the fixed-order
reduce on the gate stream after an event fence, so dL/dp and dX must be
bitwise those of the in-order entry points, on the dW-parts path (8192 tokens,
1024 -> 1024), on the fused-epilogue path (8192 tokens, 5120 -> 6144) and for a
stacked group.  The in-order entry points'
values are pinned against the oracle in test_gpu_gate_parts.py and
test_gpu_kernels.py.
"""

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant

pytestmark = pytest.mark.gpu

GGML = dict(cdequant.GGML_TYPE)
SIX = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _qbytes(types, n, d_pad, rng, dev):
    out = []
    for qt in types:
        nb = n * d_pad // 256 * (8 if qt == "Q8_0" else 1)
        qb = blocks.random_blocks(qt, nb, rng)
        for which in range(len(blocks.F16_OFFSETS[qt]) or 1):
            blocks.set_scale(qt, qb, (0x1C00 + rng.integers(0, 0x0C00, size=nb)).astype(np.uint16), which)
        out.append(torch.from_numpy(qb.reshape(-1)).to(dev))
    return out


@pytest.mark.parametrize("m, d, n", [(8192, 1024, 1024), (8192, 5120, 6144)], ids=["parts_path", "fused_epilogue"])
def test_gate_stream_backward_is_bitwise_in_order(hip, m, d, n):
    print(f"[gate stream] single M={m} D={d} N={n} K=6", flush=True)
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(m + d + n)
    qd = _qbytes(SIX, n, d, rng, dev)
    ids = [GGML[t] for t in SIX]
    g = torch.Generator(device=dev).manual_seed(1)
    probs = torch.softmax(torch.randn(6, device=dev, generator=g), 0)
    x = torch.randn(m, d, device=dev, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, device=dev, generator=g).to(torch.bfloat16)
    w_eff = torch.empty(n, d, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    hip.gated_linear_fwd(x, ids, qd, probs, n, d, w_eff, y)
    ws = torch.empty(hip.bwd_workspace_bytes(m, n, d, d, 6, False), dtype=torch.uint8, device=dev)
    dx0, dx1 = (torch.empty(m, d, dtype=torch.bfloat16, device=dev) for _ in range(2))
    dp0 = torch.full((6,), float("nan"), device=dev)
    dp1 = torch.full((6,), float("nan"), device=dev)
    hip.gated_linear_bwd(dy, x, ids, qd, probs, n, d, w_eff, dx0, dp0, ws)
    ws2 = torch.empty_like(ws)
    side = torch.cuda.Stream(device=dev)
    hip.gated_linear_bwd(dy, x, ids, qd, probs, n, d, w_eff, dx1, dp1, ws2, side)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(dp0.view(torch.int32), dp1.view(torch.int32)), (dp0, dp1)
    assert torch.equal(dx0.view(torch.int16), dx1.view(torch.int16))
    assert bool(torch.isfinite(dp1).all()) and float(dp1.abs().max()) > 0


def test_gate_stream_group_backward_is_bitwise_in_order(hip):
    m, d = 8192, 1024
    members = [(SIX, 1024), (["Q8_0", "Q4_K", "Q3_K"], 512)]
    print(f"[gate stream] group M={m} D={d} members={[n for _, n in members]}", flush=True)
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(7)
    g = torch.Generator(device=dev).manual_seed(2)
    spec, probs = [], []
    for types, n in members:
        spec.append((tuple(GGML[t] for t in types), _qbytes(types, n, d, rng, dev), n))
        probs.append(torch.softmax(torch.randn(len(types), device=dev, generator=g), 0))
    n_total = sum(n for _, n in members)
    x = torch.randn(m, d, device=dev, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n_total, device=dev, generator=g).to(torch.bfloat16)
    w_eff = torch.empty(n_total, d, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n_total, dtype=torch.bfloat16, device=dev)
    hip.gated_linear_group_fwd(x, spec, probs, d, w_eff, y)
    ws_bytes = hip.group_bwd_workspace_bytes(m, d, spec)
    outs = []
    side = torch.cuda.Stream(device=dev)
    for stream in (None, side):
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
        dps = [torch.full((len(t),), float("nan"), device=dev) for t, _ in members]
        hip.gated_linear_group_bwd(dy, x, spec, d, w_eff, dx, dps, ws, stream)
        outs.append((dx, dps, ws))
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    (dx0, dp0, _), (dx1, dp1, _) = outs
    assert torch.equal(dx0.view(torch.int16), dx1.view(torch.int16))
    for a, b in zip(dp0, dp1):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), (a, b)
        assert bool(torch.isfinite(b).all())
