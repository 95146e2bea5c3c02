"""The allocation-free backward (vq_gated_linear_bwd_static) against the
workspace one (vq_gated_linear_bwd), through the C ABI, on two calls in a row
(the second smaller, so it reuses the static scratch the first one left).

dL/dp must be bit-identical (same gate plan, same partial order, same fp64
reduce).  dX must be bit-identical to the workspace entry point's dX run with
whole tiles (the static entry point never splits dX's tail tiles: their
partials would need 16 MiB or more of scratch) and within 1e-2 relative L2 of
its split-tail dX.  A ragged shape (300 tokens, 1000 -> 1000, padded to 1024)
runs the edge tiles.
"""

import numpy as np
import pytest
import torch

from oracle import blocks

pytestmark = pytest.mark.gpu

GGML = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant import _hip

    _hip.lib()
    return _hip


def _case(types, m, n, d, seed):
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(seed)
    qd = []
    for qt in types:
        per = 8 if qt == "Q8_0" else 1
        qb = blocks.random_blocks(qt, n * d // 256 * per, rng, allow_subnormal=False)
        for off in blocks.F16_OFFSETS[qt]:
            h = qb[:, off].astype(np.uint16) | (qb[:, off + 1].astype(np.uint16) << 8)
            h = (h & 0x83FF) | (np.uint16(0x2000) + ((h >> 10) & 0x7) * np.uint16(0x0400))
            qb[:, off], qb[:, off + 1] = (h & 0xFF).astype(np.uint8), (h >> 8).astype(np.uint8)
        qd.append(torch.from_numpy(qb.reshape(-1)).to(dev))
    g = torch.Generator(device=dev).manual_seed(seed)
    probs = torch.softmax(torch.randn(len(types), device=dev, generator=g), 0)
    x = torch.randn(m, d, device=dev, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, device=dev, generator=g).to(torch.bfloat16)
    return [GGML[t] for t in types], qd, probs, x, dy


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


def test_static_backward_matches_workspace_backward(hip):
    dev = torch.device("cuda", 0)
    cases = [(["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"], 4096, 6144, 5120, 5120, 1),
             (["Q8_0", "Q6_K", "Q4_K", "Q3_K"], 512, 1024, 1024, 1024, 2),
             (["Q8_0", "Q5_K", "Q4_K", "Q2_K"], 300, 1000, 1000, 1024, 3)]
    for types, m, n, d, d_pad, seed in cases:
        print(f"[no-alloc] m={m} n={n} d={d} K={len(types)}", flush=True)
        ids, qd, probs, x, dy = _case(types, m, n, d_pad, seed)
        x = x[:, :d].contiguous()
        w_eff = hip.mix_weight(ids, qd, probs, n, d_pad)
        k = len(types)
        # the workspace entry point: dX with split tails + dL/dp, then dX alone with whole tiles
        ws = torch.empty(hip.bwd_workspace_bytes(m, n, d, d_pad, k, False), dtype=torch.uint8, device=dev)
        dx_ws = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
        dp_ws = torch.empty(k, dtype=torch.float32, device=dev)
        hip.gated_linear_bwd(dy, x, ids, qd, probs, n, d_pad, w_eff, dx_ws, dp_ws, ws)
        dx_whole = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
        hip.gated_linear_bwd(dy, x, ids, qd, probs, n, d_pad, w_eff, dx_whole, None, None)
        # the static entry point: the same outputs, filled with garbage first
        dx_st = torch.full((m, d), float("nan"), dtype=torch.bfloat16, device=dev)
        dp_st = torch.full((k,), float("nan"), dtype=torch.float32, device=dev)
        hip.gated_linear_bwd_static(dy, x, ids, qd, n, d_pad, w_eff, dx_st, dp_st)
        torch.cuda.synchronize()
        assert torch.equal(dp_st.view(torch.int32), dp_ws.view(torch.int32)), (dp_st, dp_ws)
        assert torch.equal(dx_st.view(torch.int16), dx_whole.view(torch.int16))
        assert _rel(dx_st, dx_ws) < 1e-2
        # dL/dp alone (the gate product's own launch)
        dp_only = torch.full((k,), float("nan"), dtype=torch.float32, device=dev)
        hip.gated_linear_bwd_static(dy, x, ids, qd, n, d_pad, None, None, dp_only)
        torch.cuda.synchronize()
        assert torch.equal(dp_only.view(torch.int32), dp_ws.view(torch.int32))
        print(f"[no-alloc] ok: dL/dp {dp_st.tolist()}, dX vs split-tail dX {_rel(dx_st, dx_ws):.2e}", flush=True)


def test_static_backward_rejects_sizes_beyond_the_scratch(hip):
    """Gate partials larger than the static scratch are refused on the host,
    before any launch (the small stand-in buffers are never read)."""
    dev = torch.device("cuda", 0)
    k = 12
    qd = [torch.zeros(256, dtype=torch.uint8, device=dev) for _ in range(k)]
    x = torch.zeros(256, 16384, dtype=torch.bfloat16, device=dev)
    dy = torch.zeros(256, 8, dtype=torch.bfloat16, device=dev)
    dp = torch.zeros(k, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="static scratch"):
        hip.gated_linear_bwd_static(dy, x, [8] * k, qd, 524288, 16384, None, None, dp)
    with pytest.raises(ValueError, match="w_eff"):
        hip.gated_linear_bwd_static(dy, x, [8] * k, qd, 64, 16384, None, torch.empty_like(x), None)
