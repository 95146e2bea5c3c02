"""Pins of the oracle itself (CPU only).

Dequant: the reference's own decoders (golden vectors, ``voodoo_quant/layers.py:
62-213``), closed-form field values from the independent packers, and hand-made
blocks whose values are known.  Mixture math: float64 finite differences, the
softmax-Jacobian identity of ``tests/test_ptqr.py:161-172`` and linearity.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import blocks, cdequant, mixture

GOLDEN = Path(__file__).resolve().parent / "golden" / "ref_decoders.npz"
SIX = ["Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("qt", ["Q8_0", "Q4_K", "Q5_K", "Q6_K"])
def test_oracle_matches_reference_decoders(qt):
    g = np.load(GOLDEN)
    qb, ref = g[f"{qt}_qbytes"], g[f"{qt}_out"]
    y = cdequant.oracle_dequant(qt, qb, ref.size)
    assert np.array_equal(bits(y), bits(ref)), f"{qt}: {np.sum(bits(y) != bits(ref))} mismatching weights"


GOLDEN_IQ = Path(__file__).resolve().parent / "golden" / "ref_iq_decoders.npz"


@pytest.mark.parametrize("qt", blocks.IQ_TYPES)
def test_oracle_matches_reference_iq_decoders(qt):
    """Bit-exact against the reference's IQ decoders (quants/gpu_dequant.py:53-519)
    on 128 random blocks and six edge blocks (zero/all-ones payload, subnormal,
    largest finite and signed-zero scales)."""
    g = np.load(GOLDEN_IQ)
    qb, ref = g[f"{qt}_qbytes"], g[f"{qt}_out"]
    y = cdequant.oracle_dequant(qt, qb, ref.size)
    assert np.array_equal(bits(y), bits(ref)), f"{qt}: {np.sum(bits(y) != bits(ref))} mismatching weights"


@pytest.mark.parametrize("qt", blocks.IQ_TYPES)
def test_iq_scale_linearity(qt):
    """Every IQ weight is the super-block scale d times a factor fixed by the
    other bytes: raising d's exponent by one doubles every weight exactly."""
    rng = np.random.default_rng(11)
    blk = blocks.random_blocks(qt, 16, rng)
    h = (0x3000 + rng.integers(0, 0x400, size=16)).astype(np.uint16)  # 2^-3 <= d < 2^-2
    blocks.set_scale(qt, blk, h)
    y1 = cdequant.oracle_dequant(qt, blk, 16 * 256)
    blocks.set_scale(qt, blk, h + np.uint16(0x400))
    y2 = cdequant.oracle_dequant(qt, blk, 16 * 256)
    assert np.array_equal(bits(y2), bits(2 * y1))
    if qt not in ("IQ4_XS",):  # IQ4_XS sub-block scales (ls - 32) can be 0
        assert np.all(y1 != 0)


@pytest.mark.parametrize("qt", ["IQ2_XXS", "IQ2_XS", "IQ3_XXS"])
def test_iq_stored_signs_have_even_parity(qt):
    """Formats that store 7 of 8 signs make the eighth even the count of
    negative weights in every group of 8 (positive d, nonzero grid values)."""
    rng = np.random.default_rng(12)
    blk = blocks.random_blocks(qt, 32, rng)
    blocks.set_scale(qt, blk, 0x3C00)
    y = cdequant.oracle_dequant(qt, blk, 32 * 256).reshape(-1, 8)
    assert np.all(y != 0)
    assert np.all((y < 0).sum(axis=1) % 2 == 0)


@pytest.mark.parametrize("qt", SIX)
@pytest.mark.parametrize("seed", [0, 1])
def test_oracle_matches_closed_form(qt, seed):
    rng = np.random.default_rng(seed)
    nb = 40 if qt != "Q8_0" else 320
    packed, vals = blocks.packed_and_values(qt, nb, rng)
    y = cdequant.oracle_dequant(qt, packed, vals.size)
    assert np.array_equal(bits(y), bits(vals.reshape(-1)))


def test_planted_layout_mistake_is_caught():
    """A packer that swaps Q4_K nibble halves must disagree with the decoder."""
    rng = np.random.default_rng(3)
    f = blocks.random_fields("Q4_K", 8, rng, allow_subnormal=False)
    packed = blocks.pack_q4_K(**f)
    qs = packed[:, 16:144].copy()
    packed[:, 16:144] = ((qs >> 4) | (qs << 4)).astype(np.uint8)  # swap nibbles: wrong layout
    y = cdequant.oracle_dequant("Q4_K", packed, 8 * 256)
    assert not np.array_equal(bits(y), bits(blocks.value_q4_K(**f).reshape(-1)))


def _block(qt, fill, d, dmin=0x3C00):
    b = np.full((1, blocks.BLOCK_BYTES[qt]), fill, np.uint8)
    for off, h in zip(blocks.F16_OFFSETS[qt], (d, dmin)):
        b[0, off], b[0, off + 1] = h & 0xFF, h >> 8
    return b


def test_known_values():
    # Q8_0 with d = 0.5 and qs = 0xFF (-1) -> -0.5 everywhere
    y = cdequant.oracle_dequant("Q8_0", np.tile(_block("Q8_0", 0xFF, 0x3800), (8, 1)), 256)
    assert np.all(y == -0.5)
    # Q8_0 all-zero codes with a negative scale: 0 * -1 = -0.0 (signed zero, as ggml)
    y = cdequant.oracle_dequant("Q8_0", np.tile(_block("Q8_0", 0x00, 0xBC00), (8, 1)), 256)
    assert np.all(y == 0) and np.all(np.signbit(y))
    # Q6_K with every byte 0x00 except d = 1: scales are 0 -> 0 * (0 - 32) = -0.0
    y = cdequant.oracle_dequant("Q6_K", _block("Q6_K", 0x00, 0x3C00), 256)
    assert np.all(y == 0) and np.all(np.signbit(y))
    # Q2_K all bytes 0xFF with d = dmin = 1: sc = m = 15, q = 3 -> 15*3 - 15 = 30
    y = cdequant.oracle_dequant("Q2_K", _block("Q2_K", 0xFF, 0x3C00, 0x3C00), 256)
    assert np.all(y == 30.0)
    # Q3_K all bytes 0xFF, d = 1: scale code 63 -> 31, q = 3 with hmask set -> 93
    y = cdequant.oracle_dequant("Q3_K", _block("Q3_K", 0xFF, 0x3C00), 256)
    assert np.all(y == 93.0)
    # Q4_K all 0xFF, d = dmin = 1: sc = m = 63, q = 15 -> 63*15 - 63 = 882
    y = cdequant.oracle_dequant("Q4_K", _block("Q4_K", 0xFF, 0x3C00, 0x3C00), 256)
    assert np.all(y == 882.0)
    # Q5_K all 0xFF: q = 31 -> 63*31 - 63 = 1890
    y = cdequant.oracle_dequant("Q5_K", _block("Q5_K", 0xFF, 0x3C00, 0x3C00), 256)
    assert np.all(y == 1890.0)


def test_fp16_widening_subnormal():
    assert cdequant.half_to_float(0x0001) == 2.0 ** -24
    assert cdequant.half_to_float(0x8001) == -(2.0 ** -24)
    assert cdequant.half_to_float(0x03FF) == 1023 * 2.0 ** -24
    assert cdequant.half_to_float(0x7BFF) == 65504.0


def test_parallel_decoder_agrees():
    rng = np.random.default_rng(5)
    for qt in SIX:
        nb = 300 if qt != "Q8_0" else 2400
        qb = blocks.random_blocks(qt, nb, rng)
        n = nb * blocks.BLOCK_SIZE[qt]
        a = cdequant.oracle_dequant(qt, qb, n)
        b = cdequant.oracle_dequant_parallel(qt, qb, n, nthreads=4)
        assert np.array_equal(bits(a), bits(b))


# ------------------------------------------------------------------ mixture math
def _toy(seed=0, k=3, n=8, d=16, m=5, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    cands = [torch.randn(n, d, generator=g, dtype=dtype) for _ in range(k)]
    x = torch.randn(m, d, generator=g, dtype=dtype)
    dy = torch.randn(m, n, generator=g, dtype=dtype)
    gates = torch.randn(k, generator=g, dtype=dtype)
    return cands, x, dy, gates


@pytest.mark.parametrize("temperature", [1.0, 0.37, 2.5])
def test_gate_gradient_finite_differences(temperature):
    cands, x, dy, gates = _toy()

    def loss(gv):
        p = mixture.soft_probs(gv, temperature)
        w = sum(p[k] * cands[k] for k in range(len(cands)))
        return (dy * mixture.forward(x, w, torch.float64)).sum()

    p = mixture.soft_probs(gates, temperature)
    w = sum(p[k] * cands[k] for k in range(len(cands)))
    _, _, gp = mixture.backward(dy, x, w, cands, torch.float64)
    analytic = mixture.gates_grad(gp, p, temperature)
    eps = 1e-6
    fd = torch.zeros_like(gates)
    for k in range(len(gates)):
        e = torch.zeros_like(gates)
        e[k] = eps
        fd[k] = (loss(gates + e) - loss(gates - e)) / (2 * eps)
    assert torch.allclose(analytic, fd, rtol=1e-6, atol=1e-8)


def test_softmax_jacobian_identity():
    """gates.grad = (diag p - p p^T) gp at T = 1 (tests/test_ptqr.py:161-172)."""
    cands, x, dy, gates = _toy(1)
    g = gates.clone().requires_grad_(True)
    p = torch.softmax(g, 0)
    w = sum(p[k] * cands[k] for k in range(len(cands)))
    (dy * (x @ w.t())).sum().backward()
    gp = torch.stack([(dy * (x @ c.t())).sum() for c in cands])
    pd = p.detach()
    assert torch.allclose(g.grad, (torch.diag(pd) - torch.outer(pd, pd)) @ gp, rtol=1e-10)
    # the oracle's own formula agrees with autograd
    assert torch.allclose(g.grad, mixture.gates_grad(gp, pd, 1.0), rtol=1e-10)


def test_dx_and_dw_closed_form():
    cands, x, dy, gates = _toy(2)
    p = mixture.soft_probs(gates, 1.0)
    w = sum(p[k] * cands[k] for k in range(len(cands)))
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    (dy * (xr @ wr.t())).sum().backward()
    dx, dw, gp = mixture.backward(dy, x, w, cands, torch.float64)
    assert torch.allclose(dx, xr.grad) and torch.allclose(dw, wr.grad)
    # linearity of the gate gradient in the candidates: gp_k = <G, x W_k^T>
    assert torch.allclose(gp, torch.stack([(dy * (x @ c.t())).sum() for c in cands]))


def test_mix_weight_is_k_ordered_fp32():
    g = torch.Generator().manual_seed(4)
    cands = [torch.randn(64, 64, generator=g) for _ in range(4)]
    p = torch.softmax(torch.randn(4, generator=g), 0)
    w = mixture.mix_weight(cands, p)
    ref = torch.zeros(64, 64)
    for k in range(4):
        ref = ref + p[k] * cands[k]
    assert torch.equal(w, ref)


def test_anneal_and_size_loss():
    assert mixture.anneal_temperature(0, 200, 2.0, 0.1) == 2.0
    assert abs(mixture.anneal_temperature(199, 200, 2.0, 0.1) - 0.1) < 1e-12
    assert mixture.anneal_temperature(5, 1, 2.0, 0.1) == 0.1
    assert float(mixture.size_loss(torch.tensor(101.0), 100.0, 0.02)) == 0.0
    assert abs(float(mixture.size_loss(torch.tensor(110.0, dtype=torch.float64), 100.0, 0.02)) - 0.08 ** 2) < 1e-12


def test_planted_sign_error_in_jacobian_is_caught():
    """A gate gradient with the wrong sign of the <p, gp> term fails the FD pin."""
    cands, x, dy, gates = _toy(6)
    p = mixture.soft_probs(gates, 1.0)
    w = sum(p[k] * cands[k] for k in range(len(cands)))
    _, _, gp = mixture.backward(dy, x, w, cands, torch.float64)
    wrong = p * (gp + (p * gp).sum())
    right = mixture.gates_grad(gp, p, 1.0)
    assert not torch.allclose(wrong, right, rtol=1e-3)
