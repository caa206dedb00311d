"""Pins oracle/dit.py (the DiT residual stream) without restating its formula: float64
brute force from the same bf16 inputs (the oracle may differ only by its bf16 rounding
points), and the invariants that fix the operation's structure."""

import torch

from oracle import dit


def _inputs(rows, dim, seed, spread=3.0):
    g = torch.Generator().manual_seed(seed)
    x = (spread * torch.randn(rows, dim, generator=g) + 0.5 * spread).bfloat16()
    y = torch.randn(rows, dim, generator=g).bfloat16()
    gate, scale, shift = (0.3 * torch.randn(3, dim, generator=g)).bfloat16().unbind(0)
    return x, y, gate, scale, shift


def test_against_float64():
    # dim 8 tells the biased variance from the unbiased one; a spread of 1e-3 (variance
    # 1e-6, the size of eps) tells where eps enters
    for rows, dim, seed, spread in [(7, 64, 0, 3.0), (5, 2048, 1, 3.0), (3, 5120, 2, 3.0), (6, 8, 4, 3.0),
                                    (4, 256, 5, 1e-3)]:
        x, y, gate, scale, shift = _inputs(rows, dim, seed, spread)
        y = y * spread
        xn, h = dit.adaln_residual(x, y, gate, scale, shift, 1e-6)
        x64 = x.double() + gate.double() * y.double()
        # two bf16 roundings (unit roundoff 2^-8): of the product, then of the sum
        prod = (gate.double() * y.double()).abs()
        assert ((xn.double() - x64).abs() <= 1.01 * 2.0 ** -8 * (prod + x64.abs())).all()
        xd = xn.double()
        ln = (xd - xd.mean(-1, keepdim=True)) / torch.sqrt(xd.var(-1, unbiased=False, keepdim=True) + 1e-6)
        h64 = ln * (1 + scale.double()) + shift.double()
        # four bf16 roundings on values bounded by |ln| * |1 + scale| + |shift|
        bound = 4 * 2.0 ** -8 * (ln.abs() * (1 + scale.double()).abs() + shift.double().abs()) + 1e-6
        assert ((h.double() - h64).abs() <= bound).all()


def test_a_zero_gate_keeps_the_stream_and_a_plain_norm_standardises():
    x, y, gate, scale, shift = _inputs(9, 1024, 3)
    zero = torch.zeros_like(gate)
    xn, h = dit.adaln_residual(x, y, zero, zero, zero, 1e-6)
    assert torch.equal(xn, x)
    hf = h.float()
    assert hf.mean(-1).abs().max() < 2e-2 and (hf.var(-1, unbiased=False) - 1).abs().max() < 2e-2
    # a residual but no norm: the stream alone
    xn2, none = dit.adaln_residual(x, y, gate, None, None, 1e-6)
    assert none is None and torch.equal(xn2, dit.adaln_residual(x, y, gate, scale, shift, 1e-6)[0])
    # shift moves the output by itself where scale is zero
    shifted = dit.adaln_residual(x, None, None, zero, shift, 1e-6)[1]
    assert (shifted.float() - h.float() - shift.float()).abs().max() <= 2.0 ** -6 * (h.float().abs().max() + 1)
