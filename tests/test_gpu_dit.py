"""The DiT residual stream kernel (fm_adaln_residual) against oracle/dit.py: the stream
x' = x + gate * y bit-exact (its two bf16 roundings are fixed), the modulated norm h
within what a one-ulp flip of the LayerNorm output can move it, per element (the
statistics' summation order differs), on fewer than 1 % of elements, across row widths from 8 to 8192, with and without each part, in place."""

import pytest
import torch

from oracle import dit

pytestmark = pytest.mark.gpu


def _inputs(rows, dim, seed):
    g = torch.Generator().manual_seed(seed)
    x = (2 * torch.randn(rows, dim, generator=g) + 0.25).bfloat16()
    y = torch.randn(rows, dim, generator=g).bfloat16()
    gate, scale, shift = (0.3 * torch.randn(3, dim, generator=g)).bfloat16().unbind(0)
    return x, y, gate, scale, shift


def _h_close(got, want, shift):
    """Per element of h = mod + shift: within what one bf16 ulp of the LayerNorm output
    (carried through the modulation) plus the final rounding can move it, i.e. 2^-7 of
    |mod| + |h| (mod = h - shift can cancel against shift); and the fraction of elements
    that differ at all."""
    g, w = got.float(), want.float()
    bound = 2.0 ** -7 * ((w - shift.float()).abs() + w.abs())
    return bool(((g - w).abs() <= bound).all()), float((g != w).float().mean())


@pytest.mark.parametrize("rows,dim", [(1, 8), (5, 136), (16, 1024), (1024, 2048), (33, 4096), (64, 5120),
                                      (7, 8192)])
def test_residual_and_norm(dev, rows, dim):
    print(f"adaln_residual rows={rows} dim={dim}", flush=True)
    from flashmap_amd import ops

    x, y, gate, scale, shift = _inputs(rows, dim, rows + dim)
    want_x, want_h = dit.adaln_residual(x, y, gate, scale, shift, 1e-6)
    got_x, got_h = ops.adaln_residual(x.to(dev), y.to(dev), gate.to(dev), (scale.to(dev), shift.to(dev)), 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(got_x.cpu(), want_x)
    ok, frac = _h_close(got_h.cpu(), want_h, shift)
    print(f"  h: {100 * frac:.3f} % of elements differ from the oracle", flush=True)
    assert ok and frac < 0.01


def test_parts_alone_and_in_place(dev):
    from flashmap_amd import ops

    rows, dim = 48, 2048
    x, y, gate, scale, shift = _inputs(rows, dim, 9)
    xd, yd, gd, sd, td = (t.to(dev) for t in (x, y, gate, scale, shift))
    # the norm alone (the first norm of a layer)
    none, h = ops.adaln_residual(xd, None, None, (sd, td), 1e-6)
    assert none is None
    assert _h_close(h.cpu(), dit.adaln_residual(x, None, None, scale, shift, 1e-6)[1], shift)[0]
    # the residual alone (a layer's last sublayer without a following norm)
    xo, no_h = ops.adaln_residual(xd, yd, gd, None, 1e-6)
    assert no_h is None and torch.equal(xo.cpu(), dit.adaln_residual(x, y, gate, None, None, 1e-6)[0])
    # in place on a (B, T, dim) stream, strided y rows
    stream = xd.view(3, 16, dim).clone()
    wide = torch.zeros(rows, dim + 64, dtype=torch.bfloat16, device=dev)
    wide[:, :dim] = yd
    out, h2 = ops.adaln_residual(stream, wide[:, :dim], gd, (sd, td), 1e-6, x_out=stream)
    torch.cuda.synchronize()
    assert out.data_ptr() == stream.data_ptr()
    want_x, want_h = dit.adaln_residual(x, y, gate, scale, shift, 1e-6)
    assert torch.equal(stream.view(rows, dim).cpu(), want_x)
    assert _h_close(h2.view(rows, dim).cpu(), want_h, shift)[0]


def test_rejects_unsupported_shapes(dev):
    from flashmap_amd import ops

    x = torch.zeros(4, 12, dtype=torch.bfloat16, device=dev)
    v = torch.zeros(12, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="multiple of 8"):
        ops.adaln_residual(x, x, v, (v, v), 1e-6)
    x16 = torch.zeros(4, 16, dtype=torch.bfloat16, device=dev)
    v16 = torch.zeros(16, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="one per channel"):
        ops.adaln_residual(x16, x16, v16[:8], (v16, v16), 1e-6)
