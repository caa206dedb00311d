"""The load-time folds (flashmap_amd/fold.py, restating flashmap/vllm/fold.py), pinned by
the identities that define them, in float64 on the CPU:

- fold_noise: ``rsqrt(z^2 @ lambda/H + eps) * (z @ M^T) + b`` equals the unfolded
  ``x_embed(noise_norm(z @ A))`` for any z, and ``A`` factors ``E^T E`` with ``A A^T``
  diagonal (so ``z @ A`` has the covariance of ``x0 @ E``);
- fold_head: one GEMM with the folded weight and bias equals the DiT head followed by the
  LM head, over all rows or a row subset;
- timestep_embedding: the closed form; quantize_fp8_per_channel: the round trip."""

import math

import torch

from flashmap_amd import fold


def _e(v, h, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(v, h, generator=g, dtype=torch.float64).to(dtype)


def test_noise_factor_factors_the_gram_matrix():
    e = _e(300, 24, 0)
    a, lam = fold.noise_factor(e, chunk=64)
    gram = e.T @ e  # the fold accumulates E^T E in float32, as the reference does
    tol = 1e-6 * float(gram.abs().max())
    assert torch.allclose(a.T @ a, gram, rtol=0, atol=tol)
    assert torch.allclose(a @ a.T, torch.diag(lam), rtol=0, atol=tol)
    assert (lam >= 0).all()


def test_folded_noise_equals_the_unfolded_read_out():
    v, h, d, eps = 300, 24, 16, 1e-6
    e = _e(v, h, 1)
    g = torch.Generator().manual_seed(2)
    w = 0.5 + torch.rand(h, generator=g, dtype=torch.float64)
    wx = torch.randn(d, h, generator=g, dtype=torch.float64) * 0.1
    bx = torch.randn(d, generator=g, dtype=torch.float64)
    m, lam_h = fold.fold_noise(e, w, wx)
    a, _ = fold.noise_factor(e)
    z = torch.randn(7, h, generator=g, dtype=torch.float64)
    y = z @ a
    unfolded = (w * y / torch.sqrt(y.pow(2).mean(-1, keepdim=True) + eps)) @ wx.T + bx
    folded = torch.rsqrt((z * z) @ lam_h.double() + eps)[:, None] * (z @ m.double().T) + bx
    assert torch.allclose(folded, unfolded, rtol=1e-5, atol=1e-6)  # lam_h is float32
    assert m.dtype == e.dtype and lam_h.dtype == torch.float32 and m.shape == (d, h)


def test_folded_head_equals_head_then_lm_head():
    g = torch.Generator().manual_seed(3)
    v, h, d = 500, 32, 24
    lm = torch.randn(v, h, generator=g)
    hw, hb = torch.randn(h, d, generator=g), torch.randn(h, generator=g)
    x = torch.randn(9, d, generator=g)
    w, b = fold.fold_head(lm, hw, hb, chunk=128)
    want = (x.double() @ hw.double().T + hb.double()) @ lm.double().T
    assert torch.allclose(torch.nn.functional.linear(x, w, b).double(), want, rtol=1e-4, atol=1e-3)
    rows = torch.tensor([5, 0, 499, 17])
    wr, br = fold.fold_head(lm, hw, hb, rows=rows, chunk=3)
    assert torch.allclose(wr, w[rows], rtol=1e-5, atol=1e-5) and torch.allclose(br, b[rows], rtol=1e-5, atol=1e-5)


def test_timestep_embedding_closed_form_and_fp8_round_trip():
    t = torch.tensor([0.0, 0.25, 900.0])
    emb = fold.timestep_embedding(t, 8)
    f = torch.tensor([10000.0 ** (-i / 4) for i in range(4)], dtype=torch.float64)
    want = torch.cat([torch.cos(t.double()[:, None] * f), torch.sin(t.double()[:, None] * f)], -1)
    assert emb.shape == (3, 8) and torch.allclose(emb.double(), want, atol=1e-4)
    wt = torch.randn(6, 40, generator=torch.Generator().manual_seed(4))
    q, s = fold.quantize_fp8_per_channel(wt)
    assert q.shape == (40, 6) and s.shape == (6, 1)
    back = q.t().float() * s
    assert ((back - wt).abs() <= 0.07 * wt.abs().amax(1, keepdim=True)).all()
    assert math.isclose(float(q.t().float().abs().amax()), 448.0)
