"""Pins of the oracle's QK-RMSNorm (+ RoPE) (a2/a3): a float64 restatement with the
reference's rounding points (scale rounded to bf16, product rounded to bf16) and the
unit-RMS invariant. Dropping the scale rounding or the mean (vs. sum) fails here."""

import torch

from oracle import attention as ref


def _closed_form(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xd = x.double()
    r = 1.0 / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    scale = (w.double() * r).float().bfloat16()  # rounded to x's dtype before the multiply
    return (xd * scale.double()).bfloat16()


def test_rms_norm_matches_float64_closed_form():
    g = torch.Generator().manual_seed(0)
    for d in [64, 128]:
        x = (torch.randn(257, d, generator=g) * 3).bfloat16()
        w = torch.rand(d, generator=g) + 0.5
        got = ref.rms_norm(x, w, 1e-6)
        want = _closed_form(x, w, 1e-6)
        # fp32 vs fp64 accumulation of the mean may move a value by one bf16 step
        diff = (got.float() - want.float()).abs()
        ulp = want.float().abs() * 2.0 ** -7 + 1e-30
        assert bool((diff <= ulp).all())
        assert (diff == 0).float().mean().item() > 0.97


def test_scale_is_rounded_before_the_multiply():
    # one channel, weight chosen so that w * r is not a bf16 number
    x = torch.tensor([[3.0, 4.0]]).bfloat16()
    w = torch.tensor([1.0 / 3.0, 1.0])
    got = ref.rms_norm(x, w, 0.0)
    r = 1.0 / (12.5 ** 0.5)
    s0 = torch.tensor(w[0].item() * r).bfloat16().double().item()
    assert got[0, 0].item() == torch.tensor(3.0 * s0).bfloat16().item()


def test_unit_rms_at_unit_weight():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(64, 128, generator=g) * 10).bfloat16()
    y = ref.rms_norm(x, torch.ones(128), 1e-6).double()
    rms = y.pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-2)


def test_norm_then_rope_float64():
    """rms_norm_rope_vllm == float64 rotation of the float64 closed-form norm, to bf16."""
    g = torch.Generator().manual_seed(2)
    d, tokens, heads = 64, 9, 3
    x = torch.randn(tokens, heads, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(512, d, 1e6)
    pos = torch.randint(0, 512, (tokens,), generator=g)
    got = ref.rms_norm_rope_vllm(x, w, table, pos, 1e-6).double()
    n = _closed_form(x, w, 1e-6).double()
    ang = pos.double()[:, None] * ref.inv_freq(d, 1e6).double()
    c, s = ang.cos()[:, None, :], ang.sin()[:, None, :]
    n1, n2 = n.unflatten(-1, (-1, 2)).unbind(-1)
    want = torch.stack([n1 * c - n2 * s, n2 * c + n1 * s], -1).flatten(-2)
    assert (got - want).abs().max().item() <= 2.0 ** -7 * want.abs().max().item() + 1e-6


def test_sglang_prologue_equals_vllm_prologue():
    g = torch.Generator().manual_seed(3)
    d = 128
    x = torch.randn(2, 16, 8, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    pos = torch.randint(0, 1000, (2, 16), generator=g)
    freqs = ref.rope_freqs(pos, d, 1e6)
    table = ref.rope_table(1000, d, 1e6)
    a = ref.rms_norm_rope_sglang(x, w, freqs, 1e-6)
    b = ref.rms_norm_rope_vllm(x.reshape(32, 8, d), w, table, pos.reshape(32), 1e-6).reshape(2, 16, 8, d)
    assert torch.equal(a, b)
