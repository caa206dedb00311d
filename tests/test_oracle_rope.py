"""Pins of the oracle's RoPE (a1): closed forms and invariants, independent of the
oracle's own formulas. A swapped sign, a half-split instead of interleaved pairs, or a
wrong frequency exponent each fails one of these."""

import math

import numpy as np
import torch

from oracle import attention as ref


def test_inv_freq_closed_form():
    for d, theta in [(64, 1e4), (128, 1e6), (128, 5e5)]:
        got = ref.inv_freq(d, theta).double()
        want = torch.tensor([theta ** (-(2.0 * i) / d) for i in range(d // 2)], dtype=torch.float64)
        assert torch.allclose(got, want, rtol=2e-7, atol=0)
        assert got[0] == 1.0 and bool((got[1:] < got[:-1]).all())


def test_rotation_of_each_pair_float64():
    """Pair (x[2i], x[2i+1]) -> (x0 c - x1 s, x1 c + x0 s): a 2x2 rotation by +angle."""
    g = torch.Generator().manual_seed(0)
    d = 16
    x = torch.randn(3, d, generator=g)
    ang = torch.rand(3, d // 2, generator=g, dtype=torch.float64) * 6.0
    got = ref.apply_rope(x, ang.cos().float(), ang.sin().float()).double()
    xd = x.double()
    for r in range(3):
        for i in range(d // 2):
            c, s = math.cos(ang[r, i]), math.sin(ang[r, i])
            x0, x1 = xd[r, 2 * i].item(), xd[r, 2 * i + 1].item()
            assert abs(got[r, 2 * i].item() - (x0 * c - x1 * s)) < 1e-5
            assert abs(got[r, 2 * i + 1].item() - (x1 * c + x0 * s)) < 1e-5


def test_quarter_turn_moves_unit_vectors():
    # angle pi/2 on every pair: (1, 0) -> (0, 1) and (0, 1) -> (-1, 0)
    x = torch.tensor([[1.0, 0.0, 0.0, 1.0]])
    c = torch.zeros(1, 2)
    s = torch.ones(1, 2)
    assert torch.equal(ref.apply_rope(x, c, s), torch.tensor([[0.0, 1.0, -1.0, 0.0]]))


def test_position_zero_is_identity_in_bf16():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 5, 4, 128, generator=g).bfloat16()
    cos, sin = ref.rope_tables(torch.zeros(2, 5, dtype=torch.long), 128, 1e6)
    assert torch.equal(ref.apply_rope(x, cos, sin), x)


def test_pair_norm_preserved():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 7, 1, 64, generator=g)
    pos = torch.randint(0, 100000, (4, 7), generator=g)
    cos, sin = ref.rope_tables(pos, 64, 1e6)
    y = ref.apply_rope(x, cos, sin)
    n0 = x.double().unflatten(-1, (-1, 2)).pow(2).sum(-1)
    n1 = y.double().unflatten(-1, (-1, 2)).pow(2).sum(-1)
    assert torch.allclose(n0, n1, rtol=1e-5, atol=1e-6)


def test_dot_product_depends_on_offset_only():
    g = torch.Generator().manual_seed(3)
    d = 64
    q = torch.randn(d, generator=g).double()
    k = torch.randn(d, generator=g).double()

    def rot(v, p):
        f = ref.inv_freq(d, 1e4).double() * p
        v1, v2 = v.unflatten(-1, (-1, 2)).unbind(-1)
        return torch.stack([v1 * f.cos() - v2 * f.sin(), v2 * f.cos() + v1 * f.sin()], -1).flatten()

    base = rot(q, 17) @ rot(k, 5)
    for shift in [1, 100, 4096]:
        assert abs((rot(q, 17 + shift) @ rot(k, 5 + shift)).item() - base.item()) < 1e-9


def test_table_formats_agree():
    d, theta, n = 128, 1e6, 300
    pos = torch.arange(n)
    cos, sin = ref.rope_tables(pos[None], d, theta)
    table = ref.rope_table(n, d, theta)
    assert torch.equal(table[..., 0], cos[0, :, 0])
    assert torch.equal(table[..., 1], sin[0, :, 0])
    assert torch.equal(ref.rope_freqs(pos, d, theta), table)
    cat = ref.rope_cat_table(n, d, theta)
    assert torch.equal(cat[:, : d // 2], table[..., 0]) and torch.equal(cat[:, d // 2:], table[..., 1])


def test_rope_descriptors_address_the_tables():
    """The host-side rope descriptors (row/pair strides, sin address) read the same
    (cos, sin) values as the table formats they wrap (CPU tensors, read by address)."""
    import ctypes

    from flashmap_amd import ops

    d, n = 64, 50
    table = ref.rope_table(n, d, 1e6)
    cat = ref.rope_cat_table(n, d, 1e6)
    cos, sin = table[..., 0].contiguous(), table[..., 1].contiguous()
    rng = np.random.default_rng(0)
    for desc in [ops.rope_from_table(table), ops.rope_from_cat(cat), ops.rope_from_split(cos, sin)]:
        assert desc.rows == n
        cbase = desc.cos.data_ptr()
        for _ in range(25):
            r, i = int(rng.integers(n)), int(rng.integers(d // 2))
            j = r * desc.row_stride + i * desc.pair_stride
            assert ctypes.c_float.from_address(cbase + 4 * j).value == table[r, i, 0].item()
            assert ctypes.c_float.from_address(desc.sin_ptr + 4 * j).value == table[r, i, 1].item()


def test_rotation_without_rounding_rounds_to_apply_rope():
    """rotate_f32 (the fp8 writers' unrounded rotation) is apply_rope before its rounding,
    and agrees with float64 on the same pairs."""
    g = torch.Generator().manual_seed(9)
    y = torch.randn(5, 3, 64, generator=g).bfloat16()
    ang = torch.rand(5, 1, 32, generator=g) * 6.3
    cos, sin = ang.cos(), ang.sin()
    got = ref.rotate_f32(y, cos, sin)
    assert got.dtype == torch.float32
    assert torch.equal(got.bfloat16(), ref.apply_rope(y, cos, sin))
    e, o = y[..., 0::2].double(), y[..., 1::2].double()
    c, s = cos.double(), sin.double()
    assert torch.allclose(got[..., 0::2].double(), e * c - o * s, atol=1e-5)
    assert torch.allclose(got[..., 1::2].double(), o * c + e * s, atol=1e-5)
