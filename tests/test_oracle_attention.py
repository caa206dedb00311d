"""Pins of the oracle's attention (a5/a6/a7), its split/merge (the LSE combine) and its
paged gathers: float64 brute force on tiny shapes and the invariants the mathematics
fixes. A transposed operand, a wrong scale, a GQA map of h % G instead of h // G, a
merge weight of exp(lse) without the max shift or an off-by-one page index each fails
one of these."""

import math

import numpy as np
import torch

from _inputs import paged_layout, token_pool_from_contig, vllm_cache_from_contig
from oracle import attention as ref


def _brute(q, k, v, scale):
    """Per-row float64 loops: q (Hq, T, D), k/v (Hkv, L, D)."""
    hq, t_, d = q.shape
    hkv, n, _ = k.shape
    out = torch.zeros(hq, t_, d, dtype=torch.float64)
    for h in range(hq):
        kh = h // (hq // hkv)
        for t in range(t_):
            s = [sum(q[h, t, j].item() * k[kh, p, j].item() for j in range(d)) * scale for p in range(n)]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            for j in range(d):
                out[h, t, j] = sum(e[p] * v[kh, p, j].item() for p in range(n)) / z
    return out


def test_attention_float64_brute_force_gqa():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(4, 3, 8, generator=g)
    k = torch.randn(2, 5, 8, generator=g)
    v = torch.randn(2, 5, 8, generator=g)
    want = _brute(q, k, v, 8 ** -0.5)
    got = ref.attention(q, k, v)
    assert (got.double() - want).abs().max().item() < 1e-5


def test_probabilities_sum_to_one_and_single_key():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, 4, 16, generator=g)
    k = torch.randn(2, 9, 16, generator=g)
    ones = torch.ones(2, 9, 16)
    assert torch.allclose(ref.attention(q, k, ones), torch.ones(2, 4, 16), atol=1e-6)
    v1 = torch.randn(2, 1, 16, generator=g)
    out = ref.attention(q, k[:, :1], v1)
    assert torch.allclose(out, v1.expand(2, 4, 16), atol=1e-7)


def test_key_permutation_invariance():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(4, 16, 32, generator=g)
    k = torch.randn(4, 40, 32, generator=g)
    v = torch.randn(4, 40, 32, generator=g)
    perm = torch.randperm(40, generator=g)
    assert torch.allclose(ref.attention(q, k, v), ref.attention(q, k[:, perm], v[:, perm]), atol=1e-6)


def test_gqa_equals_mha_on_repeated_kv():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(8, 16, 32, generator=g)
    k = torch.randn(2, 30, 32, generator=g)
    v = torch.randn(2, 30, 32, generator=g)
    rep_k = k.repeat_interleave(4, dim=0)
    rep_v = v.repeat_interleave(4, dim=0)
    assert torch.equal(ref.attention(q, k, v), ref.attention(q, rep_k, rep_v))
    # head h reads KV head h // 4: query head 5 attends to KV head 1 only
    only = ref.attention(q[5:6], k[1:2], v[1:2])
    assert torch.allclose(ref.attention(q, k, v)[5:6], only, atol=1e-6)


def test_default_scale_is_inverse_sqrt_head_dim():
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, 2, 64, generator=g) for _ in range(3))
    assert torch.equal(ref.attention(q, k, v), ref.attention(q, k, v, 0.125))


def test_lse_is_float64_logsumexp():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 3, 16, generator=g)
    k = torch.randn(2, 11, 16, generator=g)
    v = torch.randn(2, 11, 16, generator=g)
    _, lse = ref.attention_lse(q, k, v)
    s = (q.double() @ k.double().transpose(-1, -2)) * 0.25
    assert torch.allclose(lse.double(), torch.logsumexp(s, -1), atol=1e-5)


def test_merge_of_splits_equals_unsplit():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(4, 16, 64, generator=g)
    k = torch.randn(1, 200, 64, generator=g) * 3
    v = torch.randn(1, 200, 64, generator=g)
    want = ref.attention(q, k, v)
    for cuts in [[0, 200], [0, 37, 200], [0, 1, 64, 65, 199, 200], [0, 100, 100, 200]]:
        outs, lses = [], []
        for a, b in zip(cuts[:-1], cuts[1:]):
            o, l = ref.attention_lse(q, k[:, a:b], v[:, a:b])
            outs.append(o)
            lses.append(l)
        assert torch.allclose(ref.lse_merge(outs, lses), want, atol=2e-6), cuts


def test_merge_weights_are_shift_invariant():
    # large lse values (exp overflows without the max shift) merge to a convex combination
    o1, o2 = torch.full((1, 4), 1.0), torch.full((1, 4), 3.0)
    l1, l2 = torch.tensor([1000.0]), torch.tensor([1000.0 + math.log(3.0)])
    got = ref.lse_merge([o1, o2], [l1, l2])
    assert torch.allclose(got, torch.full((1, 4), 2.5), atol=1e-5)


def test_contig_seqlens_truncate_and_empty_is_zero():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(3, 16, 4, 32, generator=g)
    k = torch.randn(3, 2, 50, 32, generator=g)
    v = torch.randn(3, 2, 50, 32, generator=g)
    lens = torch.tensor([50, 17, 0])
    out = ref.block_attention_contig(q, k, v, lens)
    want1 = ref.attention(q[1].transpose(0, 1), k[1, :, :17], v[1, :, :17]).transpose(0, 1)
    assert torch.equal(out[1], want1)
    assert torch.equal(out[2], torch.zeros(16, 4, 32))


def test_vllm_paged_equals_contiguous_under_block_permutation():
    g = torch.Generator().manual_seed(8)
    b, hq, hkv, d, t = 3, 4, 2, 32, 5
    lens = torch.tensor([40, 16, 1])
    k = torch.randn(b, hkv, 40, d, generator=g).bfloat16()
    v = torch.randn(b, hkv, 40, d, generator=g).bfloat16()
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    for page in [16, 8]:
        bt, total = paged_layout(lens, page, g)
        cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
        cu = torch.arange(b + 1) * t
        got = ref.block_attention_paged_vllm(q.reshape(b * t, hq, d), cache, cu, lens, bt)
        want = ref.block_attention_contig(q, k, v, lens)
        assert torch.equal(got.reshape(b, t, hq, d), want)


def test_token_paged_equals_contiguous():
    g = torch.Generator().manual_seed(9)
    b, hq, hkv, d, t = 2, 4, 4, 16, 3
    lens = torch.tensor([21, 5])
    k = torch.randn(b, hkv, 21, d, generator=g).bfloat16()
    v = torch.randn(b, hkv, 21, d, generator=g).bfloat16()
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    kb, vb, pt = token_pool_from_contig(k, v, lens, g)
    got = ref.block_attention_token_paged(q, kb, vb, lens, pt)
    assert torch.equal(got, ref.block_attention_contig(q, k, v, lens))


def test_vllm_gather_slots_closed_form():
    rng = np.random.default_rng(10)
    bt = rng.integers(0, 1000, size=(4, 9)).astype(np.int32)
    for page in [1, 16, 32]:
        for b in range(4):
            n = min(9 * page, 70)
            idx = ref.vllm_gather_slots(bt, n, page, b)
            for p in range(n):
                assert idx[p, 0] == bt[b, p // page] and idx[p, 1] == p % page
