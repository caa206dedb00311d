"""Pins of the oracle's K-side writers (a4) and block self-attention (a8): write then
read back equals the projected keys / raw values at the written slots, skips are
honoured, and the self-attention composes the pinned norm, rope and attention."""

import torch

from oracle import attention as ref


def test_vllm_writer_round_trip_and_head_mapping():
    g = torch.Generator().manual_seed(0)
    tokens, layers, heads, d, page = 7, 2, 3, 32, 4
    kv = torch.randn(tokens, layers, 2, heads, d, generator=g).bfloat16()
    knorm = torch.rand(layers, d, generator=g) + 0.5
    table = ref.rope_table(64, d, 1e6)
    pos = torch.randint(0, 64, (tokens,), generator=g)
    slots = torch.tensor([0, 5, -1, 9, 3, 12, 1])
    hpc = 2  # 6 global heads over 3 caches of 2 heads
    caches = [torch.zeros(4, hpc, page, 2 * d).bfloat16() for _ in range(3)]
    ref.write_context_kv_vllm(kv, pos, slots, knorm, table, caches, page, 1e-6, heads_per_cache=hpc)
    rows = table[pos]
    cos, sin = rows[..., 0][:, None, :], rows[..., 1][:, None, :]
    written = torch.zeros(4, page, dtype=torch.bool)
    for t in range(tokens):
        s = int(slots[t])
        if s < 0:
            continue
        blk, tok = divmod(s, page)
        written[blk, tok] = True
        for l in range(layers):
            keys = ref.project_keys(kv[t, l, 0][None], knorm[l], cos[t:t + 1], sin[t:t + 1], 1e-6)[0]
            for h in range(heads):
                gh = l * heads + h
                c, hs = gh // hpc, gh % hpc
                assert torch.equal(caches[c][blk, hs, tok, :d], keys[h])
                assert torch.equal(caches[c][blk, hs, tok, d:], kv[t, l, 1, h])
    for c in caches:  # nothing else was touched
        rest = c.transpose(1, 2)[~written]  # (unwritten slots, hpc, 2D)
        assert torch.equal(rest, torch.zeros_like(rest))


def test_pool_writer_skips_negative_and_uncommitted():
    g = torch.Generator().manual_seed(1)
    tokens, layers, heads, d = 6, 2, 2, 16
    kv_size = heads * d
    kv = torch.randn(tokens, layers * 2 * kv_size, generator=g).bfloat16()
    knorm = torch.rand(layers, d, generator=g) + 0.5
    cat = ref.rope_cat_table(32, d, 1e6)
    pos = torch.arange(tokens) + 3
    locs = torch.tensor([4, 1, 8, -1, 2, 6])
    commit = torch.tensor([2, 3])  # rows of width 3: token 2 (col 2 of row 0) is uncommitted
    kb = [torch.zeros(10, heads, d).bfloat16() for _ in range(layers)]
    vb = [torch.zeros(10, heads, d).bfloat16() for _ in range(layers)]
    ref.write_context_kv_pool(kv, kb, vb, knorm, cat, pos, locs, layers, kv_size, d, 1e-6, commit, 3)
    half = d // 2
    rows = cat[pos.long()]
    for t in range(tokens):
        committed = t % 3 < int(commit[t // 3]) and int(locs[t]) >= 0
        for l in range(layers):
            k = kv[t, l * 2 * kv_size:l * 2 * kv_size + kv_size].view(heads, d)
            v = kv[t, l * 2 * kv_size + kv_size:(l + 1) * 2 * kv_size].view(heads, d)
            if not committed:
                continue
            loc = int(locs[t])
            want = ref.project_keys(k[None], knorm[l], rows[t:t + 1, None, :half], rows[t:t + 1, None, half:], 1e-6)[0]
            assert torch.equal(kb[l][loc], want) and torch.equal(vb[l][loc], v)
    for l in range(layers):  # token 2's slot (uncommitted) and slot 0 (nobody's) stay empty
        assert kb[l][8].abs().sum() == 0 and vb[l][8].abs().sum() == 0
        assert kb[l][0].abs().sum() == 0


def test_block_self_attention_composition_float64():
    g = torch.Generator().manual_seed(2)
    blocks, t, h, d = 2, 5, 3, 16
    qkv = torch.randn(blocks, t, 3, h, d, generator=g).bfloat16()
    qn, kn = torch.rand(d, generator=g) + 0.5, torch.rand(d, generator=g) + 0.5
    ang = torch.rand(blocks, t, d // 2, generator=g) * 3
    got = ref.block_self_attention(qkv, qn, kn, ang.cos(), ang.sin(), 1e-6)
    q = ref.apply_rope(ref.rms_norm(qkv[:, :, 0], qn, 1e-6), ang.cos()[:, :, None], ang.sin()[:, :, None])
    k = ref.apply_rope(ref.rms_norm(qkv[:, :, 1], kn, 1e-6), ang.cos()[:, :, None], ang.sin()[:, :, None])
    v = qkv[:, :, 2]
    s = torch.einsum("bthd,bshd->bhts", q.double(), k.double()) * d ** -0.5
    want = torch.einsum("bhts,bshd->bthd", s.softmax(-1), v.double())
    assert (got.double() - want).abs().max().item() < 1e-5
