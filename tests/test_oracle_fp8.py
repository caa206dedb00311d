"""Pins the fp8 (OCP e4m3) parts of the oracle: the quantizer against a brute-force
nearest-code search, the fp8 pool writer's norm rounding against a float64
restatement, and both fp8 writers by dequantized round trips against the bf16 key
projection (flashmap/vllm/kernels.py:276-299, flashmap/sglang/kernels.py:283-357)."""

import math

import torch

from _inputs import gen
from oracle import attention as ref

CODES = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double()
FINITE = [(c, float(v)) for c, v in enumerate(CODES.tolist()) if math.isfinite(v)]


def _nearest_code(x: float) -> int:
    """Nearest finite e4m3 value, ties to the even code (even mantissa), saturating."""
    x = max(-448.0, min(448.0, x))
    best = min(FINITE, key=lambda cv: (abs(cv[1] - x), cv[0] & 1, cv[0]))
    d = abs(best[1] - x)
    ties = [c for c, v in FINITE if abs(v - x) == d]
    if len(ties) > 1:  # ties to even mantissa; +0 / -0 by the sign of x
        even = [c for c in ties if c & 1 == 0]
        if len(even) > 1:
            even = [c for c in even if (c >> 7) == (1 if math.copysign(1, x) < 0 else 0)] or even
        return even[0]
    return best[0]


def test_to_e4m3_is_nearest_code_ties_to_even_saturating():
    g = gen(1)
    xs = torch.cat([
        torch.randn(3000, generator=g) * 3,
        torch.randn(500, generator=g) * 200,
        torch.rand(300, generator=g) * 0.01,
        torch.tensor([448.0, 449.0, 464.0, 470.0, 1000.0, -1000.0, 0.0, 2 ** -10, 3 * 2 ** -10, 1.0625, 1.1875,
                      -1.0625, 0.0009765625, 240.0, 248.0]),
    ])
    # exact midpoints between neighbouring codes
    pos = sorted(v for _, v in FINITE if v > 0)
    mids = torch.tensor([(a + b) / 2 for a, b in zip(pos[:40], pos[1:41])] + [(a + b) / 2 for a, b in zip(pos[-20:], pos[-19:])])
    xs = torch.cat([xs, mids, -mids])
    got = ref.to_e4m3(xs).view(torch.uint8).tolist()
    want = [_nearest_code(float(x)) for x in xs.tolist()]
    assert got == want


def test_sglang_fp8_norm_rounds_once():
    g = gen(2)
    k = torch.randn(64, 128, generator=g).bfloat16() * 2
    w = torch.rand(128, generator=g) + 0.5
    got = ref.norm_sglang_fp8(k, w, 1e-6)
    kd = k.double()
    inv = 1.0 / torch.sqrt((kd * kd).mean(-1, keepdim=True) + 1e-6)
    want = (kd * inv * w.double()).to(torch.bfloat16)
    # float32 evaluation of the same expression: equal up to a last-bit flip of the bf16 rounding
    diff = (got.float() - want.float()).abs()
    assert (got == want).float().mean() > 0.99
    assert (diff <= want.float().abs() * 2 ** -7 + 1e-30).all()
    # and it is not the bf16 paths' rounding
    assert (got != ref.rms_norm(k, w, 1e-6)).any()


def _rope(d, n, theta=1e6):
    return ref.rope_table(n, d, theta)


def test_vllm_fp8_writer_round_trip_and_skip():
    g = gen(3)
    tokens, layers, heads, d, page = 9, 2, 4, 64, 4
    kv = torch.randn(tokens, layers, 2, heads, d, generator=g).bfloat16()
    pos = torch.randint(0, 100, (tokens,), generator=g)
    slots = torch.randperm(16, generator=g)[:tokens].long()
    slots[3] = -1
    kn = torch.rand(layers, d, generator=g) + 0.5
    table = _rope(d, 128)
    scales = torch.tensor([[0.5, 2.0], [1.5, 0.25]])
    caches = [torch.zeros(4, heads, page, 2 * d, dtype=torch.float8_e4m3fn) for _ in range(layers)]
    ref.write_context_kv_vllm_fp8(kv, pos, slots, kn, table, caches, page, 1e-6, scales)
    cos, sin = table[pos][..., 0][:, None], table[pos][..., 1][:, None]
    for t in range(tokens):
        s = int(slots[t])
        for l in range(layers):
            blk, tok = divmod(s, page) if s >= 0 else (None, None)
            if s < 0:
                continue
            want_k = ref.rotate_f32(ref.rms_norm(kv[t, l, 0], kn[l], 1e-6), cos[t], sin[t])
            got_k = caches[l][blk, :, tok, :d].float() * scales[l, 0]
            got_v = caches[l][blk, :, tok, d:].float() * scales[l, 1]
            # half an e4m3 step: relative 2^-4 for normals, 2^-10 absolute at the bottom
            assert ((got_k - want_k).abs() <= want_k.abs() * 2 ** -4 + 2 ** -10 * scales[l, 0]).all()
            want_v = kv[t, l, 1].float()
            assert ((got_v - want_v).abs() <= want_v.abs() * 2 ** -4 + 2 ** -10 * scales[l, 1]).all()
    # exactly the live tokens' slots were written (the skipped token's stays zero)
    for c in caches:
        written = (c.view(torch.uint8).reshape(4, heads, page, 2 * d) != 0).any(-1).any(1)  # (blocks, page)
        assert int(written.sum()) == tokens - 1


def test_pool_fp8_writer_round_trip_and_commit_lens():
    g = gen(4)
    tokens, layers, heads, d = 8, 2, 2, 128
    kv_size = heads * d
    kv = torch.randn(tokens, layers * 2 * kv_size, generator=g).bfloat16()
    pos = torch.randint(0, 60, (tokens,), generator=g)
    locs = torch.arange(tokens) * 2 + 1
    kn = torch.rand(layers, d, generator=g) + 0.5
    cat = ref.rope_cat_table(64, d, 1e6)
    kb = [torch.zeros(20, heads, d, dtype=torch.float8_e4m3fn) for _ in range(layers)]
    vb = [torch.zeros(20, heads, d, dtype=torch.float8_e4m3fn) for _ in range(layers)]
    commit = torch.tensor([3, 4])  # two rows of width 4: token 3 is uncommitted
    ref.write_context_kv_pool_fp8(kv, kb, vb, kn, cat, pos, locs, layers, kv_size, d, 1e-6, k_scale=0.75,
                                  v_scale=1.25, commit_lens=commit, locs_row_width=4)
    half = d // 2
    for t in range(tokens):
        loc = int(locs[t])
        for l in range(layers):
            if t == 3:
                assert kb[l][loc].view(torch.uint8).sum() == 0
                continue
            k = kv[t, l * 2 * kv_size:l * 2 * kv_size + kv_size].view(heads, d)
            want = ref.rotate_f32(ref.norm_sglang_fp8(k, kn[l], 1e-6), cat[pos[t], :half], cat[pos[t], half:])
            got = kb[l][loc].float() * 0.75
            assert ((got - want).abs() <= want.abs() * 2 ** -4 + 2 ** -10 * 0.75).all()


def test_query_quantization_per_head():
    g = gen(5)
    q = (torch.randn(3, 16, 4, 64, generator=g) * torch.tensor([0.1, 1.0, 10.0, 300.0])[None, None, :, None]).bfloat16()
    q8, scale = ref.quantize_query_per_head(q)
    # each (request, head)'s largest |q| becomes 448 exactly
    assert torch.equal(q8.float().abs().amax(dim=(1, 3)), torch.full((3, 4), 448.0))
    want = q.float().abs().amax(dim=(1, 3)) / 448.0
    assert torch.equal(scale, want)
    deq = q8.float() * scale[:, None, :, None]
    assert ((deq - q.float()).abs() <= q.float().abs() * 2 ** -4 + scale[:, None, :, None] * 2 ** -10).all()


def test_fp8_attention_is_attention_on_dequantized_operands():
    g = gen(6)
    bs, t, hq, hkv, d, page = 2, 16, 4, 2, 64, 8
    lens = [13, 21]
    cache = ref.to_e4m3(torch.randn(6, hkv, page, 2 * d, generator=g) * 2)
    bt = torch.tensor([[3, 0, 5], [1, 4, 2]], dtype=torch.int32)
    q8 = ref.to_e4m3(torch.randn(bs * t, hq, d, generator=g) * 2)
    cu = torch.tensor([0, t, 2 * t], dtype=torch.int32)
    desc = torch.rand(3, bs, hkv, generator=g) + 0.25
    got = ref.block_attention_paged_vllm_fp8(q8, cache, cu, torch.tensor(lens), bt, 0.125, desc)
    # the same from float64 tensors dequantized by hand
    for b in range(bs):
        k, v = ref.gather_vllm(cache.float().double(), bt.numpy(), lens[b], b)
        k = k * desc[1, b].double()[:, None, None]
        v = v * desc[2, b].double()[:, None, None]
        q = q8[b * t:(b + 1) * t].float().double().transpose(0, 1) * desc[0, b].double().repeat_interleave(2)[:, None, None]
        kk, vv = k.repeat_interleave(2, 0), v.repeat_interleave(2, 0)
        want = torch.softmax(q @ kk.transpose(-1, -2) * 0.125, -1) @ vv
        assert torch.allclose(got[b * t:(b + 1) * t].double(), want.transpose(0, 1), atol=1e-5)
