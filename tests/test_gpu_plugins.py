"""GPU parity of the drop-in op layer: the plugin ops registered under the reference
names (``torch.ops.flashmap_vllm.*``, ``torch.ops.flashmap_sglang.*``) and the writers,
end to end through the C ABI, against the oracle. Tolerance as in the kernel tests
(bf16 outputs: max-abs 2e-2, mean-abs 2e-3 of fp32); the writers are bit-exact."""

import pytest
import torch

from _inputs import check_close, gen, paged_layout
from oracle import attention as ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def plugin_ops():
    from flashmap_amd import sglang as fs
    from flashmap_amd import vllm as fv

    fv.register()
    fs.register()
    return torch.ops.flashmap_vllm, torch.ops.flashmap_sglang, fv, fs


def test_vllm_write_then_paged_cross_attention(dev, plugin_ops):
    v, _, fv, _ = plugin_ops
    g = gen(11)
    b, hq, hkv, d, k_rows, page, eps = 5, 8, 2, 128, 16, 16, 1e-6
    lens = torch.tensor([3, 40, 17, 64, 1])
    bt, total = paged_layout(lens, page, g)
    table = ref.rope_table(200, d, 1e6)
    knorm = torch.rand(1, d, generator=g) + 0.5
    # context rows of every sequence, written through the drop-in writer
    toks = int(lens.sum())
    kv = torch.randn(toks, 1, 2, hkv, d, generator=g).bfloat16()
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    slots = torch.cat([bt[i, torch.arange(int(n)) // page].long() * page + torch.arange(int(n)) % page
                       for i, n in enumerate(lens)])
    cache = torch.zeros(total, hkv, page, 2 * d, dtype=torch.bfloat16, device=dev)
    ptrs = torch.tensor([cache.data_ptr()], dtype=torch.int64, device=dev)
    fv.write_context_kv(kv.to(dev), pos.to(dev), slots.to(dev), knorm.to(dev), table.to(dev), ptrs,
                        (cache.stride(0), cache.stride(1), cache.stride(2), d), page, eps)
    want_cache = torch.zeros(total, hkv, page, 2 * d, dtype=torch.bfloat16)
    ref.write_context_kv_vllm(kv, pos, slots, knorm, table, [want_cache], page, eps)
    assert torch.equal(cache.cpu(), want_cache)
    # queries: prologue op then the paged op, with the step's plan
    q = torch.randn(b * k_rows, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    qpos = torch.cat([int(n) + torch.arange(k_rows) for n in lens])
    qn = v.rms_norm_rope(q.to(dev), w.to(dev), table.to(dev), qpos.to(dev), eps)
    cu = (torch.arange(b + 1, dtype=torch.int32) * k_rows).to(dev)
    sk = lens.to(dev, torch.int32)
    plan = fv.cross_attention_schedule(sk)
    out = v.paged_cross_attention(qn, cache, cu, sk, bt.to(dev), plan, None, k_rows, 64, d ** -0.5, 3)
    want_q = ref.rms_norm_rope_vllm(q, w, table, qpos, eps)
    want = ref.block_attention_paged_vllm(want_q, want_cache, cu.cpu(), lens, bt)
    check_close(out, want)
    # without a plan: identical bits
    out2 = v.paged_cross_attention(qn, cache, cu, sk, bt.to(dev), None, None, k_rows, 64, d ** -0.5, 3)
    assert torch.equal(out, out2)


def test_vllm_block_self_attention_op(dev, plugin_ops):
    v, _, _, _ = plugin_ops
    g = gen(12)
    blocks, t, h, d = 6, 16, 4, 128
    qkv = torch.randn(blocks, t, 3, h, d, generator=g).bfloat16()
    qn, kn = torch.rand(d, generator=g) + 0.5, torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(400, d, 1e6)
    pos = torch.randint(0, 400, (blocks * t,), generator=g)
    got = v.block_self_attention(qkv.to(dev), qn.to(dev), kn.to(dev), table.to(dev), pos.to(dev), 1e-6)
    rows = table[pos].view(blocks, t, d // 2, 2)
    want = ref.block_self_attention(qkv, qn, kn, rows[..., 0], rows[..., 1], 1e-6)
    assert got.shape == (blocks * t, h * d)
    check_close(got.view(blocks, t, h, d), want)


def test_sglang_ops_and_pool_write(dev, plugin_ops):
    _, s, _, fs = plugin_ops
    g = gen(13)
    bs, k_rows, hq, hkv, d, eps, layers = 3, 16, 8, 2, 128, 1e-6, 2
    lens = torch.tensor([33, 5, 70])
    pool = int(lens.sum()) + 9
    locs_all = torch.randperm(pool, generator=g)[: int(lens.sum())]
    pt = torch.zeros(bs, int(lens.max()), dtype=torch.int32)
    o = 0
    for b in range(bs):
        pt[b, : int(lens[b])] = locs_all[o:o + int(lens[b])].int()
        o += int(lens[b])
    # pools written through the drop-in fused writer (interleaved RoPE)
    kv_size = hkv * d
    toks = int(lens.sum())
    kv = torch.randn(toks, layers * 2 * kv_size, generator=g).bfloat16()
    knorm = torch.rand(layers, d, generator=g) + 0.5
    cat = ref.rope_cat_table(128, d, 1e6)
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    kbufs = [torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    vbufs = [torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    meta = torch.tensor([[kb.data_ptr(), vb.data_ptr(), kb.stride(0), vb.stride(0)] for kb, vb in zip(kbufs, vbufs)],
                        dtype=torch.int64, device=dev)
    fs.fused_kv_norm_rope_write(kv.to(dev), meta, knorm.to(dev), cat.to(dev), pos.to(dev),
                                locs_all.to(dev), layers, kv_size, d, eps)
    wk = [torch.zeros(pool, hkv, d, dtype=torch.bfloat16) for _ in range(layers)]
    wv = [torch.zeros(pool, hkv, d, dtype=torch.bfloat16) for _ in range(layers)]
    ref.write_context_kv_pool(kv, wk, wv, knorm, cat, pos, locs_all, layers, kv_size, d, eps)
    for l in range(layers):
        assert torch.equal(kbufs[l].cpu(), wk[l]) and torch.equal(vbufs[l].cpu(), wv[l])
    # draft queries: prologue op with per-token freqs, then the token-paged op on layer 1
    q = torch.randn(bs, k_rows, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    qpos = torch.stack([int(n) + torch.arange(k_rows) for n in lens])
    freqs = fs.rope_freqs(qpos.to(dev), d, 1e6)
    qn = s.rms_norm_rope(q.to(dev), w.to(dev), freqs, eps)
    want_q = ref.rms_norm_rope_sglang(q, w, ref.rope_freqs(qpos, d, 1e6), eps)
    assert (qn.cpu().float() - want_q.float()).abs().max().item() <= 2 ** -7 * want_q.float().abs().max().item()
    sl = lens.to(dev, torch.int32)
    out = s.paged_cross_attention(qn, kbufs[1], vbufs[1], sl, pt.to(dev), fs.cross_attention_schedule(sl))
    want = ref.block_attention_token_paged(want_q, wk[1], wv[1], lens, pt)
    check_close(out, want)


def test_sglang_block_self_attention_op(dev, plugin_ops):
    _, s, _, _ = plugin_ops
    g = gen(14)
    blocks, t, h, d = 4, 16, 4, 64
    qkv = torch.randn(blocks, t, 3, h, d, generator=g).bfloat16()
    qn, kn = torch.rand(d, generator=g) + 0.5, torch.rand(d, generator=g) + 0.5
    pos = torch.randint(0, 1000, (blocks, t), generator=g)
    freqs = ref.rope_freqs(pos, d, 1e6)
    got = s.block_self_attention(qkv.to(dev), qn.to(dev), kn.to(dev), freqs.to(dev), 1e-6)
    want = ref.block_self_attention(qkv, qn, kn, freqs[..., 0], freqs[..., 1], 1e-6)
    check_close(got, want)


def test_vllm_fp8_write_then_paged_cross_attention(dev, plugin_ops):
    """The fp8 flow of the vLLM plugin (flashmap/vllm/model.py:863-873): an e4m3 cache
    written with per-layer scales, the query quantized by the caller with its static
    scale, the attention op given descales (3, requests, heads)."""
    v, _, fv, _ = plugin_ops
    g = gen(21)
    b, h, d, k_rows, page, eps = 4, 8, 128, 16, 16, 1e-6
    lens = torch.tensor([33, 100, 7, 64])
    bt, total = paged_layout(lens, page, g)
    table = ref.rope_table(200, d, 1e6)
    knorm = torch.rand(1, d, generator=g) + 0.5
    toks = int(lens.sum())
    kv = torch.randn(toks, 1, 2, h, d, generator=g).bfloat16()
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    slots = torch.cat([bt[i, torch.arange(int(n)) // page].long() * page + torch.arange(int(n)) % page
                       for i, n in enumerate(lens)])
    scales = torch.tensor([[0.8, 1.25]])
    cache = torch.zeros(total, h, page, 2 * d, dtype=torch.uint8, device=dev)
    ptrs = torch.tensor([cache.data_ptr()], dtype=torch.int64, device=dev)
    fv.write_context_kv(kv.to(dev), pos.to(dev), slots.to(dev), knorm.to(dev), table.to(dev), ptrs,
                        (cache.stride(0), cache.stride(1), cache.stride(2), d), page, eps, scales=scales.to(dev))
    q = torch.randn(b * k_rows, h, d, generator=g).bfloat16()
    q_scale = 0.05
    q8 = (q.float() / q_scale).to(torch.float8_e4m3fn)
    descales = torch.stack([torch.tensor(q_scale), scales[0, 0], scales[0, 1]])[:, None, None].expand(3, b, h)
    cu = (torch.arange(b + 1, dtype=torch.int32) * k_rows).to(dev)
    sk = lens.to(dev, torch.int32)
    out = v.paged_cross_attention(q8.to(dev), cache, cu, sk, bt.to(dev), fv.cross_attention_schedule(sk),
                                  descales.to(dev), k_rows, 128, d ** -0.5, 3)
    want_cache = torch.zeros(total, h, page, 2 * d, dtype=torch.float8_e4m3fn)
    ref.write_context_kv_vllm_fp8(kv, pos, slots, knorm, table, [want_cache], page, eps, scales)
    want = ref.block_attention_paged_vllm_fp8(q8, want_cache, cu.cpu(), lens, bt, d ** -0.5, descales.contiguous())
    check_close(out, want)


def test_sglang_fp8_pool_write_then_attention(dev, plugin_ops):
    """kv_norm_rope_write_fp8 into e4m3 pools, then flashmap_sglang::paged_cross_attention_fp8
    (flashmap/sglang/model.py:154-181, flashmap/sglang/kernels.py:336-357)."""
    _, s, _, fs = plugin_ops
    g = gen(22)
    bs, k_rows, h, d, eps = 3, 16, 4, 128, 1e-6
    lens = torch.tensor([50, 17, 90])
    pool = int(lens.sum()) + 20
    kv_size = h * d
    toks = int(lens.sum())
    kv = torch.randn(toks, 2 * kv_size, generator=g).bfloat16()
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    locs = torch.randperm(pool, generator=g)[:toks].long()
    knorm = torch.rand(1, d, generator=g) + 0.5
    cat = ref.rope_cat_table(256, d, 1e6)
    kb = torch.zeros(pool, h, d, dtype=torch.uint8, device=dev)
    vb = torch.zeros(pool, h, d, dtype=torch.uint8, device=dev)
    meta = torch.tensor([[kb.data_ptr(), vb.data_ptr(), kb.stride(0), vb.stride(0)]], dtype=torch.int64, device=dev)
    fs.kv_norm_rope_write_fp8(kv.to(dev), meta, knorm.to(dev), cat.to(dev), pos.to(dev), locs.to(dev), 1, kv_size,
                              d, eps)
    pt = torch.zeros(bs, int(lens.max()), dtype=torch.int32)
    o = 0
    for i in range(bs):
        pt[i, :int(lens[i])] = locs[o:o + int(lens[i])].int()
        o += int(lens[i])
    q = torch.randn(bs, k_rows, h, d, generator=g).bfloat16()
    sl = lens.to(dev, torch.int32)
    out = s.paged_cross_attention_fp8(q.to(dev), kb.view(torch.float8_e4m3fn), vb.view(torch.float8_e4m3fn), sl,
                                      pt.to(dev), fs.cross_attention_schedule(sl))
    wk = [torch.zeros(pool, h, d, dtype=torch.float8_e4m3fn)]
    wv = [torch.zeros(pool, h, d, dtype=torch.float8_e4m3fn)]
    ref.write_context_kv_pool_fp8(kv, wk, wv, knorm, cat, pos, locs, 1, kv_size, d, eps)
    want = ref.block_attention_token_paged_fp8(q, wk[0], wv[0], lens, pt)
    check_close(out.float(), want)
