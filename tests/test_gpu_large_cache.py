"""Caches past 4 GiB. A vLLM layer cache or an SGLang token pool of a long-context server
easily exceeds 2^32 bytes; the kernels form page and pool-row offsets in 64 bits. Here every
page (pool row) the calls touch lies past byte 2^32 of a 5 GiB cache (pool), where a 32-bit
offset would wrap:

- the context writers' rows there against the oracle writers on a compact copy (the bar of
  the writer tests: >= 99 % of the elements equal, the rest within 2e-2);
- attention over those pages (rows) against the float32 oracle on the gathered K/V
  (max-abs 2e-2, mean-abs 2e-3), bf16 and e4m3.
"""

import pytest
import torch

from _inputs import check_close, gen
from flashmap_amd import ops
from oracle import attention as ref

pytestmark = pytest.mark.gpu

GIB = 1 << 30
HKV, HQ, D, PAGE, K_ROWS = 8, 32, 128, 16, 16


def _past_4gib(count: int, unit_bytes: int, total: int, g) -> torch.Tensor:
    """``count`` distinct indices of units (pages, pool rows) lying wholly past byte 2^32,
    among ``total`` units of ``unit_bytes``."""
    first = -(-(4 * GIB) // unit_bytes)
    assert first + count <= total
    return (first + torch.randperm(total - first, generator=g)[:count]).long()


def _positions(lens):
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    seq = torch.cat([torch.full((int(n),), b) for b, n in enumerate(lens)])
    return pos, seq


def _check_rows(got, want):
    assert (got == want).float().mean().item() > 0.99
    assert (got.float() - want.float()).abs().max().item() <= 2e-2


def test_vllm_cache_past_4gib(dev):
    print("vLLM layer cache of 5 GiB, pages past 2^32", flush=True)
    g = gen(120)
    block_bytes = HKV * PAGE * 2 * D * 2
    blocks = 5 * GIB // block_bytes
    lens = torch.tensor([300, 1000, 57, 700])
    npages = [-(-int(n) // PAGE) for n in lens]
    ids = _past_4gib(sum(npages), block_bytes, blocks, g)
    bt = torch.zeros(len(lens), max(npages), dtype=torch.int32)
    compact = torch.zeros_like(bt)  # the same pages numbered 0 .. in a compact copy
    o = 0
    for b, n in enumerate(npages):
        bt[b, :n] = ids[o:o + n].int()
        compact[b, :n] = torch.arange(o, o + n, dtype=torch.int32)
        o += n
    pos, seq = _positions(lens)
    slots = bt[seq, pos // PAGE].long() * PAGE + pos % PAGE
    slots_c = compact[seq, pos // PAGE].long() * PAGE + pos % PAGE
    kv = torch.randn(len(pos), 1, 2, HKV, D, generator=g).bfloat16()
    kn = torch.rand(1, D, generator=g) + 0.5
    table = ref.rope_table(1024, D, 1e6)
    cache = torch.zeros(blocks, HKV, PAGE, 2 * D, dtype=torch.bfloat16, device=dev)
    ptrs = torch.tensor([cache.data_ptr()], dtype=torch.int64, device=dev)
    ops.write_context_kv(kv.to(dev), pos.to(dev), slots.to(dev), kn.to(dev), ops.rope_from_table(table.to(dev)), ptrs,
                         (cache.stride(0), cache.stride(1), cache.stride(2), D), PAGE, 1e-6)
    want = [torch.zeros(sum(npages), HKV, PAGE, 2 * D, dtype=torch.bfloat16)]
    ref.write_context_kv_vllm(kv, pos, slots_c, kn, table, want, PAGE, 1e-6)
    torch.cuda.synchronize()
    written = cache[ids.to(dev)].cpu()  # the used pages in compact order
    _check_rows(written, want[0])

    q = torch.randn(len(lens) * K_ROWS, HQ, D, generator=g).bfloat16()
    cu = torch.arange(0, len(lens) * K_ROWS + 1, K_ROWS, dtype=torch.int32)
    out = ops.block_attention_paged(q.to(dev), cache, cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), K_ROWS,
                                    int(lens.max()), D ** -0.5)
    torch.cuda.synchronize()
    got = out.cpu().float()
    for b, n in enumerate(lens.tolist()):
        rows = written[compact[b, :npages[b]].long()].float().transpose(1, 2).reshape(-1, HKV, 2 * D)[:n]
        k, v = rows[..., :D].transpose(0, 1), rows[..., D:].transpose(0, 1)
        qb = q[b * K_ROWS:(b + 1) * K_ROWS].float().transpose(0, 1)
        check_close(got[b * K_ROWS:(b + 1) * K_ROWS], ref.attention(qb, k, v, D ** -0.5).transpose(0, 1))


def test_vllm_fp8_cache_past_4gib(dev):
    print("vLLM e4m3 layer cache of 5 GiB, pages past 2^32", flush=True)
    g = gen(121)
    block_bytes = HKV * PAGE * 2 * D
    blocks = 5 * GIB // block_bytes
    lens = torch.tensor([512, 33, 1400])
    npages = [-(-int(n) // PAGE) for n in lens]
    ids = _past_4gib(sum(npages), block_bytes, blocks, g)
    bt = torch.zeros(len(lens), max(npages), dtype=torch.int32)
    o = 0
    for b, n in enumerate(npages):
        bt[b, :n] = ids[o:o + n].int()
        o += n
    pages = ref.to_e4m3(torch.randn(sum(npages), HKV, PAGE, 2 * D, generator=g))
    cache = torch.zeros(blocks, HKV, PAGE, 2 * D, dtype=torch.uint8, device=dev)
    cache[ids.to(dev)] = pages.view(torch.uint8).to(dev)
    q8 = ref.to_e4m3(torch.randn(len(lens) * K_ROWS, HQ, D, generator=g))
    cu = torch.arange(0, len(lens) * K_ROWS + 1, K_ROWS, dtype=torch.int32)
    desc = torch.rand(3, len(lens), HKV, generator=g) + 0.25
    out = ops.block_attention_paged_fp8(q8.to(dev), cache, cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), K_ROWS,
                                        int(lens.max()), D ** -0.5, descales=desc.to(dev))
    torch.cuda.synchronize()
    compact_bt = torch.zeros_like(bt)
    o = 0
    for b, n in enumerate(npages):
        compact_bt[b, :n] = torch.arange(o, o + n, dtype=torch.int32)
        o += n
    want = ref.block_attention_paged_vllm_fp8(q8, pages, cu, lens, compact_bt, D ** -0.5, desc)
    check_close(out.cpu().float(), want)


def test_token_pool_past_4gib(dev):
    print("SGLang token pools of 5 GiB each, rows past 2^32", flush=True)
    g = gen(122)
    row_bytes = HKV * D * 2
    pool = 5 * GIB // row_bytes
    lens = torch.tensor([300, 1000, 57, 700])
    rows = _past_4gib(int(lens.sum()), row_bytes, pool, g)
    pt = torch.zeros(len(lens), int(lens.max()), dtype=torch.int32)
    pt_c = torch.zeros_like(pt)  # the same rows numbered 0 .. in a compact copy
    o = 0
    for b, n in enumerate(lens.tolist()):
        pt[b, :n] = rows[o:o + n].int()
        pt_c[b, :n] = torch.arange(o, o + n, dtype=torch.int32)
        o += n
    pos, seq = _positions(lens)
    kv_size = HKV * D
    kv = torch.randn(len(pos), 2 * kv_size, generator=g).bfloat16()
    kn = torch.rand(1, D, generator=g) + 0.5
    cat = ref.rope_cat_table(1024, D, 1e6)
    kbuf = torch.zeros(pool, HKV, D, dtype=torch.bfloat16, device=dev)
    vbuf = torch.zeros_like(kbuf)
    meta = torch.tensor([[kbuf.data_ptr(), vbuf.data_ptr(), kbuf.stride(0), vbuf.stride(0)]], dtype=torch.int64,
                        device=dev)
    locs = pt[seq, pos].long()
    ops.write_context_kv_pool(kv.to(dev), meta, kn.to(dev), ops.rope_from_cat(cat.to(dev)), pos.to(dev), locs.to(dev),
                              1, kv_size, D, 1e-6)
    wk = [torch.zeros(len(pos), HKV, D, dtype=torch.bfloat16)]
    wv = [torch.zeros_like(wk[0])]
    ref.write_context_kv_pool(kv, wk, wv, kn, cat, pos, pt_c[seq, pos].long(), 1, kv_size, D, 1e-6)
    torch.cuda.synchronize()
    wrote_k, wrote_v = kbuf[rows.to(dev)].cpu(), vbuf[rows.to(dev)].cpu()  # compact order
    _check_rows(wrote_k, wk[0])
    _check_rows(wrote_v, wv[0])

    q = torch.randn(len(lens), K_ROWS, HQ, D, generator=g).bfloat16()
    out = ops.block_attention_token_paged(q.to(dev), kbuf, vbuf, lens.to(dev, torch.int32), pt.to(dev))
    torch.cuda.synchronize()
    got = out.cpu().float()
    for b, n in enumerate(lens.tolist()):
        k = wrote_k[pt_c[b, :n].long()].float().transpose(0, 1)
        v = wrote_v[pt_c[b, :n].long()].float().transpose(0, 1)
        check_close(got[b], ref.attention(q[b].float().transpose(0, 1), k, v, D ** -0.5).transpose(0, 1))
