"""The benchmark configurations at their full sizes on the GPU (C3: 64 x U[256, 8192]; C4:
8 x 32768; C5: GQA 5, 32 x U[1024, 8192]; R8B: MHA 16/16, 64 x U[256, 8192]; vLLM pages of
16; and LONG, 2 x 131072, each unit split over about 32 shares, the combine merging
them in four batches of eight), checked through properties that hold at any size, since the
oracle over a whole batch would take minutes:

- sampled sequences (the shortest, a median one, the longest) against the float32 oracle
  on the same K/V (max-abs 2e-2, mean-abs 2e-3);
- the block table's page order: moving every page elsewhere in the cache and rewriting the
  table accordingly gives the very same bits;
- the split: an odd number of workgroups (other share boundaries, other partials merged)
  stays within the same bar of the default split.
"""

import pytest
import torch

from _inputs import check_close, paged_layout
from flashmap_amd import ops
from oracle import attention as ref

pytestmark = pytest.mark.gpu

CONFIGS = {
    "C3": (64, 32, 8, 256, 8192),
    "C4": (8, 32, 8, 32768, 32768),
    "C5": (32, 40, 8, 1024, 8192),
    "R8B": (64, 16, 16, 256, 8192),
    "LONG": (2, 32, 8, 131072, 131072),
}
K_ROWS, D, PAGE = 16, 128, 16


def _inputs(dev, name, fp8=False):
    batch, hq, hkv, lo, hi = CONFIGS[name]
    g = torch.Generator().manual_seed(7)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g)
    bt, total = paged_layout(lens.tolist(), PAGE, g)
    gd = torch.Generator(device=dev).manual_seed(7)
    cache = torch.randn(total, hkv, PAGE, 2 * D, generator=gd, device=dev)
    q = torch.randn(batch * K_ROWS, hq, D, generator=gd, device=dev)
    if fp8:  # the cache as uint8 bytes (indexing works on them), the queries as e4m3
        cache, q = cache.to(torch.float8_e4m3fn).view(torch.uint8), q.to(torch.float8_e4m3fn)
    else:
        cache, q = cache.bfloat16(), q.bfloat16()
    cu = torch.arange(0, batch * K_ROWS + 1, K_ROWS, dtype=torch.int32, device=dev)
    return lens, bt, cache, q, cu, hi


def _run(q, cache, cu, lens, bt, hi, fp8):
    args = (cu, lens.to(cache.device, torch.int32), bt.to(cache.device), K_ROWS, hi, D ** -0.5)
    if fp8:
        return ops.block_attention_paged_fp8(q, cache, *args)
    return ops.block_attention_paged(q, cache, *args)


def _check_sampled(out, q, cache, lens, bt):
    order = torch.argsort(lens)
    picks = sorted({int(order[0]), int(order[len(order) // 2]), int(order[-1])})
    for b in picks:
        n = int(lens[b])
        pages = bt[b, :(n + PAGE - 1) // PAGE].long().to(cache.device)
        rows = cache[pages]
        rows = rows.view(torch.float8_e4m3fn) if rows.dtype == torch.uint8 else rows
        rows = rows.float().transpose(1, 2).reshape(-1, cache.shape[1], 2 * D)[:n]  # (n, Hkv, 2D)
        k, v = rows[..., :D].transpose(0, 1).cpu(), rows[..., D:].transpose(0, 1).cpu()
        qb = q[b * K_ROWS:(b + 1) * K_ROWS].float().cpu().transpose(0, 1)
        want = ref.attention(qb, k, v, D ** -0.5).transpose(0, 1)
        check_close(out[b * K_ROWS:(b + 1) * K_ROWS].cpu().float(), want)


def _check_permuted(out, q, cache, cu, lens, bt, hi, fp8):
    g = torch.Generator().manual_seed(11)
    perm = torch.randperm(cache.shape[0], generator=g).to(cache.device)
    moved = torch.empty_like(cache)
    moved[perm] = cache  # page i now lives at perm[i]
    bt2 = perm.int().cpu()[bt.long()]
    again = _run(q, moved, cu, lens, bt2, hi, fp8)
    torch.cuda.synchronize()
    assert torch.equal(again, out)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_full_size_bf16(dev, tuning, name):
    print(f"full size {name}", flush=True)
    lens, bt, cache, q, cu, hi = _inputs(dev, name)
    out = _run(q, cache, cu, lens, bt, hi, False)
    torch.cuda.synchronize()
    _check_sampled(out, q, cache, lens, bt)
    _check_permuted(out, q, cache, cu, lens, bt, hi, False)
    tuning("FLASHMAP_SPLITKV_WORKGROUPS", "61")
    split = _run(q, cache, cu, lens, bt, hi, False)
    torch.cuda.synchronize()
    check_close(split.cpu().float(), out.cpu().float())
    assert not torch.equal(split, out)  # the other split did take effect


def test_full_size_c3_e4m3(dev):
    lens, bt, cache, q, cu, hi = _inputs(dev, "C3", fp8=True)
    out = _run(q, cache, cu, lens, bt, hi, True)
    torch.cuda.synchronize()
    _check_sampled(out, q, cache, lens, bt)
    _check_permuted(out, q, cache, cu, lens, bt, hi, True)


def test_full_size_token_pool_drafter_and_verify(dev):
    """C3's contexts in an SGLang token pool at permuted slots: the drafter's token-paged
    call and the verify call (17 chain tokens, causal) on the same pool, each against the
    oracle on sampled requests and bit-identical after the pool's rows move."""
    batch, hq, hkv, lo, hi = CONFIGS["C3"]
    length = 17
    g = torch.Generator().manual_seed(9)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g)
    ctx = int(lens.sum())
    slots = torch.randperm(ctx, generator=g).int()
    pt = torch.zeros(batch, hi, dtype=torch.int32)
    o = 0
    for b in range(batch):
        pt[b, :int(lens[b])] = slots[o:o + int(lens[b])]
        o += int(lens[b])
    gd = torch.Generator(device=dev).manual_seed(9)
    rnd = lambda *shape: torch.randn(*shape, generator=gd, device=dev).bfloat16()
    kb, vb = rnd(ctx, hkv, D), rnd(ctx, hkv, D)
    q = rnd(batch, K_ROWS, hq, D)
    qv, k_ext, v_ext = rnd(batch * length, hq, D), rnd(batch * length, hkv, D), rnd(batch * length, hkv, D)
    indptr = torch.zeros(batch + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(lens, 0)
    lens_d, pt_d, ip_d, idx_d = lens.to(dev, torch.int32), pt.to(dev), indptr.to(dev), slots.to(dev)

    def run(kb_, vb_, pt_, idx_):
        drafter = ops.block_attention_token_paged(q, kb_, vb_, lens_d, pt_)
        verify = ops.verify_attention(qv, k_ext, v_ext, kb_, vb_, ip_d, idx_, None, None, False, max_context=hi)
        torch.cuda.synchronize()
        return drafter, verify

    drafter, verify = run(kb, vb, pt_d, idx_d)
    order = torch.argsort(lens)
    for b in sorted({int(order[0]), int(order[batch // 2]), int(order[-1])}):
        n = int(lens[b])
        rows = pt[b, :n].long().to(dev)
        k, v = kb[rows].float().cpu(), vb[rows].float().cpu()
        want = ref.attention(q[b].float().cpu().transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), D ** -0.5)
        check_close(drafter[b].cpu().float(), want.transpose(0, 1))
        tok = slice(b * length, (b + 1) * length)
        want_v = ref.verify_attention(qv[tok].cpu(), k_ext[tok].cpu(), v_ext[tok].cpu(), kb[rows].cpu(), vb[rows].cpu(),
                                      torch.tensor([0, n], dtype=torch.int32), torch.arange(n), None, None, False)
        check_close(verify[tok].cpu().float(), want_v)
    perm = torch.randperm(ctx, generator=g).to(dev)
    kb2, vb2 = torch.empty_like(kb), torch.empty_like(vb)
    kb2[perm], vb2[perm] = kb, vb  # pool row i now lives at perm[i]
    drafter2, verify2 = run(kb2, vb2, perm.int()[pt_d.long()], perm.int()[idx_d.long()])
    assert torch.equal(drafter2, drafter)
    assert torch.equal(verify2, verify)
