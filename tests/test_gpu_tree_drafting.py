"""Tree drafting's cross-attention on the GPU: a request's n_cand candidate blocks sit
side by side in the query axis, ``(requests, n_cand * K, heads, head_dim)``
(flashmap/sglang/model.py:866-873, 1031-1040), so each request's context is attended by
n_cand * K rows at once (up to G * n_cand * K rows per KV head, several units of 128).

Checked against the float32 oracle (max-abs 2e-2, mean-abs 2e-3), bf16 and e4m3 pools;
and each candidate's rows equal to a call with that candidate alone within the same bar
(the rows are independent: non-causal attention, no mask)."""

import pytest
import torch

from _inputs import check_close, gen
from flashmap_amd import sglang as fs
from oracle import attention as ref

pytestmark = pytest.mark.gpu


def _pool(lens, hkv, d, g, dtype=torch.bfloat16):
    pool = int(sum(int(n) for n in lens)) + 11
    perm = torch.randperm(pool, generator=g)
    pt = torch.zeros(len(lens), max(int(max(lens)), 1), dtype=torch.int32)
    o = 0
    for b, n in enumerate(lens):
        pt[b, :int(n)] = perm[o:o + int(n)].int()
        o += int(n)
    if dtype == torch.float8_e4m3fn:
        kb = ref.to_e4m3(torch.randn(pool, hkv, d, generator=g))
        vb = ref.to_e4m3(torch.randn(pool, hkv, d, generator=g))
    else:
        kb = torch.randn(pool, hkv, d, generator=g).to(dtype)
        vb = torch.randn(pool, hkv, d, generator=g).to(dtype)
    return kb, vb, pt


@pytest.mark.parametrize("n_cand,hq,hkv", [(2, 16, 16), (8, 16, 16), (32, 16, 16), (8, 32, 8), (32, 32, 8)])
def test_candidates_side_by_side(dev, n_cand, hq, hkv):
    print(f"tree n_cand={n_cand} hq={hq} hkv={hkv}", flush=True)
    g = gen(200 + n_cand + hq)
    requests, k_rows, d = 3, 16, 128
    lens = torch.randint(20, 500, (requests,), generator=g)
    kb, vb, pt = _pool(lens.tolist(), hkv, d, g)
    blocks = torch.randn(requests * n_cand, k_rows, hq, d, generator=g).bfloat16()
    query = blocks.reshape(requests, n_cand * k_rows, hq, d)  # candidate-major per request
    args = (kb.to(dev), vb.to(dev), lens.to(dev, torch.int32), pt.to(dev))
    got = fs.paged_cross_attention(query.to(dev), *args, None)
    # candidate c of every request alone
    c = n_cand // 2
    alone = fs.paged_cross_attention(query[:, c * k_rows:(c + 1) * k_rows].contiguous().to(dev), *args, None)
    torch.cuda.synchronize()
    want = ref.block_attention_token_paged(query, kb, vb, lens, pt)
    check_close(got.cpu().float(), want)
    check_close(alone.cpu().float(), got[:, c * k_rows:(c + 1) * k_rows].cpu().float())


@pytest.mark.parametrize("n_cand", [4, 32])
def test_candidates_side_by_side_fp8_pool(dev, n_cand):
    g = gen(300 + n_cand)
    requests, k_rows, hq, hkv, d = 2, 16, 32, 8, 128
    lens = torch.randint(20, 500, (requests,), generator=g)
    kb, vb, pt = _pool(lens.tolist(), hkv, d, g, torch.float8_e4m3fn)
    query = torch.randn(requests, n_cand * k_rows, hq, d, generator=g).bfloat16()
    got = fs.paged_cross_attention_fp8(query.to(dev), kb.to(dev), vb.to(dev), lens.to(dev, torch.int32),
                                       pt.to(dev), None)
    torch.cuda.synchronize()
    check_close(got.cpu().float(), ref.block_attention_token_paged_fp8(query, kb, vb, lens, pt))
