"""fm_block_attn_paged_static, the attention entry point that allocates nothing (its
split-KV scratch is the library's static per-GPU array), against fm_block_attn_paged on
the same inputs: identical bits, since both run the same kernels on the same grid. Two
calls in a row, the second with a smaller batch (the array keeps the first call's
contents), with the query prologue and with the step plan; and a call whose scratch would
not fit the array fails with FM_ERR_WORKSPACE before anything is launched."""

import pytest
import torch

from _inputs import check_close, paged_layout
from oracle import attention as ref

pytestmark = pytest.mark.gpu

D, PAGE, K_ROWS = 128, 16, 16


def _case(dev, batch, hq, hkv, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g)
    bt, total = paged_layout(lens.tolist(), PAGE, g)
    cache = torch.randn(total, hkv, PAGE, 2 * D, generator=g).bfloat16()
    q = torch.randn(batch * K_ROWS, hq, D, generator=g).bfloat16()
    table = ref.rope_table(hi + K_ROWS + 1, D, 1e6)
    pos = torch.cat([int(n) + torch.arange(K_ROWS) for n in lens])
    cu = torch.arange(batch + 1, dtype=torch.int32) * K_ROWS
    return dict(lens=lens, bt=bt, cache=cache, q=q, table=table, pos=pos, cu=cu, hi=hi)


def _both(dev, c, with_plan):
    from flashmap_amd import ops

    w = torch.ones(D, device=dev)
    pro = ops.Prologue(w, ops.rope_from_table(c["table"].to(dev)), c["pos"].to(dev), 1e-6)
    lens = c["lens"].to(dev, torch.int32)
    args = (c["q"].to(dev), c["cache"].to(dev), c["cu"].to(dev), lens, c["bt"].to(dev), K_ROWS, c["hi"], D ** -0.5)
    plan = ops.attention_plan(lens) if with_plan else None
    want = ops.block_attention_paged(*args, prologue=pro, plan=plan)
    out = torch.full_like(want, float("nan"))
    got = ops.block_attention_paged_static(*args, prologue=pro, plan=plan, out=out)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    return got, want


def test_static_scratch_matches_workspace_call_twice(dev):
    print("static scratch: C3-like batch 64, then batch 5", flush=True)
    big = _case(dev, 64, 32, 8, 256, 8192, 3)
    got, want = _both(dev, big, with_plan=True)
    assert torch.equal(got, want)
    b = 7  # one sequence against the oracle
    n = int(big["lens"][b])
    k, v = ref.gather_vllm(big["cache"], big["bt"], n, b)
    qn = ref.rms_norm_rope_vllm(big["q"][b * K_ROWS:(b + 1) * K_ROWS], torch.ones(D), big["table"],
                                big["pos"][b * K_ROWS:(b + 1) * K_ROWS], 1e-6)
    check_close(got[b * K_ROWS:(b + 1) * K_ROWS].cpu(), ref.attention(qn.float().transpose(0, 1), k, v).transpose(0, 1))
    small = _case(dev, 5, 32, 8, 1, 700, 4)  # smaller input, the array still holds the first call's data
    got, want = _both(dev, small, with_plan=False)
    assert torch.equal(got, want)


def test_static_scratch_too_small_raises(dev):
    from flashmap_amd import _native, ops

    limit = _native.lib().fm_static_scratch_bytes()
    assert limit == 32 << 20
    batch, hq, hkv = 600, 32, 8  # 4800 units of 64 rows: ~90 MB of partials
    lens = torch.full((batch,), 64, dtype=torch.int32, device=dev)
    bt = torch.arange(batch * 4, dtype=torch.int32, device=dev).view(batch, 4)
    cache = torch.zeros(batch * 4, hkv, PAGE, 2 * D, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(batch * K_ROWS, hq, D, dtype=torch.bfloat16, device=dev)
    cu = torch.arange(batch + 1, dtype=torch.int32, device=dev) * K_ROWS
    out = torch.zeros_like(q)
    with pytest.raises(_native.NativeError, match="static scratch") as e:
        ops.block_attention_paged_static(q, cache, cu, lens, bt, K_ROWS, 64, D ** -0.5, out=out)
    assert e.value.code == _native.FM_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert (out == 0).all()  # nothing was launched
