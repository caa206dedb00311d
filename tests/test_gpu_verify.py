"""GPU parity of the target verify attention (fm_verify_attention; SplitKVVerify of
flashmap/sglang/verify_attention.py) against the CPU oracle, through the C ABI.

Tolerance (written here, the bar for bf16 outputs): max-abs 2e-2 and mean-abs 2e-3
against the float32 oracle on the same bf16 inputs. The CSR context layout is checked
bit-exactly against the draft path's page-table layout on the same data (same grid, so
the same splits and the same partials).
"""

import pytest
import torch

from _inputs import check_close, gen, verify_case
from oracle import attention as ref

pytestmark = pytest.mark.gpu


def ops():
    from flashmap_amd import ops as o

    return o


def _to(case, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}


def _verify(c, **kw):
    return ops().verify_attention(c["q"], c["k"], c["v"], c["key_buffer"], c["value_buffer"], c["kv_indptr"],
                                  c["kv_indices"], c["custom_mask"], c["mask_indptr"], c["qlen_mask"], **kw)


def _oracle(case, **kw):
    return ref.verify_attention(case["q"], case["k"], case["v"], case["key_buffer"], case["value_buffer"],
                                case["kv_indptr"], case["kv_indices"], case["custom_mask"], case["mask_indptr"],
                                case["qlen_mask"], **kw)


def _contexts(bs, lo, hi, seed, zero_first=False):
    c = torch.randint(lo, hi + 1, (bs,), generator=gen(seed)).tolist()
    if zero_first:
        c[0] = 0
    return c


# id: (bs, L, Hq, Hkv, D, (ctx lo, ctx hi), mask, index dtype, (k_scale, v_scale))
CASES = {
    "gqa4_chain_causal": (4, 17, 32, 8, 128, (0, 700), "causal", torch.int32, (1.0, 1.0)),
    "gqa4_tree_rows_int64": (4, 17, 32, 8, 128, (1, 700), "rows", torch.int64, (1.0, 1.0)),
    "mha_tree_qlen": (3, 17, 16, 16, 128, (1, 500), "qlen", torch.int32, (1.0, 1.0)),
    "gqa5_tree_rows": (3, 17, 40, 8, 128, (0, 400), "rows", torch.int32, (1.0, 1.0)),
    "d64_causal_scales": (5, 8, 8, 2, 64, (0, 300), "causal", torch.int32, (0.5, 2.0)),
    "wide_tree_two_row_groups": (2, 64, 8, 2, 128, (1, 333), "qlen", torch.int64, (1.0, 1.0)),
    "d64_tree_rows_scales": (6, 12, 16, 4, 64, (0, 260), "rows", torch.int64, (1.25, 0.75)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_verify_parity(dev, name):
    bs, length, hq, hkv, d, (lo, hi), mask, idt, (ks, vs) = CASES[name]
    print(f"verify case {name}", flush=True)
    case = verify_case(bs, length, hq, hkv, d, _contexts(bs, lo, hi, 11, zero_first=lo == 0), mask=mask,
                       index_dtype=idt, seed=12)
    got = _verify(_to(case, dev), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    check_close(got.cpu().float(), _oracle(case, k_scale=ks, v_scale=vs))


def test_verify_long_contexts(dev):
    """Contexts of 2k-8k positions (several shares per unit, the stream split evenly)."""
    case = verify_case(6, 17, 32, 8, 128, _contexts(6, 2048, 8192, 13), mask="rows", seed=14)
    got = _verify(_to(case, dev))
    torch.cuda.synchronize()
    check_close(got.cpu().float(), _oracle(case))


def test_verify_no_context_and_blind_rows(dev):
    """Requests without context, rows that see no verify token: zeros exactly where the
    row sees nothing at all, the token-only attention elsewhere."""
    case = verify_case(3, 5, 8, 2, 128, [0, 0, 9], mask="qlen", seed=15)
    mask = case["custom_mask"].clone()
    mask[0:5] = False  # request 0, token 0: nothing
    mask[25 + 10:25 + 15] = False  # request 1, token 2: nothing
    mask[50 + 5:50 + 10] = False  # request 2, token 1: its context only
    case["custom_mask"] = mask
    got = _verify(_to(case, dev)).cpu()
    torch.cuda.synchronize()
    assert torch.count_nonzero(got[0]) == 0 and torch.count_nonzero(got[5 + 2]) == 0
    check_close(got.float(), _oracle(case))


def test_verify_large_batch(dev):
    """More requests than the kernel stages in LDS (sequence metadata by scalar loads)."""
    bs = 1100
    case = verify_case(bs, 4, 8, 2, 64, _contexts(bs, 0, 64, 16), seed=17)
    got = _verify(_to(case, dev))
    torch.cuda.synchronize()
    check_close(got.cpu().float(), _oracle(case))


def test_verify_context_equals_token_paged_draft_path(dev):
    """With every verify token masked out, each row attends to its context alone: the
    draft path's token-paged attention over the same pool rows, given as a page table
    instead of CSR. Same sizes, same grid: bit-identical."""
    bs, length, hq, hkv, d = 5, 17, 32, 8, 128
    ctx = _contexts(bs, 1, 900, 18)
    case = verify_case(bs, length, hq, hkv, d, ctx, mask="qlen", seed=19)
    case["custom_mask"] = torch.zeros_like(case["custom_mask"])
    c = _to(case, dev)
    pool = case["key_buffer"].shape[0]
    got = _verify(c)
    table = torch.zeros(bs, max(ctx), dtype=torch.int32)
    for b in range(bs):
        lo, hi = int(case["kv_indptr"][b]), int(case["kv_indptr"][b + 1])
        table[b, :hi - lo] = case["kv_indices"][lo:hi]
    seqlens = torch.tensor(ctx, dtype=torch.int32)
    want = ops().block_attention_token_paged(c["q"].view(bs, length, hq, d), c["key_buffer"], c["value_buffer"],
                                             seqlens.to(dev), table.to(dev), max_seqlen_k=pool)
    torch.cuda.synchronize()
    assert torch.equal(got.view(bs, length, hq, d).cpu(), want.cpu())


def test_split_kv_verify_extend_arguments(dev):
    """SplitKVVerify with extend_attention_fwd's arguments writes o in place and returns
    True; a case it declines returns False and leaves o untouched."""
    from flashmap_amd.verify_attention import SplitKVVerify

    bs, length, hq, hkv, d = 3, 17, 32, 8, 128
    case = verify_case(bs, length, hq, hkv, d, _contexts(bs, 0, 500, 20), mask="rows", seed=21)
    c = _to(case, dev)
    o = torch.full((bs * length, hq * d), 7.0, dtype=torch.bfloat16, device=dev)
    qo_indptr = torch.arange(0, bs * length + 1, length, dtype=torch.int32, device=dev)
    fwd = SplitKVVerify()
    args = (c["q"], c["k"].view(-1, hkv * d), c["v"].view(-1, hkv * d), o, c["key_buffer"], c["value_buffer"],
            qo_indptr, c["kv_indptr"], c["kv_indices"], c["custom_mask"], True, c["mask_indptr"], length)
    assert fwd(*args, logit_cap=30.0) is False
    assert fwd(*args, sinks=torch.zeros(hq, device=dev)) is False
    assert fwd(*args, k_scale=None) is False
    torch.cuda.synchronize()
    assert bool((o == 7.0).all())
    assert fwd(*args, sm_scale=0.1) is True
    torch.cuda.synchronize()
    check_close(o.view(-1, hq, d).cpu().float(), _oracle(case, sm_scale=0.1))


def test_split_kv_verify_graph_replay(dev):
    """Captured once, replayed over new contexts, queries and masks of the same shapes:
    every replay matches the oracle (only shapes are read on the host)."""
    from flashmap_amd.verify_attention import SplitKVVerify

    bs, length, hq, hkv, d = 4, 9, 16, 4, 128
    fwd = SplitKVVerify()
    fwd.qlen_mask = True

    def make(seed):
        ctx = _contexts(bs, 0, 400, seed)
        case = verify_case(bs, length, hq, hkv, d, ctx, mask="qlen", seed=seed, pool_slack=1700 - sum(ctx))
        return case

    first = make(30)
    c = _to(first, dev)
    indices = torch.zeros(1700, dtype=torch.int32, device=dev)
    n = first["kv_indices"].numel()
    indices[:n] = c["kv_indices"]
    o = torch.empty(bs * length, hq, d, dtype=torch.bfloat16, device=dev)
    qo_indptr = torch.arange(0, bs * length + 1, length, dtype=torch.int32, device=dev)
    args = (c["q"], c["k"], c["v"], o, c["key_buffer"], c["value_buffer"], qo_indptr, c["kv_indptr"], indices,
            c["custom_mask"], True, None, length)
    assert fwd(*args)  # warm-up: the workspace is sized outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert fwd(*args)
    for seed in (31, 32, 33):
        case = make(seed)
        for key in ("q", "k", "v", "key_buffer", "value_buffer", "kv_indptr", "custom_mask"):
            c[key].copy_(case[key].to(dev))
        indices[:case["kv_indices"].numel()].copy_(case["kv_indices"].to(dev))
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay {seed}", flush=True)
        check_close(o.cpu().float(), _oracle(case))
        _ = (c["q"].float() * 2).sum().item()  # eager work between replays
