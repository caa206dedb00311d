"""GPU parity of one-launch attention over vLLM's virtual context-cache layout
(fm_block_attn_paged_runs through flashmap_amd.context_cache.cross_attention_by_segments
and the plugin op flashmap_vllm::paged_cross_attention_runs).

Each layer of each case is checked four ways: against the oracle's per-run attention
(max-abs 2e-2, mean-abs 2e-3 of float32); bit-exact against the per-layer paged kernel on
a cache that holds the same heads (the same kernel and splits, other addresses);
against per-run calls of the paged op as attend_by_segments makes them (same bar); and
the plugin op equal to the direct call."""

import pytest
import torch

from _inputs import check_close, gen, paged_layout
from flashmap_amd import context_cache as cc
from flashmap_amd import ops
from oracle import attention as ref

pytestmark = pytest.mark.gpu

# layers, KV heads per layer, heads per cache, query heads per KV head, head_dim, page
CASES = [
    (3, 5, 3, 1, 128, 16),   # runs 3+2, 1+3+1, 2+3
    (2, 8, 3, 4, 128, 16),   # GQA 4; runs 3+3+2, 1+3+3+1
    (3, 12, 5, 1, 64, 8),    # page 8 (no 16-position page blocks); up to 4 runs
    (2, 20, 8, 1, 128, 16),  # the reference's example: 20 heads in caches of 8
]


def _case(layers, heads, hpc, group, d, page, seed):
    g = gen(seed)
    lens = torch.randint(1, 400, (4,), generator=g)
    lens[1] = 0
    bt, total = paged_layout(lens.tolist(), page, g)
    plan = cc.ContextCachePlan(layers, heads, -(-layers * heads // hpc), hpc, True, "")
    caches = [torch.randn(total, hpc, page, 2 * d, generator=g).bfloat16() for _ in range(plan.num_caches)]
    k_rows = 16
    q = torch.randn(4 * k_rows, group * heads, d, generator=g).bfloat16()
    cu = torch.arange(0, 4 * k_rows + 1, k_rows, dtype=torch.int32)
    return plan, caches, q, cu, lens.int(), bt


@pytest.mark.parametrize("layers,heads,hpc,group,d,page", CASES)
def test_runs_attention(dev, layers, heads, hpc, group, d, page):
    print(f"runs layers={layers} heads={heads} hpc={hpc} group={group} d={d} page={page}", flush=True)
    plan, caches, q, cu, lens, bt = _case(layers, heads, hpc, group, d, page, 100 + heads + hpc)
    gc = [c.to(dev) for c in caches]
    qd, cud, lensd, btd = q.to(dev), cu.to(dev), lens.to(dev), bt.to(dev)
    sched = ops.attention_plan(lensd)
    scale = d ** -0.5
    for layer, runs in enumerate(plan.segments):
        got = cc.cross_attention_by_segments(qd, gc, runs, cud, lensd, btd, 16, 400, scale, scheduler_metadata=sched)
        # the layer's heads in a per-layer cache, by the closed-form (cache, slot) map
        own = torch.stack([gc[c][:, s] for c, s in (plan.locate(layer, h) for h in range(heads))], dim=1)
        single = ops.block_attention_paged(qd, own, cud, lensd, btd, 16, 400, scale, plan=sched)
        per_run = cc.attend_by_segments(
            qd, gc, runs, lambda qp, cp, n: ops.block_attention_paged(qp, cp, cud, lensd, btd, 16, 400, scale))
        torch.cuda.synchronize()
        assert len(runs) > 1 or heads <= hpc
        assert torch.equal(got, single), f"layer {layer}: runs != per-layer cache"
        want = ref.block_attention_paged_segments(q, caches, runs, cu, lens, bt, scale)
        check_close(got, want)
        check_close(per_run, want)
        assert torch.count_nonzero(got[16:32]) == 0  # the empty context


def test_runs_with_fused_prologue_and_plugin_op(dev):
    from flashmap_amd import vllm as fv

    layers, heads, hpc, group, d, page = 2, 8, 3, 4, 128, 16
    plan, caches, q, cu, lens, bt = _case(layers, heads, hpc, group, d, page, 7)
    gc = [c.to(dev) for c in caches]
    qd, cud, lensd, btd = q.to(dev), cu.to(dev), lens.to(dev), bt.to(dev)
    g = gen(8)
    w = (torch.rand(d, generator=g) + 0.5).to(dev)
    table = ref.rope_table(512, d, 1e6).to(dev)
    pos = torch.randint(0, 512, (q.shape[0],), generator=g).to(dev)
    pro = ops.Prologue(w, ops.rope_from_table(table), pos, 1e-6)
    runs = plan.segments[1]
    fused = cc.cross_attention_by_segments(qd, gc, runs, cud, lensd, btd, 16, 400, 0.1, prologue=pro)
    normed = ops.rms_norm_rope(qd, w, ops.rope_from_table(table), pos, 1e-6)
    plain = cc.cross_attention_by_segments(normed, gc, runs, cud, lensd, btd, 16, 400, 0.1)
    fv.register()
    flat = [x for run in runs for x in run]
    op = torch.ops.flashmap_vllm.paged_cross_attention_runs(normed, gc, flat, cud, lensd, btd, None, 16, 400, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(fused, plain)
    assert torch.equal(op, plain)


def test_more_runs_than_one_launch_takes(dev):
    """A layer of 10 runs (20 heads in caches of 2) is attended in launches of at most
    ops.MAX_RUNS runs over consecutive head ranges: each range against the oracle, and
    the whole layer equal to per-run calls' concatenation within the same bar."""
    from flashmap_amd import vllm as fv

    layers, heads, hpc, group, d, page = 2, 20, 2, 2, 64, 16
    print(f"runs layers={layers} heads={heads} hpc={hpc} group={group} (10 runs per layer)", flush=True)
    plan, caches, q, cu, lens, bt = _case(layers, heads, hpc, group, d, page, 31)
    gc = [c.to(dev) for c in caches]
    qd, cud, lensd, btd = q.to(dev), cu.to(dev), lens.to(dev), bt.to(dev)
    scale = d ** -0.5
    fv.register()
    for layer, runs in enumerate(plan.segments):
        assert len(runs) > ops.MAX_RUNS
        got = cc.cross_attention_by_segments(qd, gc, runs, cud, lensd, btd, 16, 400, scale)
        flat = [x for run in runs for x in run]
        op = torch.ops.flashmap_vllm.paged_cross_attention_runs(qd, gc, flat, cud, lensd, btd, None, 16, 400, scale)
        torch.cuda.synchronize()
        want = ref.block_attention_paged_segments(q, caches, runs, cu, lens, bt, scale)
        check_close(got, want)
        assert torch.equal(op, got)
        assert torch.count_nonzero(got[16:32]) == 0
