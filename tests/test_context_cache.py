"""The virtual context-cache layout (flashmap/vllm/context_cache.py): the oracle's runs
pinned by the invariants that fix them, its per-run attention pinned against the
per-layer paged oracle, and the host plan (flashmap_amd.context_cache) checked against
both and against the reference's layout rules."""

import itertools

import pytest
import torch

from _inputs import gen, paged_layout
from flashmap_amd import context_cache as cc
from flashmap_amd import ops
from oracle import attention as ref


def _shapes():
    for layers, heads, hpc in itertools.product((1, 2, 3, 6), (1, 3, 5, 8, 20), (1, 2, 3, 5, 8, 16)):
        yield layers, heads, hpc


def test_oracle_segments_are_fixed_by_their_invariants():
    for layers, heads, hpc in _shapes():
        for layer, runs in enumerate(ref.context_segments(layers, heads, hpc)):
            # the runs cover heads 0 .. heads-1 in order
            assert runs[0][3] == 0 and sum(r[2] for r in runs) == heads
            for a, b in zip(runs, runs[1:]):
                assert b[3] == a[3] + a[2]
                assert b[0] != a[0]  # maximal: neighbours lie in different caches
            # every head at the closed-form (cache, slot)
            for cache, slot, count, first in runs:
                for i in range(count):
                    assert (cache, slot + i) == divmod(layer * heads + first + i, hpc)


def test_plan_segments_and_maps_match_the_oracle():
    for layers, heads, hpc in _shapes():
        plan = cc.ContextCachePlan(layers, heads, -(-layers * heads // hpc), hpc, hpc != heads, "")
        assert plan.segments == ref.context_segments(layers, heads, hpc)
        for l, h in itertools.product(range(layers), range(heads)):
            assert (plan.cache[l][h], plan.slot[l][h]) == divmod(l * heads + h, hpc)


def test_plan_rules():
    kw = dict(hybrid=True, target_attention_layers=16, target_kv_heads=4, target_head_size=256, bf16_cache=True)
    # the reference's example: 6 layers x 20 heads of 128 next to 16 layers of 4 x 256
    plan = cc.plan_context_cache(6, 20, 128, **kw, mode="auto")
    assert plan.virtual and plan.num_caches == 16 and plan.heads_per_cache == 8
    assert plan.segments[0] == [(0, 0, 8, 0), (1, 0, 8, 8), (2, 0, 4, 16)]
    assert plan.segments[1] == [(2, 4, 4, 0), (3, 0, 8, 4), (4, 0, 8, 12)]
    per_layer = lambda p: (not p.virtual and p.num_caches == 6 and p.heads_per_cache == 20
                           and p.segments == [[(l, 0, 20, 0)] for l in range(6)])
    assert per_layer(cc.plan_context_cache(6, 20, 128, **kw, mode="layers"))
    assert per_layer(cc.plan_context_cache(6, 20, 128, **{**kw, "hybrid": False}, mode="auto"))
    assert cc.plan_context_cache(6, 20, 128, **{**kw, "hybrid": False}, mode="virtual").virtual
    assert per_layer(cc.plan_context_cache(6, 20, 128, **{**kw, "bf16_cache": False}, mode="virtual"))
    assert per_layer(cc.plan_context_cache(6, 20, 128, **{**kw, "target_head_size": 200}, mode="virtual"))
    assert per_layer(cc.plan_context_cache(6, 20, 128, **{**kw, "target_attention_layers": 14}, mode="virtual"))
    assert per_layer(cc.plan_context_cache(6, 20, 128, **{**kw, "target_attention_layers": 0}, mode="virtual"))
    with pytest.raises(ValueError):
        cc.plan_context_cache(6, 20, 128, **kw, mode="bogus")


def test_plan_mode_from_environment(monkeypatch):
    kw = dict(hybrid=True, target_attention_layers=16, target_kv_heads=4, target_head_size=256, bf16_cache=True)
    monkeypatch.setenv("FLASHMAP_CONTEXT_CACHE", "layers")
    assert not cc.plan_context_cache(6, 20, 128, **kw).virtual
    monkeypatch.setenv("FLASHMAP_CONTEXT_CACHE", "auto")
    assert cc.plan_context_cache(6, 20, 128, **kw).virtual


def _virtual_case(seed, layers, heads, hpc, group, d, page, lens):
    g = gen(seed)
    bt, total = paged_layout(lens, page, g)
    ncache = -(-layers * heads // hpc)
    caches = [torch.randn(total, hpc, page, 2 * d, generator=g).bfloat16() for _ in range(ncache)]
    k_rows = 16
    q = torch.randn(len(lens) * k_rows, group * heads, d, generator=g).bfloat16()
    cu = torch.arange(0, len(lens) * k_rows + 1, k_rows, dtype=torch.int32)
    return caches, bt, q, cu, torch.tensor(lens, dtype=torch.int32)


def _per_layer_cache(caches, layer, heads, hpc):
    """The layer's heads gathered into one (blocks, heads, page, 2D) cache by the
    closed-form (cache, slot) map."""
    return torch.stack([caches[c][:, s] for c, s in (divmod(layer * heads + h, hpc) for h in range(heads))], dim=1)


@pytest.mark.parametrize("layers,heads,hpc,group", [(2, 3, 2, 1), (3, 5, 3, 2), (2, 4, 4, 1)])
def test_oracle_segment_attention_equals_per_layer_cache(layers, heads, hpc, group):
    caches, bt, q, cu, lens = _virtual_case(layers * 10 + heads, layers, heads, hpc, group, 32, 4, [9, 0, 23])
    for layer, runs in enumerate(ref.context_segments(layers, heads, hpc)):
        got = ref.block_attention_paged_segments(q, caches, runs, cu, lens, bt, 0.2)
        want = ref.block_attention_paged_vllm(q, _per_layer_cache(caches, layer, heads, hpc), cu, lens, bt, 0.2)
        assert torch.allclose(got, want, atol=1e-6)


def test_attend_by_segments_slices_like_the_reference():
    layers, heads, hpc, group = 3, 5, 3, 2
    caches, bt, q, cu, lens = _virtual_case(7, layers, heads, hpc, group, 32, 4, [5, 17])
    calls = []

    def attend(q_part, c_part, count):
        calls.append((tuple(q_part.shape), tuple(c_part.shape), count))
        return ref.block_attention_paged_vllm(q_part, c_part, cu, lens, bt, 0.2)

    plan = cc.ContextCachePlan(layers, heads, 5, hpc, True, "")
    for layer in range(layers):
        calls.clear()
        got = cc.attend_by_segments(q, caches, plan.segments[layer], attend)
        want = ref.block_attention_paged_segments(q, caches, plan.segments[layer], cu, lens, bt, 0.2)
        assert torch.equal(got, want)
        assert [c[2] for c in calls] == [r[2] for r in plan.segments[layer]]
        assert all(qs[1] == group * n and cs[1] == n for qs, cs, n in calls)
    # a run that covers the whole query and its whole cache passes both unsliced
    seen = []
    cc.attend_by_segments(q[:, :2], [caches[0][:, :1]], [(0, 0, 1, 0)], lambda a, b, n: seen.append((a, b)) or a)
    assert seen[0][0].data_ptr() == q.data_ptr() and seen[0][1].data_ptr() == caches[0].data_ptr()


def test_runs_op_rejects_bad_runs_before_launching():
    c = torch.zeros(2, 4, 4, 64, dtype=torch.bfloat16)
    q = torch.zeros(16, 4, 32, dtype=torch.bfloat16)
    args = (None, torch.zeros(1, dtype=torch.int32), torch.zeros(1, 1, dtype=torch.int32), 16, 4, 0.1)
    with pytest.raises(ValueError, match="at most"):
        ops.block_attention_paged_runs(q, [c] * 9, [(i, 0, 1, i) for i in range(9)], *args)
    with pytest.raises(ValueError, match="continue"):
        ops.block_attention_paged_runs(q, [c, c], [(0, 0, 2, 0), (1, 0, 2, 1)], *args)
    with pytest.raises(ValueError, match="continue"):
        ops.block_attention_paged_runs(q, [c, c], [(0, 3, 2, 0), (1, 0, 2, 2)], *args)
    with pytest.raises(ValueError, match="share"):
        ops.block_attention_paged_runs(q, [c, c[:1]], [(0, 0, 2, 0), (1, 0, 2, 2)], *args)
    with pytest.raises(TypeError):
        ops.block_attention_paged_runs(q, [c.float()], [(0, 0, 4, 0)], *args)
