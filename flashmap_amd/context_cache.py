"""Where a drafter layer's cross-attention context lives in vLLM's paged KV cache, and
attention over it in one launch.

Two layouts (flashmap/vllm/context_cache.py:1-19, 33-117):

- per layer: DiT layer ``l``'s heads are the heads of attention cache ``l``;
- virtual: the DiT's heads, layer-major (global head ``l * heads + h``), are packed into
  as many caches as the target has full-attention layers, each with the target's page
  per token (``target_kv_heads * target_head_size`` elements, i.e. ``heads_per_cache``
  DiT heads). A layer's heads may then span two or more caches.

:func:`plan_context_cache` picks the layout by the reference's rules, and
:class:`ContextCachePlan` maps heads to (cache, slot) and lists each layer's heads as
runs ``(cache, first slot, count, first head)``. :func:`attend_by_segments` keeps the
reference's per-run calling convention; :func:`cross_attention_by_segments` attends to
all of a layer's runs in one kernel launch (``fm_block_attn_paged_runs``).
"""

from __future__ import annotations

import os
from collections.abc import Callable
from dataclasses import dataclass

import torch

from . import ops

__all__ = ["ContextCachePlan", "attend_by_segments", "cross_attention_by_segments", "plan_context_cache"]

# Values of FLASHMAP_CONTEXT_CACHE. "layers": one cache per DiT layer; "virtual": DiT
# heads packed into the target's own caches; "auto": virtual only beside a hybrid target.
MODES = ("auto", "layers", "virtual")


@dataclass(frozen=True)
class ContextCachePlan:
    """``num_caches`` caches of ``heads_per_cache`` heads hold the context of
    ``num_layers`` DiT layers of ``heads`` heads (flashmap/vllm/context_cache.py:33-73)."""

    num_layers: int
    heads: int
    num_caches: int
    heads_per_cache: int
    virtual: bool
    reason: str

    def locate(self, layer: int, head: int) -> tuple[int, int]:
        """(cache, slot) of DiT head ``head`` of layer ``layer``."""
        return divmod(layer * self.heads + head, self.heads_per_cache)

    @property
    def cache(self) -> list[list[int]]:
        return [[self.locate(l, h)[0] for h in range(self.heads)] for l in range(self.num_layers)]

    @property
    def slot(self) -> list[list[int]]:
        return [[self.locate(l, h)[1] for h in range(self.heads)] for l in range(self.num_layers)]

    @property
    def segments(self) -> list[list[tuple[int, int, int, int]]]:
        """Per layer, its heads as runs ``(cache, first slot, count, first head)``: the
        layer's range of global heads cut at the caches' boundaries."""
        out = []
        for layer in range(self.num_layers):
            start = layer * self.heads
            end = start + self.heads
            runs = []
            g = start
            while g < end:
                cache, slot = divmod(g, self.heads_per_cache)
                count = min(end, (cache + 1) * self.heads_per_cache) - g
                runs.append((cache, slot, count, g - start))
                g += count
            out.append(runs)
        return out


def plan_context_cache(
    num_layers: int,
    heads: int,
    head_dim: int,
    *,
    hybrid: bool,
    target_attention_layers: int,
    target_kv_heads: int,
    target_head_size: int,
    bf16_cache: bool,
    mode: str | None = None,
) -> ContextCachePlan:
    """The context layout for a DiT of ``num_layers`` x ``heads`` heads of ``head_dim``
    beside a target with ``target_attention_layers`` full-attention layers of
    ``target_kv_heads`` heads of ``target_head_size`` (flashmap/vllm/context_cache.py:76-117).
    ``mode`` (default ``FLASHMAP_CONTEXT_CACHE``, else "auto"): "layers" always takes the
    per-layer layout, "auto" the virtual one on hybrid targets, "virtual" always where
    the shapes allow it. The virtual layout needs a bf16 cache, a target page whose
    elements are a whole number of DiT heads, and room for every DiT head."""
    mode = mode or os.environ.get("FLASHMAP_CONTEXT_CACHE", "auto")
    if mode not in MODES:
        raise ValueError(f"unknown context-cache mode {mode!r} (FLASHMAP_CONTEXT_CACHE takes {', '.join(MODES)})")

    def per_layer(reason: str) -> ContextCachePlan:
        return ContextCachePlan(num_layers, heads, num_layers, heads, False, reason)

    if mode == "layers":
        return per_layer("FLASHMAP_CONTEXT_CACHE=layers")
    if mode == "auto" and not hybrid:
        return per_layer("the target has no linear-attention or Mamba layers")
    if not bf16_cache:
        return per_layer("the KV cache is fp8")
    page_elems = target_kv_heads * target_head_size
    if target_attention_layers <= 0 or page_elems <= 0 or page_elems % head_dim:
        return per_layer(f"a target page of {target_kv_heads} x {target_head_size} does not hold whole heads of "
                         f"{head_dim}")
    hpc = page_elems // head_dim
    if target_attention_layers * hpc < num_layers * heads:
        return per_layer(f"{target_attention_layers} caches of {hpc} heads are fewer than {num_layers} x {heads} "
                         f"DiT heads")
    return ContextCachePlan(num_layers, heads, target_attention_layers, hpc, True,
                            f"{target_attention_layers} caches of {hpc} heads of {head_dim} (the target's page)")


def _group(query: torch.Tensor, segments) -> int:
    kv_heads = sum(run[2] for run in segments)
    if kv_heads <= 0 or query.shape[1] % kv_heads:
        raise ValueError(f"{query.shape[1]} query heads are not a multiple of the runs' {kv_heads} heads")
    return query.shape[1] // kv_heads


def attend_by_segments(
    query: torch.Tensor,
    caches: list[torch.Tensor],
    segments: list[tuple[int, int, int, int]],
    attend: Callable[[torch.Tensor, torch.Tensor, int], torch.Tensor],
) -> torch.Tensor:
    """One layer's cross-attention of ``query (tokens, heads, head_dim)`` as
    ``attend(query heads, cache heads, count)`` per run, outputs concatenated along the
    heads (flashmap/vllm/context_cache.py:120-139); a run covering the whole query and
    its whole cache passes both unsliced. With grouped queries (``G`` query heads per
    KV head) a run of ``count`` KV heads takes its ``G * count`` query heads."""
    group = _group(query, segments)
    parts = []
    for cache_id, first_slot, count, first_head in segments:
        cache = caches[cache_id]
        q_part = query
        if group * count != query.shape[1]:
            q_part = query[:, group * first_head:group * (first_head + count)].contiguous()
        c_part = cache if count == cache.shape[1] else cache[:, first_slot:first_slot + count]
        parts.append(attend(q_part, c_part, count))
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)


def cross_attention_by_segments(
    query: torch.Tensor,
    caches: list[torch.Tensor],
    segments: list[tuple[int, int, int, int]],
    cu_seqlens_q: torch.Tensor | None,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    scheduler_metadata: torch.Tensor | None = None,
    prologue: ops.Prologue | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`attend_by_segments` with ``flashmap_vllm::paged_cross_attention`` as the
    per-run call, in one launch per ``ops.MAX_RUNS`` runs of the layer (bf16 caches; the
    virtual layout is not used with fp8 caches). A layer of more runs is attended in
    consecutive head ranges, each launch reading and writing its range of query and
    output heads in place. ``scheduler_metadata``: the step's plan from
    ``cross_attention_schedule(seqused_k)``."""
    group = _group(query, segments)
    if len(segments) <= ops.MAX_RUNS:
        return ops.block_attention_paged_runs(query, caches, segments, cu_seqlens_q, seqused_k, block_table,
                                              max_seqlen_q, max_seqlen_k, softmax_scale, prologue=prologue,
                                              plan=scheduler_metadata, out=out)
    if out is None:
        out = torch.empty(query.shape, dtype=torch.bfloat16, device=query.device)
    for i in range(0, len(segments), ops.MAX_RUNS):
        chunk = segments[i:i + ops.MAX_RUNS]
        h0 = chunk[0][3]
        h1 = h0 + sum(run[2] for run in chunk)
        rebased = [(c, slot, count, head - h0) for c, slot, count, head in chunk]
        heads = slice(group * h0, group * h1)
        ops.block_attention_paged_runs(query[:, heads], caches, rebased, cu_seqlens_q, seqused_k, block_table,
                                       max_seqlen_q, max_seqlen_k, softmax_scale, prologue=prologue,
                                       plan=scheduler_metadata, out=out[:, heads])
    return out
