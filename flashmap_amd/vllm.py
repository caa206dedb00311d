"""Drop-in torch custom ops for FlashMap's vLLM plugin, over the gfx950 kernels.

:func:`register` defines the plugin's ops under their names and signatures, with fake
(meta) implementations so that ``torch.compile(fullgraph=True)`` traces through them
and engine graphs capture them:

- ``flashmap_vllm::rms_norm_rope``          (flashmap/vllm/kernels.py:101-124)
- ``flashmap_vllm::block_self_attention``   (flashmap/vllm/kernels.py:194-232)
- ``flashmap_vllm::paged_cross_attention``  (flashmap/vllm/model.py:93-139), bf16
  caches and e4m3 caches with ``descales``

plus ``flashmap_vllm::paged_cross_attention_runs``, one DiT layer's cross-attention
over the virtual context-cache layout in one launch (what attend_by_segments does with
one call per run, flashmap/vllm/context_cache.py:120-139), and the plain functions
:func:`write_context_kv` (flashmap/vllm/kernels.py:311-364; bf16, or e4m3 with
``scales``) and :func:`cross_attention_schedule`, the per-step plan that takes the place
of FlashAttention's ``get_scheduler_metadata`` (flashmap/vllm/model.py:967-989): pass
its result as ``scheduler_metadata``. Registration is explicit (not on import) so the
package can sit beside the reference plugin; it is idempotent.
"""

from __future__ import annotations

import torch

from . import ops

NAMESPACE = "flashmap_vllm"


def rms_norm_rope(
    x: torch.Tensor, weight: torch.Tensor, cos_sin: torch.Tensor, positions: torch.Tensor, eps: float
) -> torch.Tensor:
    """RMSNorm then RoPE at ``positions (tokens,)`` of ``x (tokens, heads, head_dim)``
    with the ``rope_table`` ``cos_sin (P, head_dim/2, 2)``, in one launch."""
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous():
        raise ValueError("cos_sin must be a contiguous float32 (P, head_dim/2, 2) table")
    return ops.rms_norm_rope(x, weight, ops.rope_from_table(cos_sin), positions, eps)


def block_self_attention(
    qkv: torch.Tensor,
    q_norm: torch.Tensor,
    k_norm: torch.Tensor,
    cos_sin: torch.Tensor,
    positions: torch.Tensor,
    eps: float,
) -> torch.Tensor:
    """Unmasked self-attention within each draft block of ``qkv (blocks, T, 3, heads,
    head_dim)`` after the q/k RMSNorms and RoPE at ``positions (blocks * T,)``;
    returns ``(blocks * T, heads * head_dim)``."""
    blocks, t, _, heads, d = qkv.shape
    out = ops.block_self_attention(qkv, q_norm, k_norm, ops.rope_from_table(cos_sin), positions, eps)
    return out.view(blocks * t, heads * d)


def cross_attention_schedule(seqused_k: torch.Tensor) -> torch.Tensor:
    """The step's split plan from the context lengths, computed once per draft step
    and shared by every layer's :func:`paged_cross_attention`."""
    return ops.attention_plan(seqused_k)


def _plan(meta: torch.Tensor | None, batch: int) -> torch.Tensor | None:
    if meta is None:
        return None
    if meta.dtype != torch.int32 or meta.dim() != 1 or meta.numel() != 2 * (batch + 1):
        raise ValueError("scheduler_metadata must be cross_attention_schedule(seqused_k) or None")
    return meta


def paged_cross_attention(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    scheduler_metadata: torch.Tensor | None,
    descales: torch.Tensor | None,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    fa_version: int,
) -> torch.Tensor:
    """Non-causal attention of ``query (tokens, heads, head_dim)`` onto the first
    ``seqused_k`` cached positions of each request (vLLM's ``(blocks, kv_heads, page,
    2 * head_dim)`` cache, K then V in each row). An fp8 cache takes an e4m3 ``query``
    and ``descales (3, requests, kv_heads)`` for the query, keys and values
    (flashmap/vllm/model.py:93-134). ``fa_version`` is accepted and ignored."""
    del fa_version
    if descales is not None:
        return ops.block_attention_paged_fp8(
            query, kv_cache, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k,
            softmax_scale, descales=descales, plan=_plan(scheduler_metadata, seqused_k.shape[0]),
        )
    return ops.block_attention_paged(
        query, kv_cache, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k,
        softmax_scale, plan=_plan(scheduler_metadata, seqused_k.shape[0]),
    )


def paged_cross_attention_runs(
    query: torch.Tensor,
    kv_caches: list[torch.Tensor],
    runs: list[int],
    cu_seqlens_q: torch.Tensor,
    seqused_k: torch.Tensor,
    block_table: torch.Tensor,
    scheduler_metadata: torch.Tensor | None,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
) -> torch.Tensor:
    """:func:`paged_cross_attention` of one DiT layer whose KV heads lie in runs over
    several bf16 caches (``ContextCachePlan.segments[layer]`` flattened, four ints per
    run: cache, first slot, count, first head), in one launch per ``ops.MAX_RUNS`` runs;
    the output is what attend_by_segments concatenates from one call per run
    (flashmap/vllm/context_cache.py:120-139)."""
    from .context_cache import cross_attention_by_segments

    if len(runs) % 4:
        raise ValueError("runs must hold four ints per run (cache, first slot, count, first head)")
    segments = [tuple(runs[i:i + 4]) for i in range(0, len(runs), 4)]
    return cross_attention_by_segments(
        query, kv_caches, segments, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k,
        softmax_scale, scheduler_metadata=_plan(scheduler_metadata, seqused_k.shape[0]),
    )


def write_context_kv(
    kv: torch.Tensor,
    positions: torch.Tensor,
    slots: torch.Tensor,
    k_norm: torch.Tensor,
    cos_sin: torch.Tensor,
    cache_ptrs: torch.Tensor,
    cache_strides: tuple[int, int, int, int],
    block_size: int,
    eps: float,
    scales: torch.Tensor | None = None,
    heads_per_cache: int | None = None,
) -> None:
    """Every layer's context keys (k-normed, rotated) and values of ``kv (tokens,
    layers, 2, heads, head_dim)`` written into the paged caches at ``slots`` (negative
    slots skipped), heads in layer-major order, ``heads_per_cache`` per cache. With
    ``scales (layers, 2)`` the caches are e4m3 and keys / values are divided by the
    layer's scales (flashmap/vllm/kernels.py:292-299)."""
    if scales is not None:
        ops.write_context_kv_fp8(kv, positions, slots, k_norm, ops.rope_from_table(cos_sin), cache_ptrs,
                                 cache_strides, block_size, eps, scales, heads_per_cache)
        return
    ops.write_context_kv(kv, positions, slots, k_norm, ops.rope_from_table(cos_sin), cache_ptrs,
                         cache_strides, block_size, eps, heads_per_cache)


def split_argmax(logits: torch.Tensor, chunks: int = 128) -> torch.Tensor:
    """``logits.argmax(-1)`` of ``(rows, vocab)`` logits, the first index among equals
    (flashmap/vllm/fold.py:117-128). ``chunks`` is accepted for the signature: the kernel
    splits the vocabulary into tiles of its own, which does not change the result."""
    del chunks
    return ops.argmax_rows(logits)


def seeded_normal(
    seeds: torch.Tensor, rows: torch.Tensor, positions: torch.Tensor, n_cols: int, scale: float = 1.0
) -> torch.Tensor:
    """Standard normals ``(len(rows), n_cols)`` in float32, row ``i`` keyed by
    ``seeds[rows[i]]`` (0 where ``rows[i] < 0``) and ``positions[i]``
    (flashmap/vllm/kernels.py:394-410), the reference's random stream."""
    return ops.seeded_normal(seeds, rows, positions, n_cols, scale)


_OPS: dict[str, object] = {}


def register(namespace: str = NAMESPACE) -> dict[str, object]:
    """Define the custom ops under ``namespace`` (the reference plugin's by default)
    and return them by name. Idempotent."""
    if namespace in _OPS:
        return _OPS[namespace]
    lib = torch.library

    norm = lib.custom_op(f"{namespace}::rms_norm_rope", mutates_args=())(rms_norm_rope)
    norm.register_fake(lambda x, weight, cos_sin, positions, eps: torch.empty_like(x))

    self_attn = lib.custom_op(f"{namespace}::block_self_attention", mutates_args=())(block_self_attention)

    def _self_fake(qkv, q_norm, k_norm, cos_sin, positions, eps):
        blocks, t, _, heads, d = qkv.shape
        return qkv.new_empty((blocks * t, heads * d))

    self_attn.register_fake(_self_fake)

    cross = lib.custom_op(f"{namespace}::paged_cross_attention", mutates_args=())(paged_cross_attention)

    def _cross_fake(query, kv_cache, cu_seqlens_q, seqused_k, block_table, *args):
        return torch.empty(query.shape, dtype=torch.bfloat16, device=query.device)

    cross.register_fake(_cross_fake)

    runs = lib.custom_op(f"{namespace}::paged_cross_attention_runs", mutates_args=())(paged_cross_attention_runs)
    runs.register_fake(lambda query, *args: torch.empty_like(query))
    _OPS[namespace] = {"rms_norm_rope": norm, "block_self_attention": self_attn,
                       "paged_cross_attention": cross, "paged_cross_attention_runs": runs}
    return _OPS[namespace]


__all__ = ["block_self_attention", "cross_attention_schedule", "paged_cross_attention",
           "paged_cross_attention_runs", "register", "rms_norm_rope", "seeded_normal", "split_argmax",
           "write_context_kv"]


def plugin() -> None:
    """The vLLM general plugin (`vllm.general_plugins`) entry point of this package (``pyproject.toml``), called
    by the engine at start-up in every process: defines the ops under the reference's
    namespace ``flashmap_vllm``, unless ops of that namespace exist already (the reference's
    own plugin registered first); never raises, as an engine plugin must not."""
    import logging

    try:
        getattr(torch.ops, NAMESPACE).rms_norm_rope
        return  # the namespace is taken
    except (AttributeError, RuntimeError):
        pass
    try:
        register()
    except Exception as err:  # noqa: BLE001 -- a plugin must not take the engine down
        logging.getLogger(__name__).warning("flashmap_amd: flashmap_vllm ops not registered: %s", err)
