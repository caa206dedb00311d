"""Drop-in torch custom ops for FlashMap's SGLang plugin, over the gfx950 kernels.

:func:`register` defines, with fake implementations for ``torch.compile(dynamic=True)``:

- ``flashmap_sglang::rms_norm_rope``          (flashmap/sglang/kernels.py:171-189)
- ``flashmap_sglang::block_self_attention``   (flashmap/sglang/kernels.py:84-120)
- ``flashmap_sglang::paged_cross_attention``  (flashmap/sglang/model.py:127-151)

and the plain functions :func:`rope_freqs` (flashmap/sglang/model.py:116-123),
:func:`cross_attention_schedule` (the per-step plan in place of
``get_scheduler_metadata``, flashmap/sglang/model.py:189-204) and
:func:`fused_kv_norm_rope_write`, the bf16 pool write the plugin takes from sglang
(called at flashmap/sglang/model.py:746-766, interleaved RoPE), with the e4m3 pool
variants ``paged_cross_attention_fp8`` (flashmap/sglang/model.py:154-186) and
``kv_norm_rope_write_fp8`` (flashmap/sglang/kernels.py:283-357). Registration is
explicit and idempotent.
"""

from __future__ import annotations

import torch

from . import ops

NAMESPACE = "flashmap_sglang"


def rope_freqs(positions: torch.Tensor, head_dim: int, theta: float) -> torch.Tensor:
    """``(..., head_dim/2, [cos, sin])`` float32 at ``positions``: angle
    ``position / theta ** (2 i / head_dim)``, built with the reference's torch ops."""
    inv_freq = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=positions.device).float() / head_dim)
    angles = positions.float()[..., None] * inv_freq
    return torch.stack([angles.cos(), angles.sin()], dim=-1)


def rms_norm_rope(x: torch.Tensor, weight: torch.Tensor, freqs: torch.Tensor, eps: float) -> torch.Tensor:
    """RoPE of RMSNorm(x) for ``x (..., T, heads, head_dim)`` with one ``freqs (..., T,
    head_dim/2, [cos, sin])`` row per token."""
    *lead, heads, d = x.shape
    if freqs.dtype != torch.float32 or not freqs.is_contiguous():
        raise ValueError("freqs must be contiguous float32 (..., T, head_dim/2, 2)")
    flat = x.reshape(-1, heads, d)
    out = ops.rms_norm_rope(flat, weight, ops.rope_from_table(freqs), None, eps)
    return out.view(*lead, heads, d)


def block_self_attention(
    qkv: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, freqs: torch.Tensor, eps: float
) -> torch.Tensor:
    """Self-attention within each draft block of ``qkv (blocks, T, 3, heads, head_dim)``
    with ``freqs (blocks, T, head_dim/2, 2)``; returns ``(blocks, T, heads, head_dim)``."""
    return ops.block_self_attention(qkv, q_norm, k_norm, ops.rope_from_table(freqs), None, eps)


def cross_attention_schedule(cache_seqlens: torch.Tensor) -> torch.Tensor:
    """The step's split plan from the context lengths (shared by every layer)."""
    return ops.attention_plan(cache_seqlens)


def paged_cross_attention(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    cache_seqlens: torch.Tensor,
    page_table: torch.Tensor,
    scheduler_metadata: torch.Tensor | None,
) -> torch.Tensor:
    """``query (bs, K, heads, head_dim)`` onto each request's first ``cache_seqlens``
    pool rows of ``key_buffer / value_buffer (pool, kv_heads, head_dim)``, listed by
    ``page_table`` (page size 1)."""
    plan = scheduler_metadata
    if plan is not None and (plan.dtype != torch.int32 or plan.numel() != 2 * (cache_seqlens.shape[0] + 1)):
        raise ValueError("scheduler_metadata must be cross_attention_schedule(cache_seqlens) or None")
    return ops.block_attention_token_paged(query, key_buffer, value_buffer, cache_seqlens, page_table,
                                           plan=plan)


def paged_cross_attention_fp8(
    query: torch.Tensor,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    cache_seqlens: torch.Tensor,
    page_table: torch.Tensor,
    scheduler_metadata: torch.Tensor | None,
) -> torch.Tensor:
    """:func:`paged_cross_attention` onto an e4m3 pool written with scale 1: the bf16
    query is quantized per (request, head) with scale amax / 448 and every operand
    descaled (flashmap/sglang/model.py:154-181); returns the query's dtype."""
    plan = scheduler_metadata
    if plan is not None and (plan.dtype != torch.int32 or plan.numel() != 2 * (cache_seqlens.shape[0] + 1)):
        raise ValueError("scheduler_metadata must be cross_attention_schedule(cache_seqlens) or None")
    return ops.block_attention_token_paged_fp8(query, key_buffer, value_buffer, cache_seqlens, page_table,
                                               plan=plan)


def kv_norm_rope_write_fp8(
    kv: torch.Tensor,
    meta: torch.Tensor,
    k_norm_weights: torch.Tensor,
    cos_sin: torch.Tensor,
    positions: torch.Tensor,
    locs: torch.Tensor,
    num_layers: int,
    kv_size: int,
    head_dim: int,
    eps: float,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    commit_lens: torch.Tensor | None = None,
    locs_row_width: int | None = None,
) -> None:
    """:func:`fused_kv_norm_rope_write` (same arguments, interleaved RoPE) for e4m3 pools:
    keys k-normed (one rounding, bf16(x r w)) and rotated, keys and values divided by
    their static scale (flashmap/sglang/kernels.py:336-357)."""
    if kv.shape[0] == 0:
        return
    ops.write_context_kv_pool_fp8(kv, meta, k_norm_weights, ops.rope_from_cat(cos_sin), positions, locs,
                                  num_layers, kv_size, head_dim, eps, k_scale=k_scale, v_scale=v_scale,
                                  commit_lens=commit_lens, locs_row_width=locs_row_width)


def fused_kv_norm_rope_write(
    kv: torch.Tensor,
    meta: torch.Tensor,
    k_norm_weights: torch.Tensor,
    cos_sin: torch.Tensor,
    positions: torch.Tensor,
    locs: torch.Tensor,
    num_layers: int,
    kv_size: int,
    head_dim: int,
    eps: float,
    is_neox_style: bool = False,
    commit_lens: torch.Tensor | None = None,
    locs_row_width: int | None = None,
) -> None:
    """Every layer's keys (k-normed, rotated at ``positions`` with the ``(P, head_dim)``
    ``[cos | sin]`` table) and values of ``kv (tokens, layers * 2 * kv_size)`` written
    to pool rows ``locs``, per layer at the buffers ``meta (layers, 4)`` = (key ptr,
    value ptr, key row stride, value row stride); negative locations and, with
    ``commit_lens``, uncommitted verify columns are skipped."""
    if is_neox_style:
        raise NotImplementedError("FlashMap rotates interleaved pairs (is_neox_style=False)")
    ops.write_context_kv_pool(kv, meta, k_norm_weights, ops.rope_from_cat(cos_sin), positions, locs,
                              num_layers, kv_size, head_dim, eps, commit_lens, locs_row_width)


def sample_rows(
    logits: torch.Tensor,
    temperatures: torch.Tensor,
    greedy: torch.Tensor,
    seed: torch.Tensor,
    block_v: int = 4096,
) -> torch.Tensor:
    """A token per row of contiguous ``logits (rows, V)``: the argmax for ``greedy`` rows,
    else a sample of ``softmax(logits / temperature)`` (Gumbel-max), with Philox noise
    seeded by the int64 scalar tensor ``seed`` (flashmap/sglang/kernels.py:222-247); the
    tokens equal the reference's for the same seed wherever the winning key is not
    within float rounding of the runner-up. ``block_v`` is accepted for the signature
    (the tiling does not change the result). Reads the logits once; no noise buffer."""
    del block_v
    if not logits.is_contiguous():
        raise ValueError("logits must be contiguous")
    return ops.sample_rows(logits, temperatures, greedy, seed)


_OPS: dict[str, object] = {}


def register(namespace: str = NAMESPACE) -> dict[str, object]:
    """Define the custom ops under ``namespace`` (the reference plugin's by default)
    and return them by name. Idempotent."""
    if namespace in _OPS:
        return _OPS[namespace]
    lib = torch.library
    norm = lib.custom_op(f"{namespace}::rms_norm_rope", mutates_args=())(rms_norm_rope)
    norm.register_fake(lambda x, weight, freqs, eps: torch.empty_like(x))
    self_attn = lib.custom_op(f"{namespace}::block_self_attention", mutates_args=())(block_self_attention)

    def _self_fake(qkv, q_norm, k_norm, freqs, eps):
        blocks, t, _, heads, d = qkv.shape
        return qkv.new_empty((blocks, t, heads, d))

    self_attn.register_fake(_self_fake)
    cross = lib.custom_op(f"{namespace}::paged_cross_attention", mutates_args=())(paged_cross_attention)
    cross.register_fake(lambda query, key_buffer, value_buffer, cache_seqlens, page_table, meta:
                        torch.empty_like(query))
    cross8 = lib.custom_op(f"{namespace}::paged_cross_attention_fp8", mutates_args=())(paged_cross_attention_fp8)
    cross8.register_fake(lambda query, key_buffer, value_buffer, cache_seqlens, page_table, meta:
                         torch.empty_like(query))
    _OPS[namespace] = {"rms_norm_rope": norm, "block_self_attention": self_attn,
                       "paged_cross_attention": cross, "paged_cross_attention_fp8": cross8}
    return _OPS[namespace]


__all__ = ["block_self_attention", "cross_attention_schedule", "fused_kv_norm_rope_write",
           "kv_norm_rope_write_fp8", "paged_cross_attention", "paged_cross_attention_fp8", "register",
           "rms_norm_rope", "rope_freqs", "sample_rows"]


def plugin() -> None:
    """The SGLang plugin (`sglang.srt.plugins`) entry point of this package (``pyproject.toml``), called
    by the engine at start-up in every process: defines the ops under the reference's
    namespace ``flashmap_sglang``, unless ops of that namespace exist already (the reference's
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
        logging.getLogger(__name__).warning("flashmap_amd: flashmap_sglang ops not registered: %s", err)
