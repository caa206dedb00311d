"""CPU restatement of the reference drafter-attention math (torch on the CPU).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Each function cites the reference
lines it restates. Pinning (tests/test_oracle_*.py): closed forms, invariants and
float64 brute force on tiny inputs; which check pins which function is listed in the
functions' docstrings under "Pinned by".

Numerics follow the reference modules:
  * RMSNorm: ``x * to_dtype(w_f32 * rsqrt(mean(x_f32^2) + eps))``
    (flashmap/modeling_flashmap.py:79-80);
  * RoPE: interleaved pairs ``(2i, 2i+1)`` rotated in float32, rounded to x's dtype
    (flashmap/modeling_flashmap.py:61-66);
  * attention: non-causal ``softmax(q k^T * scale) v`` in float32, GQA by repeating
    each KV head over its group of query heads (the fp32 reference of
    ``F.scaled_dot_product_attention`` at flashmap/modeling_flashmap.py:146).
"""

from __future__ import annotations

import math

import numpy as np
import torch

# ----------------------------------------------------------------------------- rope


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """``1 / theta ** (arange(0, D, 2) / D)`` in float32 (flashmap/modeling_flashmap.py:56).
    Pinned by: closed form against float64 (test_oracle_rope)."""
    return 1.0 / theta ** (torch.arange(0, head_dim, 2).float() / head_dim)


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float):
    """``(cos, sin)`` each ``(B, T, 1, D/2)`` float32 at ``positions (B, T)``
    (flashmap/modeling_flashmap.py:53-58). Pinned by: identity at position 0, pair-norm
    preservation, relative-position invariance of q.k (test_oracle_rope)."""
    angles = positions.float()[..., None, None] * inv_freq(head_dim, theta)
    return angles.cos(), angles.sin()


def rope_table(max_positions: int, head_dim: int, base: float) -> torch.Tensor:
    """vLLM table ``(P, D/2, 2)`` of ``(cos, sin)`` (flashmap/vllm/kernels.py:26-33).
    Pinned by: equality with rope_tables rows (test_oracle_rope)."""
    angles = torch.arange(max_positions).float()[:, None] * inv_freq(head_dim, base)
    return torch.stack([angles.cos(), angles.sin()], dim=-1).contiguous()


def rope_freqs(positions: torch.Tensor, head_dim: int, theta: float) -> torch.Tensor:
    """SGLang per-position table ``(..., D/2, 2)`` (flashmap/sglang/model.py:116-123).
    Pinned by: equality with rope_table rows (test_oracle_rope)."""
    angles = positions.float()[..., None] * inv_freq(head_dim, theta)
    return torch.stack([angles.cos(), angles.sin()], dim=-1)


def rope_cat_table(max_positions: int, head_dim: int, theta: float) -> torch.Tensor:
    """SGLang writer table ``(P, D)``: ``[cos(D/2) | sin(D/2)]`` per row
    (flashmap/sglang/model.py:814-817). Pinned by: equality with rope_table rows."""
    freqs = rope_freqs(torch.arange(max_positions), head_dim, theta)
    return torch.cat([freqs[..., 0], freqs[..., 1]], dim=-1).contiguous()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate interleaved pairs ``(x[2i], x[2i+1])`` of ``x (..., D)`` by angles with
    ``cos``/``sin`` broadcastable to ``(..., D/2)``, in float32, result in x's dtype
    (flashmap/modeling_flashmap.py:61-66). Pinned by: a 2x2 rotation per pair checked
    against float64 (test_oracle_rope)."""
    x1, x2 = x.float().unflatten(-1, (-1, 2)).unbind(-1)
    return torch.stack([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).flatten(-2).type_as(x)


# -------------------------------------------------------------------------- norms


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``x * to_dtype(w_f32 * rsqrt(mean(x_f32^2) + eps))`` over the last dim
    (flashmap/modeling_flashmap.py:69-80). Pinned by: float64 closed form with the
    bf16 rounding points, unit RMS of the output at w = 1 (test_oracle_norm)."""
    rms = torch.rsqrt(x.float().pow(2).mean(dim=-1, keepdim=True) + eps)
    return x * (weight.float() * rms).to(x.dtype)


def rms_norm_rope_vllm(x, weight, cos_sin, positions, eps):
    """flashmap_vllm::rms_norm_rope on ``x (tokens, H, D)``: rope rows gathered at
    ``positions`` of the ``(P, D/2, 2)`` table (flashmap/vllm/kernels.py:67-124).
    Pinned by: composition of the pinned rms_norm and apply_rope (test_oracle_norm)."""
    rows = cos_sin[positions.long()]  # (tokens, D/2, 2)
    cos, sin = rows[..., 0][:, None, :], rows[..., 1][:, None, :]
    return apply_rope(rms_norm(x, weight, eps), cos, sin)


def rms_norm_rope_sglang(x, weight, freqs, eps):
    """flashmap_sglang::rms_norm_rope on ``x (..., T, H, D)`` with one table row per token
    ``freqs (..., T, D/2, 2)`` (flashmap/sglang/kernels.py:149-189). Pinned by: equal to
    rms_norm_rope_vllm on the same rows with the vLLM table layout (test_oracle_norm)."""
    cos, sin = freqs[..., 0].unsqueeze(-2), freqs[..., 1].unsqueeze(-2)
    return apply_rope(rms_norm(x, weight, eps), cos, sin)


# ---------------------------------------------------------------------- attention


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None) -> torch.Tensor:
    """Non-causal ``softmax(q k^T * scale) v`` in float32 for ``q (..., Hq, T, D)`` and
    ``k, v (..., Hkv, L, D)``; query head h reads KV head ``h // (Hq / Hkv)``
    (flashmap/modeling_flashmap.py:146; the GQA convention of
    flashmap/sglang/verify_attention.py:77-79). Returns float32 ``(..., Hq, T, D)``.
    Pinned by: float64 brute force, rows of P sum to 1, one key -> v, key permutation
    invariance, GQA == MHA on repeated KV (test_oracle_attention)."""
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    hq, hkv = q.shape[-3], k.shape[-3]
    if hq != hkv:
        k = k.repeat_interleave(hq // hkv, dim=-3)
        v = v.repeat_interleave(hq // hkv, dim=-3)
    s = (q.float() @ k.float().transpose(-1, -2)) * scale
    return s.softmax(dim=-1) @ v.float()


def attention_lse(q, k, v, scale=None):
    """``(out, lse)`` of :func:`attention` with lse the natural log-sum-exp of the
    scaled scores per row; -inf (and out 0) for an empty key set. The partial a split
    of the context hands to the merge (flashmap/sglang/verify_attention.py:172-181).
    Pinned by: merge of splits == unsplit attention (test_oracle_attention)."""
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    hq, hkv = q.shape[-3], k.shape[-3]
    if hq != hkv:
        k = k.repeat_interleave(hq // hkv, dim=-3)
        v = v.repeat_interleave(hq // hkv, dim=-3)
    if k.shape[-2] == 0:
        shape = (*q.shape[:-1],)
        return torch.zeros((*shape, v.shape[-1])), torch.full(shape, -math.inf)
    s = (q.float() @ k.float().transpose(-1, -2)) * scale
    lse = torch.logsumexp(s, dim=-1)
    return (s - lse[..., None]).exp() @ v.float(), lse


def lse_merge(outs: list[torch.Tensor], lses: list[torch.Tensor]) -> torch.Tensor:
    """Merge split partials ``O = sum_s exp(lse_s - m) O_s / sum_s exp(lse_s - m)``,
    skipping splits with lse = -inf (flashmap/sglang/verify_attention.py:184-233).
    Pinned by: merge of splits == unsplit attention (test_oracle_attention)."""
    lse = torch.stack(lses)
    m = lse.max(dim=0).values
    m = torch.where(torch.isinf(m), torch.zeros_like(m), m)
    w = torch.exp(lse - m)  # exp(-inf) = 0 for empty splits
    num = sum(wi[..., None] * oi for wi, oi in zip(w, outs))
    den = w.sum(dim=0)
    return num / torch.where(den > 0, den, torch.ones_like(den))[..., None]


def block_attention_contig(query, keys, values, seqlens_k=None, scale=None):
    """a5: ``query (B, T, Hq, D)`` onto FlashMapCache views ``keys/values (B, Hkv, L, D)``,
    sequence b reading its first ``seqlens_k[b]`` positions (all L by default)
    (flashmap/modeling_flashmap.py:144-147, 218-219). Returns float32 (B, T, Hq, D);
    zeros for an empty context. Pinned by: its attention core against float64 brute force,
    seqlens truncation and empty contexts (test_oracle_attention)."""
    b_, t_, hq, d = query.shape
    out = torch.zeros((b_, t_, hq, d))
    for b in range(b_):
        n = keys.shape[2] if seqlens_k is None else int(seqlens_k[b])
        if n <= 0:
            continue
        out[b] = attention(query[b].transpose(0, 1), keys[b, :, :n], values[b, :, :n], scale).transpose(0, 1)
    return out


# ----------------------------------------------------------------- paged layouts


def vllm_gather_slots(block_table: np.ndarray, seqlen: int, page_size: int, b: int) -> np.ndarray:
    """Physical (page, in-page token) of positions ``0..seqlen-1`` of request ``b``:
    ``(block_table[b, p // page], p % page)`` (the block-table addressing of
    flashmap/vllm/model.py:107-134). Pinned by: exact integer closed form checked
    elementwise against a direct loop (test_oracle_layouts)."""
    p = np.arange(seqlen)
    return np.stack([block_table[b, p // page_size], p % page_size], axis=-1)


def gather_vllm(kv_cache: torch.Tensor, block_table, seqlen: int, b: int):
    """K and V ``(Hkv, seqlen, D)`` of request ``b`` from a vLLM cache
    ``(num_blocks, Hkv, page, 2D)`` whose rows hold K then V
    (flashmap/vllm/model.py:107-112: ``kv_cache.transpose(1, 2).split(D, -1)``). Pinned
    by: the gather closed form and paged == contiguous under block permutations
    (test_oracle_attention)."""
    d = kv_cache.shape[-1] // 2
    page = kv_cache.shape[2]
    idx = vllm_gather_slots(np.asarray(block_table), seqlen, page, b)
    rows = kv_cache[torch.as_tensor(idx[:, 0]), :, torch.as_tensor(idx[:, 1])]  # (seqlen, Hkv, 2D)
    return rows[..., :d].transpose(0, 1), rows[..., d:].transpose(0, 1)


def block_attention_paged_vllm(query, kv_cache, cu_seqlens_q, seqused_k, block_table, scale=None):
    """a6: flashmap_vllm::paged_cross_attention (flashmap/vllm/model.py:93-134): request b's
    query rows ``cu_seqlens_q[b]:cu_seqlens_q[b+1]`` of ``query (tokens, Hq, D)`` attend
    non-causally to its first ``seqused_k[b]`` paged positions. Returns float32 (tokens, Hq,
    D), zeros for empty contexts. Pinned by: equal to block_attention_contig under any block
    permutation (test_oracle_attention)."""
    out = torch.zeros(query.shape)
    bt = np.asarray(block_table)
    for b in range(len(seqused_k)):
        lo, hi = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        n = int(seqused_k[b])
        if n <= 0 or hi <= lo:
            continue
        k, v = gather_vllm(kv_cache, bt, n, b)
        out[lo:hi] = attention(query[lo:hi].transpose(0, 1), k, v, scale).transpose(0, 1)
    return out


def block_attention_token_paged(query, key_buffer, value_buffer, cache_seqlens, page_table, scale=None):
    """a7: flashmap_sglang::paged_cross_attention (flashmap/sglang/model.py:127-146): request b
    (``query (bs, T, Hq, D)``) reads pool rows ``page_table[b, :cache_seqlens[b]]`` of
    ``key_buffer/value_buffer (pool, Hkv, D)``. Returns float32 (bs, T, Hq, D). Pinned by:
    equal to block_attention_contig on the same K/V at shuffled pool slots
    (test_oracle_attention)."""
    out = torch.zeros(query.shape)
    for b in range(query.shape[0]):
        n = int(cache_seqlens[b])
        if n <= 0:
            continue
        rows = torch.as_tensor(np.asarray(page_table)[b, :n]).long()
        k = key_buffer[rows].transpose(0, 1)
        v = value_buffer[rows].transpose(0, 1)
        out[b] = attention(query[b].transpose(0, 1), k, v, scale).transpose(0, 1)
    return out


# --------------------------------------------------------------- verify attention


def verify_visibility(b: int, length: int, context: int, custom_mask=None, mask_indptr=None,
                      qlen_mask: bool = False) -> torch.Tensor:
    """``(L, L)`` bool: verify token t of request b sees verify token j. No mask: causal
    (j <= t). sglang's layout: request b's rows start at ``mask_indptr[b]``, each
    ``context + L`` entries of which the last L apply (the context columns are never
    read: the context is always visible). QLEN_ONLY: request b's ``L x L`` block at
    ``b * L * L`` (flashmap/sglang/verify_attention.py:143-164).
    Pinned by: causal == the lower-triangular mask in both layouts, context columns
    ignored (test_oracle_verify)."""
    if custom_mask is None:
        return torch.ones(length, length, dtype=torch.bool).tril()
    m = torch.as_tensor(custom_mask).reshape(-1)
    if qlen_mask:
        return m[b * length * length:(b + 1) * length * length].reshape(length, length) != 0
    start = int(mask_indptr[b])
    rows = m[start:start + length * (context + length)].reshape(length, context + length)
    return rows[:, context:] != 0


def verify_attention(q, k_ext, v_ext, key_buffer, value_buffer, kv_indptr, kv_indices, custom_mask=None,
                     mask_indptr=None, qlen_mask=False, sm_scale=None, k_scale=1.0, v_scale=1.0):
    """Target verify attention, SplitKVVerify (flashmap/sglang/verify_attention.py:35-233,
    360-474): ``q (bs * L, Hq, D)`` row ``b * L + t`` (query head hq, KV head
    ``hq // (Hq / Hkv)``) attends to request b's context, pool rows
    ``kv_indices[kv_indptr[b]:kv_indptr[b + 1]]`` of ``key_buffer/value_buffer (pool,
    Hkv, D)`` with scores scaled by ``sm_scale * k_scale`` and values by ``v_scale``, and
    to the verify tokens j of ``k_ext/v_ext (bs * L, Hkv, D)`` that
    :func:`verify_visibility` allows, scores scaled by ``sm_scale``; one softmax over
    both (the reference splits it into partials merged by LSE, which is the same
    function). A row that sees nothing is zero. Returns float32 (bs * L, Hq, D).
    Pinned by: float64 brute force per row; == lse_merge of the context and verify
    partials (the reference's split form); L = 1 causal == :func:`attention` onto the
    context plus the token; k_scale / v_scale == pre-scaled pool; GQA == MHA on repeated
    KV (test_oracle_verify)."""
    bs = len(kv_indptr) - 1
    tokens, hq, d = q.shape
    length = tokens // bs
    hkv = key_buffer.shape[1]
    g = hq // hkv
    scale = d ** -0.5 if sm_scale is None else sm_scale
    out = torch.zeros((tokens, hq, v_ext.shape[-1]))
    for b in range(bs):
        lo, hi = int(kv_indptr[b]), int(kv_indptr[b + 1])
        n = max(hi - lo, 0)
        rows = torch.as_tensor(np.asarray(kv_indices)[lo:lo + n]).long()
        kp, vp = key_buffer[rows].float(), value_buffer[rows].float()  # (n, Hkv, D)
        ke, ve = k_ext[b * length:(b + 1) * length].float(), v_ext[b * length:(b + 1) * length].float()
        vis = verify_visibility(b, length, n, custom_mask, mask_indptr, qlen_mask)
        qb = q[b * length:(b + 1) * length].float()  # (L, Hq, D)
        for h in range(hq):
            kh = h // g
            sp = (qb[:, h] @ kp[:, kh].T) * (scale * k_scale)  # (L, n)
            se = (qb[:, h] @ ke[:, kh].T) * scale  # (L, L)
            se = se.masked_fill(~vis, -math.inf)
            s = torch.cat([sp, se], dim=1)
            m = s.max(dim=1, keepdim=True).values
            m = torch.where(torch.isinf(m), torch.zeros_like(m), m)
            p = torch.exp(s - m)
            den = p.sum(dim=1, keepdim=True)
            o = p[:, :n] @ vp[:, kh] * v_scale + p[:, n:] @ ve[:, kh]
            out[b * length:(b + 1) * length, h] = o / torch.where(den > 0, den, torch.ones_like(den))
    return out


# -------------------------------------------------------------- self-attention (a8)


def block_self_attention(qkv, q_norm, k_norm, cos, sin, eps, scale=None):
    """a8: q/k RMSNorm + RoPE then unmasked softmax attention within each block of
    ``qkv (blocks, T, 3, H, D)``; ``cos/sin (blocks, T, D/2)`` per slot. Returns float32
    (blocks, T, H, D) (flashmap/vllm/kernels.py:127-191, flashmap/sglang/kernels.py:18-75;
    transformers: flashmap/modeling_flashmap.py:188). Pinned by: composition of pinned
    rms_norm / apply_rope / attention."""
    q, k, v = qkv.unbind(2)  # (blocks, T, H, D)
    c, s = cos[:, :, None, :], sin[:, :, None, :]
    q = apply_rope(rms_norm(q, q_norm, eps), c, s)
    k = apply_rope(rms_norm(k, k_norm, eps), c, s)
    return attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale).transpose(1, 2)


# ------------------------------------------------------------------ writers (a4)


def project_keys(k_rows, k_norm_w, cos, sin, eps):
    """The K side of the prologue: ``apply_rope(k_norm(k))`` of ``k_rows (..., H, D)`` with
    ``cos/sin`` broadcastable to ``(..., 1, D/2)`` (flashmap/modeling_flashmap.py:139-142;
    flashmap/vllm/kernels.py:276-290). Pinned by: composition of rms_norm and apply_rope,
    each pinned (test_oracle_norm, test_oracle_rope)."""
    return apply_rope(rms_norm(k_rows, k_norm_w, eps), cos, sin)


def write_context_kv_vllm(kv, positions, slots, k_norm, cos_sin, caches, block_size, eps, heads_per_cache=None):
    """vLLM ``write_context_kv`` for bf16 caches (flashmap/vllm/kernels.py:235-364):
    ``kv (tokens, L, 2, H, D)``; head h of layer l (global head l*H + h) goes to cache
    ``g // HPC`` head ``g % HPC`` at slot ``slots[t]`` (skipped if negative); caches are
    ``(num_blocks, HPC, page, 2D)`` tensors, updated in place. Pinned by: write then
    gather round trip equals project_keys / v (test_oracle_layouts)."""
    tokens, layers, _, heads, d = kv.shape
    hpc = heads_per_cache or heads
    rows = cos_sin[positions.long()]  # (tokens, D/2, 2)
    cos, sin = rows[..., 0][:, None, :], rows[..., 1][:, None, :]
    for t in range(tokens):
        slot = int(slots[t])
        if slot < 0:
            continue
        page, tok = divmod(slot, block_size)
        for l in range(layers):
            keys = project_keys(kv[t, l, 0][None], k_norm[l], cos[t:t + 1], sin[t:t + 1], eps)[0]
            for h in range(heads):
                g = l * heads + h
                c, s = divmod(g, hpc)
                caches[c][page, s, tok, :d] = keys[h]
                caches[c][page, s, tok, d:] = kv[t, l, 1, h]


# ------------------------------------------------------ virtual context-cache layout


def context_segments(num_layers: int, heads: int, heads_per_cache: int):
    """Per DiT layer, its heads as runs ``(cache, first slot, count, first head)``, built
    head by head as ``ContextCachePlan.segments`` does (flashmap/vllm/context_cache.py:56-68):
    global head ``l * heads + h`` sits at ``divmod(., heads_per_cache)`` (:60-73), and a
    head in the same cache as the previous one extends its run. Pinned by: the runs
    cover the heads in order, give each head the closed-form (cache, slot), and
    neighbouring runs lie in different caches, which fixes them (test_context_cache)."""
    out = []
    for layer in range(num_layers):
        runs: list[tuple[int, int, int, int]] = []
        for head in range(heads):
            cache, slot = divmod(layer * heads + head, heads_per_cache)
            if runs and runs[-1][0] == cache:
                c, first_slot, count, first_head = runs[-1]
                runs[-1] = (c, first_slot, count + 1, first_head)
            else:
                runs.append((cache, slot, 1, head))
        out.append(runs)
    return out


def block_attention_paged_segments(query, caches, segments, cu_seqlens_q, seqused_k, block_table, scale=None):
    """One layer's cross-attention over the virtual layout: block_attention_paged_vllm
    per run, on the run's query heads and cache heads, concatenated along the heads
    (flashmap/vllm/context_cache.py:120-139 with the op of flashmap/vllm/model.py:876-890;
    ``G`` query heads per KV head). Pinned by: equal to block_attention_paged_vllm on a
    per-layer cache that holds the same heads, gathered by the closed-form (cache, slot)
    map (test_context_cache)."""
    kv_heads = sum(run[2] for run in segments)
    group = query.shape[1] // kv_heads
    parts = []
    for cache_id, first_slot, count, first_head in segments:
        q = query[:, group * first_head:group * (first_head + count)]
        c = caches[cache_id][:, first_slot:first_slot + count]
        parts.append(block_attention_paged_vllm(q, c, cu_seqlens_q, seqused_k, block_table, scale))
    return torch.cat(parts, dim=1)


# ------------------------------------------------------------------- fp8 (e4m3) KV


E4M3_MAX = 448.0


def to_e4m3(x: torch.Tensor) -> torch.Tensor:
    """Round to OCP e4m3 (nearest even) saturating at +-448, the conversion the
    reference's Triton writers use for fp8 caches (flashmap/vllm/kernels.py:292-299,
    flashmap/sglang/kernels.py:330-335). Returns a float8_e4m3fn tensor.
    Pinned by: nearest-code brute force over all 256 codes with ties to even
    (test_oracle_fp8)."""
    return x.float().clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)


def rotate_f32(y: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair RoPE of ``y`` in float32 without the final rounding (the fp8
    writers quantize the rotated keys directly: flashmap/vllm/kernels.py:287-296,
    flashmap/sglang/kernels.py:330-331). Pinned by: its result rounded
    to bf16 equals apply_rope (test_oracle_rope), and float64 on the same pairs."""
    e, o = y[..., 0::2].float(), y[..., 1::2].float()
    out = torch.empty(y.shape, dtype=torch.float32)
    out[..., 0::2] = e * cos - o * sin
    out[..., 1::2] = o * cos + e * sin
    return out


def norm_sglang_fp8(k: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """The fp8 pool writer's RMSNorm: ``bf16((x * r) * w)`` with ``r = 1 / sqrt(mean(x^2)
    + eps)``, one rounding (flashmap/sglang/kernels.py:325-329), where the bf16 paths
    round the scale first (:func:`rms_norm`). Pinned by: float64 restatement; differs
    from rms_norm on some inputs (test_oracle_fp8)."""
    kf = k.float()
    inv = 1.0 / torch.sqrt((kf * kf).mean(dim=-1, keepdim=True) + eps)
    return (kf * inv * weight.float()).to(torch.bfloat16)


def write_context_kv_vllm_fp8(kv, positions, slots, k_norm, cos_sin, caches, block_size, eps, scales,
                              heads_per_cache=None):
    """vLLM ``write_context_kv`` for e4m3 caches (flashmap/vllm/kernels.py:276-299):
    keys k-normed (bf16 rounding as :func:`rms_norm`), rotated in float32, divided by the
    layer's key scale; values divided by its value scale; both :func:`to_e4m3`.
    ``caches`` are float8_e4m3fn ``(num_blocks, HPC, page, 2D)`` tensors, updated in place;
    ``scales (L, 2)``. Pinned by: dequantized round trip == project_keys / v within half
    an e4m3 step (test_oracle_fp8)."""
    tokens, layers, _, heads, d = kv.shape
    hpc = heads_per_cache or heads
    rows = cos_sin[positions.long()]
    cos, sin = rows[..., 0][:, None, :], rows[..., 1][:, None, :]
    for t in range(tokens):
        slot = int(slots[t])
        if slot < 0:
            continue
        page, tok = divmod(slot, block_size)
        for l in range(layers):
            ks, vs = float(scales[l, 0]), float(scales[l, 1])
            keys = rotate_f32(rms_norm(kv[t, l, 0], k_norm[l], eps), cos[t], sin[t])
            for h in range(heads):
                g = l * heads + h
                c, s_ = divmod(g, hpc)
                caches[c][page, s_, tok, :d] = to_e4m3(keys[h] / ks)
                caches[c][page, s_, tok, d:] = to_e4m3(kv[t, l, 1, h].float() / vs)


def write_context_kv_pool_fp8(kv, k_bufs, v_bufs, k_norm, cos_sin_cat, positions, locs, num_layers, kv_size,
                              head_dim, eps, k_scale=1.0, v_scale=1.0, commit_lens=None, locs_row_width=None):
    """``kv_norm_rope_write_fp8`` (flashmap/sglang/kernels.py:283-357): as
    :func:`write_context_kv_pool` into float8_e4m3fn pools, keys normed by
    :func:`norm_sglang_fp8`, rotated in float32, both divided by their static scale
    and :func:`to_e4m3`. Pinned by: dequantized round trip (test_oracle_fp8)."""
    heads = kv_size // head_dim
    half = head_dim // 2
    rows = cos_sin_cat[positions.long()]
    cos, sin = rows[:, None, :half], rows[:, None, half:]
    for t in range(kv.shape[0]):
        loc = int(locs[t])
        if loc < 0:
            continue
        if commit_lens is not None and t % locs_row_width >= int(commit_lens[t // locs_row_width]):
            continue
        for l in range(num_layers):
            base = l * 2 * kv_size
            k = kv[t, base:base + kv_size].view(heads, head_dim)
            v = kv[t, base + kv_size:base + 2 * kv_size].view(heads, head_dim)
            keys = rotate_f32(norm_sglang_fp8(k, k_norm[l], eps), cos[t], sin[t])
            k_bufs[l][loc] = to_e4m3(keys / k_scale)
            v_bufs[l][loc] = to_e4m3(v.float() / v_scale)


def quantize_query_per_head(query: torch.Tensor):
    """``query (bs, T, H, D)`` -> (e4m3 query, scale (bs, H)): scale = max(amax |q| over
    (T, D), 1e-12) / 448, q8 = q / scale rounded to e4m3, as
    flashmap_sglang::paged_cross_attention_fp8 quantizes (flashmap/sglang/model.py:167-169).
    Pinned by: each head's largest |q| maps to 448; dequantized within half an e4m3 step
    (test_oracle_fp8)."""
    scale = query.float().abs().amax(dim=(1, 3)).clamp_min(1e-12) / 448.0
    return (query.float() / scale[:, None, :, None]).to(torch.float8_e4m3fn), scale


def block_attention_paged_vllm_fp8(query, kv_cache, cu_seqlens_q, seqused_k, block_table, scale, descales=None):
    """a6 onto an e4m3 cache with FlashAttention's descales (flashmap/vllm/model.py:93-134,
    863-873): ``query (tokens, Hq, D)`` e4m3, ``descales (3, requests, Hkv)`` (query, key,
    value; None = 1); attention of the dequantized operands q8 q_d, k8 k_d, v8 v_d in
    float32. Returns float32 (tokens, Hq, D). Pinned by: :func:`attention` (pinned) on
    exactly dequantized e4m3 values (test_oracle_fp8)."""
    tokens, hq, d = query.shape
    hkv = kv_cache.shape[1]
    g = hq // hkv
    qf = query.float()
    cache = kv_cache.float()
    out = torch.zeros(tokens, hq, d)
    bt = np.asarray(block_table)
    for b in range(len(seqused_k)):
        lo, hi = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        n = int(seqused_k[b])
        if n <= 0 or hi <= lo:
            continue
        k, v = gather_vllm(cache, bt, n, b)  # (Hkv, n, D)
        q = qf[lo:hi].transpose(0, 1).clone()  # (Hq, T, D)
        if descales is not None:
            qd, kd, vd = (descales[i, b].float() for i in range(3))
            q = q * qd.repeat_interleave(g)[:, None, None]
            k = k * kd[:, None, None]
            v = v * vd[:, None, None]
        out[lo:hi] = attention(q, k, v, scale).transpose(0, 1)
    return out


def block_attention_token_paged_fp8(query, key_buffer, value_buffer, cache_seqlens, page_table, scale=None,
                                    descales=None):
    """a7 onto e4m3 pools as flashmap_sglang::paged_cross_attention_fp8 computes it
    (flashmap/sglang/model.py:154-181): the bf16 ``query (bs, T, Hq, D)`` quantized by
    :func:`quantize_query_per_head`, keys and values descaled by ``descales[1:]`` (None =
    1, the pool written with scale 1), attention of the dequantized operands in float32.
    Returns float32 (bs, T, Hq, D). Pinned by: composition of pinned parts (test_oracle_fp8)."""
    q8, qs = quantize_query_per_head(query)
    qd = q8.float() * qs[:, None, :, None]
    kf, vf = key_buffer.float(), value_buffer.float()
    out = torch.zeros(query.shape)
    for b in range(query.shape[0]):
        n = int(cache_seqlens[b])
        if n <= 0:
            continue
        rows = torch.as_tensor(np.asarray(page_table)[b, :n]).long()
        k, v = kf[rows].transpose(0, 1), vf[rows].transpose(0, 1)
        if descales is not None:
            k = k * descales[1, b].float()[:, None, None]
            v = v * descales[2, b].float()[:, None, None]
        out[b] = attention(qd[b].transpose(0, 1), k, v, scale).transpose(0, 1)
    return out


def write_context_kv_pool(kv, k_bufs, v_bufs, k_norm, cos_sin_cat, positions, locs, num_layers, kv_size,
                          head_dim, eps, commit_lens=None, locs_row_width=None):
    """SGLang pool write (fused_kv_norm_rope_write as flashmap/sglang/model.py:746-766
    calls it, interleaved RoPE; the reference's rounding of the norm, scale rounded to
    bf16 first, flashmap/modeling_flashmap.py:79-80): ``kv (tokens, L*2*kv_size)``,
    per layer keys then values; token t goes to pool row ``locs[t]`` unless negative or
    past its request's ``commit_lens`` column. Pinned by: write then read back equals project_keys
    / the values at committed slots, uncommitted tokens untouched (test_oracle_layouts)."""
    heads = kv_size // head_dim
    half = head_dim // 2
    rows = cos_sin_cat[positions.long()]
    cos, sin = rows[:, None, :half], rows[:, None, half:]
    for t in range(kv.shape[0]):
        loc = int(locs[t])
        if loc < 0:
            continue
        if commit_lens is not None and t % locs_row_width >= int(commit_lens[t // locs_row_width]):
            continue
        for l in range(num_layers):
            base = l * 2 * kv_size
            k = kv[t, base:base + kv_size].view(heads, head_dim)
            v = kv[t, base + kv_size:base + 2 * kv_size].view(heads, head_dim)
            k_bufs[l][loc] = project_keys(k[None], k_norm[l], cos[t:t + 1], sin[t:t + 1], eps)[0]
            v_bufs[l][loc] = v
