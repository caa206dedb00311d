"""Seeded input builders shared by the tests (drawn on the CPU, moved to the GPU)."""

from __future__ import annotations

import math

import torch

from oracle import attention as ref

MAX_ABS = 2e-2  # bf16 output vs fp32 oracle, max |diff|
MEAN_ABS = 2e-3  # bf16 output vs fp32 oracle, mean |diff|


def gen(seed: int = 0) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def paged_layout(lens, page: int, g: torch.Generator):
    """A randomly permuted block table for contexts ``lens`` (padding entries 0)."""
    pages = [max(1, math.ceil(int(n) / page)) for n in lens]
    total = sum(pages)
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n].int()
        o += n
    return bt, total


def vllm_cache_from_contig(keys, values, lens, page, bt, total):
    """A vLLM cache (total, Hkv, page, 2D) holding contiguous keys/values (B, Hkv, L, D)."""
    b_, hkv, _, d = keys.shape
    cache = torch.zeros(total, hkv, page, 2 * d, dtype=keys.dtype)
    for b in range(b_):
        for p in range(int(lens[b])):
            blk, t = int(bt[b, p // page]), p % page
            cache[blk, :, t, :d] = keys[b, :, p]
            cache[blk, :, t, d:] = values[b, :, p]
    return cache


def token_pool_from_contig(keys, values, lens, g):
    """SGLang pools (pool, Hkv, D) and a page table of shuffled token slots."""
    b_, hkv, lmax, d = keys.shape
    pool = int(sum(int(n) for n in lens)) + 7
    perm = torch.randperm(pool, generator=g)
    width = max(int(lens.max()), 1)
    pt = torch.zeros(b_, width, dtype=torch.int32)
    kb = torch.zeros(pool, hkv, d, dtype=keys.dtype)
    vb = torch.zeros(pool, hkv, d, dtype=keys.dtype)
    o = 0
    for b in range(b_):
        n = int(lens[b])
        slots = perm[o:o + n]
        o += n
        pt[b, :n] = slots.int()
        kb[slots] = keys[b, :, :n].transpose(0, 1)
        vb[slots] = values[b, :, :n].transpose(0, 1)
    return kb, vb, pt


def normed_keys(b, hkv, lmax, d, g, theta=1e6, eps=1e-6):
    """Context keys as the drafter caches them: RMS-normed and rotated at their
    positions (weight 1), bf16 (B, Hkv, L, D)."""
    k = torch.randn(b, lmax, hkv, d, generator=g).bfloat16()
    cos, sin = ref.rope_tables(torch.arange(lmax)[None].expand(b, -1), d, theta)
    return ref.project_keys(k, torch.ones(d), cos, sin, eps).transpose(1, 2).contiguous()


def check_close(got: torch.Tensor, want: torch.Tensor, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    err = (got.float().cpu() - want.float()).abs()
    assert torch.isfinite(got.float()).all(), "non-finite output"
    assert err.max().item() <= max_abs, f"max-abs {err.max().item():.3e} > {max_abs}"
    assert err.mean().item() <= mean_abs, f"mean-abs {err.mean().item():.3e} > {mean_abs}"
    return err


def tree_visibility(length: int, g: torch.Generator) -> torch.Tensor:
    """``(L, L)`` bool visibility of a random draft tree: node 0 is the root, node j's
    parent is drawn from nodes 0..j-1, and a node sees itself and its ancestors."""
    parent = [-1] + [int(torch.randint(0, j, (1,), generator=g)) for j in range(1, length)]
    vis = torch.zeros(length, length, dtype=torch.bool)
    for j in range(length):
        a = j
        while a >= 0:
            vis[j, a] = True
            a = parent[a]
    return vis


def verify_case(bs, length, hq, hkv, d, contexts, mask="causal", index_dtype=torch.int32, seed=0,
                pool_slack=37, dtype=torch.bfloat16):
    """Seeded inputs of a verify call in sglang's extend_attention_fwd layout:
    q ``(bs * L, Hq, D)``, the verify tokens' k/v ``(bs * L, Hkv, D)``, a pool
    ``(pool, Hkv, D)`` whose rows hold every request's context at randomly permuted slots
    (plus unused rows), ``kv_indptr``/``kv_indices`` and, for ``mask`` "rows" (sglang's
    layout, the context columns filled with junk the kernels must not read) or "qlen"
    (L x L blocks), per-request random tree masks."""
    g = gen(seed)
    contexts = [int(c) for c in contexts]
    total = sum(contexts)
    pool = total + pool_slack
    q = torch.randn(bs * length, hq, d, generator=g).to(dtype)
    k = torch.randn(bs * length, hkv, d, generator=g).to(dtype)
    v = torch.randn(bs * length, hkv, d, generator=g).to(dtype)
    key_buffer = torch.randn(pool, hkv, d, generator=g).to(dtype)
    value_buffer = torch.randn(pool, hkv, d, generator=g).to(dtype)
    kv_indptr = torch.zeros(bs + 1, dtype=torch.int32)
    kv_indptr[1:] = torch.cumsum(torch.tensor(contexts, dtype=torch.int64), 0).to(torch.int32)
    kv_indices = torch.randperm(pool, generator=g)[:total].to(index_dtype)
    case = dict(q=q, k=k, v=v, key_buffer=key_buffer, value_buffer=value_buffer, kv_indptr=kv_indptr,
                kv_indices=kv_indices, custom_mask=None, mask_indptr=None, qlen_mask=False)
    if mask == "rows":
        rows, starts = [], [0]
        for b in range(bs):
            junk = torch.randint(0, 2, (length, contexts[b]), generator=g).bool()
            rows.append(torch.cat([junk, tree_visibility(length, g)], dim=1).reshape(-1))
            starts.append(starts[-1] + length * (contexts[b] + length))
        case["custom_mask"] = torch.cat(rows)
        case["mask_indptr"] = torch.tensor(starts, dtype=torch.int64)
    elif mask == "qlen":
        case["custom_mask"] = torch.cat([tree_visibility(length, g).reshape(-1) for _ in range(bs)])
        case["qlen_mask"] = True
    return case
