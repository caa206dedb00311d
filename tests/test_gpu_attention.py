"""GPU parity of the block attention kernels (a5/a6/a7) and the Q prologue (a2/a3)
against the CPU oracle, through the C ABI (flashmap_amd.ops -> ctypes).

Tolerance (written here, from the bar for bf16 outputs): max-abs 2e-2 and mean-abs 2e-3
against the float32 oracle on the same bf16 inputs. Integer/layout properties
(paged == contiguous on the same data, fused == unfused prologue) are bit-exact.
"""

import math

import pytest
import torch

from _inputs import (check_close, gen, normed_keys, paged_layout, token_pool_from_contig,
                     vllm_cache_from_contig)
from oracle import attention as ref

pytestmark = pytest.mark.gpu


def ops():
    from flashmap_amd import ops as o

    return o


# ------------------------------------------------------------------- Q prologue


@pytest.mark.parametrize("d", [64, 128])
def test_rms_norm_rope_vllm_table(dev, d):
    g = gen(1)
    tokens, heads = 37, 6
    x = torch.randn(tokens, heads, d, generator=g).bfloat16() * 3
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(4096, d, 1e6)
    pos = torch.randint(0, 4096, (tokens,), generator=g)
    want = ref.rms_norm_rope_vllm(x, w, table, pos, 1e-6)
    got = ops().rms_norm_rope(x.to(dev), w.to(dev), ops().rope_from_table(table.to(dev)), pos.to(dev), 1e-6)
    diff = (got.cpu().float() - want.float()).abs()
    # Bit-exact except where a last-ulp difference of the fp32 mean flips a rounding.
    exact = (got.cpu() == want).float().mean().item()
    assert exact > 0.99, f"only {exact:.4f} of elements bit-exact"
    ulp = want.float().abs() * 2.0 ** -7 + 1e-30
    assert (diff <= 2 * ulp).all()


def test_rms_norm_rope_sglang_freqs(dev):
    g = gen(2)
    bs, t, heads, d = 3, 16, 4, 128
    x = torch.randn(bs, t, heads, d, generator=g).bfloat16()
    w = torch.ones(d)
    freqs = ref.rope_freqs(torch.arange(bs * t).view(bs, t) * 7 + 3, d, 1e6)
    want = ref.rms_norm_rope_sglang(x, w, freqs, 1e-6)
    got = ops().rms_norm_rope(
        x.view(-1, heads, d).to(dev), w.to(dev), ops().rope_from_table(freqs.contiguous().to(dev)), None, 1e-6
    ).view(bs, t, heads, d)
    assert (got.cpu() == want).float().mean().item() > 0.99


# ------------------------------------------------------------ contiguous (a5)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (8, 4), (32, 8), (40, 8)])
@pytest.mark.parametrize("d", [64, 128])
def test_contig_attention(dev, hq, hkv, d):
    g = gen(3)
    b, t, lmax = 2, 16, 300
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    want = ref.block_attention_contig(q, k, v)
    got = ops().block_attention_contig(q.to(dev), k.to(dev), v.to(dev))
    check_close(got, want)


def test_contig_attention_seqlens_and_empty(dev):
    g = gen(4)
    b, t, hq, hkv, d, lmax = 4, 16, 8, 2, 128, 200
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    lens = torch.tensor([200, 0, 1, 77])
    want = ref.block_attention_contig(q, k, v, lens)
    got = ops().block_attention_contig(q.to(dev), k.to(dev), v.to(dev), seqlens_k=lens.to(dev))
    check_close(got, want)
    assert (got[1] == 0).all(), "an empty context must give zeros"


def test_fused_prologue_is_bit_identical(dev):
    g = gen(5)
    b, t, hq, hkv, d, lmax = 3, 16, 32, 8, 128, 160
    q_pre = torch.randn(b, t, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(lmax + t + 1, d, 1e6)
    pos = (lmax + torch.arange(t))[None].expand(b, -1).reshape(-1)
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    o = ops()
    rope = o.rope_from_table(table.to(dev))
    qn = o.rms_norm_rope(q_pre.view(-1, hq, d).to(dev), w.to(dev), rope, pos.to(dev), 1e-6).view(b, t, hq, d)
    unfused = o.block_attention_contig(qn, k.to(dev), v.to(dev))
    fused = o.block_attention_contig(
        q_pre.to(dev), k.to(dev), v.to(dev), prologue=o.Prologue(w.to(dev), rope, pos.to(dev), 1e-6)
    )
    assert torch.equal(fused, unfused)
    want = ref.block_attention_contig(ref.rms_norm_rope_vllm(q_pre.view(-1, hq, d), w, table, pos, 1e-6).view(b, t, hq, d), k, v)
    check_close(fused, want)


# ----------------------------------------------------------------- paged (a6)


@pytest.mark.parametrize("hq,hkv,page", [(32, 8, 16), (16, 16, 16), (40, 8, 16), (8, 2, 32), (8, 2, 8), (8, 2, 64),
                                          (8, 2, 128), (8, 2, 24), (8, 2, 1)])
def test_paged_vllm_matches_oracle_and_contig(dev, hq, hkv, page):
    g = gen(6)
    d, t = 128, 16
    lens = torch.tensor([1, 16, 17, 300, 513, 95])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    want = ref.block_attention_paged_vllm(q, cache, cu, lens, bt)
    o = ops()
    got = o.block_attention_paged(
        q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), t, lmax, d ** -0.5
    )
    check_close(got, want)
    contig = o.block_attention_contig(q.view(b, t, hq, d).to(dev), k.to(dev), v.to(dev), seqlens_k=lens.to(dev))
    assert torch.equal(got.view(b, t, hq, d), contig), "paged and contiguous layouts must agree bit for bit"


@pytest.mark.parametrize("hq,hkv", [(64, 8), (56, 8), (48, 8)])
def test_one_replica_double_tiles(dev, hq, hkv):
    """Units of 6-8 row blocks run one replica per workgroup with 64-position line tiles
    (two 32-position stages each): lengths on either side of every 32- and 64-position
    boundary (the second stage empty, partial or full), and a long one; against the oracle,
    and paged == contiguous bit for bit, and the token pool (SGLang) against the oracle."""
    g = gen(61)
    d, t, page = 128, 16, 16
    lens = torch.tensor([1, 31, 32, 33, 63, 64, 65, 95, 96, 97, 129, 0, 513, 1000])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    want = ref.block_attention_paged_vllm(q, cache, cu, lens, bt)
    o = ops()
    got = o.block_attention_paged(
        q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), t, lmax, d ** -0.5
    )
    check_close(got, want)
    contig = o.block_attention_contig(q.view(b, t, hq, d).to(dev), k.to(dev), v.to(dev), seqlens_k=lens.to(dev))
    assert torch.equal(got.view(b, t, hq, d), contig), "paged and contiguous layouts must agree bit for bit"
    kp, vp, pt = token_pool_from_contig(k, v, lens, g)
    want_p = ref.block_attention_token_paged(q.view(b, t, hq, d), kp, vp, lens, pt)
    got_p = o.block_attention_token_paged(q.view(b, t, hq, d).to(dev), kp.to(dev), vp.to(dev),
                                          lens.to(dev, torch.int32), pt.to(dev))
    check_close(got_p, want_p)


def test_paged_zero_length_gives_zeros(dev):
    g = gen(7)
    hq, hkv, d, t, page = 8, 2, 128, 16, 16
    lens = torch.tensor([0, 40, 0])
    b = len(lens)
    bt, total = paged_layout(lens, page, g)
    cache = torch.randn(total, hkv, page, 2 * d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    want = ref.block_attention_paged_vllm(q, cache, cu, lens, bt)
    got = ops().block_attention_paged(
        q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), t, 64, d ** -0.5
    )
    check_close(got, want)
    assert (got[:t] == 0).all() and (got[2 * t:] == 0).all()


def test_paged_large_batch(dev):
    """More sequences than the streaming kernel stages in LDS (1024): the plan and the
    lengths are then read with scalar loads. Short and empty sequences mixed."""
    g = gen(17)
    hq, hkv, d, t, page = 8, 2, 64, 16, 16
    lens = torch.randint(0, 70, (1100,), generator=g)
    lens[::97] = 0
    b = len(lens)
    bt, total = paged_layout(lens, page, g)
    cache = torch.randn(total, hkv, page, 2 * d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    want = ref.block_attention_paged_vllm(q, cache, cu, lens, bt)
    got = ops().block_attention_paged(
        q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), t, 70, d ** -0.5
    )
    check_close(got, want)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 2)])
def test_paged_ragged_query_rows(dev, hq, hkv):
    """FlashAttention's varlen queries: requests with 16, 3, 0, 16, 9, 1 and 12 rows
    (max_seqlen_q 16), contexts including an empty one; every row of ``cu_seqlens_q``'s
    ranges against the oracle."""
    g = gen(23)
    d, page = 128, 16
    rows = [16, 3, 0, 16, 9, 1, 12]
    lens = torch.tensor([40, 700, 33, 0, 129, 16, 1])
    b = len(rows)
    cu = torch.zeros(b + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(rows), 0)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(int(cu[-1]), hq, d, generator=g).bfloat16()
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
    want = ref.block_attention_paged_vllm(q, cache, cu, lens, bt)
    o = ops()
    got = o.block_attention_paged(q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), 16,
                                  lmax, d ** -0.5)
    check_close(got, want)
    assert (got[int(cu[3]):int(cu[4])] == 0).all()  # the empty context's 16 rows


@pytest.mark.parametrize("t", [1, 5, 33, 48])
def test_query_lengths_contig_and_token_paged(dev, t):
    """Query blocks other than 16 rows (a head's rows spanning row blocks and units):
    the contiguous and the token-paged layouts against the oracle and each other."""
    g = gen(24 + t)
    hq, hkv, d = 32, 8, 128
    lens = torch.tensor([77, 1, 260])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    want = ref.block_attention_contig(q, k, v, lens)
    o = ops()
    got = o.block_attention_contig(q.to(dev), k.to(dev), v.to(dev), seqlens_k=lens.to(dev))
    check_close(got, want)
    kb, vb, pt = token_pool_from_contig(k, v, lens, g)
    tok = o.block_attention_token_paged(q.to(dev), kb.to(dev), vb.to(dev), lens.to(dev, torch.int32), pt.to(dev))
    assert torch.equal(tok, got), "token-paged and contiguous layouts must agree bit for bit"


# ----------------------------------------------------------- token paged (a7)


@pytest.mark.parametrize("hq,hkv", [(16, 16), (32, 8)])
def test_token_paged_sglang(dev, hq, hkv):
    g = gen(8)
    d, t = 128, 16
    lens = torch.tensor([5, 64, 333, 1])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    kb, vb, pt = token_pool_from_contig(k, v, lens, g)
    want = ref.block_attention_token_paged(q, kb, vb, lens, pt)
    got = ops().block_attention_token_paged(q.to(dev), kb.to(dev), vb.to(dev), lens.to(dev, torch.int32), pt.to(dev))
    check_close(got, want)


# ------------------------------------------------------------ self-attention (a8)


@pytest.mark.parametrize("heads,d", [(16, 128), (4, 64)])
def test_block_self_attention(dev, heads, d):
    g = gen(9)
    blocks, t = 5, 16
    qkv = torch.randn(blocks, t, 3, heads, d, generator=g).bfloat16()
    qn = torch.rand(d, generator=g) + 0.5
    kn = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(2048, d, 1e6)
    pos = torch.randint(0, 2000, (blocks * t,), generator=g)
    rows = table[pos].view(blocks, t, d // 2, 2)
    want = ref.block_self_attention(qkv, qn, kn, rows[..., 0], rows[..., 1], 1e-6)
    o = ops()
    got = o.block_self_attention(qkv.to(dev), qn.to(dev), kn.to(dev), o.rope_from_table(table.to(dev)), pos.to(dev), 1e-6)
    check_close(got, want)


# ---------------------------------------------------------------- writers (a4)


def test_write_context_kv_vllm(dev):
    g = gen(10)
    tokens, layers, heads, d, page = 9, 3, 4, 128, 16
    kv = torch.randn(tokens, layers, 2, heads, d, generator=g).bfloat16()
    kn = torch.rand(layers, d, generator=g) + 0.5
    table = ref.rope_table(1024, d, 1e6)
    pos = torch.randint(0, 1000, (tokens,), generator=g)
    slots = torch.randperm(4 * page, generator=g)[:tokens]
    slots[3] = -1
    hpc = 6  # virtual packing: heads of a layer span caches
    ncache = math.ceil(layers * heads / hpc)
    caches = [torch.zeros(4, hpc, page, 2 * d, dtype=torch.bfloat16) for _ in range(ncache)]
    want = [c.clone() for c in caches]
    ref.write_context_kv_vllm(kv, pos, slots, kn, table, want, page, 1e-6, hpc)
    o = ops()
    dcaches = [c.to(dev) for c in caches]
    ptrs = torch.tensor([c.data_ptr() for c in dcaches], dtype=torch.int64, device=dev)
    key = dcaches[0][..., :d]
    strides = (key.stride(0), key.stride(1), key.stride(2), d)
    o.write_context_kv(kv.to(dev), pos.to(dev), slots.to(dev), kn.to(dev), o.rope_from_table(table.to(dev)),
                       ptrs, strides, page, 1e-6, hpc)
    torch.cuda.synchronize()
    for got, exp in zip(dcaches, want):
        diff = (got.cpu().float() - exp.float()).abs()
        assert (got.cpu() == exp).float().mean().item() > 0.99
        assert diff.max().item() <= 2e-2


def test_write_context_kv_pool_sglang(dev):
    g = gen(11)
    tokens, layers, heads, d, width = 8, 2, 4, 128, 4
    kv_size = heads * d
    kv = torch.randn(tokens, layers * 2 * kv_size, generator=g).bfloat16()
    kn = torch.rand(layers, d, generator=g) + 0.5
    cat = ref.rope_cat_table(512, d, 1e6)
    pos = torch.randint(0, 500, (tokens,), generator=g)
    locs = torch.randperm(32, generator=g)[:tokens]
    commit = torch.tensor([3, 1], dtype=torch.int32)
    kbufs = [torch.zeros(32, heads, d, dtype=torch.bfloat16) for _ in range(layers)]
    vbufs = [torch.zeros(32, heads, d, dtype=torch.bfloat16) for _ in range(layers)]
    wk = [x.clone() for x in kbufs]
    wv = [x.clone() for x in vbufs]
    ref.write_context_kv_pool(kv, wk, wv, kn, cat, pos, locs, layers, kv_size, d, 1e-6, commit, width)
    o = ops()
    dk = [x.to(dev) for x in kbufs]
    dv = [x.to(dev) for x in vbufs]
    meta = torch.tensor([[a.data_ptr(), b.data_ptr(), a.stride(0), b.stride(0)] for a, b in zip(dk, dv)],
                        dtype=torch.int64, device=dev)
    o.write_context_kv_pool(kv.to(dev), meta, kn.to(dev), o.rope_from_cat(cat.to(dev)), pos.to(dev),
                            locs.to(dev), layers, kv_size, d, 1e-6, commit.to(dev), width)
    torch.cuda.synchronize()
    for got, exp in zip(dk + dv, wk + wv):
        assert (got.cpu() == exp).float().mean().item() > 0.99
        assert (got.cpu().float() - exp.float()).abs().max().item() <= 2e-2


# ------------------------------------------- query rows: direct (in-kernel prologue) vs pass


def _tables(kind, rows, d):
    table = ref.rope_table(rows, d, 1e6)
    if kind == "interleaved":
        return table, ops().rope_from_table
    if kind == "cat":  # [cos | sin] rows
        return table, lambda t: ops().rope_from_cat(torch.cat([t[..., 0], t[..., 1]], dim=-1).contiguous())
    return table, lambda t: ops().rope_from_split(t[..., 0].contiguous(), t[..., 1].contiguous())


@pytest.mark.parametrize("kind", ["interleaved", "cat", "split"])
@pytest.mark.parametrize("layout", ["contig", "paged"])
def test_direct_rows_equal_query_pass(dev, tuning, kind, layout):
    """The attention kernel applies the prologue to the caller's rows itself (direct rows)
    or reads rows a separate query pass normed and rotated: the same bits either way,
    for every rotary table layout, with ragged draft rows (cu_seqlens_q shorter than q_len)."""
    g = gen(41)
    hq, hkv, d, t, page = 32, 8, 128, 16, 16
    lens = torch.tensor([700, 33, 1, 260])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q_pre = torch.randn(b * t, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table, make = _tables(kind, lmax + t + 1, d)
    rope = make(table.to(dev))
    rows = torch.tensor([16, 9, 16, 3]) if layout == "paged" else torch.full((b,), t)
    cu = torch.cat([torch.zeros(1, dtype=torch.int32), rows.cumsum(0).to(torch.int32)])
    pos = torch.cat([int(n) + torch.arange(int(r)) for n, r in zip(lens, rows)])
    n_tok = int(cu[-1])
    o = ops()
    pro = o.Prologue(w.to(dev), rope, pos.to(dev), 1e-6)
    if layout == "paged":
        bt, total = paged_layout(lens, page, g)
        cache = vllm_cache_from_contig(k, v, lens, page, bt, total).to(dev)

        def run():
            return o.block_attention_paged(q_pre[:n_tok].to(dev), cache, cu.to(dev), lens.to(dev, torch.int32),
                                           bt.to(dev), t, lmax, d ** -0.5, prologue=pro)
    else:
        def run():
            return o.block_attention_contig(q_pre.view(b, t, hq, d).to(dev), k.to(dev), v.to(dev),
                                            seqlens_k=lens.to(dev), prologue=pro)
    outs = {}
    tuning("FLASHMAP_SMALL_TILES", "0")  # the persistent kernel (the small-call one reads rows directly)
    tuning("FLASHMAP_SHARE_COST", "2")  # one cut of the line for both (their default costs differ)
    for mode in ("1", "0"):
        tuning("FLASHMAP_QUERY_PASS", mode)
        outs[mode] = run()
    assert torch.equal(outs["0"], outs["1"]), f"{kind}/{layout}: direct rows differ from the query pass"
    qn = ref.rms_norm_rope_vllm(q_pre[:n_tok], w, table, pos, 1e-6)
    got = outs["0"].cpu().view(-1, hq, d)
    for i in range(b):
        s, e = int(cu[i]), int(cu[i + 1])
        if layout == "contig":
            s, e = i * t, (i + 1) * t
        want = ref.attention(qn[s:e].transpose(0, 1), k[i, :, : int(lens[i])], v[i, :, : int(lens[i])])
        check_close(got[s:e], want.transpose(0, 1))


@pytest.mark.parametrize("layout", ["contig", "paged"])
@pytest.mark.parametrize("hq,hkv", [(40, 8), (48, 8), (64, 8)])
@pytest.mark.parametrize("workgroups", ["6", ""])
def test_one_replica_direct_rows_equal_query_pass(dev, tuning, layout, hq, hkv, workgroups):
    """One-replica workgroups (GQA 5-8: 64-position line tiles) with direct rows, with few
    workgroups (long shares, several units and segment starts each) and with the default
    split: the same bits as the query pass, and the oracle's attention."""
    g = gen(43)
    d, t, page = 128, 16, 16
    lens = torch.tensor([1500, 700, 33, 1, 260, 95])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q_pre = torch.randn(b * t, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table, make = _tables("interleaved", lmax + t + 1, d)
    rope = make(table.to(dev))
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    pos = torch.cat([int(n) + torch.arange(t) for n in lens])
    o = ops()
    pro = o.Prologue(w.to(dev), rope, pos.to(dev), 1e-6)
    if layout == "paged":
        bt, total = paged_layout(lens, page, g)
        cache = vllm_cache_from_contig(k, v, lens, page, bt, total).to(dev)

        def run():
            return o.block_attention_paged(q_pre.to(dev), cache, cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), t,
                                           lmax, d ** -0.5, prologue=pro)
    else:
        def run():
            return o.block_attention_contig(q_pre.view(b, t, hq, d).to(dev), k.to(dev), v.to(dev),
                                            seqlens_k=lens.to(dev), prologue=pro)
    tuning("FLASHMAP_SMALL_TILES", "0")
    tuning("FLASHMAP_SHARE_COST", "2")
    tuning("FLASHMAP_SPLITKV_WORKGROUPS", workgroups)
    outs = {}
    for mode in ("1", "0"):
        tuning("FLASHMAP_QUERY_PASS", mode)
        outs[mode] = run()
    assert torch.equal(outs["0"], outs["1"]), f"{hq}/{hkv} {layout}: direct rows differ from the query pass"
    qn = ref.rms_norm_rope_vllm(q_pre, w, table, pos, 1e-6)
    got = outs["0"].cpu().view(-1, hq, d)
    for i in range(b):
        s, e = i * t, (i + 1) * t
        want = ref.attention(qn[s:e].transpose(0, 1), k[i, :, : int(lens[i])], v[i, :, : int(lens[i])])
        check_close(got[s:e], want.transpose(0, 1))


@pytest.mark.parametrize("layout", ["contig", "paged"])
@pytest.mark.parametrize("hq,hkv,lens", [(8, 2, [700, 33, 0, 260]), (32, 8, [1100, 5])])
def test_small_call_kernel(dev, tuning, layout, hq, hkv, lens):
    """Calls whose K/V fits one pass of a few-tile workgroups over the CUs run the small-call
    kernel: against the oracle at 1, 3 and 8 tiles per share and with that kernel off (the
    persistent one), max_seqlen_k far above the lengths (more shares than tiles, so empty
    shares whose partial slots the merge must skip), ragged draft rows, an empty context
    and the fused prologue."""
    g = gen(43)
    d, t, page, max_k = 128, 16, 16, 4096
    lens = torch.tensor(lens)
    b = len(lens)
    k = normed_keys(b, hkv, max_k, d, g)
    v = torch.randn(b, hkv, max_k, d, generator=g).bfloat16()
    q_pre = torch.randn(b * t, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table, make = _tables("interleaved", int(lens.max()) + t + 1, d)
    rope = make(table.to(dev))
    rows = torch.tensor([16, 9, 16, 3][:b]) if layout == "paged" else torch.full((b,), t)
    cu = torch.cat([torch.zeros(1, dtype=torch.int32), rows.cumsum(0).to(torch.int32)])
    pos = torch.cat([int(n) + torch.arange(int(r)) for n, r in zip(lens, rows)])
    n_tok = int(cu[-1])
    o = ops()
    pro = o.Prologue(w.to(dev), rope, pos.to(dev), 1e-6)
    if layout == "paged":
        bt, total = paged_layout(lens, page, g)
        cache = vllm_cache_from_contig(k, v, lens, page, bt, total).to(dev)

        def run():
            return o.block_attention_paged(q_pre[:n_tok].to(dev), cache, cu.to(dev), lens.to(dev, torch.int32),
                                           bt.to(dev), t, max_k, d ** -0.5, prologue=pro)
    else:
        def run():
            return o.block_attention_contig(q_pre.view(b, t, hq, d).to(dev), k.to(dev), v.to(dev),
                                            seqlens_k=lens.to(dev), prologue=pro)
    qn = ref.rms_norm_rope_vllm(q_pre[:n_tok], w, table, pos, 1e-6)
    for tiles in ("1", "3", "8", "0"):
        tuning("FLASHMAP_SMALL_TILES", tiles)
        got = run().cpu().view(-1, hq, d)
        print(f"small-call kernel {layout} hq={hq} hkv={hkv} lens={lens.tolist()} tiles per share={tiles}",
              flush=True)
        for i in range(b):
            s, e = (int(cu[i]), int(cu[i + 1])) if layout == "paged" else (i * t, (i + 1) * t)
            if int(lens[i]) == 0:
                assert (got[s:e] == 0).all(), "an empty context gives zeros"
                continue
            want = ref.attention(qn[s:e].transpose(0, 1), k[i, :, : int(lens[i])], v[i, :, : int(lens[i])])
            check_close(got[s:e], want.transpose(0, 1))


@pytest.mark.parametrize("tiles", ["", "1"])
def test_small_call_fits_the_queried_workspace(dev, monkeypatch, tuning, tiles):
    """fm_attn_workspace_bytes covers the small-call kernel at any tiles per share: a
    workspace of exactly the queried size runs the same kernel and split as the pool's
    larger one (identical bits), at C2's shape."""
    g = gen(44)
    b, hq, hkv, d, t, ctx = 1, 32, 8, 128, 16, 2048
    q = torch.randn(b, t, hq, d, generator=g).bfloat16()
    k = normed_keys(b, hkv, ctx, d, g)
    v = torch.randn(b, hkv, ctx, d, generator=g).bfloat16()
    o = ops()
    tuning("FLASHMAP_SMALL_TILES", tiles)
    pooled = o.block_attention_contig(q.to(dev), k.to(dev), v.to(dev))
    monkeypatch.setattr(o._WORKSPACES, "get",
                        lambda device, nbytes: torch.empty(nbytes, dtype=torch.uint8, device=device))
    exact = o.block_attention_contig(q.to(dev), k.to(dev), v.to(dev))
    assert torch.equal(pooled, exact), "the queried workspace must fit the small-call kernel"
    check_close(exact, ref.block_attention_contig(q, k, v))


@pytest.mark.parametrize("tiles", ["1", "0"])
def test_lengths_past_max_seqlen_k(dev, tuning, tiles):
    """Lengths beyond ``max_seqlen_k`` (the caller's bound, used to size the split): the
    shares then hold more tiles than planned (more than the small-call kernel's 8 stages,
    so it walks them in chunks); the results still match the oracle. 0: the persistent
    kernel."""
    g = gen(45)
    hq, hkv, d, t, page = 32, 8, 128, 16, 16
    lens = torch.tensor([700, 300, 33])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    want = ref.block_attention_paged_vllm(q, cache, cu, lens, bt)
    tuning("FLASHMAP_SMALL_TILES", tiles)
    got = ops().block_attention_paged(q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                      t, 1, d ** -0.5)
    check_close(got, want)


@pytest.mark.parametrize("qpass", ["1", "0"])
@pytest.mark.parametrize("cost", ["0", "1", "3", "6", "40"])
def test_share_cost_cuts(dev, tuning, cost, qpass):
    """The persistent kernel cuts its line of tiles into shares by cost (every unit counts
    its tiles plus a fixed cost): at any cost, including one that outweighs the tiles,
    every tile is computed once and every partial merged, for sequences of 0 to 2000
    positions, through the query pass (1) and with direct rows (0)."""
    g = gen(47)
    hq, hkv, d, t, page = 32, 8, 128, 16, 16
    lens = torch.tensor([0, 5, 33, 700, 1, 64, 2000, 31, 0, 129, 16, 450])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(lmax + t + 1, d, 1e6)
    pos = torch.cat([int(n) + torch.arange(t) for n in lens])
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    qn = ref.rms_norm_rope_vllm(q, w, table, pos, 1e-6)
    want = ref.block_attention_paged_vllm(qn, cache, cu, lens, bt)
    o = ops()
    pro = o.Prologue(w.to(dev), o.rope_from_table(table.to(dev)), pos.to(dev), 1e-6)
    tuning("FLASHMAP_SMALL_TILES", "0")
    tuning("FLASHMAP_SHARE_COST", cost)
    tuning("FLASHMAP_QUERY_PASS", qpass)
    got = o.block_attention_paged(q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                  t, lmax, d ** -0.5, prologue=pro)
    check_close(got, want)


@pytest.mark.parametrize("workgroups", ["128", "127"])
@pytest.mark.parametrize("lens", [[2048] * 4, [2048, 1500, 64, 1999]], ids=["equal", "ragged"])
def test_four_shares_per_unit_cut(dev, tuning, workgroups, lens):
    """Units that span four or more shares each are cut by tiles, fewer by cost: 32 units
    (4 sequences x 8 KV heads, one-replica workgroups, so shares = workgroups) over 128
    shares take the tile cut, over 127 the cost cut. Either way every tile is computed once
    and every partial merged, with equal lengths (every unit split at the same tiles) and
    ragged ones."""
    g = gen(53)
    hq, hkv, d, t, page = 32, 8, 128, 16, 16
    lens = torch.tensor(lens)
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(lmax + t + 1, d, 1e6)
    pos = torch.cat([int(n) + torch.arange(t) for n in lens])
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total)
    cu = torch.arange(b + 1, dtype=torch.int32) * t
    want = ref.block_attention_paged_vllm(ref.rms_norm_rope_vllm(q, w, table, pos, 1e-6), cache, cu, lens, bt)
    o = ops()
    pro = o.Prologue(w.to(dev), o.rope_from_table(table.to(dev)), pos.to(dev), 1e-6)
    tuning("FLASHMAP_SMALL_TILES", "0")
    tuning("FLASHMAP_SPLITKV_WORKGROUPS", workgroups)
    got = o.block_attention_paged(q.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                  t, lmax, d ** -0.5, prologue=pro)
    check_close(got, want)


@pytest.mark.parametrize("qpass", ["1", "0"])
def test_own_plan_equals_step_plan(dev, tuning, qpass):
    """A call given no step plan computes its own (in one extra workgroup of its query pass
    when it has one, else with a launch of its own): the same bits as the call given the
    step plan of ops.attention_plan."""
    g = gen(49)
    hq, hkv, d, t, page = 32, 8, 128, 16, 16
    lens = torch.tensor([0, 5, 700, 1, 2000, 31, 129, 450])
    b = len(lens)
    lmax = int(lens.max())
    k = normed_keys(b, hkv, lmax, d, g)
    v = torch.randn(b, hkv, lmax, d, generator=g).bfloat16()
    q = torch.randn(b * t, hq, d, generator=g).bfloat16()
    bt, total = paged_layout(lens, page, g)
    cache = vllm_cache_from_contig(k, v, lens, page, bt, total).to(dev)
    cu = (torch.arange(b + 1, dtype=torch.int32) * t).to(dev)
    lens_d = lens.to(dev, torch.int32)
    tuning("FLASHMAP_SMALL_TILES", "0")
    tuning("FLASHMAP_QUERY_PASS", qpass)
    o = ops()
    own = o.block_attention_paged(q.to(dev), cache, cu, lens_d, bt.to(dev), t, lmax, d ** -0.5)
    step = o.block_attention_paged(q.to(dev), cache, cu, lens_d, bt.to(dev), t, lmax, d ** -0.5,
                                   plan=o.attention_plan(lens_d))
    assert torch.equal(own, step)
