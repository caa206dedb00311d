"""GPU parity of the fp8 (OCP e4m3) KV paths against the CPU oracle, through the C ABI:
the fp8 context writers (vLLM per-layer scales; the SGLang pool writer with its own norm
rounding) and the block attention onto e4m3 caches (vLLM's paged cache with
FlashAttention descales and e4m3 queries; SGLang's pool with the queries quantized per
(request, head) inside the call).

Tolerances (written here): written e4m3 bytes equal the oracle's for >= 99 % of the
elements, the rest one code away (a last-ulp difference of the fp32 arithmetic flipping
a rounding); attention outputs within max-abs 2e-2, mean-abs 2e-3 of the float32 oracle
on the same e4m3 inputs (the scores are exact products of e4m3 values; P is bf16).
"""

import pytest
import torch

from _inputs import check_close, gen, paged_layout
from oracle import attention as ref

pytestmark = pytest.mark.gpu


def ops():
    from flashmap_amd import ops as o

    return o


def _codes_close(got: torch.Tensor, want: torch.Tensor):
    g8, w8 = got.cpu().view(torch.uint8).long(), want.cpu().view(torch.uint8).long()
    same = (g8 == w8).float().mean().item()
    assert same >= 0.99, f"only {same:.4f} of the e4m3 bytes equal"
    off = g8 != w8
    # one code apart with the same sign (the codes of one sign are monotone in value)
    assert ((g8[off] - w8[off]).abs() == 1).all() and ((g8[off] >> 7) == (w8[off] >> 7)).all()


@pytest.mark.parametrize("d", [64, 128])
def test_vllm_fp8_writer(dev, d):
    g = gen(40 + d)
    tokens, layers, heads, page, blocks = 37, 2, 4, 16, 5
    kv = torch.randn(tokens, layers, 2, heads, d, generator=g).bfloat16()
    pos = torch.randint(0, 500, (tokens,), generator=g)
    slots = torch.randperm(blocks * page, generator=g)[:tokens].long()
    slots[5] = -1
    kn = torch.rand(layers, d, generator=g) + 0.5
    table = ref.rope_table(512, d, 1e6)
    scales = torch.tensor([[0.75, 1.5], [2.0, 0.5]])
    caches = [torch.zeros(blocks, heads, page, 2 * d, dtype=torch.uint8, device=dev) for _ in range(layers)]
    ptrs = torch.tensor([c.data_ptr() for c in caches], dtype=torch.int64, device=dev)
    c0 = caches[0]
    ops().write_context_kv_fp8(kv.to(dev), pos.to(dev), slots.to(dev), kn.to(dev), ops().rope_from_table(table.to(dev)),
                               ptrs, (c0.stride(0), c0.stride(1), c0.stride(2), d), page, 1e-6, scales.to(dev))
    torch.cuda.synchronize()
    want = [torch.zeros(blocks, heads, page, 2 * d, dtype=torch.float8_e4m3fn) for _ in range(layers)]
    ref.write_context_kv_vllm_fp8(kv, pos, slots, kn, table, want, page, 1e-6, scales)
    for got_c, want_c in zip(caches, want):
        _codes_close(got_c, want_c)


def test_pool_fp8_writer(dev):
    g = gen(50)
    tokens, layers, heads, d, pool = 24, 2, 2, 128, 64
    kv_size = heads * d
    kv = torch.randn(tokens, layers * 2 * kv_size, generator=g).bfloat16()
    pos = torch.randint(0, 300, (tokens,), generator=g)
    locs = torch.randperm(pool, generator=g)[:tokens].long()
    kn = torch.rand(layers, d, generator=g) + 0.5
    cat = ref.rope_cat_table(512, d, 1e6)
    kb = [torch.zeros(pool, heads, d, dtype=torch.uint8, device=dev) for _ in range(layers)]
    vb = [torch.zeros(pool, heads, d, dtype=torch.uint8, device=dev) for _ in range(layers)]
    meta = torch.tensor([[k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0)] for k, v in zip(kb, vb)],
                        dtype=torch.int64, device=dev)
    commit = torch.tensor([5, 8, 2], dtype=torch.int32)
    ops().write_context_kv_pool_fp8(kv.to(dev), meta, kn.to(dev), ops().rope_from_cat(cat.to(dev)), pos.to(dev),
                                    locs.to(dev), layers, kv_size, d, 1e-6, k_scale=0.625, v_scale=1.25,
                                    commit_lens=commit.to(dev), locs_row_width=8)
    torch.cuda.synchronize()
    wk = [torch.zeros(pool, heads, d, dtype=torch.float8_e4m3fn) for _ in range(layers)]
    wv = [torch.zeros(pool, heads, d, dtype=torch.float8_e4m3fn) for _ in range(layers)]
    ref.write_context_kv_pool_fp8(kv, wk, wv, kn, cat, pos, locs, layers, kv_size, d, 1e-6, k_scale=0.625,
                                  v_scale=1.25, commit_lens=commit, locs_row_width=8)
    for l in range(layers):
        _codes_close(kb[l], wk[l])
        _codes_close(vb[l], wv[l])


def _e4m3(shape, g, scale=1.0):
    """Unit-scale e4m3 data: outputs stay of order 1, where the absolute bar applies (at
    larger scales the bf16 rounding of the output alone approaches it)."""
    return ref.to_e4m3(torch.randn(*shape, generator=g) * scale)


@pytest.mark.parametrize("page,d,hq,hkv", [(16, 128, 32, 8), (8, 64, 8, 2), (16, 128, 16, 16), (32, 64, 40, 8),
                                         (16, 128, 48, 8), (8, 128, 24, 4), (64, 128, 8, 2), (128, 64, 16, 16),
                                         (24, 128, 8, 2)])
def test_paged_fp8_attention_descales(dev, page, d, hq, hkv):
    print(f"fp8 paged page={page} d={d} hq={hq} hkv={hkv}", flush=True)
    g = gen(60 + page + d + hq)
    bs, k_rows = 5, 16
    lens = torch.randint(1, 700, (bs,), generator=g)
    lens[2] = 0
    bt, total = paged_layout(lens.tolist(), page, g)
    cache = _e4m3((total, hkv, page, 2 * d), g)
    q8 = _e4m3((bs * k_rows, hq, d), g)
    cu = torch.arange(0, bs * k_rows + 1, k_rows, dtype=torch.int32)
    desc = torch.rand(3, bs, hkv, generator=g) + 0.25
    got = ops().block_attention_paged_fp8(q8.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                          k_rows, 700, d ** -0.5, descales=desc.to(dev))
    torch.cuda.synchronize()
    want = ref.block_attention_paged_vllm_fp8(q8, cache, cu, lens, bt, d ** -0.5, desc)
    check_close(got.cpu().float(), want)
    assert torch.count_nonzero(got[2 * k_rows:3 * k_rows]) == 0  # empty context: zeros


def test_paged_fp8_attention_expanded_scalar_descales(dev):
    """vLLM passes per-layer scalar scales expanded to (3, requests, heads)."""
    g = gen(70)
    bs, k_rows, hq, hkv, d, page = 3, 16, 16, 16, 128, 16
    lens = torch.randint(100, 900, (bs,), generator=g)
    bt, total = paged_layout(lens.tolist(), page, g)
    cache = _e4m3((total, hkv, page, 2 * d), g)
    q8 = _e4m3((bs * k_rows, hq, d), g)
    cu = torch.arange(0, bs * k_rows + 1, k_rows, dtype=torch.int32)
    scal = torch.tensor([0.8, 1.2, 0.6])
    desc = scal[:, None, None].expand(3, bs, hkv)
    got = ops().block_attention_paged_fp8(q8.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                          k_rows, 900, d ** -0.5, descales=desc.to(dev))
    torch.cuda.synchronize()
    check_close(got.cpu().float(), ref.block_attention_paged_vllm_fp8(q8, cache, cu, lens, bt, d ** -0.5, desc.contiguous()))


@pytest.mark.parametrize("q_len,hq,hkv", [(16, 16, 16), (32, 32, 8), (16, 40, 8)])
def test_token_paged_fp8_attention_quantizes_queries(dev, q_len, hq, hkv):
    print(f"fp8 token-paged q_len={q_len} hq={hq} hkv={hkv}", flush=True)
    g = gen(80 + q_len + hq)
    bs, d = 4, 128
    lens = torch.randint(1, 600, (bs,), generator=g)
    pool = int(lens.sum()) + 50
    perm = torch.randperm(pool, generator=g)
    pt = torch.zeros(bs, int(lens.max()), dtype=torch.int32)
    o = 0
    for b in range(bs):
        pt[b, :int(lens[b])] = perm[o:o + int(lens[b])].int()
        o += int(lens[b])
    kb, vb = _e4m3((pool, hkv, d), g), _e4m3((pool, hkv, d), g)
    query = (torch.randn(bs, q_len, hq, d, generator=g) * 3).bfloat16()
    got = ops().block_attention_token_paged_fp8(query.to(dev), kb.to(dev), vb.to(dev), lens.to(dev, torch.int32),
                                                pt.to(dev))
    torch.cuda.synchronize()
    check_close(got.cpu().float(), ref.block_attention_token_paged_fp8(query, kb, vb, lens, pt))


def test_token_paged_fp8_fused_prologue_equals_standalone(dev):
    g = gen(90)
    bs, q_len, hq, hkv, d = 3, 16, 16, 16, 128
    lens = torch.randint(50, 400, (bs,), generator=g)
    pool = int(lens.sum())
    pt = torch.arange(pool, dtype=torch.int32)
    pt = torch.stack([torch.nn.functional.pad(pt[int(lens[:b].sum()):int(lens[:b + 1].sum())], (0, int(lens.max()) - int(lens[b])))
                      for b in range(bs)])
    kb, vb = _e4m3((pool, hkv, d), g), _e4m3((pool, hkv, d), g)
    x = torch.randn(bs, q_len, hq, d, generator=g).bfloat16().to(dev)
    w = (torch.rand(d, generator=g) + 0.5).to(dev)
    table = ref.rope_table(1024, d, 1e6).to(dev)
    pos = torch.randint(0, 1024, (bs * q_len,), generator=g).to(dev)
    rope = ops().rope_from_table(table)
    args = (kb.to(dev), vb.to(dev), lens.to(dev, torch.int32), pt.to(dev))
    fused = ops().block_attention_token_paged_fp8(x, *args, prologue=ops().Prologue(w, rope, pos, 1e-6))
    normed = ops().rms_norm_rope(x.view(-1, hq, d), w, rope, pos, 1e-6).view(bs, q_len, hq, d)
    plain = ops().block_attention_token_paged_fp8(normed, *args)
    torch.cuda.synchronize()
    assert torch.equal(fused.cpu(), plain.cpu())


def test_paged_fp8_large_batch(dev):
    """More requests than the kernel stages in LDS (sequence metadata by scalar loads)."""
    g = gen(95)
    bs, k_rows, hq, hkv, d, page = 1100, 16, 8, 2, 64, 16
    lens = torch.randint(0, 80, (bs,), generator=g)
    bt, total = paged_layout(lens.tolist(), page, g)
    cache = _e4m3((total, hkv, page, 2 * d), g)
    q8 = _e4m3((bs * k_rows, hq, d), g)
    cu = torch.arange(0, bs * k_rows + 1, k_rows, dtype=torch.int32)
    got = ops().block_attention_paged_fp8(q8.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                          k_rows, 80, d ** -0.5)
    torch.cuda.synchronize()
    check_close(got.cpu().float(), ref.block_attention_paged_vllm_fp8(q8, cache, cu, lens, bt, d ** -0.5))



@pytest.mark.parametrize("cost", ["0", "1", "4", "40"])
def test_paged_fp8_share_cost_cuts(dev, tuning, cost):
    """The e4m3 kernel's line of 64-position tiles cut into shares by cost at any per-unit
    cost (0: by tiles; 40: the cost outweighs the tiles): every tile computed once and
    every partial merged, for sequences of 0 to 3000 positions."""
    print(f"fp8 share cost {cost}", flush=True)
    g = gen(97)
    hq, hkv, d, page, k_rows = 32, 8, 128, 16, 16
    lens = torch.tensor([0, 5, 65, 700, 1, 128, 3000, 63, 0, 129, 16, 450])
    bs = len(lens)
    bt, total = paged_layout(lens.tolist(), page, g)
    cache = _e4m3((total, hkv, page, 2 * d), g)
    q8 = _e4m3((bs * k_rows, hq, d), g)
    cu = torch.arange(0, bs * k_rows + 1, k_rows, dtype=torch.int32)
    desc = torch.rand(3, bs, hkv, generator=g) + 0.25
    tuning("FLASHMAP_SHARE_COST", cost)
    got = ops().block_attention_paged_fp8(q8.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev),
                                          k_rows, 3000, d ** -0.5, descales=desc.to(dev))
    torch.cuda.synchronize()
    check_close(got.cpu().float(), ref.block_attention_paged_vllm_fp8(q8, cache, cu, lens, bt, d ** -0.5, desc))


def test_paged_fp8_own_plan_equals_step_plan(dev):
    """An e4m3 call given no step plan computes its own in its query pass: the same bits as
    the call given ops.attention_plan's (whose second prefix counts 64-position tiles)."""
    g = gen(98)
    hq, hkv, d, page, k_rows = 32, 8, 128, 16, 16
    lens = torch.tensor([0, 5, 65, 700, 1, 3000, 63, 450])
    bs = len(lens)
    bt, total = paged_layout(lens.tolist(), page, g)
    cache = _e4m3((total, hkv, page, 2 * d), g).to(dev)
    q8 = _e4m3((bs * k_rows, hq, d), g).to(dev)
    cu = torch.arange(0, bs * k_rows + 1, k_rows, dtype=torch.int32).to(dev)
    lens_d = lens.to(dev, torch.int32)
    o = ops()
    own = o.block_attention_paged_fp8(q8, cache, cu, lens_d, bt.to(dev), k_rows, 3000, d ** -0.5)
    step = o.block_attention_paged_fp8(q8, cache, cu, lens_d, bt.to(dev), k_rows, 3000, d ** -0.5,
                                       plan=o.attention_plan(lens_d))
    assert torch.equal(own, step)


@pytest.mark.parametrize("q_len", [16, 32])
def test_paged_fp8_call_quantization_equals_callers(dev, q_len):
    """bf16 queries quantized inside the call (per (request, query head): scale = max(amax,
    1e-12) / 448, q / scale rounded to nearest even; flashmap/sglang/model.py:167-169) give
    the bits of the same queries quantized on the CPU by the oracle (float32 division,
    torch's e4m3 conversion) and passed as e4m3 with that scale as the query descale:
    the call's scale and codes equal the CPU's exactly. One query head per KV head, so
    that the descales' (request, KV head) grid holds every head's scale. Heads span 1e-14
    (below the 1e-12 floor) to 1e3, and one is all zeros."""
    print(f"fp8 call quantization q_len={q_len}", flush=True)
    g = gen(99 + q_len)
    bs, h, d, page = 4, 8, 128, 16
    lens = torch.tensor([37, 600, 0, 255])
    bt, total = paged_layout(lens.tolist(), page, g)
    cache = _e4m3((total, h, page, 2 * d), g)
    mag = torch.tensor([1e-3, 3.0, 1e3, 0.0, 1e-14, 0.25, 40.0, 1.0])
    q = (torch.randn(bs, q_len, h, d, generator=g) * mag[None, None, :, None]).bfloat16()
    q8, qscale = ref.quantize_query_per_head(q)  # (bs, T, H, D) e4m3, (bs, H)
    kv_desc = torch.rand(2, bs, h, generator=g) + 0.25
    cu = torch.arange(0, bs * q_len + 1, q_len, dtype=torch.int32)
    args = (cache.to(dev), cu.to(dev), lens.to(dev, torch.int32), bt.to(dev), q_len, 600, d ** -0.5)
    in_call = ops().block_attention_paged_fp8(q.view(-1, h, d).to(dev), *args,
                                              descales=torch.cat([torch.ones(1, bs, h), kv_desc]).to(dev))
    by_caller = ops().block_attention_paged_fp8(q8.view(-1, h, d).to(dev), *args,
                                                descales=torch.cat([qscale[None], kv_desc]).to(dev))
    torch.cuda.synchronize()
    assert torch.count_nonzero(by_caller[2 * q_len:3 * q_len]) == 0  # a request without context
    assert torch.equal(in_call.cpu(), by_caller.cpu())


@pytest.mark.parametrize("descales", [False, True])
@pytest.mark.parametrize("layout,d,hq,hkv", [("paged", 128, 32, 8), ("pool", 128, 32, 8), ("paged", 64, 8, 2),
                                            ("pool", 64, 40, 8)])
def test_fp8_direct_rows_equal_query_pass(dev, tuning, layout, d, hq, hkv, descales):
    """e4m3 calls with bf16 queries: the attention kernel normalizes, rotates and quantizes
    each (request, query head) of the caller's rows itself (direct rows), or the query pass
    does: the same bits either way (the same prologue arithmetic, the same amax, the same
    correctly rounded divisions), for ragged draft rows, a request without context and,
    on vLLM's layout, key descales; both within the bar of the dequantized oracle."""
    print(f"fp8 direct rows {layout} d={d} hq={hq} hkv={hkv} descales={descales}", flush=True)
    g = gen(99 + descales + d)
    page, k_rows = 16, 16
    lens = torch.tensor([700, 33, 1, 260, 0, 1500])
    bs = len(lens)
    o = ops()
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(int(lens.max()) + k_rows + 1, d, 1e6)
    pro_rows = torch.tensor([16, 9, 16, 3, 16, 16]) if layout == "paged" else torch.full((bs,), k_rows)
    cu = torch.cat([torch.zeros(1, dtype=torch.int32), pro_rows.cumsum(0).to(torch.int32)])
    pos = torch.cat([int(n) + torch.arange(int(r)) for n, r in zip(lens, pro_rows)])
    n_tok = int(cu[-1])
    q_pre = (torch.randn(n_tok, hq, d, generator=g) * 2).bfloat16()
    pro = o.Prologue(w.to(dev), o.rope_from_table(table.to(dev)), pos.to(dev), 1e-6)
    desc = (torch.rand(3, bs, hkv, generator=g) + 0.25) if descales else None
    if layout == "paged":
        bt, total = paged_layout(lens.tolist(), page, g)
        cache = _e4m3((total, hkv, page, 2 * d), g)

        def run():
            return o.block_attention_paged_fp8(q_pre.to(dev), cache.to(dev), cu.to(dev), lens.to(dev, torch.int32),
                                               bt.to(dev), k_rows, int(lens.max()), d ** -0.5, prologue=pro,
                                               descales=None if desc is None else desc.to(dev))
    else:
        if descales:
            pytest.skip("the pool call takes no descales (its pools are written with scale 1)")
        pool = int(lens.sum()) + 11
        perm = torch.randperm(pool, generator=g)
        pt = torch.zeros(bs, int(lens.max()), dtype=torch.int32)
        off = 0
        for b in range(bs):
            pt[b, :int(lens[b])] = perm[off:off + int(lens[b])].int()
            off += int(lens[b])
        kb, vb = _e4m3((pool, hkv, d), g), _e4m3((pool, hkv, d), g)

        def run():
            return o.block_attention_token_paged_fp8(q_pre.view(bs, k_rows, hq, d).to(dev), kb.to(dev), vb.to(dev),
                                                     lens.to(dev, torch.int32), pt.to(dev), prologue=pro)
    tuning("FLASHMAP_SHARE_COST", "4")  # one cut of the line for both
    outs = {}
    for mode in ("1", "0"):
        tuning("FLASHMAP_QUERY_PASS", mode)
        outs[mode] = run()
    torch.cuda.synchronize()
    assert torch.equal(outs["0"], outs["1"]), "direct rows differ from the query pass"
    qn = ref.rms_norm_rope_vllm(q_pre, w, table, pos, 1e-6)
    got = outs["0"].cpu().float().view(-1, hq, d)
    if layout == "paged":
        for b in range(bs):
            s, e = int(cu[b]), int(cu[b + 1])
            q8, qs = ref.quantize_query_per_head(qn[s:e][None])  # per (request, query head)
            qdq = q8[0].float() * qs[0][None, :, None]
            kv_desc = torch.ones(3, 1, hkv)
            if desc is not None:
                kv_desc[1:, 0] = desc[1:, b]
            want = ref.block_attention_paged_vllm_fp8(qdq, cache, torch.tensor([0, e - s], dtype=torch.int32),
                                                      lens[b:b + 1], bt[b:b + 1], d ** -0.5, kv_desc)
            check_close(got[s:e], want)
    else:
        want = ref.block_attention_token_paged_fp8(qn.view(bs, k_rows, hq, d), kb, vb, lens, pt)
        check_close(got.view(bs, k_rows, hq, d), want)

