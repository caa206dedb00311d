"""The benchmark configurations, each run as its own call on the GPU and checked against
the float32 oracle (max-abs 2e-2, mean-abs 2e-3 on the bf16 outputs):

- C1's shape: hidden 1024, 16 q / 8 KV heads, head_dim 64, K = 16 draft rows, batch 1,
  512 context positions, drawn as the configuration states it (hidden states N(0, 1),
  projection weights N(0, 0.02), QK-RMSNorm weight 1, eps 1e-6, RoPE theta 1e6, query
  positions 512 + 0..15); keys k-normed and rotated by the GPU prologue, the queries'
  prologue fused into the contiguous attention call;
- C2 at its full size: contiguous batch 1 x 2048 positions, 32 q / 8 KV heads, head_dim
  128, fused prologue, query positions 2048 + 0..15;
- C3 (batch 64, contexts U[256, 8192]), C4 (batch 8 x 32768), C5 (GQA 5, batch 32,
  U[1024, 8192]) and R8B (MHA 16/16, batch 64, U[256, 8192]; its 1024 units take the query
  pass): exactly the call bench.py times -- the query prologue fused, the step
  plan computed once and passed in, the paged op over the cache the context writer
  filled -- with every sequence of the batch checked against the oracle's prologue,
  block-table gather and attention; and C3's call on an e4m3 cache the same way;
- the SGLang drafter's call on token pools at C3's shape (bf16 and e4m3 pools) and the
  tree-drafting calls, every request against the oracle's gather and attention;
- the target verify call (64 requests x 17 chain tokens on a pool), every request against
  the verify oracle;
- C3 through the virtual context-cache layout (4 runs), bit-identical to the per-layer call.
"""

import pytest
import torch

from _inputs import check_close
from oracle import attention as ref

pytestmark = pytest.mark.gpu

EPS, THETA = 1e-6, 1e6


def _ops():
    from flashmap_amd import ops

    return ops


def test_c1_shape_fused_prologue(dev):
    ops = _ops()
    hidden, hq, hkv, d, k_rows, ctx = 1024, 16, 8, 64, 16, 512
    print("C1 shape: hidden 1024, 16/8 heads, D 64, ctx 512", flush=True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, k_rows, hidden, generator=g)
    h = torch.randn(1, ctx, hidden, generator=g)
    wq = torch.randn(hq * d, hidden, generator=g) * 0.02
    wk = torch.randn(hkv * d, hidden, generator=g) * 0.02
    wv = torch.randn(hkv * d, hidden, generator=g) * 0.02
    q_pre = (x @ wq.T).bfloat16().view(1, k_rows, hq, d)
    k_pre = (h @ wk.T).bfloat16().view(ctx, hkv, d)
    v = (h @ wv.T).bfloat16().view(1, ctx, hkv, d).transpose(1, 2).contiguous()
    w = torch.ones(d)
    table = ref.rope_table(ctx + k_rows + 1, d, THETA)
    kpos, qpos = torch.arange(ctx), ctx + torch.arange(k_rows)

    rope = ops.rope_from_table(table.to(dev))
    keys = ops.rms_norm_rope(k_pre.to(dev), w.to(dev), rope, kpos.to(dev), EPS)
    want_keys = ref.rms_norm_rope_vllm(k_pre, w, table, kpos, EPS)
    assert (keys.cpu() == want_keys).float().mean() > 0.99
    keys = keys.view(1, ctx, hkv, d).transpose(1, 2).contiguous()
    got = ops.block_attention_contig(q_pre.to(dev), keys, v.to(dev), d ** -0.5,
                                     prologue=ops.Prologue(w.to(dev), rope, qpos.to(dev), EPS))
    qn = ref.rms_norm_rope_vllm(q_pre.view(k_rows, hq, d), w, table, qpos, EPS).view(1, k_rows, hq, d)
    want = ref.block_attention_contig(qn, want_keys.view(1, ctx, hkv, d).transpose(1, 2), v)
    err = check_close(got, want)
    print(f"C1: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)


def test_c2_full_size_fused_prologue(dev):
    ops = _ops()
    hq, hkv, d, k_rows, ctx = 32, 8, 128, 16, 2048
    print("C2 full size: contiguous 1 x 2048, 32/8 heads, D 128", flush=True)
    g = torch.Generator().manual_seed(0)
    q_pre = torch.randn(1, k_rows, hq, d, generator=g).bfloat16()
    keys = torch.randn(1, hkv, ctx, d, generator=g).bfloat16()
    values = torch.randn(1, hkv, ctx, d, generator=g).bfloat16()
    w = torch.rand(d, generator=g) + 0.5
    table = ref.rope_table(ctx + k_rows + 1, d, THETA)
    qpos = ctx + torch.arange(k_rows)
    pro = ops.Prologue(w.to(dev), ops.rope_from_table(table.to(dev)), qpos.to(dev), EPS)
    got = ops.block_attention_contig(q_pre.to(dev), keys.to(dev), values.to(dev), d ** -0.5, prologue=pro)
    qn = ref.rms_norm_rope_vllm(q_pre.view(k_rows, hq, d), w, table, qpos, EPS).view(1, k_rows, hq, d)
    want = ref.block_attention_contig(qn, keys, values)
    err = check_close(got, want)
    print(f"C2: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)


def _bench_call(dev, workload, fp8=False):
    """The inputs and the output of bench.py's timed call for ``workload`` (``fp8``: its
    e4m3 twin, the cache written by the fp8 context writer with scales 1)."""
    import bench

    ops = _ops()
    inp = bench.build_inputs(workload)
    batch, hkv, d, k_rows, page = (inp[k] for k in ("batch", "hkv", "d", "k_rows", "page"))
    table = ref.rope_table(inp["hi"] + k_rows + 1, d, THETA)
    rope = ops.rope_from_table(table.to(dev))
    w = torch.ones(d, device=dev)
    lens = inp["lens"].to(dev, torch.int32)
    cache = torch.zeros(inp["total"], hkv, page, 2 * d, dtype=torch.uint8 if fp8 else torch.bfloat16, device=dev)
    ptrs = torch.tensor([cache.data_ptr()], dtype=torch.int64, device=dev)
    writer_args = (inp["kv_pre"].to(dev), inp["positions"].to(dev), inp["slots"].to(dev),
                   w[None].expand(1, d).contiguous(), rope, ptrs,
                   (cache.stride(0), cache.stride(1), cache.stride(2), d), page, EPS)
    if fp8:
        ops.write_context_kv_fp8(*writer_args, torch.ones(1, 2, device=dev))
    else:
        ops.write_context_kv(*writer_args)
    qpos = torch.cat([int(n) + torch.arange(k_rows) for n in inp["lens"]])
    cu = (torch.arange(batch + 1, dtype=torch.int32) * k_rows).to(dev)
    pro = ops.Prologue(w, rope, qpos.to(dev), EPS)
    plan = ops.attention_plan(lens)
    call = ops.block_attention_paged_fp8 if fp8 else ops.block_attention_paged
    out = call(inp["q_pre"].to(dev), cache, cu, lens, inp["bt"].to(dev), k_rows, inp["hi"], d ** -0.5, prologue=pro,
               plan=plan)
    torch.cuda.synchronize()
    return inp, table, qpos, cache, out


@pytest.mark.parametrize("workload", [
    "c3-qwen3-8b-paged-b64", "c4-qwen3-8b-long-b8", "c5-27b-gqa5-b32", "r8b-mha-b64"])
def test_bench_call_every_sequence(dev, workload):
    print(f"bench call {workload}", flush=True)
    inp, table, qpos, cache, out = _bench_call(dev, workload)
    k_rows, d, hq = inp["k_rows"], inp["d"], inp["hq"]
    w = torch.ones(d)
    qn = ref.rms_norm_rope_vllm(inp["q_pre"], w, table, qpos, EPS)
    bt = inp["bt"]
    worst = 0.0
    for b in range(inp["batch"]):
        n = int(inp["lens"][b])
        pages = bt[b, :(n + inp["page"] - 1) // inp["page"]].long().to(dev)
        rows = cache[pages].transpose(1, 2).reshape(-1, inp["hkv"], 2 * d)[:n].float().cpu()  # (n, Hkv, 2D)
        k, v = rows[..., :d].transpose(0, 1), rows[..., d:].transpose(0, 1)
        want = ref.attention(qn[b * k_rows:(b + 1) * k_rows].float().transpose(0, 1), k, v, d ** -0.5)
        err = check_close(out[b * k_rows:(b + 1) * k_rows].cpu().float(), want.transpose(0, 1))
        worst = max(worst, err.max().item())
    assert out.shape == (inp["batch"] * k_rows, hq, d)
    print(f"{workload}: {inp['batch']} sequences, worst max-abs {worst:.3e}", flush=True)


def test_bench_call_every_sequence_e4m3(dev):
    """The e4m3 call bench.py times (c3-qwen3-8b-paged-b64-fp8): C3's draw, the cache written
    by the fp8 context writer with scales 1, the bf16 queries normed, rotated and quantized
    per (sequence, query head) inside the call. Every sequence against the oracle's
    prologue, its per-head quantization (flashmap/sglang/model.py:167-169, the bits the
    call's own are pinned to) and the attention of the dequantized operands in float32."""
    print("bench call c3-qwen3-8b-paged-b64-fp8", flush=True)
    inp, table, qpos, cache, out = _bench_call(dev, "c3-qwen3-8b-paged-b64", fp8=True)
    batch, k_rows, d, hq, hkv = inp["batch"], inp["k_rows"], inp["d"], inp["hq"], inp["hkv"]
    qn = ref.rms_norm_rope_vllm(inp["q_pre"], torch.ones(d), table, qpos, EPS)
    q8, qs = ref.quantize_query_per_head(qn.view(batch, k_rows, hq, d))
    qd = q8.float() * qs[:, None, :, None]  # the queries as the call's scores see them
    bt = inp["bt"]
    worst = 0.0
    for b in range(batch):
        n = int(inp["lens"][b])
        pages = bt[b, :(n + inp["page"] - 1) // inp["page"]].long().to(dev)
        rows = cache[pages].view(torch.float8_e4m3fn).transpose(1, 2).reshape(-1, hkv, 2 * d)[:n].float().cpu()
        k, v = rows[..., :d].transpose(0, 1), rows[..., d:].transpose(0, 1)
        want = ref.attention(qd[b].transpose(0, 1), k, v, d ** -0.5)
        err = check_close(out[b * k_rows:(b + 1) * k_rows].cpu().float(), want.transpose(0, 1))
        worst = max(worst, err.max().item())
    assert out.shape == (batch * k_rows, hq, d)
    print(f"c3 e4m3: {batch} sequences, worst max-abs {worst:.3e}", flush=True)


@pytest.mark.parametrize("workload", ["c3shape-sglang-pool-b64", "c3shape-sglang-pool-b64-fp8", "tree-r8b-b4-n8",
                                      "tree-r8b-b1-n32"])
def test_token_pool_bench_call_every_request(dev, workload):
    """The SGLang drafter's cross-attention on token pools as bench.py times it
    (``bench.tree_inputs``; at C3's shape: 64 requests, contexts U[256, 8192] at permuted
    slots of (pool, 8, 128) pools, 16 rows x 32 heads each; tree drafting: 4 requests x 8
    candidates and 1 x 32, 16/16 heads, the candidates' rows side by side; the step plan
    passed in): every request against the oracle's gather and attention. e4m3 pools: the queries quantized per
    (request, query head) by the oracle (the bits the call's own are pinned to), the pools
    dequantized."""
    import bench

    print(f"bench call {workload}", flush=True)
    ops = _ops()
    lens, pt, q, kb, vb = bench.tree_inputs(workload)
    fp8 = kb.dtype == torch.float8_e4m3fn
    lens_d = lens.to(dev, torch.int32)
    call = ops.block_attention_token_paged_fp8 if fp8 else ops.block_attention_token_paged
    out = call(q.to(dev), kb.to(dev), vb.to(dev), lens_d, pt.to(dev), plan=ops.attention_plan(lens_d))
    torch.cuda.synchronize()
    requests, q_len, hq, d = q.shape
    if fp8:
        q8, qs = ref.quantize_query_per_head(q)
        qd = q8.float() * qs[:, None, :, None]
        kb, vb = kb.view(torch.uint8), vb.view(torch.uint8)  # gathered as bytes, then widened
    else:
        qd = q.float()
    out = out.cpu().float()
    worst = 0.0
    for b in range(requests):
        rows = pt[b, :int(lens[b])].long()
        k, v = kb[rows], vb[rows]
        if fp8:
            k, v = k.view(torch.float8_e4m3fn), v.view(torch.float8_e4m3fn)
        want = ref.attention(qd[b].transpose(0, 1), k.float().transpose(0, 1), v.float().transpose(0, 1), d ** -0.5)
        err = check_close(out[b], want.transpose(0, 1))
        worst = max(worst, err.max().item())
    print(f"{workload}: {requests} requests, worst max-abs {worst:.3e}", flush=True)


def test_verify_bench_call_every_request(dev):
    """The target verify call as bench.py times it (``bench.verify_inputs`` of
    verify-qwen3-8b-chain-b64: 64 requests x 17 chain tokens, 32/8 heads, contexts
    U[256, 8192] at permuted slots of (pool, 8, 128) pools, causal among the verify tokens):
    every request against the verify oracle on its gathered context."""
    import bench

    print("bench call verify-qwen3-8b-chain-b64", flush=True)
    ops = _ops()
    lens, q, k_ext, v_ext, kb, vb, indptr, indices, cmask = bench.verify_inputs("verify-qwen3-8b-chain-b64")
    assert cmask is None
    length = q.shape[0] // len(lens)
    out = ops.verify_attention(q.to(dev), k_ext.to(dev), v_ext.to(dev), kb.to(dev), vb.to(dev), indptr.to(dev),
                               indices.to(dev), None, None, False, max_context=int(lens.max()))
    out = out.cpu().float()
    worst = 0.0
    for b in range(len(lens)):
        lo_, hi_ = int(indptr[b]), int(indptr[b + 1])
        rows = indices[lo_:hi_].long()
        tok = slice(b * length, (b + 1) * length)
        want = ref.verify_attention(q[tok], k_ext[tok], v_ext[tok], kb[rows], vb[rows],
                                    torch.tensor([0, hi_ - lo_], dtype=torch.int32), torch.arange(hi_ - lo_))
        err = check_close(out[tok], want)
        worst = max(worst, err.max().item())
    print(f"verify: {len(lens)} requests, worst max-abs {worst:.3e}", flush=True)


def test_virtual_layout_bench_call_equals_per_layer(dev):
    """The virtual context-cache call as bench.py times it (c3-qwen3-8b-virtual-hpc3: C3's
    draw written for 2 DiT layers into caches of 3 heads each, layer 1's 8 KV heads in 4
    runs, flashmap/vllm/context_cache.py): the same bits as the per-layer call on a cache of
    the layer's 8 heads, which test_bench_call_every_sequence checks against the oracle."""
    import bench
    from flashmap_amd import context_cache as cc

    print("bench call c3-qwen3-8b-virtual-hpc3", flush=True)
    ops = _ops()
    _, hpc, layer = bench.VIRTUAL_WORKLOADS["c3-qwen3-8b-virtual-hpc3"]
    inp, _, qpos, _, per_layer = _bench_call(dev, "c3-qwen3-8b-paged-b64")
    hkv, d, k_rows, page = inp["hkv"], inp["d"], inp["k_rows"], inp["page"]
    table = ref.rope_table(inp["hi"] + k_rows + 1, d, THETA)
    rope = ops.rope_from_table(table.to(dev))
    w = torch.ones(d, device=dev)
    vplan = cc.ContextCachePlan(layer + 1, hkv, -(-(layer + 1) * hkv // hpc), hpc, True, "")
    caches = [torch.zeros(inp["total"], hpc, page, 2 * d, dtype=torch.bfloat16, device=dev)
              for _ in range(vplan.num_caches)]
    c0 = caches[0]
    ops.write_context_kv(inp["kv_pre"].to(dev).repeat(1, layer + 1, 1, 1, 1), inp["positions"].to(dev),
                         inp["slots"].to(dev), w[None].expand(layer + 1, d).contiguous(), rope,
                         torch.tensor([c.data_ptr() for c in caches], dtype=torch.int64, device=dev),
                         (c0.stride(0), c0.stride(1), c0.stride(2), d), page, EPS, heads_per_cache=hpc)
    runs = vplan.segments[layer]
    assert len(runs) == 4
    lens = inp["lens"].to(dev, torch.int32)
    cu = (torch.arange(inp["batch"] + 1, dtype=torch.int32) * k_rows).to(dev)
    pro = ops.Prologue(w, rope, qpos.to(dev), EPS)
    got = ops.block_attention_paged_runs(inp["q_pre"].to(dev), caches, runs, cu, lens, inp["bt"].to(dev), k_rows,
                                         inp["hi"], d ** -0.5, prologue=pro, plan=ops.attention_plan(lens))
    torch.cuda.synchronize()
    assert torch.equal(got, per_layer)
