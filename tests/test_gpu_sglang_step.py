"""The SGLang plugin's one-jump draft step (flashmap_amd.sglang_step.SGLangDraftStep,
flashmap/sglang/model.py:837-1057) on the GPU, against the oracle's SGLang composition
(oracle/draft_step.py ``pool_*``: the DiT of the draft-step oracle, which the reference's
own ``draft`` fixtures pin on the CPU, over token pools) prepared from the drafter's raw
weights: the pools' context and anchor rows, the final hidden rows, the logits and the
greedy tokens; one candidate per request and tree drafting's candidates side by side
(each request's blocks attending together to its one context); the sampler over the
step's logits.

Bars as the vLLM step's (tests/test_gpu_draft_step.py): pool rows within two bf16 ulps
plus one ulp of the row's RMS; hidden rows within four ulps plus 2 % of the row's RMS per
element and 1 % in RMS over the row; logits within 1 % of the largest and 1 % of the mean
|logit|; greedy tokens equal on every row whose top-2 margin exceeds twice the logit
error."""

import math

import pytest
import torch

from _inputs import gen
from flashmap_amd import drafter as d
from flashmap_amd import fold
from flashmap_amd.sglang_step import SGLangDraftStep
from oracle import draft_step as oracle

pytestmark = pytest.mark.gpu

BASE = dict(target_hidden_size=128, vocab_size=512, target_layer_ids=[0, 1], block_size=16, hidden_size=256,
            num_hidden_layers=2, num_attention_heads=2, intermediate_size=512, cond_dim=32, time_embed_dim=32,
            rope_theta=1e6)


def _model(over, dev, seed):
    torch.manual_seed(seed)
    m = d.FlashMapDraftModel(dict(BASE, **over))
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight") or name == "noise_gate":
                p.copy_(0.75 + 0.5 * torch.rand(p.shape))
            elif name.endswith(".bias"):
                p.copy_(0.02 * torch.randn(p.shape))
            elif "adaln.linear" in name:
                p.normal_(0.0, 0.05)
            else:
                p.normal_(0.0, 1.0 / math.sqrt(p.shape[-1]))
    return m.to(dev, torch.bfloat16)


def _close_rows(got, want, what, ulps=2, rel=2.0 ** -7, row_rel=None):
    w = want.float().reshape(-1, want.shape[-1])
    g = got.float().cpu().reshape(w.shape)
    err = (g - w).abs()
    rms = w.pow(2).mean(-1, keepdim=True).sqrt()
    bad = err > ulps * 2.0 ** -7 * w.abs() + rel * rms
    row = err.pow(2).mean(-1).sqrt() / rms.squeeze(-1).clamp_min(1e-30)
    print(f"  {what}: max err {err.max():.4f}, worst row RMS error {row.max():.4f}, {int(bad.sum())} past the bar",
          flush=True)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {err.max():.4f}"
    if row_rel is not None:
        assert row.max() <= row_rel, f"{what}: a row's RMS error is {row.max():.4f} of its RMS"


@pytest.mark.parametrize("name,over,n_cand", [
    ("gelu_full_vocab", dict(mlp_type="gelu"), 1),
    ("swiglu_state_vocab", dict(mlp_type="swiglu", state_vocab_size=200), 1),
    ("gelu_tree", dict(mlp_type="gelu"), 4),
])
def test_sglang_step_matches_the_oracle(dev, name, over, n_cand):
    print(f"sglang draft step {name}, {n_cand} candidate(s) per request", flush=True)
    model = _model(over, dev, 17)
    cfg = model.config
    g = gen(21)
    embed = torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g).bfloat16().to(dev)
    lm_head = (torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g) / 8).bfloat16().to(dev)
    hot = torch.arange(1, 2 * cfg.state_vocab_size, 2).to(dev) if cfg.state_vocab_size else None
    step = SGLangDraftStep(model, embed, lm_head, max_positions=400, hot_ids=hot)
    lens = torch.tensor([45, 0, 130, 77])  # context positions before each anchor
    requests, k = len(lens), cfg.block_size
    pool = int(lens.sum()) + requests + 9
    perm = torch.randperm(pool, generator=g)
    page_table = torch.zeros(requests, int(lens.max()) + 1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(lens.tolist()):
        page_table[r, :n + 1] = perm[o:o + n + 1].int()  # the context, then the anchor's row
        o += n + 1
    heads, hd = step.heads, step.head_dim
    k_bufs = [torch.zeros(pool, heads, hd, dtype=torch.bfloat16, device=dev) for _ in model.layers]
    v_bufs = [torch.zeros_like(b) for b in k_bufs]
    meta = step.pool_meta(k_bufs, v_bufs)
    pos = torch.cat([torch.arange(n) for n in lens.tolist()])
    req = torch.cat([torch.full((n,), r) for r, n in enumerate(lens.tolist())])
    locs = page_table[req, pos].long()
    feats = torch.randn(len(pos), len(cfg.target_layer_ids) * cfg.target_hidden_size, generator=g).bfloat16()
    step.write_context(feats.to(dev), pos.to(dev), locs.to(dev), meta)
    anchors = torch.randint(0, cfg.vocab_size, (requests,), generator=g)
    a_locs = page_table[torch.arange(requests), lens].long()
    z = torch.randn(requests * n_cand * k, cfg.target_hidden_size, generator=g)
    hidden = step(anchors.to(dev), lens.to(dev), a_locs.to(dev), z.to(dev), k_bufs, v_bufs, page_table.to(dev),
                  n_cand=n_cand, meta=meta)
    logits = step.logits(hidden)
    greedy = torch.ones(hidden.shape[0], dtype=torch.bool, device=dev)
    tokens = step.sample(hidden, torch.ones(hidden.shape[0], device=dev), greedy,
                         torch.tensor(5, dtype=torch.int64, device=dev))
    torch.cuda.synchronize()

    sd = {key: v.detach().cpu() for key, v in model.state_dict().items()}
    w = oracle.prepare(sd, dict(vars(cfg)), embed.cpu(), lm_head.cpu(), None if hot is None else hot.cpu(), 1, 400)
    rk = [torch.zeros(pool, heads, hd, dtype=torch.bfloat16) for _ in model.layers]
    rv = [torch.zeros_like(b) for b in rk]
    oracle.pool_write_context(w, feats, pos, locs, rk, rv)
    oracle.pool_write_anchors(w, anchors, lens, a_locs, rk, rv)
    for i in range(len(rk)):
        _close_rows(k_bufs[i], rk[i], f"keys {i}")
        _close_rows(v_bufs[i], rv[i], f"values {i}")
    state_rows = embed[hot] if hot is not None else embed
    noise_embeds = (z.to(dev).double() @ fold.noise_factor(state_rows)[0]).bfloat16().cpu()
    want_h, want = oracle.pool_draft(w, lens, rk, rv, page_table, noise_embeds, n_cand)
    _close_rows(hidden, want_h, "hidden", ulps=4, rel=2e-2, row_rel=1e-2)
    got = logits.float().cpu()
    want = want.float()
    err = (got - want).abs()
    top2 = want.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * err.max()
    want_tok = want.argmax(-1) if hot is None else hot.cpu()[want.argmax(-1)]
    same = tokens.cpu() == want_tok
    print(f"  logits max err {err.max():.4f} (max |logit| {want.abs().max():.3f}), mean err {err.mean():.5f} "
          f"(mean |logit| {want.abs().mean():.4f}); clear-margin rows {clear.float().mean():.3f}; greedy tokens "
          f"equal on {same.float().mean():.3f}", flush=True)
    assert err.max() <= 0.01 * want.abs().max() and err.mean() <= 0.01 * want.abs().mean()
    assert clear.float().mean() >= 0.6 and same[clear].all()


def test_sglang_step_candidates_are_independent_blocks(dev):
    """Tree drafting: a request's candidate blocks side by side give each block what it
    gives drafted alone (one candidate, its own noise), within the bf16 bar."""
    model = _model(dict(mlp_type="gelu"), dev, 19)
    cfg = model.config
    g = gen(23)
    embed = torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g).bfloat16().to(dev)
    lm_head = (torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g) / 8).bfloat16().to(dev)
    step = SGLangDraftStep(model, embed, lm_head, max_positions=400)
    n, k, n_cand = 150, cfg.block_size, 3
    heads, hd = step.heads, step.head_dim
    k_bufs = [torch.zeros(n + 8, heads, hd, dtype=torch.bfloat16, device=dev) for _ in model.layers]
    v_bufs = [torch.zeros_like(b) for b in k_bufs]
    meta = step.pool_meta(k_bufs, v_bufs)
    page_table = torch.randperm(n + 8, generator=g)[:n + 1].int()[None].to(dev)
    pos = torch.arange(n, device=dev)
    feats = torch.randn(n, len(cfg.target_layer_ids) * cfg.target_hidden_size, generator=g).bfloat16().to(dev)
    step.write_context(feats, pos, page_table[0, :n].long(), meta)
    anchor = torch.randint(0, cfg.vocab_size, (1,), generator=g).to(dev)
    a_pos = torch.tensor([n], device=dev)
    a_loc = page_table[0, n:n + 1].long()
    z = torch.randn(n_cand * k, cfg.target_hidden_size, generator=g).to(dev)
    together = step(anchor, a_pos, a_loc, z, k_bufs, v_bufs, page_table, n_cand=n_cand, meta=meta)
    for c in range(n_cand):
        alone = step(anchor, a_pos, a_loc, z[c * k:(c + 1) * k].contiguous(), k_bufs, v_bufs, page_table,
                     meta=meta)
        # the same attention split differently (48 rows of a unit, or 16): merges in another order
        _close_rows(together[c * k:(c + 1) * k], alone.cpu(), f"candidate {c}", ulps=4, rel=2e-2, row_rel=1e-2)
