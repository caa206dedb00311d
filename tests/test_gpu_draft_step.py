"""The one-jump draft step (flashmap_amd.draft_step.DraftStep, the vLLM plugin's step of
flashmap/vllm/model.py:779-925, 1039-1041) against the oracle (oracle/draft_step.py) on
tiny random drafters: the anchors' rows written into the paged caches, the final AdaLN
output, the draft logits and the greedy draft tokens; and the noise read-out's row pass
(fm_noise_rows) against its definition.

Bars: cache rows within two bf16 ulps of their magnitude per element (projections and
norms round on GPU and CPU in different summation orders), hidden rows (two DiT layers of
such roundings) within four ulps plus 1 % of their mean magnitude, both with mean-abs
within 2e-3 of the values' scale; logits within 1 % of the largest logit (max) and 0.3 % of
the mean |logit| (mean; a bf16 ulp is 0.4-0.8 % of a logit); greedy tokens equal wherever the oracle's top-2 margin exceeds twice the
observed logit error."""

import math
from types import SimpleNamespace

import pytest
import torch

from _inputs import gen, paged_layout
from flashmap_amd import drafter as d
from flashmap_amd import ops
from flashmap_amd.draft_step import DraftStep
from oracle import draft_step as oracle

pytestmark = pytest.mark.gpu

CASES = {
    "gelu_full_vocab": dict(mlp_type="gelu"),
    "swiglu_state_vocab": dict(mlp_type="swiglu", state_vocab_size=200),
}
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


def _weights(step: DraftStep):
    """The oracle's plain-tensor view of the prepared step (CPU)."""
    m, cpu = step.model, (lambda t: t.detach().cpu())
    w = {"embed": cpu(step.embed_weight), "anchor_proj.weight": cpu(m.anchor_proj.weight),
         "anchor_proj.bias": cpu(m.anchor_proj.bias), "anchor_norm.weight": cpu(m.anchor_norm.weight),
         "anchor_norm.eps": m.anchor_norm.eps, "context_kv_weight": cpu(step.context_kv_weight),
         "context_k_norm": cpu(step.context_k_norm), "k_eps": step.k_eps, "cos_sin": cpu(step.cos_sin),
         "heads": step.heads, "block": step.block, "noise_eigvals": cpu(step.noise_eigvals),
         "noise_embed": cpu(step.noise_embed), "noise_eps": step.noise_eps, "gain": step.noise_gain,
         "first_hidden": cpu(step.first_hidden), "ln_eps": m.final_adaln.eps,
         "final_mod": [cpu(t) for t in step.final_mod], "head_weight": cpu(step.head_weight),
         "head_bias": cpu(step.head_bias), "layers": []}
    for i, layer in enumerate(m.layers):
        lw = {"mods": [[cpu(t) for t in mod] for mod in step.layer_mods[i]], "self_qkv": cpu(step.self_qkv[i]),
              "self_q_norm": cpu(layer.self_attn.q_norm.weight), "self_k_norm": cpu(layer.self_attn.k_norm.weight),
              "qk_eps": layer.self_attn.q_norm.eps, "self_o": cpu(layer.self_attn.o_proj.weight),
              "cross_q": cpu(layer.cross_attn.q_proj.weight), "cross_q_norm": cpu(layer.cross_attn.q_norm.weight),
              "cross_o": cpu(layer.cross_attn.o_proj.weight)}
        lw.update({k: cpu(v) for k, v in layer.mlp.state_dict().items()})
        w["layers"].append(lw)
    return w


def _close_rows(got, want, what, ulps=2, slack=2e-3):
    g, w = got.float().cpu(), want.float()
    err = (g - w).abs()
    bad = err > ulps * 2.0 ** -7 * w.abs() + slack * float(w.abs().mean())
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {err.max():.4f}"
    assert err.mean() <= 2e-3 * max(float(w.abs().mean()), 1.0), f"{what}: mean err {err.mean():.5f}"


@pytest.mark.parametrize("name", sorted(CASES))
def test_draft_step_matches_the_oracle(dev, name):
    print(f"draft step {name}", flush=True)
    over = CASES[name]
    model = _model(over, dev, 11)
    cfg = model.config
    g = gen(5)
    embed = torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g).bfloat16().to(dev)
    lm_head = (torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g) / 8).bfloat16().to(dev)
    hot = torch.arange(0, 2 * cfg.state_vocab_size, 2).to(dev) if cfg.state_vocab_size else None
    step = DraftStep(model, embed, lm_head, max_model_len=512, hot_ids=hot)
    lens = torch.tensor([37, 100, 0, 64])  # context positions before each anchor
    batch, page, heads, hd = len(lens), 16, cfg.num_attention_heads, cfg.hidden_size // cfg.num_attention_heads
    bt, total = paged_layout((lens + 1).tolist(), page, g)
    caches = [torch.zeros(total, heads, page, 2 * hd, dtype=torch.bfloat16, device=dev) for _ in model.layers]
    layout = step.cache_layout(caches)
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    req = torch.cat([torch.full((int(n),), b) for b, n in enumerate(lens)])
    slots = bt[req, pos // page].long() * page + pos % page
    states = torch.randn(len(pos), len(cfg.target_layer_ids) * cfg.target_hidden_size, generator=g).bfloat16()
    step.write_context(states.to(dev), pos.to(dev), slots.to(dev), layout)
    torch.cuda.synchronize()
    ref_caches = [c.cpu() for c in caches]  # the oracle starts from the same context
    anchors = torch.randint(0, cfg.vocab_size, (batch,), generator=g)
    a_slots = bt[torch.arange(batch), lens // page].long() * page + lens % page
    z = torch.randn(batch * cfg.block_size, cfg.target_hidden_size, generator=g)
    hidden = step(anchors.to(dev), lens.to(dev), a_slots.to(dev), z.to(dev), caches, bt.to(dev), layout)
    logits = step.logits(hidden)
    tokens = step.greedy(hidden)
    torch.cuda.synchronize()

    w = _weights(step)
    oracle.write_anchor_rows(w, anchors, lens, a_slots, ref_caches, page)
    for i, (c, rc) in enumerate(zip(caches, ref_caches)):
        _close_rows(c, rc, f"cache {i}")
    want_h = oracle.one_jump(w, anchors, lens, z, ref_caches, bt)
    _close_rows(hidden, want_h, "hidden", ulps=4, slack=1e-2)  # two DiT layers of roundings
    want = oracle.draft_logits(w, want_h).float()
    got = logits.float().cpu()
    err = (got - want).abs()
    assert err.max() <= 0.01 * want.abs().max(), f"max err {err.max():.4f} vs {want.abs().max():.4f}"
    assert err.mean() <= 0.003 * want.abs().mean(), f"mean err {err.mean():.5f}"
    top2 = want.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * err.max()
    want_tok = want.argmax(-1)
    if hot is not None:
        want_tok = hot.cpu()[want_tok]
    same = tokens.cpu() == want_tok
    print(f"  logits max err {err.max():.4f} (max |logit| {want.abs().max():.3f}); clear-margin rows "
          f"{clear.float().mean():.3f}; greedy tokens equal on {same.float().mean():.3f}", flush=True)
    assert clear.float().mean() >= 0.8 and same[clear].all()


def test_noise_rows_against_their_definition(dev):
    g = gen(9)
    z = torch.randn(37, 4096, generator=g)
    lam = torch.rand(4096, generator=g) * 0.01
    zb, sc = ops.noise_rows(z.to(dev), lam.to(dev), 1e-6, 0.8)
    torch.cuda.synchronize()
    assert torch.equal(zb.cpu(), z.bfloat16())
    want = (0.8 * torch.rsqrt((z.double() ** 2) @ lam.double() + 1e-6)).float().bfloat16()
    diff = (sc.cpu().view(torch.int16).int() - want.view(torch.int16).int()).abs()
    assert diff.max() <= 1  # one bf16 step: the fp32 sum's order differs from float64's
