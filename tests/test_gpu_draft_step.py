"""The vLLM plugin's draft step (flashmap_amd.draft_step.DraftStep, flashmap/vllm/model.py:
779-1041), one jump and two, on the GPU.

- Against the reference's own ``draft`` outputs (tests/golden/drafter_tiny.safetensors):
  DraftStep prepared from the fixtures' raw weights over paged caches holding the
  fixtures' context; one jump from the fixture's vocabulary noise mapped into the folded
  space (``z = (x0 @ E) A^-1`` with the step's own factor ``A``, so that ``z @ A`` is the
  ``x0 @ E`` the reference reads), two jumps from the vocabulary-sized noise itself.
- Against the oracle (oracle/draft_step.py, pinned to the same fixtures on the CPU)
  prepared from the drafter's raw weights -- not from anything DraftStep computed -- on
  two tiny random drafters with ragged contexts, one and two jumps: the anchors' cache
  rows, the final hidden rows, the logits and the greedy tokens.
- Against the drop-in ``FlashMapDraftModel.forward`` (pinned to the fixtures through
  ``draft``) on the same weights and the same effective noise, over its contiguous
  ``FlashMapCache``: the hidden rows through the DiT's head.
- ``fm_noise_rows`` against its definition, and the wrapper's checks of its output.

Bars: cache rows within two bf16 ulps of each element plus one ulp of the row's RMS
(projections and norms round on GPU and CPU in different summation orders, and a flipped
rounding of one operand moves a whole normed, rotated row by about an ulp of the row);
hidden rows (two DiT layers of such roundings, twice for two jumps, and the step's folded
noise read-out against the oracle's unfolded one) within four ulps plus 2 % of the row's
RMS per element and 1 % of it in RMS over the row (per jump); logits within 1 % of the largest logit
(max) and 1 % of the mean |logit| (mean): a bf16 ulp is 0.4-0.8 % of a logit, and the
step's folded head rounds its product once where the reference rounds the DiT head's
output and then the logits (measured against the fixture: mean error 0.6 %); greedy
tokens equal on every row whose reference top-2 margin exceeds twice the observed logit
error, and on every row where the reference's own greedy token is compared."""

import json
import math
from pathlib import Path

import pytest
import torch

from _inputs import gen, paged_layout
from flashmap_amd import drafter as d
from flashmap_amd import fold, ops
from flashmap_amd.draft_step import DraftStep
from oracle import draft_step as oracle

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "drafter_tiny.safetensors"
PAGE = 16
CASES = {
    "gelu_full_vocab": dict(mlp_type="gelu"),
    "swiglu_state_vocab": dict(mlp_type="swiglu", state_vocab_size=200),
    # vLLM's d2t: a draft vocabulary restricting the logits while the state stays on the
    # whole vocabulary (its jump head then spans every token)
    "gelu_hot_ids": dict(mlp_type="gelu"),
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


def _close_rows(got, want, what, ulps=2, rel=2.0 ** -7, row_rel=None):
    """Per element within ``ulps`` bf16 ulps of its own magnitude plus ``rel`` of its
    row's RMS (a one-ulp flip of one operand moves every element of a normed or rotated
    row by about an ulp of the row, whatever the element's own size); ``row_rel``: each
    row's RMS error within that fraction of its RMS."""
    w = want.float().reshape(-1, want.shape[-1])
    g = got.float().cpu().reshape(w.shape)
    err = (g - w).abs()
    rms = w.pow(2).mean(-1, keepdim=True).sqrt()
    bad = err > ulps * 2.0 ** -7 * w.abs() + rel * rms
    row = err.pow(2).mean(-1).sqrt() / rms.squeeze(-1).clamp_min(1e-30)
    print(f"  {what}: max err {err.max():.4f}, worst row RMS error {row.max():.4f} of the row's RMS, "
          f"{int(bad.sum())} of {err.numel()} elements past the bar", flush=True)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {err.max():.4f}"
    if row_rel is not None:
        assert row.max() <= row_rel, f"{what}: a row's RMS error is {row.max():.4f} of its RMS"


def _check_logits(got, want, hot=None, what=""):
    """The bars on logits over the draft vocabulary; ``want`` may span the target's
    vocabulary (then restricted to ``hot``). Returns the fraction of clear-margin rows."""
    got = got.float().cpu().reshape(-1, got.shape[-1])
    want = want.float().reshape(got.shape[0], -1)
    if hot is not None and want.shape[1] != got.shape[1]:
        want = want[:, hot.cpu()]
    err = (got - want).abs()
    top2 = want.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * err.max()
    same = got.argmax(-1) == want.argmax(-1)
    print(f"  {what}: logits max err {err.max():.4f} (max |logit| {want.abs().max():.3f}), mean err "
          f"{err.mean():.5f} (mean |logit| {want.abs().mean():.4f}); clear-margin rows {clear.float().mean():.3f}; "
          f"greedy tokens equal on {same.float().mean():.3f}", flush=True)
    assert err.max() <= 0.01 * want.abs().max(), f"{what} max err {err.max():.4f} vs {want.abs().max():.4f}"
    assert err.mean() <= 0.01 * want.abs().mean(), f"{what} mean err {err.mean():.5f}"
    assert same[clear].all(), f"{what}: a clear-margin greedy token differs"
    return float(clear.float().mean()), float(same.float().mean())


def _fold_space(step: DraftStep, embeds: torch.Tensor) -> torch.Tensor:
    """``z`` (float32) with ``z @ A = embeds`` for the step's own noise factor ``A`` (the
    one ``fold_noise`` folded), so that the one-jump step reads ``embeds`` as its noise."""
    factor = fold.noise_factor(_state_rows(step))[0]
    return torch.linalg.solve(factor.T, embeds.double().T).T.float()


def _state_rows(step: DraftStep) -> torch.Tensor:
    hot, cfg = step.hot_ids, step.cfg
    return step.embed_weight[hot] if (hot is not None and cfg.state_vocab_size is not None) else step.embed_weight


def _fixture(name):
    from safetensors import safe_open

    with safe_open(str(GOLDEN), "pt") as f:
        meta = json.loads(f.metadata()["cases"])[name]
        t = {k[len(name) + 1:]: f.get_tensor(k) for k in f.keys() if k.startswith(name + "/")}
    return meta, {k[len("model/"):]: v for k, v in t.items() if k.startswith("model/")}, t


def _paged_context(step, features, lens, dev, g):
    """Per-layer paged caches with each request's context features at positions 0 ..
    lens[b] - 1 (written by the step), the block table, and the anchors' slots."""
    batch = len(lens)
    bt, total = paged_layout((lens + 1).tolist(), PAGE, g)
    caches = [torch.zeros(total, step.heads, PAGE, 2 * step.head_dim, dtype=torch.bfloat16, device=dev)
              for _ in step.model.layers]
    layout = step.cache_layout(caches)
    pos = torch.cat([torch.arange(int(n)) for n in lens])
    req = torch.cat([torch.full((int(n),), b) for b, n in enumerate(lens)])
    slots = bt[req, pos // PAGE].long() * PAGE + pos % PAGE
    if len(pos):
        step.write_context(features.to(dev), pos.to(dev), slots.to(dev), layout)
    a_slots = bt[torch.arange(batch), lens // PAGE].long() * PAGE + lens % PAGE
    return caches, layout, bt, pos, slots, a_slots


@pytest.mark.parametrize("name", ["gelu_full_vocab_1step", "swiglu_state_vocab_2step"])
def test_draft_step_matches_reference_fixtures(dev, name):
    print(f"draft step on the reference fixture {name}", flush=True)
    meta, sd, t = _fixture(name)
    model = d.FlashMapDraftModel(meta["config"])
    model.load_state_dict(sd)
    model = model.to(dev, torch.bfloat16)
    cfg = model.config
    hot = model.draft_ids.to(dev) if cfg.state_vocab_size else None
    step = DraftStep(model, t["embed"].to(dev), t["lm_head"].to(dev), max_model_len=meta["context"] + 32,
                     hot_ids=hot, num_steps=meta["num_steps"])
    batch, ctx = meta["batch"], meta["context"]
    lens = torch.full((batch,), ctx)
    feats = t["features"].reshape(batch * ctx, -1)
    caches, layout, bt, _, _, a_slots = _paged_context(step, feats, lens, dev, gen(3))
    noise = t["noise"].to(dev).reshape(batch * cfg.block_size, -1)
    if step.num_steps == 1:  # the reference reads x0 only as bf16(x0) @ E
        z = _fold_space(step, noise.bfloat16() @ _state_rows(step))
    else:
        z = noise
    h = step(t["anchors"].to(dev), lens.to(dev), a_slots.to(dev), z, caches, bt.to(dev), layout)
    logits = step.logits(h)
    tokens = step.greedy(h)
    torch.cuda.synchronize()
    clear, same = _check_logits(logits, t["logits"], hot, name)
    assert clear >= 0.85
    # The vLLM step folds the DiT head into the LM head (one rounding of the product where
    # the reference rounds the head's output, then the logits), as the reference plugin
    # does: a slot within rounding of a tie may flip; every clear-margin slot is equal.
    want = t["logits"].reshape(batch * cfg.block_size, -1)
    if hot is not None:
        want = want[:, hot.cpu()]
    top2 = want.topk(2, dim=-1).values
    err = (logits.float().cpu() - want).abs().max()
    rows = (top2[:, 0] - top2[:, 1]) > 2 * err
    want_tok = want.argmax(-1) if hot is None else hot.cpu()[want.argmax(-1)]
    assert torch.equal(tokens.cpu()[rows], want_tok[rows]), "a clear-margin greedy draft token differs"


def _oracle_weights(model, embed, lm_head, hot, steps, max_positions):
    """The oracle prepared from the drafter's raw weights (its state dict on the CPU)."""
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = dict(vars(model.config))
    return oracle.prepare(sd, cfg, embed.cpu(), lm_head.cpu(), None if hot is None else hot.cpu(), steps,
                          max_positions)


@pytest.mark.parametrize("steps", [1, 2])
@pytest.mark.parametrize("name", sorted(CASES))
def test_draft_step_matches_the_oracle(dev, name, steps):
    print(f"draft step {name}, {steps} jump(s)", flush=True)
    over = dict(CASES[name])
    model = _model(over, dev, 11)
    cfg = model.config
    g = gen(5)
    embed = torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g).bfloat16().to(dev)
    lm_head = (torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g) / 8).bfloat16().to(dev)
    hot = torch.arange(0, 2 * cfg.state_vocab_size, 2).to(dev) if cfg.state_vocab_size else None
    if name == "gelu_hot_ids":
        hot = torch.arange(3, cfg.vocab_size, 3).to(dev)
    step = DraftStep(model, embed, lm_head, max_model_len=512, hot_ids=hot, num_steps=steps)
    lens = torch.tensor([37, 100, 0, 64])  # context positions before each anchor
    batch, k = len(lens), cfg.block_size
    states = torch.randn(int(lens.sum()), len(cfg.target_layer_ids) * cfg.target_hidden_size, generator=g).bfloat16()
    caches, layout, bt, pos, slots, a_slots = _paged_context(step, states, lens, dev, g)
    torch.cuda.synchronize()
    w = _oracle_weights(model, embed, lm_head, hot, steps, 512 + k + 1)
    ref_caches = [torch.zeros_like(c, device="cpu") for c in caches]
    oracle.write_context(w, states, pos, slots, ref_caches, PAGE)
    for i, (c, rc) in enumerate(zip(caches, ref_caches)):
        _close_rows(c.view(*c.shape[:-1], 2, -1), rc.view(*rc.shape[:-1], 2, -1), f"context cache {i}")
    anchors = torch.randint(0, cfg.vocab_size, (batch,), generator=g)
    if steps == 1:
        z = torch.randn(batch * k, cfg.target_hidden_size, generator=g)
        noise_embeds = (z.to(dev).double() @ fold.noise_factor(_state_rows(step))[0]).bfloat16().cpu()
    else:
        z = torch.randn(batch * k, step.noise_columns, generator=g)
    hidden = step(anchors.to(dev), lens.to(dev), a_slots.to(dev), z.to(dev), caches, bt.to(dev), layout)
    logits = step.logits(hidden)
    tokens = step.greedy(hidden)
    torch.cuda.synchronize()

    oracle.write_anchors(w, anchors, lens, a_slots, ref_caches, PAGE)
    for i, (c, rc) in enumerate(zip(caches, ref_caches)):
        _close_rows(c.view(*c.shape[:-1], 2, -1), rc.view(*rc.shape[:-1], 2, -1), f"cache {i} with the anchors")
    if steps == 1:
        want_h, want = oracle.draft(w, lens, ref_caches, bt, noise_embeds=noise_embeds)
    else:
        want_h, want = oracle.draft(w, lens, ref_caches, bt, state=z)
    _close_rows(hidden, want_h, "hidden", ulps=4, rel=2e-2 * steps, row_rel=1e-2 * steps)
    clear, _ = _check_logits(logits, want, None, f"{name} x{steps}")
    want_tok = want.float().argmax(-1)
    if hot is not None:
        want_tok = hot.cpu()[want_tok]
    assert clear >= 0.6  # not vacuous: most rows are decided by a clear margin
    top2 = want.float().topk(2, dim=-1).values
    err = (logits.float().cpu() - want.float()).abs().max()
    rows = (top2[:, 0] - top2[:, 1]) > 2 * err
    assert torch.equal(tokens.cpu()[rows], want_tok[rows])


def test_draft_step_equals_model_forward(dev):
    """The step's final hidden rows, through the DiT's head, against
    FlashMapDraftModel.forward on the same weights over a contiguous FlashMapCache, from
    the same effective noise ``z @ A`` (``mix_state`` of the uniform posterior and it)."""
    model = _model(CASES["gelu_full_vocab"], dev, 13)
    cfg = model.config
    g = gen(7)
    embed = torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g).bfloat16().to(dev)
    lm_head = (torch.randn(cfg.vocab_size, cfg.target_hidden_size, generator=g) / 8).bfloat16().to(dev)
    step = DraftStep(model, embed, lm_head, max_model_len=256)
    lens = torch.tensor([21, 77, 50])
    k = cfg.block_size
    feats = torch.randn(int(lens.sum()), len(cfg.target_layer_ids) * cfg.target_hidden_size, generator=g).bfloat16()
    caches, layout, bt, _, _, a_slots = _paged_context(step, feats, lens, dev, g)
    anchors = torch.randint(0, cfg.vocab_size, (len(lens),), generator=g).to(dev)
    z = torch.randn(len(lens) * k, cfg.target_hidden_size, generator=g).to(dev)
    h = step(anchors, lens.to(dev), a_slots.to(dev), z, caches, bt.to(dev), layout)
    got = model.head(h).float().cpu()
    factor = fold.noise_factor(embed)[0]
    uniform = torch.full((1, cfg.vocab_size), 1.0 / cfg.vocab_size, device=dev).bfloat16() @ embed
    emb_tok = torch.nn.Embedding.from_pretrained(embed)
    offsets = torch.cat([torch.zeros(1, dtype=torch.long), lens.cumsum(0)])
    for b, n in enumerate(lens.tolist()):
        cache = d.FlashMapCache(cfg, 1, n + 1, device=dev, dtype=torch.bfloat16)
        model.extend_context(cache, feats[offsets[b]:offsets[b + 1]][None].to(dev))
        positions = model._open_block(cache, anchors[b:b + 1], emb_tok)
        noise_embeds = (z[b * k:(b + 1) * k].double() @ factor).bfloat16()
        inputs = model.mix_state(uniform.expand(k, -1), noise_embeds, 0.0, 1.0)[None]
        want = model(inputs, 0.0, 1.0, positions, cache.context(cache.length + 1)).float().cpu()[0]
        _close_rows(got[b * k:(b + 1) * k], want, f"request {b}", ulps=4, rel=2e-2, row_rel=1e-2)


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


def test_noise_rows_refuses_a_wrong_output(dev):
    z = torch.zeros(8, 64, device=dev)
    lam = torch.ones(64, device=dev)
    for bad in (torch.empty(7, 64, dtype=torch.bfloat16, device=dev),  # too few rows
                torch.empty(8, 64, dtype=torch.float16, device=dev),  # not bf16
                torch.empty(8, 128, dtype=torch.bfloat16, device=dev)[:, ::2],  # strided channels
                torch.empty(8, 66, dtype=torch.bfloat16, device=dev)[:, :64]):  # row stride 66
        with pytest.raises(ValueError, match="z_bf16"):
            ops.noise_rows(z, lam, 1e-6, 1.0, z_bf16=bad)
