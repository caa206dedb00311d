"""The draft-step oracle (oracle/draft_step.py) against the reference's own ``draft``
outputs (tests/golden/drafter_tiny.safetensors, written from flashmap/modeling_flashmap.py
by tests/golden/make_drafter_golden.py), on the CPU: from the fixtures' raw weights,
context features, anchors and noise, over vLLM-layout paged caches behind a permuted block
table.

Bars: logits within 0.8 % of the largest logit (max) and 0.1 % of the mean |logit|
(mean), as for the drop-in drafter (one bf16 ulp of the largest logits is 0.4-0.8 %); the
greedy tokens equal on every slot whose reference top-2 margin exceeds twice the
observed error. Planted slips in the oracle (the first jump's modulations reused by the
second, the state update's sign, the noise gate's jump factor dropped, the wrong state
vocabulary rows) each fail these bars."""

import json
from pathlib import Path

import pytest
import torch

from _inputs import gen, paged_layout
from oracle import draft_step as oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "drafter_tiny.safetensors"
PAGE = 16


def _case(name):
    from safetensors import safe_open

    with safe_open(str(GOLDEN), "pt") as f:
        meta = json.loads(f.metadata()["cases"])[name]
        t = {k[len(name) + 1:]: f.get_tensor(k) for k in f.keys() if k.startswith(name + "/")}
    sd = {k[len("model/"):]: v for k, v in t.items() if k.startswith("model/")}
    return meta, sd, t


def _setup(name, slip=None):
    """The oracle prepared from the fixture's raw weights, with the context and anchors
    written into paged caches; ``slip`` plants a mistake."""
    meta, sd, t = _case(name)
    cfg = meta["config"]
    hot = sd["draft_ids"] if cfg.get("state_vocab_size") else None
    batch, ctx, steps = meta["batch"], meta["context"], meta["num_steps"]
    rows = hot + 1 if slip == "wrong_state_rows" else hot
    w = oracle.prepare(sd, cfg, t["embed"], t["lm_head"], rows, steps, max_positions=ctx + 64)
    if slip == "first_jump_mods":
        w["mods"] = [w["mods"][0]] * len(w["mods"])
    bt, total = paged_layout([ctx + 1] * batch, PAGE, gen(3))
    caches = [torch.zeros(total, w["heads"], PAGE, 2 * w["head_dim"], dtype=torch.bfloat16)
              for _ in range(w["layers"])]
    pos = torch.arange(ctx).repeat(batch)
    req = torch.arange(batch).repeat_interleave(ctx)
    slots = bt[req, pos // PAGE].long() * PAGE + pos % PAGE
    oracle.write_context(w, t["features"].reshape(batch * ctx, -1), pos, slots, caches, PAGE)
    a_pos = torch.full((batch,), ctx)
    a_slots = bt[torch.arange(batch), ctx // PAGE].long() * PAGE + ctx % PAGE
    oracle.write_anchors(w, t["anchors"], a_pos, a_slots, caches, PAGE)
    return meta, w, t, hot, a_pos, caches, bt


def _compare(got, want, hot):
    """(max err, mean err, clear-margin fraction, all clear-margin tokens equal) of draft
    logits over the draft vocabulary against the reference's over the full vocabulary."""
    want = want.reshape(got.shape[0], -1)
    if hot is not None:
        want = want[:, hot]
    err = (got.float() - want).abs()
    top2 = want.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * err.max()
    same = got.float().argmax(-1) == want.argmax(-1)
    ok = err.max() <= 0.008 * want.abs().max() and err.mean() <= 0.001 * want.abs().mean() and same[clear].all()
    return err.max(), err.mean(), clear.float().mean(), same.float().mean(), bool(ok)


@pytest.mark.parametrize("name", ["gelu_full_vocab_1step", "swiglu_state_vocab_2step"])
def test_oracle_draft_matches_reference(name):
    meta, w, t, hot, a_pos, caches, bt = _setup(name)
    state = t["noise"].reshape(-1, t["noise"].shape[-1])
    _, got = oracle.draft(w, a_pos, caches, bt, state=state)
    mx, mean, clear, same, ok = _compare(got, t["logits"], hot)
    print(f"{name}: max err {mx:.4f}, mean err {mean:.5f}, clear-margin {clear:.3f}, equal {same:.3f}")
    assert ok
    assert clear >= 0.85 and same >= 0.99
    if meta["num_steps"] == 1:  # the noise already through the embedding: the same computation
        _, got2 = oracle.draft(w, a_pos, caches, bt, noise_embeds=state.bfloat16() @ w["state_embed"])
        assert torch.equal(got, got2)


@pytest.mark.parametrize("name,slip", [
    ("swiglu_state_vocab_2step", "first_jump_mods"),
    ("swiglu_state_vocab_2step", "state_update_sign"),
    ("swiglu_state_vocab_2step", "constant_noise_gate"),
    ("swiglu_state_vocab_2step", "wrong_state_rows"),
])
def test_planted_slips_fail(name, slip, monkeypatch):
    if slip == "state_update_sign":
        real = oracle.logits
        monkeypatch.setattr(oracle, "logits",
                            lambda w, h, rows="draft_head": -real(w, h, rows) if rows == "state_head" else real(w, h))
    meta, w, t, hot, a_pos, caches, bt = _setup(name, slip)
    if slip == "constant_noise_gate":
        w["cfg"] = {**w["cfg"], "noise_gate": "constant"}
    state = t["noise"].reshape(-1, t["noise"].shape[-1])
    _, got = oracle.draft(w, a_pos, caches, bt, state=state)
    assert not _compare(got, t["logits"], hot)[-1], f"the slip {slip} went unnoticed"
