"""CPU restatement of the drafter's draft step over paged context caches.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Everything is computed from the
drafter's raw weights (a state dict under the reference's parameter names), its
configuration and the target's embedding and LM head, as eager bf16 torch ops on the CPU
that round where the reference's do:

- ``prepare``: per jump the AdaLN modulations of the time conditioning
  (flashmap/modeling_flashmap.py:83-117, 287-300), the embedded uniform posterior
  (``target_constants``, :396-418) and the state / draft vocabulary rows
  (``state_vocab``, :355-366);
- ``write_context`` / ``write_anchors``: the context rows ``hidden_norm(fc(features))``
  (:342-351) and the anchor rows ``anchor_norm(anchor_proj(embedding))`` (:451-457),
  projected to every layer's keys and values and stored by the vLLM writer's oracle
  (``oracle.attention.write_context_kv_vllm``) at the requests' slots;
- ``draft``: the jump loop of ``draft`` (:422-479): ``embed_state`` / ``mix_state``
  (:370-394), the DiT of ``forward`` (:302-313, layers :173-192) with the cross-attention
  over the paged caches (``oracle.attention.block_attention_paged_vllm``, each request
  attending to positions ``0 .. anchor``), the head then the LM head, and the state update
  between jumps; the one-jump draft also takes its noise already through the embedding
  (``noise_embeds = x0 @ E``), which is all a one-jump draft reads of it.

Unfolded on purpose: the plugin's draft step (flashmap/vllm/model.py:779-1041) folds the
noise read-out and the head into single GEMMs (flashmap/vllm/fold.py); this oracle keeps
the composition those folds preserve, so it checks them too.

Pinned by: the reference's own ``draft`` outputs on two tiny random drafters
(tests/golden/drafter_tiny.safetensors; tests/test_oracle_draft_step.py): one jump over
the full vocabulary and two jumps over a 200-token state vocabulary, logits within the
bf16 bar and greedy tokens equal on every clear-margin slot.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import attention as ref
from . import dit

# flashmap/configuration_flashmap.py:11-16 (the "decoding_error" schedule's grids)
DEFAULT_JUMP_GRIDS = {
    "1": [0.0, 1.0],
    "2": [0.0, 0.8172569274902344, 1.0],
    "3": [0.0, 0.8010796308517456, 0.8310279846191406, 1.0],
    "4": [0.0, 0.7906050682067871, 0.8172569274902344, 0.8379518389701843, 1.0],
}
# flashmap/configuration_flashmap.py:88-112 (the fields the draft reads)
DEFAULTS = dict(block_size=16, time_scale=1000.0, rope_theta=10000.0, rms_norm_eps=1e-6, qk_norm_eps=1e-5,
                layer_norm_eps=1e-6, noise_gate="jump", mlp_type="gelu", state_vocab_size=None)


def jump_times(grid) -> list:
    """``(s, t, next)`` per jump, ``t == next`` (flashmap/configuration_flashmap.py:23-31)."""
    g = [float(v) for v in grid]
    return [(a, b, b) for a, b in zip(g[:-1], g[1:])]


def _lin(sd, name, x):
    return F.linear(x, sd[f"{name}.weight"], sd.get(f"{name}.bias"))


def time_embedding(sd, prefix: str, t: torch.Tensor, dim: int, scale: float) -> torch.Tensor:
    """``linear_2(silu(linear_1([cos | sin](scale t f))))`` (flashmap/modeling_flashmap.py:83-99)."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half).float() / half)
    args = (t.float() * scale)[..., None] * freqs
    emb = torch.cat([args.cos(), args.sin()], dim=-1).to(sd[f"{prefix}.linear_1.weight"].dtype)
    return _lin(sd, f"{prefix}.linear_2", F.silu(_lin(sd, f"{prefix}.linear_1", emb)))


def modulations(sd, cfg: dict, s: float, t: float):
    """Per layer ``[(scale, shift, gate)]`` of its self-attention, cross-attention and MLP
    norms, and the final norm's ``(scale, shift)``, for the jump ``s -> t``
    (flashmap/modeling_flashmap.py:108-110, 287-300)."""
    times = torch.tensor([s, t])
    cond = (time_embedding(sd, "time_embed", times[:1], cfg["time_embed_dim"], cfg["time_scale"])
            + time_embedding(sd, "jump_embed", times[1:], cfg["time_embed_dim"], cfg["time_scale"]))[None]

    def mod(name):
        return tuple(m.reshape(-1) for m in _lin(sd, f"{name}.linear", F.silu(cond)).chunk(3, dim=-1))

    layers = [[mod(f"layers.{i}.{n}") for n in ("self_attn_adaln", "cross_attn_adaln", "mlp_adaln")]
              for i in range(cfg["num_hidden_layers"])]
    return layers, mod("final_adaln")[:2]


def prepare(sd: dict, cfg: dict, embed: torch.Tensor, lm_head: torch.Tensor, hot_ids=None, num_steps: int = 1,
            max_positions: int = 4096) -> dict:
    """Everything the draft needs, from the raw weights ``sd`` (bf16 CPU tensors), ``cfg``
    (the drafter's configuration; missing fields take the reference's defaults), the
    target's ``embed``/``lm_head (V, H)`` and ``hot_ids``, the draft vocabulary's token
    ids (None: all). The state lives on the state vocabulary: ``hot_ids``' rows when the
    drafter has one, else every row."""
    cfg = {**DEFAULTS, **cfg}
    grids = cfg.get("jump_grids") or DEFAULT_JUMP_GRIDS
    jumps = jump_times(grids[str(num_steps)])
    state_rows = hot_ids if (cfg["state_vocab_size"] is not None and hot_ids is not None) else None
    state_embed = embed if state_rows is None else embed[state_rows]
    vocab = state_embed.shape[0]
    uniform = torch.full((1, vocab), 1.0 / vocab).to(state_embed.dtype)
    heads = cfg["num_attention_heads"]
    return dict(sd=sd, cfg=cfg, jumps=jumps, mods=[modulations(sd, cfg, s, t) for s, t, _ in jumps],
                embed=embed, state_embed=state_embed, uniform_embeds=uniform @ state_embed,
                state_head=lm_head if state_rows is None else lm_head[state_rows],
                draft_head=lm_head if hot_ids is None else lm_head[hot_ids],
                heads=heads, head_dim=cfg["hidden_size"] // heads, layers=cfg["num_hidden_layers"],
                cos_sin=ref.rope_table(max_positions, cfg["hidden_size"] // heads, cfg["rope_theta"]))


# --------------------------------------------------------------------------- context


def _write(w: dict, rows, positions, slots, caches, page: int) -> None:
    """Every layer's keys (k-normed, rotated at ``positions``) and values of ``rows``
    stored at ``slots`` of the per-layer paged caches."""
    sd, cfg, heads, hd = w["sd"], w["cfg"], w["heads"], w["head_dim"]
    kv = torch.stack([torch.stack([_lin(sd, f"layers.{i}.cross_attn.{p}_proj", rows) for p in "kv"])
                      for i in range(w["layers"])])  # (L, 2, tokens, dim)
    kv = kv.permute(2, 0, 1, 3).reshape(rows.shape[0], w["layers"], 2, heads, hd)
    k_norm = torch.stack([sd[f"layers.{i}.cross_attn.k_norm.weight"].float() for i in range(w["layers"])])
    ref.write_context_kv_vllm(kv, positions, slots, k_norm, w["cos_sin"], caches, page, cfg["qk_norm_eps"])


def write_context(w: dict, features, positions, slots, caches, page: int) -> None:
    """The target's features ``(tokens, n_layers * H)`` at ``positions``: ``hidden_norm(fc(.))``
    then every layer's keys and values (flashmap/modeling_flashmap.py:342-351)."""
    sd, eps = w["sd"], w["cfg"]["rms_norm_eps"]
    rows = ref.rms_norm(F.linear(features, sd["fc.weight"]), sd["hidden_norm.weight"], eps)
    _write(w, rows, positions, slots, caches, page)


def write_anchors(w: dict, anchors, positions, slots, caches, page: int) -> None:
    """Each request's anchor at its position (flashmap/modeling_flashmap.py:451-457)."""
    sd, eps = w["sd"], w["cfg"]["rms_norm_eps"]
    rows = ref.rms_norm(_lin(sd, "anchor_proj", w["embed"][anchors]), sd["anchor_norm.weight"], eps)
    _write(w, rows, positions, slots, caches, page)


# ------------------------------------------------------------------------ the draft


def mix_state(w: dict, posterior_embeds, state_embeds, s: float, t: float):
    """``state_norm(posterior) + gate * noise_norm(state)``, the gate ``noise_gate * (t -
    s)`` (or alone, "constant") rounded to bf16 (flashmap/modeling_flashmap.py:388-394)."""
    sd, cfg = w["sd"], w["cfg"]
    jump = 1.0 if cfg["noise_gate"] == "constant" else t - s
    gate = (sd["noise_gate"].float() * jump).to(torch.bfloat16)
    eps = cfg["rms_norm_eps"]
    return (ref.rms_norm(posterior_embeds.to(torch.bfloat16), sd["state_norm.weight"], eps)
            + gate * ref.rms_norm(state_embeds.to(torch.bfloat16), sd["noise_norm.weight"], eps))


def embed_state(w: dict, state, s: float, t: float):
    """The DiT input of a state over the state vocabulary at ``s`` jumping to ``t``
    (flashmap/modeling_flashmap.py:370-386)."""
    e = w["state_embed"]
    if s == 0:
        posterior = w["uniform_embeds"]
    else:
        posterior = (state.float() * (s / max(1.0 - s, 1e-3) ** 2)).softmax(dim=-1).to(e.dtype) @ e
    return mix_state(w, posterior, state.to(e.dtype) @ e, s, t)


def run_dit(w: dict, inputs, jump: int, positions, cross, blocks: int):
    """The DiT's final AdaLN output ``(tokens, dim)`` bf16 for ``inputs (tokens, H)``
    (``mix_state``'s output) of ``blocks`` blocks at ``positions (tokens,)``; ``cross(i,
    q)`` is layer ``i``'s cross-attention of its normed, rotated queries ``q (tokens,
    heads, head_dim)`` onto the context (flashmap/modeling_flashmap.py:173-192, 302-313)."""
    sd, cfg = w["sd"], w["cfg"]
    heads, hd, ln = w["heads"], w["head_dim"], cfg["layer_norm_eps"]
    tokens = inputs.shape[0]
    k = tokens // blocks
    cs = w["cos_sin"][positions.long()]
    cos, sin = cs[..., 0].view(blocks, k, -1), cs[..., 1].view(blocks, k, -1)
    hidden = _lin(sd, "x_embed", inputs)
    per_layer, final = w["mods"][jump]
    for i in range(w["layers"]):
        (s_sc, s_sh, s_g), (c_sc, c_sh, c_g), (m_sc, m_sh, m_g) = per_layer[i]
        p = f"layers.{i}"
        h = dit.adaln_residual(hidden, None, None, s_sc, s_sh, ln)[1]
        qkv = torch.stack([_lin(sd, f"{p}.self_attn.{n}_proj", h) for n in "qkv"], dim=1)
        att = ref.block_self_attention(qkv.view(blocks, k, 3, heads, hd), sd[f"{p}.self_attn.q_norm.weight"],
                                       sd[f"{p}.self_attn.k_norm.weight"], cos, sin,
                                       cfg["qk_norm_eps"]).to(torch.bfloat16)
        hidden = dit.adaln_residual(hidden, _lin(sd, f"{p}.self_attn.o_proj", att.reshape(tokens, -1)), s_g,
                                    None, None, 0)[0]
        h = dit.adaln_residual(hidden, None, None, c_sc, c_sh, ln)[1]
        q = ref.rms_norm_rope_vllm(_lin(sd, f"{p}.cross_attn.q_proj", h).view(tokens, heads, hd),
                                   sd[f"{p}.cross_attn.q_norm.weight"], w["cos_sin"], positions, cfg["qk_norm_eps"])
        ctx = cross(i, q).to(torch.bfloat16)
        hidden = dit.adaln_residual(hidden, _lin(sd, f"{p}.cross_attn.o_proj", ctx.reshape(tokens, -1)), c_g,
                                    None, None, 0)[0]
        h = dit.adaln_residual(hidden, None, None, m_sc, m_sh, ln)[1]
        if cfg["mlp_type"] == "swiglu":
            gate, up = _lin(sd, f"{p}.mlp.gate_up_proj", h).chunk(2, dim=-1)
            y = _lin(sd, f"{p}.mlp.down_proj", F.silu(gate) * up)
        else:
            y = _lin(sd, f"{p}.mlp.fc2", F.gelu(_lin(sd, f"{p}.mlp.fc1", h)))
        hidden = dit.adaln_residual(hidden, y, m_g, None, None, 0)[0]
    return dit.adaln_residual(hidden, None, None, final[0], final[1], ln)[1]


def paged_cross(caches, block_table, seqused):
    """``cross`` of ``run_dit`` over per-layer vLLM paged caches: request ``b``'s rows
    attend to its first ``seqused[b]`` positions (flashmap/vllm/model.py:862-893)."""
    def cross(i, q):
        k = q.shape[0] // seqused.shape[0]
        cu = torch.arange(0, q.shape[0] + 1, k, dtype=torch.int32)
        return ref.block_attention_paged_vllm(q, caches[i], cu, seqused, block_table)
    return cross


def pool_cross(k_bufs, v_bufs, page_table, cache_seqlens, n_cand: int = 1):
    """``cross`` of ``run_dit`` over per-layer SGLang token pools: a request's ``n_cand``
    candidate blocks, side by side in the query axis, attend together to its
    ``cache_seqlens`` pool rows of ``page_table`` (flashmap/sglang/model.py:1028-1040)."""
    def cross(i, q):
        requests = cache_seqlens.shape[0]
        qr = q.view(requests, -1, *q.shape[1:])
        out = ref.block_attention_token_paged(qr, k_bufs[i], v_bufs[i], cache_seqlens, page_table)
        return out.reshape(q.shape)
    return cross


def logits(w: dict, h, rows: str = "draft_head"):
    """``lm_head[rows](head(h))``: the DiT head, then the target's LM head rows of the
    draft (or, ``rows="state_head"``, the state) vocabulary, each a bf16 linear
    (flashmap/modeling_flashmap.py:313, 468-469)."""
    return F.linear(_lin(w["sd"], "head", h), w[rows])


def draft(w: dict, anchor_positions, caches, block_table, noise_embeds=None, state=None):
    """``(final AdaLN output (B K, dim), draft logits (B K, draft vocabulary))`` of the
    block after each request's anchor at ``anchor_positions (B,)`` (anchors already
    written): a one-jump draft from ``noise_embeds (B K, H) = x0 @ E``, or any draft from
    ``state (B K, state vocabulary)`` float32, the starting noise (the loop of
    flashmap/modeling_flashmap.py:460-478)."""
    k = w["cfg"]["block_size"]
    positions = (anchor_positions[:, None] + 1 + torch.arange(k)).reshape(-1)
    seqused = anchor_positions + 1
    h = None
    for j, (s, t, nxt) in enumerate(w["jumps"]):
        if state is None:
            if len(w["jumps"]) != 1:
                raise ValueError("a draft of several jumps starts from a vocabulary-sized state")
            inputs = mix_state(w, w["uniform_embeds"].expand(noise_embeds.shape[0], -1), noise_embeds, s, t)
        else:
            inputs = embed_state(w, state, s, t)
        h = run_dit(w, inputs, j, positions, paged_cross(caches, block_table, seqused), seqused.shape[0])
        if nxt < 1.0:
            delta = logits(w, h, "state_head").float().softmax(dim=-1)
            state = ((1.0 - nxt) * state + (nxt - s) * delta) / (1.0 - s)
    return h, logits(w, h)


# ------------------------------------------------------------ the SGLang plugin's step


def pool_layout_rows(w: dict, rows, positions, locs, k_bufs, v_bufs) -> None:
    """Every layer's keys and values of ``rows`` written to pool rows ``locs`` by the
    SGLang pool writer's oracle (flashmap/sglang/model.py:725-766)."""
    sd, heads, hd = w["sd"], w["heads"], w["head_dim"]
    kv = torch.cat([torch.cat([_lin(sd, f"layers.{i}.cross_attn.{p}_proj", rows) for p in "kv"], dim=-1)
                    for i in range(w["layers"])], dim=-1)  # per layer [k | v]
    k_norm = torch.stack([sd[f"layers.{i}.cross_attn.k_norm.weight"].float() for i in range(w["layers"])])
    cs = w["cos_sin"]
    cat = torch.cat([cs[..., 0], cs[..., 1]], dim=-1)
    ref.write_context_kv_pool(kv, k_bufs, v_bufs, k_norm, cat, positions, locs, w["layers"], heads * hd, hd,
                              w["cfg"]["qk_norm_eps"])


def pool_write_context(w: dict, features, positions, locs, k_bufs, v_bufs) -> None:
    """``write_target_hidden_kv``: ``hidden_norm(fc(features))`` into the pools."""
    sd, eps = w["sd"], w["cfg"]["rms_norm_eps"]
    rows = ref.rms_norm(F.linear(features, sd["fc.weight"]), sd["hidden_norm.weight"], eps)
    pool_layout_rows(w, rows, positions, locs, k_bufs, v_bufs)


def pool_write_anchors(w: dict, anchors, positions, locs, k_bufs, v_bufs) -> None:
    """The anchors' context rows (``_anchor_kv``, flashmap/sglang/model.py:896-903)."""
    sd, eps = w["sd"], w["cfg"]["rms_norm_eps"]
    rows = ref.rms_norm(_lin(sd, "anchor_proj", w["embed"][anchors]), sd["anchor_norm.weight"], eps)
    pool_layout_rows(w, rows, positions, locs, k_bufs, v_bufs)


def pool_draft(w: dict, anchor_positions, k_bufs, v_bufs, page_table, noise_embeds, n_cand: int = 1):
    """``(final AdaLN output, draft logits)`` of the SGLang plugin's one-jump draft
    (``_draft_impl`` + ``_denoise``, flashmap/sglang/model.py:905-1057): ``n_cand`` blocks
    per request (candidate-major, the noise ``noise_embeds (requests n_cand K, H) = x0 @ E``
    drawn per block) at positions ``anchor + 1 ..``, every block of a request attending
    to its pool rows ``0 .. anchor``."""
    if len(w["jumps"]) != 1:
        raise ValueError("the SGLang step's oracle covers one jump")
    k = w["cfg"]["block_size"]
    requests = anchor_positions.shape[0]
    positions = (anchor_positions[:, None] + 1 + torch.arange(k)).repeat_interleave(n_cand, dim=0).reshape(-1)
    s, t, _ = w["jumps"][0]
    inputs = mix_state(w, w["uniform_embeds"].expand(noise_embeds.shape[0], -1), noise_embeds, s, t)
    cross = pool_cross(k_bufs, v_bufs, page_table, anchor_positions + 1, n_cand)
    h = run_dit(w, inputs, 0, positions, cross, requests * n_cand)
    return h, logits(w, h)
