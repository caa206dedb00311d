"""The SGLang plugin's one-jump draft step on the gfx950 kernels, outside SGLang.

``SGLangDraftStep`` holds what the plugin prepares once (flashmap/sglang/model.py:366-404,
533-595): the jump's AdaLN modulations, the folded noise read-out, the constant first
hidden row, one projection weight for every layer's context keys/values (rows ``[k; v]``
per layer) and one per layer for the self-attention's q/k/v, the norms' weights in
float32, the pool writer's ``[cos | sin]`` table and the folded head. A call runs
``forward`` + ``_draft_impl`` + ``_denoise`` (flashmap/sglang/model.py:837-1057) over the
per-layer token pools ``(pool, heads, head_dim)``, every non-GEMM op of the DiT on a
kernel of this library:

1. the anchors' context rows: embedding -> ``anchor_proj`` -> ``anchor_norm`` -> one GEMM
   over every layer's ``[k; v]`` weights -> ``fm_write_context_kv_pool`` (k-norm, RoPE,
   store at each anchor's pool row);
2. the noise read-out: ``fm_noise_rows`` -> the folded GEMM -> ``fm_adaln_residual``;
3. per DiT layer: the fused q/k/v GEMM -> ``fm_block_self_attention`` with the step's
   per-token rotary rows -> ``o_proj`` -> ``fm_adaln_residual`` -> ``q_proj`` ->
   ``fm_block_attn_token_paged`` with the query prologue fused, a request's ``n_cand``
   candidate blocks side by side in the query axis over its one context (tree
   drafting), the step's shared plan -> ``o_proj`` -> ``fm_adaln_residual`` -> the MLP ->
   ``fm_adaln_residual``;
4. the folded head GEMM and ``fm_sample_rows`` (greedy rows: the argmax; the others a
   Gumbel-max sample on the Philox stream).

The plugin's drafts of several jumps go through its jump bank (flashmap/sglang/
jump_bank.py), a different scheme from the vLLM plugin's vocabulary-sized state; this
step takes one jump. GEMMs are hipBLASLt through torch; bf16 only.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops
from .drafter import FlashMapDraftModel, jump_times
from .fold import fold_head, fold_noise
from .sglang import rope_freqs

__all__ = ["SGLangDraftStep"]


class SGLangDraftStep:
    """A prepared one-jump SGLang draft step (see the module docstring). ``model``: the
    drafter (bf16, on the GPU); ``embed_tokens`` / ``lm_head``: the target's ``(V, H)``
    weights; ``max_positions``: the positions the pool writer's rotary table covers (the
    server's longest request plus a block); ``hot_ids``: the draft vocabulary's token ids
    (a drafter's ``draft_ids``), else None."""

    @torch.no_grad()
    def __init__(self, model: FlashMapDraftModel, embed_tokens: torch.Tensor, lm_head: torch.Tensor,
                 max_positions: int, hot_ids: torch.Tensor | None = None):
        cfg = model.config
        if model.dtype != torch.bfloat16:
            raise TypeError("the draft step's kernels are bf16: move the drafter to torch.bfloat16")
        self.model, self.cfg = model, cfg
        self.block = cfg.block_size
        self.heads = cfg.num_attention_heads
        self.head_dim = cfg.hidden_size // self.heads
        self.dim = cfg.hidden_size
        (s, t, _), = jump_times(model._jump_grid(1))
        per_layer, final = model.time_conditioning(s, t)
        self.layer_mods = [tuple(tuple(m.reshape(-1) for m in mod) for mod in mods) for mods in per_layer]
        self.final_mod = tuple(m.reshape(-1) for m in final[:2])
        # jump_gate: the noise weight rounded to the drafter's dtype (flashmap/sglang/model.py:661-671)
        jump = 1.0 if cfg.noise_gate == "constant" else t - s
        self.noise_gain = float((model.noise_gate.float() * jump).to(model.dtype))
        self.hot_ids = hot_ids
        state_vocab = hot_ids is not None and cfg.state_vocab_size is not None
        state_embed = embed_tokens[hot_ids] if state_vocab else embed_tokens
        vocab = state_embed.shape[0]
        uniform = torch.full((1, vocab), 1.0 / vocab, device=state_embed.device).to(state_embed.dtype)
        self.first_hidden = model.x_embed(model.state_norm(uniform @ state_embed))[0].contiguous()
        self.noise_embed, self.noise_eigvals = fold_noise(state_embed, model.noise_norm.weight, model.x_embed.weight)
        self.noise_eps = model.noise_norm.eps
        self.embed_weight = embed_tokens
        layers = model.layers
        self.ctx_kv_weight = torch.cat([torch.cat([l.cross_attn.k_proj.weight, l.cross_attn.v_proj.weight])
                                        for l in layers])
        self.k_norms = torch.stack([l.cross_attn.k_norm.weight.float() for l in layers]).contiguous()
        self.k_eps = layers[0].cross_attn.k_norm.eps if len(layers) else 0.0
        self.self_qkv = [torch.cat([l.self_attn.q_proj.weight, l.self_attn.k_proj.weight, l.self_attn.v_proj.weight])
                         for l in layers]
        self.norms = [tuple(n.weight.float().contiguous() for n in (l.self_attn.q_norm, l.self_attn.k_norm,
                                                                     l.cross_attn.q_norm)) for l in layers]
        freqs = rope_freqs(torch.arange(max_positions, device=state_embed.device), self.head_dim, cfg.rope_theta)
        # the pool writer's table: row p = [cos | sin] of p (flashmap/sglang/model.py:808-817)
        self.cos_sin = torch.cat([freqs[..., 0], freqs[..., 1]], dim=-1).contiguous()
        self.writer_rope = ops.rope_from_cat(self.cos_sin)
        self.head_weight, self.head_bias = fold_head(lm_head, model.head.weight, model.head.bias, hot_ids)
        self.scale = self.head_dim ** -0.5

    # -- the context -----------------------------------------------------------------

    def pool_meta(self, k_bufs: list[torch.Tensor], v_bufs: list[torch.Tensor]) -> torch.Tensor:
        """``(layers, 4)`` int64 (key ptr, value ptr, key row stride, value row stride) of
        the per-layer pools (``_fused_write_args``, flashmap/sglang/model.py:768-799)."""
        for k, v in zip(k_bufs, v_bufs):
            if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
                raise ValueError("the draft step's pools must be bf16")
            if k.shape[1:] != (self.heads, self.head_dim) or k.stride()[1:] != (self.head_dim, 1) \
                    or v.shape != k.shape or v.stride() != k.stride():
                raise ValueError(f"pools must be (pool, {self.heads}, {self.head_dim}) with unit head_dim stride")
        return torch.tensor([[k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0)] for k, v in zip(k_bufs, v_bufs)],
                            dtype=torch.int64, device=k_bufs[0].device)

    @torch.no_grad()
    def write_rows(self, rows: torch.Tensor, positions: torch.Tensor, locs: torch.Tensor, meta: torch.Tensor) -> None:
        """Every layer's keys (k-normed, rotated) and values of ``rows (tokens, dim)``,
        stored at pool rows ``locs`` (``_kv_write``, flashmap/sglang/model.py:746-766)."""
        kv = F.linear(rows, self.ctx_kv_weight)
        ops.write_context_kv_pool(kv, meta, self.k_norms, self.writer_rope, positions, locs, len(self.model.layers),
                                  self.dim, self.head_dim, self.k_eps)

    @torch.no_grad()
    def write_context(self, states: torch.Tensor, positions: torch.Tensor, locs: torch.Tensor,
                      meta: torch.Tensor) -> None:
        """The target's hidden states ``(tokens, n_layers * H)`` at ``positions``, stored at
        pool rows ``locs`` (``write_target_hidden_kv``, flashmap/sglang/model.py:700-744)."""
        self.write_rows(self.model.hidden_norm(F.linear(states, self.model.fc.weight)), positions, locs, meta)

    # -- the step --------------------------------------------------------------------

    @torch.no_grad()
    def __call__(self, anchors: torch.Tensor, anchor_positions: torch.Tensor, anchor_locs: torch.Tensor,
                 z: torch.Tensor, k_bufs: list[torch.Tensor], v_bufs: list[torch.Tensor], page_table: torch.Tensor,
                 n_cand: int = 1, meta: torch.Tensor | None = None, plan: torch.Tensor | None = None) -> torch.Tensor:
        """One draft for ``R`` requests: writes each anchor's context row at its position
        and pool row ``anchor_locs``, then returns the final AdaLN output ``(R * n_cand *
        block_size, dim)`` of ``n_cand`` blocks per request (candidate-major) at positions
        ``anchor + 1 ..``, all of a request's blocks attending to its pool rows
        ``page_table[r, :anchor + 1]``. ``z (R * n_cand * block_size, H)`` float32 is the
        starting noise in the folded space, one row per drafted slot."""
        model = self.model
        requests, k = anchors.shape[0], self.block
        blocks = requests * n_cand
        if z.shape != (blocks * k, self.noise_embed.shape[1]) or z.dtype != torch.float32:
            raise ValueError(f"the noise must be float32 ({blocks * k}, {self.noise_embed.shape[1]}), "
                             f"got {z.dtype} {tuple(z.shape)}")
        meta = self.pool_meta(k_bufs, v_bufs) if meta is None else meta
        anchor_rows = model.anchor_norm(model.anchor_proj(F.embedding(anchors, self.embed_weight)))
        self.write_rows(anchor_rows, anchor_positions, anchor_locs, meta)
        cache_seqlens = (anchor_positions + 1).to(torch.int32)
        if plan is None:
            plan = ops.attention_plan(cache_seqlens)
        # the blocks' rotary rows: slots at anchor + 1 .. anchor + K (flashmap/sglang/model.py:925-927)
        freqs = rope_freqs(anchor_positions[:, None] + 1 + torch.arange(k, device=anchors.device), self.head_dim,
                           self.cfg.rope_theta)
        if n_cand > 1:
            freqs = freqs.repeat_interleave(n_cand, dim=0)
        rope = ops.rope_from_table(freqs.reshape(blocks * k, self.head_dim // 2, 2).contiguous())
        z16, row_scale = ops.noise_rows(z, self.noise_eigvals, self.noise_eps, self.noise_gain)
        noise = F.linear(z16, self.noise_embed)
        mods = self.layer_mods
        first = mods[0][0] if mods else self.final_mod
        eps = model.layers[0].self_attn_adaln.eps if mods else model.final_adaln.eps
        hidden, h = ops.adaln_residual(self.first_hidden, noise, row_scale, (first[0], first[1]), eps,
                                       gate_per_row=True)
        heads, hd, tokens = self.heads, self.head_dim, blocks * k
        for i, layer in enumerate(model.layers):
            (_, _, g_self), (c_scale, c_shift, g_cross), (m_scale, m_shift, g_mlp) = mods[i]
            self_qn, self_kn, cross_qn = self.norms[i]
            attn = ops.block_self_attention(F.linear(h, self.self_qkv[i]).view(blocks, k, 3, heads, hd),
                                            self_qn, self_kn, rope, None, layer.self_attn.q_norm.eps)
            y = F.linear(attn.view(tokens, self.dim), layer.self_attn.o_proj.weight)
            hidden, h = ops.adaln_residual(hidden, y, g_self, (c_scale, c_shift), layer.cross_attn_adaln.eps,
                                           x_out=hidden)
            query = F.linear(h, layer.cross_attn.q_proj.weight).view(requests, n_cand * k, heads, hd)
            prologue = ops.Prologue(cross_qn, rope, None, layer.cross_attn.q_norm.eps)
            ctx = ops.block_attention_token_paged(query, k_bufs[i], v_bufs[i], cache_seqlens, page_table,
                                                  self.scale, prologue=prologue, plan=plan)
            y = F.linear(ctx.view(tokens, self.dim), layer.cross_attn.o_proj.weight)
            hidden, h = ops.adaln_residual(hidden, y, g_cross, (m_scale, m_shift), layer.mlp_adaln.eps, x_out=hidden)
            y = layer.mlp(h)
            if i + 1 < len(model.layers):
                nxt, eps = mods[i + 1][0][:2], model.layers[i + 1].self_attn_adaln.eps
            else:
                nxt, eps = self.final_mod, model.final_adaln.eps
            hidden, h = ops.adaln_residual(hidden, y, g_mlp, nxt, eps, x_out=hidden)
        return h

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """Draft-vocabulary logits (``head_logits``, the folded head,
        flashmap/sglang/model.py:511-513)."""
        return F.linear(hidden, self.head_weight, self.head_bias)

    def sample(self, hidden: torch.Tensor, temperatures: torch.Tensor, greedy: torch.Tensor,
               seed: torch.Tensor) -> torch.Tensor:
        """A token per row (target token ids): ``fm_sample_rows`` over the draft logits
        (``sample_rows``, flashmap/sglang/kernels.py:222-247, as the plugin's sampler calls
        it), mapped through ``hot_ids``."""
        idx = ops.sample_rows(self.logits(hidden).contiguous(), temperatures, greedy, seed)
        return idx if self.hot_ids is None else self.hot_ids[idx]
