"""The vLLM plugin's one-jump draft step on the gfx950 kernels, outside vLLM.

``DraftStep`` holds what the plugin's ``prepare`` computes once (flashmap/vllm/model.py:
461-608): the jump's AdaLN modulations, the folded noise read-out and the folded head
(``flashmap_amd.fold``), the constant first hidden row, one projection weight for every
layer's context keys/values and one per layer for the self-attention's q/k/v, and the
rotary table. A call runs the step of flashmap/vllm/model.py:779-903, 915-925 and
1039-1041 over vLLM-layout paged caches (one per DiT layer, ``(blocks, heads, page,
2 head_dim)``), every non-GEMM op on a kernel of this library:

1. the anchors' context rows: embedding -> ``anchor_proj`` -> ``anchor_norm`` -> one GEMM
   over all layers' K/V weights -> ``fm_write_context_kv`` (k-norm, RoPE, store);
2. the noise read-out: ``fm_noise_rows`` (row scales, z in bf16) -> the folded GEMM ->
   ``fm_adaln_residual`` (``first_hidden + scale * noise`` and the first layer's norm);
3. per DiT layer: the fused q/k/v GEMM -> ``fm_block_self_attention`` -> ``o_proj`` ->
   ``fm_adaln_residual`` -> ``q_proj`` -> ``fm_block_attn_paged`` with the query prologue
   fused and the step's shared plan -> ``o_proj`` -> ``fm_adaln_residual`` -> the MLP ->
   ``fm_adaln_residual`` (fused with the next layer's norm, or the final one);
4. the folded head GEMM and, for greedy drafts, ``fm_argmax_rows``.

GEMMs are hipBLASLt through torch. Inputs are explicit (what vLLM's forward context
supplies): anchors and their positions and slots, the noise, the caches, the block
table. bf16 only.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops
from .drafter import FlashMapDraftModel, jump_times
from .fold import fold_head, fold_noise

__all__ = ["DraftStep"]


def _rope_table(positions: int, head_dim: int, theta: float, device) -> torch.Tensor:
    """``(positions, head_dim / 2, [cos, sin])`` float32 (flashmap/vllm/kernels.py:26-33)."""
    inv_freq = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim)
    angles = torch.arange(positions, device=device).float()[:, None] * inv_freq
    return torch.stack([angles.cos(), angles.sin()], dim=-1).contiguous()


class DraftStep:
    """A prepared one-jump draft step (see the module docstring).

    ``model``: the drafter (bf16, on the GPU); ``embed_tokens`` / ``lm_head``: the
    target's ``(V, H)`` weights; ``max_model_len``: the longest context (rotary table
    rows); ``hot_ids``: the draft vocabulary's token ids when the drafter has a state
    vocabulary (``draft_ids``) or vLLM restricts it (``d2t``), else None."""

    @torch.no_grad()
    def __init__(self, model: FlashMapDraftModel, embed_tokens: torch.Tensor, lm_head: torch.Tensor,
                 max_model_len: int, hot_ids: torch.Tensor | None = None):
        cfg = model.config
        if model.dtype != torch.bfloat16:
            raise TypeError("the draft step's kernels are bf16: move the drafter to torch.bfloat16")
        self.model, self.cfg = model, cfg
        self.block = cfg.block_size
        self.heads = cfg.num_attention_heads
        self.head_dim = cfg.hidden_size // self.heads
        self.dim = cfg.hidden_size
        grid = cfg.jump_grids["1"]
        (s, t, _), = jump_times(grid)
        per_layer, final = model.time_conditioning(s, t)
        self.layer_mods = [tuple(tuple(m.reshape(-1) for m in mod) for mod in mods) for mods in per_layer]
        self.final_mod = tuple(m.reshape(-1) for m in final[:2])
        gate = model.noise_gate.float()
        self.noise_gain = float(gate * (t - s)) if cfg.noise_gate == "jump" else float(gate)
        self.hot_ids = hot_ids
        state_embed = embed_tokens[hot_ids] if (hot_ids is not None and cfg.state_vocab_size is not None) \
            else embed_tokens
        vocab = state_embed.shape[0]
        uniform = torch.full((1, vocab), 1.0 / vocab, device=state_embed.device, dtype=state_embed.dtype)
        self.first_hidden = model.x_embed(model.state_norm(uniform @ state_embed))[0].contiguous()
        self.noise_embed, self.noise_eigvals = fold_noise(state_embed, model.noise_norm.weight, model.x_embed.weight)
        self.noise_eps = model.noise_norm.eps
        self.embed_weight = embed_tokens
        layers = model.layers
        self.context_kv_weight = torch.cat([torch.cat([l.cross_attn.k_proj.weight, l.cross_attn.v_proj.weight])
                                            for l in layers])
        self.context_k_norm = torch.stack([l.cross_attn.k_norm.weight.float() for l in layers]).contiguous()
        self.k_eps = layers[0].cross_attn.k_norm.eps if len(layers) else 0.0
        self.self_qkv = [torch.cat([l.self_attn.q_proj.weight, l.self_attn.k_proj.weight, l.self_attn.v_proj.weight])
                         for l in layers]
        # the kernels read the q/k norm weights as float32: converted once here, not per call
        self.norms = [tuple(n.weight.float().contiguous() for n in (l.self_attn.q_norm, l.self_attn.k_norm,
                                                                     l.cross_attn.q_norm)) for l in layers]
        self.cos_sin = _rope_table(max_model_len + self.block + 1, self.head_dim, cfg.rope_theta,
                                   state_embed.device)
        self.rope = ops.rope_from_table(self.cos_sin)
        self.max_model_len = max_model_len
        self.head_weight, self.head_bias = fold_head(lm_head, model.head.weight, model.head.bias, hot_ids)
        self.scale = self.head_dim ** -0.5

    # -- the context -----------------------------------------------------------------

    @staticmethod
    def cache_layout(caches: list[torch.Tensor]):
        """``(base addresses (layers,) int64 on the device, (block, head, token, value)
        strides, page size)`` of per-layer vLLM caches ``(blocks, heads, page, 2D)``
        (flashmap/vllm/model.py:707-733)."""
        c0 = caches[0]
        if any(c.shape != c0.shape or c.stride() != c0.stride() or c.dtype != torch.bfloat16 for c in caches):
            raise ValueError("the layers' caches must be bf16 and share one shape and strides")
        bases = torch.tensor([c.data_ptr() for c in caches], dtype=torch.int64, device=c0.device)
        return bases, (c0.stride(0), c0.stride(1), c0.stride(2), c0.shape[-1] // 2), c0.shape[2]

    @torch.no_grad()
    def write_rows(self, rows: torch.Tensor, positions: torch.Tensor, slots: torch.Tensor, layout) -> None:
        """Keys and values of context rows ``(tokens, dim)`` for every layer: one GEMM over
        the layers' K/V weights and one writer launch (flashmap/vllm/model.py:735-777)."""
        kv = F.linear(rows, self.context_kv_weight)
        bases, strides, page = layout
        ops.write_context_kv(kv.view(rows.shape[0], len(self.model.layers), 2, self.heads, self.head_dim),
                             positions, slots, self.context_k_norm, self.rope, bases, strides, page, self.k_eps)

    @torch.no_grad()
    def write_context(self, states: torch.Tensor, positions: torch.Tensor, slots: torch.Tensor, layout) -> None:
        """The target's hidden states ``(tokens, n_layers * H)`` at ``positions``, stored
        at ``slots`` (precompute_and_store_context_kv, flashmap/vllm/model.py:759-767)."""
        self.write_rows(self.model.hidden_norm(F.linear(states, self.model.fc.weight)), positions, slots, layout)

    # -- the step --------------------------------------------------------------------

    @torch.no_grad()
    def __call__(self, anchors: torch.Tensor, anchor_positions: torch.Tensor, anchor_slots: torch.Tensor,
                 z: torch.Tensor, caches: list[torch.Tensor], block_table: torch.Tensor, layout=None,
                 plan: torch.Tensor | None = None) -> torch.Tensor:
        """One jump for ``B`` requests: writes each anchor's context row at its position /
        slot, then returns the final AdaLN output ``(B * block_size, dim)`` of the block
        rows at positions ``anchor + 1 ..`` attending to positions ``0 .. anchor``.
        ``z (B * block_size, H)`` float32 is the starting noise in the folded space."""
        model = self.model
        batch, k = anchors.shape[0], self.block
        layout = layout or self.cache_layout(caches)
        anchor_rows = model.anchor_norm(model.anchor_proj(F.embedding(anchors, self.embed_weight)))
        self.write_rows(anchor_rows, anchor_positions, anchor_slots, layout)
        seqused_k = (anchor_positions + 1).to(torch.int32)
        if plan is None:
            plan = ops.attention_plan(seqused_k)
        slot_positions = (anchor_positions[:, None] + 1 + torch.arange(k, device=anchors.device)).reshape(-1)
        cu = torch.arange(0, batch * k + 1, k, dtype=torch.int32, device=anchors.device)
        z16, row_scale = ops.noise_rows(z, self.noise_eigvals, self.noise_eps, self.noise_gain)
        noise = F.linear(z16, self.noise_embed)
        mods = self.layer_mods
        first = mods[0][0] if mods else self.final_mod
        hidden, h = ops.adaln_residual(self.first_hidden, noise, row_scale, (first[0], first[1]),
                                       model.layers[0].self_attn_adaln.eps if mods else model.final_adaln.eps,
                                       gate_per_row=True)
        heads, hd, tokens = self.heads, self.head_dim, batch * k
        for i, layer in enumerate(model.layers):
            (_, _, g_self), (c_scale, c_shift, g_cross), (m_scale, m_shift, g_mlp) = mods[i]
            self_qn, self_kn, cross_qn = self.norms[i]
            attn = ops.block_self_attention(F.linear(h, self.self_qkv[i]).view(batch, k, 3, heads, hd),
                                            self_qn, self_kn, self.rope, slot_positions, layer.self_attn.q_norm.eps)
            y = F.linear(attn.view(tokens, self.dim), layer.self_attn.o_proj.weight)
            hidden, h = ops.adaln_residual(hidden, y, g_self, (c_scale, c_shift), layer.cross_attn_adaln.eps,
                                           x_out=hidden)
            query = F.linear(h, layer.cross_attn.q_proj.weight).view(tokens, heads, hd)
            prologue = ops.Prologue(cross_qn, self.rope, slot_positions, layer.cross_attn.q_norm.eps)
            ctx = ops.block_attention_paged(query, caches[i], cu, seqused_k, block_table, k, self.max_model_len,
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
        """Draft logits over the draft vocabulary (compute_draft_logits,
        flashmap/vllm/model.py:1039-1041)."""
        return F.linear(hidden, self.head_weight, self.head_bias)

    def greedy(self, hidden: torch.Tensor) -> torch.Tensor:
        """Greedy draft tokens ``(rows,)`` as target token ids (``split_argmax`` on the
        folded logits, mapped through ``hot_ids``)."""
        idx = ops.argmax_rows(self.logits(hidden))
        return idx if self.hot_ids is None else self.hot_ids[idx]
