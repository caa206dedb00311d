"""The vLLM plugin's draft step on the gfx950 kernels, outside vLLM.

``DraftStep`` holds what the plugin's ``prepare`` computes once (flashmap/vllm/model.py:
455-585): every jump's AdaLN modulations and noise gain, the folded noise read-out and
the folded head (``flashmap_amd.fold``), the constant first hidden row, one projection
weight for every layer's context keys/values and one per layer for the self-attention's
q/k/v, the rotary table, and for drafts of several jumps the state vocabulary's embedding
and the head the state moves with. A call runs the step of flashmap/vllm/model.py:
779-1041 over vLLM-layout paged caches (one per DiT layer, ``(blocks, heads, page,
2 head_dim)``), every non-GEMM op of the DiT on a kernel of this library:

1. the anchors' context rows: embedding -> ``anchor_proj`` -> ``anchor_norm`` -> one GEMM
   over all layers' K/V weights -> ``fm_write_context_kv`` (k-norm, RoPE, store);
2. one jump: the noise read-out, ``fm_noise_rows`` (row scales, z in bf16) -> the folded
   GEMM -> ``fm_adaln_residual`` (``first_hidden + scale * noise`` and the first layer's
   norm); several jumps (Algorithm 8): per jump the state's embedding (its sharpened
   posterior and the state itself through the state vocabulary's embedding, one GEMM),
   ``x_embed`` and the first norm, and between jumps the state's move towards the
   softmax of the jump head's logits;
3. per DiT layer: the fused q/k/v GEMM -> ``fm_block_self_attention`` -> ``o_proj`` ->
   ``fm_adaln_residual`` -> ``q_proj`` -> ``fm_block_attn_paged`` with the query prologue
   fused and the step's shared plan -> ``o_proj`` -> ``fm_adaln_residual`` -> the MLP ->
   ``fm_adaln_residual`` (fused with the next layer's norm, or the final one);
4. the folded head GEMM and, for greedy drafts, ``fm_argmax_rows``.

GEMMs are hipBLASLt through torch. With several jumps, the state's softmaxes run as two
row kernels (``ops.state_embed_rows``: posterior and state as the embedding GEMM's bf16
operand; ``ops.state_update``: the jump head's softmax and the update, in place).
Inputs are explicit (what vLLM's forward context supplies): anchors and their positions
and slots, the noise, the caches, the block table. bf16 only.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops
from .drafter import FlashMapDraftModel, jump_times
from .fold import fold_head, fold_noise

__all__ = ["DraftStep"]


def _split_k(a: torch.Tensor, w: torch.Tensor, splits: int = 4) -> torch.Tensor:
    """``a @ w`` for a long reduction (the vocabulary) and few rows: ``splits`` slices of
    the reduction as one batched GEMM with float32 partials, summed, rounded once to bf16
    (hipBLASLt's single GEMM covers a quarter of the CUs at 1024 x 4096 outputs:
    measured 2.00 -> 1.06 ms at 1024 x 151936 x 4096). Falls back to ``a @ w`` when the
    reduction does not split evenly."""
    rows, k = a.shape
    if k % splits or a.stride(-1) != 1 or not w.is_contiguous():
        return a @ w
    part = k // splits
    a3 = a.view(rows, splits, part).transpose(0, 1)  # (splits, rows, part), rows keep their stride
    w3 = w.view(splits, part, w.shape[1])             # contiguous slices: no transposed operand
    return torch.bmm(a3, w3, out_dtype=torch.float32).sum(0).to(w.dtype)


def _rope_table(positions: int, head_dim: int, theta: float, device) -> torch.Tensor:
    """``(positions, head_dim / 2, [cos, sin])`` float32 (flashmap/vllm/kernels.py:26-33)."""
    inv_freq = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim)
    angles = torch.arange(positions, device=device).float()[:, None] * inv_freq
    return torch.stack([angles.cos(), angles.sin()], dim=-1).contiguous()


class DraftStep:
    """A prepared draft step of ``num_steps`` jumps (see the module docstring).

    ``model``: the drafter (bf16, on the GPU); ``embed_tokens`` / ``lm_head``: the
    target's ``(V, H)`` weights; ``max_model_len``: the longest context (rotary table
    rows); ``hot_ids``: the draft vocabulary's token ids when the drafter has a state
    vocabulary (``draft_ids``) or vLLM restricts it (``d2t``), else None; ``num_steps``:
    the jumps per draft (the drafter's configured count when None; the config's
    ``jump_grids`` must hold a grid for it)."""

    @torch.no_grad()
    def __init__(self, model: FlashMapDraftModel, embed_tokens: torch.Tensor, lm_head: torch.Tensor,
                 max_model_len: int, hot_ids: torch.Tensor | None = None, num_steps: int | None = None):
        cfg = model.config
        if model.dtype != torch.bfloat16:
            raise TypeError("the draft step's kernels are bf16: move the drafter to torch.bfloat16")
        self.model, self.cfg = model, cfg
        self.block = cfg.block_size
        self.heads = cfg.num_attention_heads
        self.head_dim = cfg.hidden_size // self.heads
        self.dim = cfg.hidden_size
        self.num_steps = int(num_steps or cfg.num_steps)
        grid = model._jump_grid(self.num_steps)
        self.time_grid = [float(v) for v in grid]
        self.jumps = jump_times(grid)
        # per jump: per layer ((scale, shift, gate) of self, cross, MLP), and the final (scale, shift)
        self.jump_mods, self.final_mods = [], []
        for s, t, _ in self.jumps:
            per_layer, final = model.time_conditioning(s, t)
            self.jump_mods.append([tuple(tuple(m.reshape(-1) for m in mod) for mod in mods) for mods in per_layer])
            self.final_mods.append(tuple(m.reshape(-1) for m in final[:2]))
        gate = model.noise_gate.float()
        self.noise_gains = ([float(gate * (t - s)) for s, t, _ in self.jumps] if cfg.noise_gate == "jump"
                            else [float(gate)] * self.num_steps)
        self.hot_ids = hot_ids
        state_vocab = hot_ids is not None and cfg.state_vocab_size is not None
        state_embed = embed_tokens[hot_ids] if state_vocab else embed_tokens
        vocab = state_embed.shape[0]
        uniform = torch.full((1, vocab), 1.0 / vocab, device=state_embed.device, dtype=state_embed.dtype)
        self.uniform_emb = uniform @ state_embed  # the embedding of a uniform posterior (1, H)
        self.first_hidden = model.x_embed(model.state_norm(self.uniform_emb))[0].contiguous()
        self.noise_embed, self.noise_eigvals = fold_noise(state_embed, model.noise_norm.weight, model.x_embed.weight)
        self.noise_eps = model.noise_norm.eps
        self.embed_weight = embed_tokens
        # several jumps read vocabulary-sized states through the state vocabulary's rows
        self.state_weight = state_embed if self.num_steps > 1 else None
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
        # between jumps the state moves with a distribution over its own vocabulary
        self.jump_head = None
        if self.num_steps > 1:
            self.jump_head = ((self.head_weight, self.head_bias) if hot_ids is None or state_vocab
                              else fold_head(lm_head, model.head.weight, model.head.bias))
        self.scale = self.head_dim ** -0.5

    @property
    def noise_columns(self) -> int:
        """Columns of the starting noise a call takes: the folded space's (``H``) for one
        jump, the state vocabulary's for several."""
        return self.noise_embed.shape[1] if self.num_steps == 1 else self.state_weight.shape[0]

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
        """One draft for ``B`` requests: writes each anchor's context row at its position /
        slot, then returns the final AdaLN output ``(B * block_size, dim)`` of the last
        jump for the block rows at positions ``anchor + 1 ..`` attending to positions ``0 ..
        anchor``. ``z (B * block_size, noise_columns)`` float32 is the starting noise: in
        the folded space for one jump, the vocabulary-sized state for several
        (flashmap/vllm/model.py:1016-1038)."""
        model = self.model
        batch, k = anchors.shape[0], self.block
        if z.shape != (batch * k, self.noise_columns) or z.dtype != torch.float32:
            raise ValueError(f"the noise must be float32 ({batch * k}, {self.noise_columns}), "
                             f"got {z.dtype} {tuple(z.shape)}")
        layout = layout or self.cache_layout(caches)
        anchor_rows = model.anchor_norm(model.anchor_proj(F.embedding(anchors, self.embed_weight)))
        self.write_rows(anchor_rows, anchor_positions, anchor_slots, layout)
        seqused_k = (anchor_positions + 1).to(torch.int32)
        if plan is None:
            plan = ops.attention_plan(seqused_k)
        attend = (caches, block_table, seqused_k, plan,
                  (anchor_positions[:, None] + 1 + torch.arange(k, device=anchors.device)).reshape(-1),
                  torch.arange(0, batch * k + 1, k, dtype=torch.int32, device=anchors.device))
        if self.num_steps == 1:
            z16, row_scale = ops.noise_rows(z, self.noise_eigvals, self.noise_eps, self.noise_gains[0])
            noise = F.linear(z16, self.noise_embed)
            eps = model.layers[0].self_attn_adaln.eps if len(model.layers) else model.final_adaln.eps
            hidden, h = ops.adaln_residual(self.first_hidden, noise, row_scale, self._first_norm(0), eps,
                                           gate_per_row=True)
            return self._dit(hidden, h, 0, attend)
        # The state is updated in place between the jumps: a copy of the caller's noise,
        # in rows padded to a multiple of 4 values (the row kernels' 16-byte chunks).
        vocab = z.shape[1]
        state = torch.empty(z.shape[0], -(-vocab // 4) * 4, dtype=torch.float32, device=z.device)[:, :vocab]
        state.copy_(z)
        h = None
        for step, (start, _, end) in enumerate(self.jumps):
            hidden = self._embed_state(state, step)
            eps = model.layers[0].self_attn_adaln.eps if len(model.layers) else model.final_adaln.eps
            h = ops.adaln_residual(hidden, None, None, self._first_norm(step), eps)[1]
            h = self._dit(hidden, h, step, attend)
            if step + 1 < self.num_steps:
                ops.state_update(state, F.linear(h, *self.jump_head), start, end)
        return h

    def _first_norm(self, step: int):
        """``(scale, shift)`` of the norm the jump's DiT input goes through first."""
        mods = self.jump_mods[step]
        return mods[0][0][:2] if mods else self.final_mods[step]

    def _embed_state(self, state: torch.Tensor, step: int) -> torch.Tensor:
        """``x_embed`` of the state's embedding at jump ``step``: its posterior sharpened
        by the jump's start time and the state itself, both through the state
        vocabulary's embedding in one GEMM, normed and mixed with the jump's noise gain
        (flashmap/vllm/model.py:944-956)."""
        model, weight = self.model, self.state_weight
        start = self.time_grid[step]
        evidence = start / max(1.0 - start, 1e-3) ** 2
        if start == 0.0:  # evidence 0: the posterior is uniform, its embedding one row
            state_emb = _split_k(ops.state_embed_rows(state, 0.0, posterior=False), weight)
            posterior = model.state_norm(self.uniform_emb)  # (1, H), every row's
        else:
            both = ops.state_embed_rows(state, evidence) @ weight
            posterior_emb, state_emb = both.split(state.shape[0])
            posterior = model.state_norm(posterior_emb)
        embedded = (self.noise_gains[step] * model.noise_norm(state_emb)).to(weight.dtype)
        return model.x_embed(posterior + embedded)

    def _dit(self, hidden: torch.Tensor, h: torch.Tensor, step: int, attend) -> torch.Tensor:
        """The DiT layers of jump ``step`` from the residual stream ``hidden`` and its
        first norm ``h``; returns the final AdaLN output (flashmap/vllm/model.py:813-903)."""
        model = self.model
        caches, block_table, seqused_k, plan, slot_positions, cu = attend
        heads, hd, tokens = self.heads, self.head_dim, hidden.shape[0]
        batch, k = seqused_k.shape[0], self.block
        mods = self.jump_mods[step]
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
                nxt, eps = self.final_mods[step], model.final_adaln.eps
            hidden, h = ops.adaln_residual(hidden, y, g_mlp, nxt, eps, x_out=hidden)
        return h  # without layers: the first norm, which is then the final one

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """Draft logits over the draft vocabulary (compute_draft_logits,
        flashmap/vllm/model.py:1039-1041)."""
        return F.linear(hidden, self.head_weight, self.head_bias)

    def greedy(self, hidden: torch.Tensor) -> torch.Tensor:
        """Greedy draft tokens ``(rows,)`` as target token ids (``split_argmax`` on the
        folded logits, mapped through ``hot_ids``)."""
        idx = ops.argmax_rows(self.logits(hidden))
        return idx if self.hot_ids is None else self.hot_ids[idx]
